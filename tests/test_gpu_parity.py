"""GPU parity of the HIP path (libg1env.so, called through its C ABI) against the CPU oracle and the
reference's fixtures. The physics is compared bit for bit with the fp32 oracle in the kernel's
summation association, and within the reference's fp32 gate (per-state ||a-b||/||b|| <= 1e-5,
src/test_envqacc.cu:74-90) with the oracle in the reference's association; MuJoCo contact fixture
<= 2e-5 at 2000 PGS sweeps (reference worst 2.24e-5). The policy MLP runs on MFMA and is compared
within 1e-5."""
import ctypes

import numpy as np
import pytest

from conftest import relerr_rows, load_contact_validate, envqacc_states

pytestmark = pytest.mark.gpu

TOL_QACC = 1e-5


@pytest.fixture(scope="module")
def g1():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import g1env
    return g1env


def _dev(x, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def gpu_qacc(g1, qpos, qvel, tau=None, damped=True, contact=True, pgs=8, mu=0.6):
    import torch
    n = qpos.shape[0]
    q = _dev(qpos.astype(np.float32)); v = _dev(qvel.astype(np.float32))
    t = _dev(np.zeros((n, 35), np.float32) if tau is None else tau.astype(np.float32))
    out = torch.zeros(n, 35, device="cuda"); nc = torch.zeros(n, dtype=torch.int32, device="cuda")
    g1.lib.g1_probe_qacc(n, g1.dev_ptr(q), g1.dev_ptr(v), g1.dev_ptr(t), int(damped), int(contact), pgs, mu, g1.dev_ptr(out),
                          g1.dev_ptr(nc))
    torch.cuda.synchronize()
    return out.cpu().numpy(), nc.cpu().numpy()


def test_env_qacc_gate_states(g1, orc):
    """Teacher-forced env_qacc (zero torque, implicit kd damping, pgs=8) on the reference gate's
    random-state family, worst per-state relerr <= 1e-5."""
    qp, qv = envqacc_states(4096)
    Bdt = orc.bdt(np.float32)
    ref, nref = orc.qacc(qp, qv, Bdt=Bdt, pgs=8, mu=0.6, dtype=np.float32, threads=8)
    out, nc = gpu_qacc(g1, qp, qv, pgs=8, mu=0.6)
    assert np.array_equal(nc, nref)
    assert (nref > 0).mean() > 0.5     # the family exercises the contact path
    rel = relerr_rows(out, ref)
    with orc.reference_order():
        ref_r, _ = orc.qacc(qp, qv, Bdt=Bdt, pgs=8, mu=0.6, dtype=np.float32, threads=8)
    rel_r = relerr_rows(out, ref_r)
    print(f"env_qacc gate: worst relerr {rel.max():.3e} (states differing: {int((rel > 0).sum())}); against the "
          f"reference association {rel_r.max():.3e}; contact share {(nref>0).mean():.2f}")
    assert np.array_equal(out, ref)           # the kernel's association: bit for bit
    assert rel_r.max() <= TOL_QACC            # the reference's association: the fp32 gate


@pytest.mark.parametrize("mu", [0.6, 1.0])
def test_contact_config_states(g1, orc, mu):
    """Config 2 at its full size: 8192 states with 0..8 penetrating spheres and tangential foot
    velocity, pgs=8."""
    import configs
    qp, qv, k = configs.config2(lambda q: orc.fk(q, dtype=np.float64), n=8192)
    Bdt = orc.bdt(np.float32)
    ref, nref = orc.qacc(qp, qv, Bdt=Bdt, pgs=8, mu=mu, dtype=np.float32, threads=8)
    out, nc = gpu_qacc(g1, qp, qv, pgs=8, mu=mu)
    assert np.array_equal(nc, nref)
    assert set(np.unique(nref)) >= {0, 4, 8}
    with orc.reference_order():
        ref_r, _ = orc.qacc(qp, qv, Bdt=Bdt, pgs=8, mu=mu, dtype=np.float32, threads=8)
    rel, rel_r = relerr_rows(out, ref), relerr_rows(out, ref_r)
    print(f"config2 mu={mu}: worst relerr {rel.max():.3e}, reference association {rel_r.max():.3e}; "
          f"ncon hist {np.bincount(nref, minlength=9)}")
    assert np.array_equal(out, ref)
    assert rel_r.max() <= TOL_QACC


def test_smooth_qacc_config0(g1, orc):
    """No contact, plain M^-1 (tau - bias) on config-0 states: vs fp32 and fp64 oracle."""
    import configs
    qp, qv, tau = configs.config0()
    ref32, _ = orc.qacc(qp, qv, tau=tau, pgs=0, dtype=np.float32, contact=False)
    ref64, _ = orc.qacc(qp, qv, tau=tau, pgs=0, dtype=np.float64, contact=False)
    out, _ = gpu_qacc(g1, qp, qv, tau=tau, damped=False, contact=False)
    r32, r64 = relerr_rows(out, ref32), relerr_rows(out, ref64)
    print(f"config0 smooth: vs fp32 oracle {r32.max():.3e}, vs fp64 oracle {r64.max():.3e}")
    assert r32.max() <= TOL_QACC
    assert r64.max() <= 1e-4


def test_config1_dynamics_teacher_forced_and_drift(g1, orc):
    """Config 1 (no contact, plain factor, tau held, semi-implicit Euler) through g1_dynamics_bench:
    one substep from the oracle's own state is bit-identical in qpos, qvel and qacc; a 100-substep
    free run (tau held, 0.2 s) stays within fp32 drift of the oracle's free run. Full-range random
    torques on the unconstrained floating robot make explicit Euler diverge within ~50 substeps
    (fp32 and fp64 alike), so the runs use the env's velocity guard (NaN -> 0, clamp +-50)."""
    import torch
    import configs
    qp, qv, tau = configs.config0(seed=7, n=512)
    qp, qv, tau = (x.astype(np.float32) for x in (qp, qv, tau))

    def gpu(nsub):
        dq, dv, dt_ = _dev(qp), _dev(qv), _dev(tau)
        qa = torch.zeros(qp.shape[0], 35, device="cuda")
        nc = torch.zeros(qp.shape[0], dtype=torch.int32, device="cuda")
        g1.lib.g1_dynamics_bench(qp.shape[0], g1.dev_ptr(dq), g1.dev_ptr(dv), g1.dev_ptr(dt_), nsub, 0, 0, 1, 8, 0.6,
                                  g1.dev_ptr(qa), g1.dev_ptr(nc))
        torch.cuda.synchronize()
        return dq.cpu().numpy(), dv.cpu().numpy(), qa.cpu().numpy()

    gq, gv, ga = gpu(1)
    oq, ov, oa, _ = orc.dynamics(qp, qv, tau, nsub=1, guard=True, threads=8)
    assert np.array_equal(ga, oa) and np.array_equal(gv, ov) and np.array_equal(gq, oq)
    gq, gv, ga = gpu(100)
    oq, ov, oa, _ = orc.dynamics(qp, qv, tau, nsub=100, guard=True, threads=8)
    dq_, dv_ = relerr_rows(gq, oq), relerr_rows(gv, ov)
    print(f"config1: 1 substep bit-identical; 100-substep free-run drift qpos {dq_.max():.2e}, qvel {dv_.max():.2e}")
    assert np.isfinite(gq).all() and dq_.max() <= 1e-4


@pytest.mark.timeout(600)
def test_config1_full_workload_teacher_forced(g1, orc):
    """Config 1 at its full size: N=8192 worlds, 1000 substeps with tau resampled every 10 (100
    draws), no contact, plain factor, the env's velocity guard, on the GPU's own running state. At
    10 sampled segments the first substep runs as its own launch over all worlds, and 1024 sampled
    worlds are compared with the oracle's substep from the same pre-substep state: qacc, qvel and
    qpos bit for bit. The 1000-substep run stays finite."""
    import torch
    import configs
    N, seg, nseg = 8192, 10, 100
    rng = np.random.default_rng(17)
    qp, qv = configs.perturbed_states(N, rng)
    dq, dv = _dev(qp.astype(np.float32)), _dev(qv.astype(np.float32))
    qa = torch.zeros(N, 35, device="cuda")
    nc = torch.zeros(N, dtype=torch.int32, device="cuda")
    sel = np.sort(rng.choice(N, 1024, replace=False))
    check = {0, 11, 23, 37, 50, 64, 77, 88, 95, 99}

    def run(dt_, nsub):
        g1.lib.g1_dynamics_bench(N, g1.dev_ptr(dq), g1.dev_ptr(dv), g1.dev_ptr(dt_), nsub, 0, 0, 1, 8, 0.6,
                                  g1.dev_ptr(qa), g1.dev_ptr(nc))

    for k in range(nseg):
        tau = configs.random_torque(N, rng).astype(np.float32)
        dt_ = _dev(tau)
        if k in check:
            torch.cuda.synchronize()
            q0, v0 = dq.cpu().numpy()[sel], dv.cpu().numpy()[sel]
            run(dt_, 1)
            torch.cuda.synchronize()
            oq, ov, oa, _ = orc.dynamics(q0, v0, tau[sel], nsub=1, guard=True, threads=8)
            gq, gv, ga = dq.cpu().numpy()[sel], dv.cpu().numpy()[sel], qa.cpu().numpy()[sel]
            assert np.array_equal(ga, oa) and np.array_equal(gv, ov) and np.array_equal(gq, oq), k
            run(dt_, seg - 1)
        else:
            run(dt_, seg)
    torch.cuda.synchronize()
    assert np.isfinite(dq.cpu().numpy()).all() and np.isfinite(dv.cpu().numpy()).all()
    print(f"config1 N={N}: 1000 substeps; {len(check)} sampled substeps x {sel.size} worlds bit-identical")


def test_smooth_qacc_vs_mujoco(g1, ref_traj):
    sel = ref_traj["sel"]
    prev = np.maximum(sel - 1, 0)
    out, nc = gpu_qacc(g1, ref_traj["qpos"][prev], ref_traj["qvel"][prev], damped=False, contact=True)
    assert (nc == 0).all()
    rel = relerr_rows(out, ref_traj["qacc"])
    print(f"smooth qacc vs MuJoCo: worst {rel.max():.3e}")
    assert rel.max() <= 2e-5


def test_contact_vs_mujoco_fixture(g1, orc):
    """Pure foot-ground states at 2000 PGS sweeps vs MuJoCo's qacc (reference worst 2.24e-5 on its fp32
    CUDA path; the fp32 oracle with fp64 FK compositions gives 1.28e-5)."""
    cv = load_contact_validate()
    out, nc = gpu_qacc(g1, cv["qpos"], cv["qvel"], damped=False, contact=True, pgs=2000, mu=0.6)
    assert list(nc) == [0, 0, 0, 8, 8, 4, 8, 8, 8]
    rel = relerr_rows(out, cv["qacc"])
    print("contact_validate relerr:", np.array2string(rel, precision=2))
    assert rel.max() <= 2e-5
    ref32, _ = orc.qacc(cv["qpos"], cv["qvel"], pgs=2000, mu=0.6, dtype=np.float32)
    assert np.array_equal(out, ref32)


def test_substep_teacher_forced(g1, orc):
    """One env substep (FK -> clamped PD -> qacc -> guarded Euler -> integration) on config-2 states
    with random PD targets: qacc relerr <= 1e-5, next-state deviation at rounding level."""
    import torch
    import configs
    import g1_model as gm
    qp, qv, _ = configs.config2(lambda q: orc.fk(q, dtype=np.float64), n=1024, seed=5)
    rng = np.random.default_rng(6)
    tg = (gm.qpos_stand[7:][None] + 0.5 * rng.uniform(-1, 1, (1024, 29))).astype(np.float32)
    tg = np.clip(tg, gm.act_ctrl_lo, gm.act_ctrl_hi).astype(np.float32)
    q1, v1, qa_ref, n_ref = orc.substep(qp, qv, tg, pgs=8, mu=0.6, threads=8)
    q = _dev(qp.astype(np.float32)); v = _dev(qv.astype(np.float32)); t = _dev(tg)
    qa = torch.zeros(1024, 35, device="cuda"); nc = torch.zeros(1024, dtype=torch.int32, device="cuda")
    g1.lib.g1_probe_substep(1024, g1.dev_ptr(q), g1.dev_ptr(v), g1.dev_ptr(t), 1, 8, 0.6, g1.dev_ptr(qa), g1.dev_ptr(nc))
    torch.cuda.synchronize()
    assert np.array_equal(nc.cpu().numpy(), n_ref)
    rel = relerr_rows(qa.cpu().numpy(), qa_ref)
    dq = np.abs(q.cpu().numpy() - q1).max()
    dv = relerr_rows(v.cpu().numpy(), v1).max()
    print(f"substep: qacc worst {rel.max():.3e}, qpos maxabs {dq:.3e}, qvel worst rel {dv:.3e}")
    assert np.array_equal(qa.cpu().numpy(), qa_ref)
    assert np.array_equal(q.cpu().numpy(), q1) and np.array_equal(v.cpu().numpy(), v1)


@pytest.mark.parametrize("hidden,act", [((256, 256), 0), ((512, 512, 256), 1), ((48, 32), 1), ((80, 144), 0),
                                        ((512,), 0), ((512, 512, 512), 1)])
def test_policy_mlp(g1, orc, hidden, act):
    """Policy MLP on fp32 MFMA (k_policy) vs the oracle's serial MLP: config 3 and config 4 shapes,
    and narrow, single-layer and widest shapes, whose LDS tile pitch is set by the observation
    staging, the head's split-K partial tiles or the widest layer respectively."""
    import torch
    import configs
    rng = np.random.default_rng(3)
    W = configs.policy_init(rng, hidden=hidden)
    n = 1000
    x = np.clip(rng.normal(0, 1.5, (n, 100)), -10, 10).astype(np.float32)
    mu_ref, _, v_ref = orc.mlp(W, x, hidden=hidden, act=act)
    mu = torch.zeros(n, 29, device="cuda"); v = torch.zeros(n, device="cuda")
    h = np.asarray(hidden, np.int32)
    dW, dx = _dev(W), _dev(x)          # keep the device tensors alive across the call
    rc = g1.lib.g1_probe_policy(n, len(hidden), h.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), act,
                                 g1.dev_ptr(dW), g1.dev_ptr(dx), g1.dev_ptr(mu), g1.dev_ptr(v))
    assert rc == 0
    mu = mu.cpu().numpy(); v = v.cpu().numpy()
    rm = relerr_rows(mu, mu_ref)
    # the value head is one scalar per world, often near zero: relative error over the batch
    rv = np.linalg.norm(v - v_ref) / np.linalg.norm(v_ref)
    print(f"mlp {hidden}: mu worst relerr {rm.max():.3e}, v batch relerr {rv:.3e}")
    assert rm.max() <= 1e-5 and rv <= 1e-5


def test_philox_known_answers(g1):
    """Philox4x32-10 known-answer vectors (Random123 kat_vectors)."""
    import torch
    ctr = np.array([[0, 0, 0, 0], [0xffffffff] * 4, [0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344]], np.uint32)
    keys = [(0, 0), (0xffffffff, 0xffffffff), (0xa4093822, 0x299f31d0)]
    want = [[0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8], [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd],
            [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]]
    for i, (k0, k1) in enumerate(keys):
        c = torch.from_numpy(ctr[i:i + 1].view(np.int32).copy()).cuda()
        o = torch.zeros(4, dtype=torch.int32, device="cuda")
        g1.lib.g1_probe_philox(1, g1.dev_ptr(c), g1.dev_ptr(o), k0, k1)
        got = o.cpu().numpy().view(np.uint32)
        assert list(got) == want[i], [hex(x) for x in got]


def test_reciprocal_and_quotient_are_ieee(g1):
    """The physics kernel's short-chain rcp_rn / div_rn against IEEE fp32 division (numpy rounds
    float32 division correctly): every mantissa of the binades 2^-12 .. 2^12 (the divisors of the
    path: pivots, D, A_ii, impedances) and random numerators of both signs over 2^-40 .. 2^40."""
    import torch
    m = np.arange(1 << 23, dtype=np.uint32)
    bs = np.concatenate([((np.uint32(e + 127) << np.uint32(23)) | m).view(np.float32) for e in range(-12, 13, 4)])
    rng = np.random.default_rng(5)
    a = (rng.uniform(1, 2, bs.size) * np.exp2(rng.integers(-40, 41, bs.size)) *
         rng.choice([-1, 1], bs.size)).astype(np.float32)
    a[::9] = (bs[::9] * rng.integers(-1000, 1001, bs[::9].size)).astype(np.float32)   # exact quotients
    da, db = torch.from_numpy(a).cuda(), torch.from_numpy(bs).cuda()
    r, q = torch.zeros_like(db), torch.zeros_like(db)
    g1.lib.g1_probe_divide(bs.size, g1.dev_ptr(da), g1.dev_ptr(db), g1.dev_ptr(r), g1.dev_ptr(q))
    r, q = r.cpu().numpy(), q.cpu().numpy()
    with np.errstate(all="ignore"):
        assert np.array_equal(r.view(np.uint32), (np.float32(1) / bs).view(np.uint32))
        assert np.array_equal(q.view(np.uint32), (a / bs).view(np.uint32))


def test_pivot_sqrt_exhaustive(g1):
    """The Cholesky pivots' short square root against the IEEE one (numpy rounds float32 sqrt
    correctly) for EVERY float from 2^-96 up to the largest finite, plus +0 and +inf; inputs are
    generated on the device, 2^25 bit patterns per launch."""
    import torch
    lo = int(np.float32(2.0 ** -96).view(np.uint32))
    hi = int(np.float32(np.inf).view(np.uint32))
    chunk = 1 << 25
    for start in range(lo, hi + 1, chunk):
        stop = min(start + chunk, hi + 1)
        dx = torch.arange(start, stop, dtype=torch.int32, device="cuda").view(torch.float32)
        out = torch.empty_like(dx)
        g1.lib.g1_probe_sqrt(dx.numel(), g1.dev_ptr(dx), g1.dev_ptr(out))
        want = np.sqrt(np.arange(start, stop, dtype=np.uint32).view(np.float32))
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)), hex(start)
    z = torch.zeros(64, device="cuda")
    out = torch.full_like(z, 1.0)
    g1.lib.g1_probe_sqrt(z.numel(), g1.dev_ptr(z), g1.dev_ptr(out))
    assert np.array_equal(out.cpu().numpy().view(np.uint32), np.zeros(64, np.uint32))


def test_small_angle_sincos_exhaustive(g1, orc):
    """The free joint's quaternion update takes sin/cos of the half rotation per substep on a short
    fp64 path for |x| <= 1/8: bit-identical to the oracle's fp64 libm rounded once for EVERY float
    of that range (both signs, zeros and denormals), plus the library path just above it."""
    import torch
    lim = int(np.float32(0.125).view(np.uint32))          # bit patterns 0 .. lim are 0 .. 1/8
    chunk = 1 << 25
    for start in range(0, lim + 1, chunk):
        bits = np.arange(start, min(start + chunk, lim + 1), dtype=np.uint32)
        for sign in (np.uint32(0), np.uint32(0x80000000)):
            x = (bits | sign).view(np.float32)
            dx = torch.from_numpy(x).cuda()
            ds, dc = torch.zeros_like(dx), torch.zeros_like(dx)
            g1.lib.g1_probe_sincos(x.size, g1.dev_ptr(dx), g1.dev_ptr(ds), g1.dev_ptr(dc))
            want_s, want_c = orc.sincos(x)
            assert np.array_equal(ds.cpu().numpy().view(np.uint32), want_s.view(np.uint32)), start
            assert np.array_equal(dc.cpu().numpy().view(np.uint32), want_c.view(np.uint32)), start
    x = np.nextafter(np.float32(0.125), np.float32(1), dtype=np.float32) * np.arange(1, 1001, dtype=np.float32)
    dx = torch.from_numpy(x).cuda()
    ds, dc = torch.zeros_like(dx), torch.zeros_like(dx)
    g1.lib.g1_probe_sincos(x.size, g1.dev_ptr(dx), g1.dev_ptr(ds), g1.dev_ptr(dc))
    want_s, want_c = orc.sincos(x)
    assert np.array_equal(ds.cpu().numpy(), want_s) and np.array_equal(dc.cpu().numpy(), want_c)


def test_hinge_sincos_exhaustive(g1, orc):
    """The FK's hinge half-angle path (fp64 reduction by pi/2 and Taylor series, each result
    rounded once; the library above |x| = 4): bit-identical to the oracle's fp64 libm sin and cos
    rounded once for EVERY float with |x| <= 4 (both signs, zeros and denormals; hinge half-angles,
    joint ranges included), plus a sample of larger ones. The free joint's path takes the same
    function above 1/8, checked over 1/8 < |x| <= 4 through its own probe."""
    import torch
    hi = int(np.float32(4.0).view(np.uint32))
    lo8 = int(np.float32(0.125).view(np.uint32)) + 1
    chunk = 1 << 25
    for probe, lo in ((g1.lib.g1_probe_sincos_hinge, 0), (g1.lib.g1_probe_sincos, lo8)):
        for start in range(lo, hi + 1, chunk):
            bits = np.arange(start, min(start + chunk, hi + 1), dtype=np.uint32)
            for sign in (np.uint32(0), np.uint32(0x80000000)):
                x = (bits | sign).view(np.float32)
                dx = torch.from_numpy(x).cuda()
                ds, dc = torch.zeros_like(dx), torch.zeros_like(dx)
                probe(x.size, g1.dev_ptr(dx), g1.dev_ptr(ds), g1.dev_ptr(dc))
                want_s, want_c = orc.sincos(x)
                assert np.array_equal(ds.cpu().numpy().view(np.uint32), want_s.view(np.uint32)), start
                assert np.array_equal(dc.cpu().numpy().view(np.uint32), want_c.view(np.uint32)), start
    rng = np.random.default_rng(7)
    x = (rng.uniform(4, 1e4, 1 << 22) * rng.choice([-1, 1], 1 << 22)).astype(np.float32)
    dx = torch.from_numpy(x).cuda()
    for probe in (g1.lib.g1_probe_sincos_hinge, g1.lib.g1_probe_sincos):
        ds, dc = torch.zeros_like(dx), torch.zeros_like(dx)
        probe(x.size, g1.dev_ptr(dx), g1.dev_ptr(ds), g1.dev_ptr(dc))
        want_s, want_c = orc.sincos(x)
        assert np.array_equal(ds.cpu().numpy(), want_s) and np.array_equal(dc.cpu().numpy(), want_c)


def test_policy_mlp_trained_checkpoint(g1, orc):
    """The reference's trained policy (converted checkpoint) through the MFMA policy kernel vs the
    oracle's fp32 MLP on normalised observations of perturbed stand states."""
    import os
    import torch
    from conftest import ROOT
    tp = np.load(os.path.join(ROOT, "g1.cu_amd", "data", "trained_policy_finish_best.npz"))
    W = tp["W"]
    rng = np.random.default_rng(9)
    n = 1000
    x = np.clip(rng.normal(0, 1.0, (n, 100)), -10, 10).astype(np.float32)
    mu_ref, _, v_ref = orc.mlp(W, x, hidden=(256, 256), act=0)
    mu = torch.zeros(n, 29, device="cuda"); v = torch.zeros(n, device="cuda")
    h = np.asarray((256, 256), np.int32)
    dW, dx = _dev(W), _dev(x)
    rc = g1.lib.g1_probe_policy(n, 2, h.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), 0, g1.dev_ptr(dW), g1.dev_ptr(dx),
                                 g1.dev_ptr(mu), g1.dev_ptr(v))
    assert rc == 0
    rm = relerr_rows(mu.cpu().numpy(), mu_ref)
    rv = np.linalg.norm(v.cpu().numpy() - v_ref) / np.linalg.norm(v_ref)
    print(f"trained mlp: mu worst relerr {rm.max():.3e}, v batch relerr {rv:.3e}")
    assert rm.max() <= 1e-5 and rv <= 1e-5
