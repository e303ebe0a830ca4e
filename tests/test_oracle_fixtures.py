"""Pin the CPU oracle against the reference's own golden data (MuJoCo fp64 and the reference's fp32
CUDA outputs). Fixture semantics: MuJoCo records kinematics/bias/qacc of the PRE-step state after
mj_step, so per-state quantities at index t belong to qpos/qvel[t-1] (t >= 1)."""
import os

import numpy as np
import pytest

from conftest import GOLDEN, relerr_rows, load_contact_validate


def _prestep(ref):
    sel = ref["sel"]
    prev = np.maximum(sel - 1, 0)
    return ref["qpos"][prev], ref["qvel"][prev]


def test_fk_matches_mujoco(orc, ref_traj):
    q, _ = _prestep(ref_traj)
    xp, xq, xi = orc.fk(q, dtype=np.float64)
    assert np.abs(xp - ref_traj["xpos"]).max() < 1e-8
    assert np.abs(xq - ref_traj["xquat"]).max() < 1e-8
    assert np.abs(xi - ref_traj["xipos"]).max() < 1e-8


def test_fk_doubling_matches_recursion(orc, ref_traj):
    """FK by ancestor doubling with fp64 compositions (the GPU's form) against the reference's root
    -> leaf recursion in fp32: the same transforms, so the frames agree to fp32 rounding (a wrong
    ancestor, composition order or missing round would be off by O(1)); and both are pinned to
    MuJoCo's fp64 frames at the same fp32 tolerance."""
    rng = np.random.default_rng(3)
    q = np.tile(ref_traj["qpos"][0], (512, 1)).astype(np.float64)
    q[:, 7:] += rng.uniform(-1.0, 1.0, (512, 29))
    q[:, 3:7] = rng.normal(size=(512, 4)); q[:, 3:7] /= np.linalg.norm(q[:, 3:7], axis=1, keepdims=True)
    q = q.astype(np.float32)
    a = orc.fk(q, dtype=np.float32)
    b = orc.fk_recursive(q)
    for x, y in zip(a, b):
        assert np.abs(x - y).max() <= 2e-6, np.abs(x - y).max()
    assert not all(np.array_equal(x, y) for x, y in zip(a, b))   # the associations do differ
    # fp64 compositions: closer to the fp64 frames than the fp32 recursion (an fp32 composition in
    # either association fails this: its mean position error is 8e-8 against 4.8e-8)
    c = orc.fk(q.astype(np.float64), dtype=np.float64)
    ea, eb = np.abs(a[0] - c[0]).mean(), np.abs(b[0] - c[0]).mean()
    assert ea < 0.7 * eb, (ea, eb)
    assert np.abs(a[0] - c[0]).max() < 1e-6 and np.abs(a[2] - c[2]).max() < 1e-6
    qf, _ = _prestep(ref_traj)
    for f in (lambda: orc.fk(qf.astype(np.float32), dtype=np.float32), lambda: orc.fk_recursive(qf.astype(np.float32))):
        xp, xq, xi = f()
        assert np.abs(xp - ref_traj["xpos"]).max() < 1e-5
        assert np.abs(xq - ref_traj["xquat"]).max() < 1e-5


def test_bias_matches_mujoco(orc, ref_traj):
    q, v = _prestep(ref_traj)
    _, b = orc.bias(q, v, dtype=np.float64)
    assert relerr_rows(b, ref_traj["qfrc_bias"]).max() < 1e-8


def test_mass_matrix_matches_mujoco(orc, ref_traj):
    M = orc.mass(ref_traj["qpos"][0], dtype=np.float64)[0]
    assert np.linalg.norm(M - ref_traj["M0"]) / np.linalg.norm(ref_traj["M0"]) < 1e-9
    assert np.array_equal(M, M.T)


def test_smooth_qacc_matches_mujoco(orc, ref_traj):
    q, v = _prestep(ref_traj)
    qa, nc = orc.qacc(q, v, dtype=np.float64)          # no actuation, plain factor, lifted base
    assert (nc == 0).all()
    assert relerr_rows(qa, ref_traj["qacc"]).max() < 1e-8
    qa32, _ = orc.qacc(q, v, dtype=np.float32)
    assert relerr_rows(qa32, ref_traj["qacc"]).max() < 2e-5   # fp32 path accuracy (~2.5e-6)


def test_smooth_trajectory_matches_mujoco(orc, ref_traj):
    qo, _ = orc.smooth_traj(ref_traj["qpos_init"], ref_traj["qvel_init"], 300, dtype=np.float64)
    assert np.abs(qo - ref_traj["qpos"]).max() < 1e-8


def test_fp32_trajectory_matches_reference_cuda(orc, ref_traj):
    """300-step fp32 smooth trajectory vs the reference's fp32 CUDA dumps (dense and ABA)."""
    qo, _ = orc.smooth_traj(ref_traj["qpos_init"], ref_traj["qvel_init"], 300, dtype=np.float32)
    for name in ("cuda_traj.bin", "aba_traj.bin"):
        ct = np.fromfile(os.path.join(GOLDEN, name), np.float32).reshape(301, 36)
        assert np.abs(qo - ct).max() < 2e-6, name
    assert np.abs(qo - ref_traj["qpos"]).max() < 2e-6


def test_fp32_bias_and_mass_match_reference_cuda(orc, ref_traj):
    cf = np.fromfile(os.path.join(GOLDEN, "cuda_fk.bin"), np.float32)
    Mc, bc, qc = cf[:1225].reshape(35, 35), cf[1225:1260], cf[1260:1295]
    init = np.fromfile(os.path.join(GOLDEN, "init_state.bin"), np.float64)
    q0, v0 = init[:36], init[36:]
    assert np.array_equal(q0, ref_traj["qpos_init"]) and np.array_equal(v0, ref_traj["qvel_init"])
    _, b = orc.bias(q0, v0, dtype=np.float32)
    assert relerr_rows(b, bc[None]).max() < 1e-6
    M = orc.mass(q0, dtype=np.float32)[0]
    assert np.linalg.norm(M - Mc) / np.linalg.norm(Mc) < 1e-6
    qa, _ = orc.qacc(q0, v0, dtype=np.float32)
    assert relerr_rows(qa, qc[None]).max() < 1e-5
    aq = np.fromfile(os.path.join(GOLDEN, "aba_qacc.bin"), np.float32)
    assert relerr_rows(qa, aq[None]).max() < 1e-5


def test_implicit_pd_matches_mujoco_implicitfast(orc):
    """Damped (M + dt*kd) factor + clamped PD torque vs MuJoCo implicitfast (contacts off)."""
    d = np.load(os.path.join(GOLDEN, "implicit_ref.npz"), allow_pickle=False)
    Bdt = d["Bdiag"] * float(d["dt"])
    qo, vo = orc.implicit_traj(d["qpos"][0], d["qvel"][0], Bdt, d["targets"], dtype=np.float64)
    # single-step qvel error (the reference's gate: scripts/test_implicit.py:53-55, < 1e-3;
    # measured 1.32e-5 on its fp32 CUDA path)
    assert np.abs(vo[1] - d["qvel"][1]).max() < 1e-3
    assert np.abs(vo[1] - d["qvel"][1]).max() < 5e-5
    assert np.abs(qo[-1] - d["qpos"][-1]).max() < 2e-3
    # fp32 oracle vs the reference's fp32 CUDA replay of the same controls
    raw = open(os.path.join(GOLDEN, "implicit_cuda.bin"), "rb").read()
    n = int(np.frombuffer(raw[:4], np.int32)[0])
    cq = np.frombuffer(raw[4:4 + (n + 1) * 36 * 4], np.float32).reshape(n + 1, 36)
    cv = np.frombuffer(raw[4 + (n + 1) * 36 * 4:], np.float32).reshape(n + 1, 35)
    qo32, vo32 = orc.implicit_traj(d["qpos"][0], d["qvel"][0], Bdt.astype(np.float32), d["targets"],
                                   dtype=np.float32)
    # fp32 rounding of a stiff (kp=500) step: ~1e-5 abs on |qvel| ~ 2.5, i.e. qacc relerr ~1e-5
    assert np.abs(vo32[1] - cv[1]).max() < 5e-5
    assert np.abs(qo32[1] - cq[1]).max() < 1e-7
    # implicit_cuda.bin drifts from MuJoCo from step ~2 on (3.2e-4 qpos at step 100, a stale run);
    # the fp32 oracle instead tracks MuJoCo over all 100 steps
    assert np.abs(cq[-1] - d["qpos"][-1]).max() > 1e-4
    assert np.abs(qo32 - d["qpos"]).max() < 1e-6


@pytest.mark.parametrize("dtype,tol", [(np.float64, 1.2e-5), (np.float32, 1.5e-5)])
def test_contact_qacc_matches_mujoco(orc, dtype, tol):
    """Pure foot-ground states vs MuJoCo's converged qacc at 2000 PGS sweeps (reference worst
    relerr 2.24e-5 on its fp32 CUDA path, DEVLOG.md:250-251; this fp32 path composes FK's first
    three doubling rounds in fp64, the feet's frames among them, and measures 1.27e-5)."""
    cv = load_contact_validate()
    qa, nc = orc.qacc(cv["qpos"], cv["qvel"], pgs=2000, mu=0.6, dtype=dtype)
    assert list(nc) == [0, 0, 0, 8, 8, 4, 8, 8, 8]
    rel = relerr_rows(qa, cv["qacc"])
    assert rel.max() < tol, rel
    # 8 unconverged sweeps stay far from MuJoCo: the sweep count is a real parameter
    qa8, _ = orc.qacc(cv["qpos"], cv["qvel"], pgs=8, mu=0.6, dtype=dtype)
    assert relerr_rows(qa8, cv["qacc"])[3:].min() > 1e-3


def test_kernel_association_matches_reference_association(orc):
    """The oracle's default association (the GPU kernel's: single-RHS contact solves, butterfly PGS
    row sums and reward totals) against the reference's serial association: the same algorithm, so
    per-state qacc agrees within the fp32 gate (1e-5, src/test_envqacc.cu:74-90) on the gate's
    state family, and both meet the MuJoCo contact fixture's bound; the two are not bit-identical
    (the switch takes effect)."""
    from conftest import envqacc_states
    qp, qv = envqacc_states(2048)
    Bdt = orc.bdt(np.float32)
    dev, nd = orc.qacc(qp, qv, Bdt=Bdt, pgs=8, mu=0.6, dtype=np.float32, threads=8)
    with orc.reference_order():
        ref, nr = orc.qacc(qp, qv, Bdt=Bdt, pgs=8, mu=0.6, dtype=np.float32, threads=8)
    assert np.array_equal(nd, nr) and (nd > 0).mean() > 0.5
    rel = relerr_rows(dev, ref)
    assert rel.max() <= 1e-5, rel.max()
    assert not np.array_equal(dev, ref)
    cv = load_contact_validate()
    for ctx in (None, orc.reference_order()):
        if ctx:
            ctx.__enter__()
        qa, _ = orc.qacc(cv["qpos"], cv["qvel"], pgs=2000, mu=0.6, dtype=np.float32)
        if ctx:
            ctx.__exit__(None, None, None)
        assert relerr_rows(qa, cv["qacc"]).max() < 1.5e-5
