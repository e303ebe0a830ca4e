"""Fused rollout through the reference's ABI (g1_rollout / g1_rollout_ex into torch buffers) against
the CPU oracle on identical states and pre-generated noise.

Teacher forcing: every control step starts the oracle from the GPU's own state before that step
(g1_env_get_state). The policy runs on MFMA and its outputs are held to the per-step bound (A/LP/V
within 1e-5, O bitwise). The physics of a step is driven by the GPU's own actions and compared bit
for bit with the oracle in the kernel's summation association: qpos, qvel, reward, done, step
counters and reset states.
"""
import os

import numpy as np
import pytest

from conftest import relerr_rows

pytestmark = pytest.mark.gpu

NTHREADS = min(16, os.cpu_count() or 1)
TOL = 1e-5


@pytest.fixture(scope="module")
def g1():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import g1env
    return g1env


def _dev(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _rollout(g1, env, W, mean, var, H, act_noise=None, reset_noise=None):
    import torch
    tr = g1.Trajectory(H, env.N)
    keep = [_dev(x) for x in (W, mean, var)]
    an = None if act_noise is None else _dev(act_noise)
    rn = None if reset_noise is None else _dev(reset_noise)
    tr.run(env, *keep, act_noise=an, reset_noise=rn)
    torch.cuda.synchronize()
    assert env.check() == 0
    return tr.numpy()


def _setup(N, H, seed, hidden=(256, 256)):
    import configs
    rng = np.random.default_rng(seed)
    qp, qv, pa, steps = configs.reset_states(rng, N)
    W = configs.policy_init(rng, hidden=hidden)
    mean = rng.normal(0, 0.1, 100).astype(np.float32)
    var = rng.uniform(0.5, 2.0, 100).astype(np.float32)
    an, rn = configs.rollout_noise(rng, H, N)
    return qp, qv, pa, steps, W, mean, var, an, rn


def _targets(act):
    """PD joint targets of a control step, as the kernel forms them: clamp(stand + 0.5 a)."""
    import g1_model as gm
    t = np.float32(0.5) * act.astype(np.float32) + gm.qpos_stand[7:].astype(np.float32)
    return np.clip(t, gm.act_ctrl_lo, gm.act_ctrl_hi).astype(np.float32)


def _substeps_teacher_forced(g1, orc, qp, qv, act, S, pgs=8, mu=0.6):
    """S env substeps of the given worlds, each started on the GPU from the GPU's state after the
    previous one and compared with the oracle's substep from that same state. Returns the worst
    per-world relerr of qacc, qpos and qvel over the substeps."""
    import torch
    n = qp.shape[0]
    tg = _targets(act)
    dq, dv, dt_ = _dev(qp), _dev(qv), _dev(tg)
    qa = torch.zeros(n, 35, device="cuda")
    nc = torch.zeros(n, dtype=torch.int32, device="cuda")
    worst = np.zeros(3)
    for _ in range(S):
        q0, v0 = dq.cpu().numpy(), dv.cpu().numpy()
        g1.lib.g1_probe_substep(n, g1.dev_ptr(dq), g1.dev_ptr(dv), g1.dev_ptr(dt_), 1, pgs, mu, g1.dev_ptr(qa),
                                g1.dev_ptr(nc))
        torch.cuda.synchronize()
        q1, v1, qa_ref, n_ref = orc.substep(q0, v0, tg, pgs=pgs, mu=mu, threads=NTHREADS)
        assert np.array_equal(nc.cpu().numpy(), n_ref)
        worst = np.maximum(worst, [relerr_rows(qa.cpu().numpy(), qa_ref).max(),
                                   relerr_rows(dq.cpu().numpy(), q1).max(), relerr_rows(dv.cpu().numpy(), v1).max()])
    return worst


def _teacher_forced_run(g1, orc, env, n_check, H, W, mean, var, hidden, act, seed, substep_probe=()):
    """H control steps of g1_rollout_ex (one launch sequence per step, H = 1) over all env.N worlds;
    the first n_check worlds of every step are compared with the oracle from the GPU's pre-step
    state. Returns per-step worst errors."""
    import configs
    rng = np.random.default_rng(seed)
    rows = []
    for t in range(H):
        an, rn = configs.rollout_noise(rng, 1, env.N)
        pre = env.get_state()
        out = _rollout(g1, env, W, mean, var, 1, an, rn)
        post = env.get_state()
        k = slice(0, n_check)
        pq, pv, ppa, pst = (np.ascontiguousarray(x[k]) for x in pre)
        # policy outputs from the same pre-step state
        ref = orc.rollout(pq.copy(), pv.copy(), ppa.copy(), pst.copy(), W, mean, var,
                          np.ascontiguousarray(an[:, k]), np.ascontiguousarray(rn[:, k]), 1, hidden=hidden, act=act,
                          threads=NTHREADS)
        O, A, LP, V, R, D = (out[f][0, k] for f in ("O", "A", "LP", "V", "R", "D"))
        assert np.array_equal(O, ref["O"][0]), t
        e_a = relerr_rows(A, ref["A"][0]).max()
        e_lp = (np.abs(LP - ref["LP"][0]) / np.abs(ref["LP"][0])).max()
        e_v = np.abs(V - ref["V"][0]).max() / max(1.0, np.abs(ref["V"][0]).max())
        # the step's physics driven by the GPU's actions, from the same pre-step state
        oq, ov, opa, ost = pq.copy(), pv.copy(), ppa.copy(), pst.copy()
        rr, dd = orc.env_advance(oq, ov, opa, ost, A, np.ascontiguousarray(rn[0, k]), threads=NTHREADS)
        assert np.array_equal(D, dd), t
        e_r = (np.abs(R - rr) / np.maximum(1.0, np.abs(rr))).max()
        gq, gv, gpa, gst = (x[k] for x in post)
        assert np.array_equal(gst, ost) and np.array_equal(gpa, opa), t
        e_q, e_qd = relerr_rows(gq, oq).max(), relerr_rows(gv, ov).max()
        nbit = int((~(gq == oq).all(1) | ~(gv == ov).all(1) | (R != rr)).sum())
        row = dict(t=t, A=e_a, LP=e_lp, V=e_v, R=e_r, qpos=e_q, qvel=e_qd, done=int(dd.sum()), nbit=nbit)
        if t in substep_probe:
            sel = np.arange(0, n_check, max(1, n_check // 256))[:256]
            row["substep"] = _substeps_teacher_forced(g1, orc, pq[sel], pv[sel], A[sel], env.S)
        rows.append(row)
        print(f"step {t:2d}: A {e_a:.1e} LP {e_lp:.1e} V {e_v:.1e} R {e_r:.1e} qpos {e_q:.1e} qvel {e_qd:.1e} "
              f"done {row['done']} worlds not bit-identical {nbit}" + (f" | substeps qacc/qpos/qvel {np.array2string(row['substep'], precision=1)}"
                                        if "substep" in row else ""), flush=True)
    return rows


def _assert_rows(rows):
    """Policy outputs within 1e-5; the physics of each step (driven by the GPU's own actions) and
    its reward bit for bit."""
    for r in rows:
        for key in ("A", "LP", "V"):
            assert r[key] <= TOL, (r["t"], key, r[key])
        assert r["nbit"] == 0, (r["t"], r["nbit"], r["qpos"], r["qvel"], r["R"])
        if "substep" in r:
            assert (r["substep"] == 0).all(), (r["t"], r["substep"])


@pytest.mark.timeout(900)
def test_rollout_teacher_forced_config3(g1, orc):
    """Config 3 (N=8192, H=32, S=10, pgs=8, 100-256-256 tanh) step by step against the oracle, with
    the per-substep qacc/qpos/qvel of 256 sampled worlds teacher-forced on steps 0, 15 and 31."""
    N, H = 8192, 32
    qp, qv, pa, steps, W, mean, var, _, _ = _setup(N, 1, 41)
    with g1.Env(N, substeps=10, pgs_iters=8, seed=1) as env:
        env.set_state(qp, qv, pa, steps)
        rows = _teacher_forced_run(g1, orc, env, N, H, W, mean, var, (256, 256), 0, seed=42,
                                   substep_probe=(0, 15, 31))
    assert sum(r["done"] for r in rows) > 0     # the done path and auto-reset ran
    _assert_rows(rows)


@pytest.mark.timeout(1200)
def test_rollout_teacher_forced_config4_slice(g1, orc):
    """Config 4 (N=131072, 100-512-512-256 ELU through g1_env_set_policy): the first 8192 worlds of
    every control step of the full-size launch against the oracle."""
    import configs
    N, H, n = 131072, 32, 8192
    rng = np.random.default_rng(51)
    qp, qv, pa, steps = configs.reset_states(rng, N)
    W = configs.policy_init(rng, hidden=(512, 512, 256))
    mean = rng.normal(0, 0.1, 100).astype(np.float32)
    var = rng.uniform(0.5, 2.0, 100).astype(np.float32)
    with g1.Env(N, substeps=10, pgs_iters=8, seed=1) as env:
        env.set_policy((512, 512, 256), 1)
        assert env.policy_params() == W.size
        env.set_state(qp, qv, pa, steps)
        rows = _teacher_forced_run(g1, orc, env, n, H, W, mean, var, (512, 512, 256), 1, seed=52,
                                   substep_probe=(31,))
    _assert_rows(rows)


@pytest.mark.parametrize("hidden,act", [((48, 32), 1), ((80, 144), 0), ((100, 60), 0), ((256, 17), 1),
                                        ((512, 512, 256), 1), ((300,), 0), ((64, 48, 32), 1), ((512, 70), 0)])
def test_rollout_teacher_forced_one_launch_shapes(g1, orc, hidden, act):
    """The one-launch rollout's policy tiles on shapes other than 256-256: two layers of at most 256
    run on the register-resident tile at 256-256 with zero padding (widths that are and are not
    multiples of 16, ELU and tanh); one to three layers of up to 512 on the wide tile (activations
    staged in global memory, output tiles padded to multiples of 64 rows), config 4's 512-512-256
    ELU among them. N=512, 4 control steps against the oracle."""
    import configs
    N, H = 512, 4
    rng = np.random.default_rng(61)
    qp, qv, pa, steps = configs.reset_states(rng, N)
    W = configs.policy_init(rng, hidden=hidden)
    mean = rng.normal(0, 0.1, 100).astype(np.float32)
    var = rng.uniform(0.5, 2.0, 100).astype(np.float32)
    with g1.Env(N, substeps=10, pgs_iters=8, seed=1) as env:
        env.set_policy(hidden, act)
        assert env.policy_params() == W.size
        assert env.set_fused(True)          # the shape runs in the one-launch form
        env.set_state(qp, qv, pa, steps)
        rows = _teacher_forced_run(g1, orc, env, N, H, W, mean, var, hidden, act, seed=62)
    _assert_rows(rows)


def test_one_launch_rollout_equals_step_by_step(g1):
    """The one-launch rollout cuts a control step into work items by the work per wave: at the
    benchmark's shape (N=8192, H=32) every step but the last is one item and the last two (6 and 4
    substeps); a launch per control step (H=1) cuts each step into 3,3,2,2. From its second step on
    the one launch also pairs each tile's worlds by their contact state (the worlds in contact at
    the end of the previous step share waves), while a launch's first step keeps the fixed pairs.
    Item boundaries only hand a pair's state over, which two worlds share a wave changes no result,
    and the policy tiles are the same, so one H=32 launch equals 32 H=1 launches bit for bit: every
    trajectory output, the bootstrap value and the final state (with timeouts and auto-resets inside
    the horizon)."""
    N, H = 8192, 32
    qp, qv, pa, steps, W, mean, var, an, rn = _setup(N, H, 71)
    steps[::7] = 969 + np.arange(steps[::7].size) % 31   # timeouts and auto-resets inside the horizon
    with g1.Env(N, substeps=10, pgs_iters=8, seed=1) as env:
        env.set_state(qp, qv, pa, steps)
        one = _rollout(g1, env, W, mean, var, H, an, rn)
        end_one = env.get_state()
        env.set_state(qp, qv, pa, steps)
        parts = [_rollout(g1, env, W, mean, var, 1, an[t:t + 1], rn[t:t + 1]) for t in range(H)]
        end_steps = env.get_state()
    for f in ("O", "A", "LP", "V", "R", "D"):
        step_by_step = np.concatenate([q[f] for q in parts], 0)
        assert np.array_equal(one[f].view(np.uint32), step_by_step.view(np.uint32)), f
    assert np.array_equal(one["Vlast"].view(np.uint32), parts[-1]["Vlast"].view(np.uint32))
    for a, b in zip(end_one, end_steps):
        assert np.array_equal(a, b)
    assert one["D"].sum() > 0


@pytest.mark.parametrize("fences,fused", [(0, True), (1, True), (0, False), (1, False)])
def test_rollout_matches_oracle_free_run(g1, orc, fences, fused):
    """A short rollout (N=96, H=3) with no teacher forcing: every output equals the oracle's own
    rollout within the per-step bound, in both rollout forms (one persistent launch, or policy and
    physics launches per control step), through the L2 state hand-over (fences=0) and through the
    agent-scope fence hand-over that the work queue falls back to off the round-robin placement."""
    N, H = 96, 3
    qp, qv, pa, steps, W, mean, var, an, rn = _setup(N, H, 11)
    with g1.Env(N, substeps=10, pgs_iters=8, seed=1) as env:
        env.set_handover(fences)
        assert env.set_fused(fused) == fused
        env.set_state(qp, qv, pa, steps)
        out = _rollout(g1, env, W, mean, var, H, an, rn)
        g = env.get_state()
    o = [x.copy() for x in (qp, qv, pa, steps)]
    ref = orc.rollout(*o, W, mean, var, an, rn, H, threads=NTHREADS)
    assert np.array_equal(out["O"][0], ref["O"][0]) and np.array_equal(out["D"], ref["D"])
    for t in range(H):
        assert relerr_rows(out["A"][t], ref["A"][t]).max() <= TOL
        assert (np.abs(out["R"][t] - ref["R"][t]) / np.maximum(1, np.abs(ref["R"][t]))).max() <= TOL
        assert relerr_rows(out["O"][t], ref["O"][t]).max() <= TOL
    assert relerr_rows(g.qpos, o[0]).max() <= TOL and relerr_rows(g.qvel, o[1]).max() <= TOL
    assert np.array_equal(g.steps, o[3])


def test_termination_reset_and_reward_closed_form(g1, orc):
    """Each termination cause on the GPU: the 1000th step, the finish line, a pelvis below 0.45 m and
    a 70 degree roll, beside alive worlds whose reward is known in closed form
    (tests/reward_spec.py, src/g1_env.cu:164-211). A zero policy with log_std 0 makes the sampled
    action equal the injected noise, so each world takes its planned action. R and D equal the
    oracle's and the closed form; finished worlds restart bit for bit at the stand pose + 0.05 x
    their injected reset noise."""
    import g1_model as gm
    import configs
    from reward_spec import crafted_cases, reward_spec
    c = crafted_cases()
    n = len(c["steps"])
    W = np.zeros_like(configs.policy_init(np.random.default_rng(0)))   # mu = 0, V = 0, log_std = 0
    mean, var = np.zeros(100, np.float32), np.ones(100, np.float32)
    an = c["act"][None].copy()
    rn = np.random.default_rng(3).uniform(-1, 1, (1, n, 29)).astype(np.float32)
    with g1.Env(n, substeps=10, pgs_iters=8, seed=2) as env:
        env.set_state(c["qp"], c["qv"], c["pa"], c["steps"])
        out = _rollout(g1, env, W, mean, var, 1, an, rn)
        post = env.get_state()
    assert np.array_equal(out["A"][0], c["act"])
    o = [x.copy() for x in (c["qp"], c["qv"], c["pa"], c["steps"])]
    ref = orc.rollout(*o, W, mean, var, an, rn, 1)
    R, D = out["R"][0], out["D"][0]
    assert np.array_equal(D, ref["D"][0])
    assert (np.abs(R - ref["R"][0]) <= 1e-6 + np.spacing(np.abs(ref["R"][0]).astype(np.float32))).all()
    live = D == 0
    r_spec, d_spec = reward_spec(post.qpos, post.qvel, c["qv"][:, 0], c["act"], c["pa"], c["steps"])
    assert list(D.astype(bool)) == [False] * 8 + [True] * 4 and list(d_spec[live]) == [False] * 8
    assert (np.abs(R[live] - r_spec[live]) <= 1e-6).all(), np.abs(R[live] - r_spec[live])
    assert R[c["names"].index("fallen (height)")] == -5.0 and R[c["names"].index("fallen (tilt)")] == -5.0
    assert R[c["names"].index("finish line")] > 50.0
    for w in np.flatnonzero(~live):
        exp = gm.qpos_stand.astype(np.float32).copy()
        exp[7:] += np.float32(0.05) * rn[0, w]
        assert np.array_equal(post.qpos[w], exp) and not post.qvel[w].any() and not post.prev_act[w].any()
        assert post.steps[w] == 0
        assert np.array_equal(post.qpos[w], o[0][w])
    for w in np.flatnonzero(live):
        assert post.steps[w] == c["steps"][w] + 1 and np.array_equal(post.prev_act[w], c["act"][w])
    print("rewards:", dict(zip(c["names"], np.round(R, 5).tolist())))


def test_rollout_deterministic_and_world_independent(g1):
    """Bitwise run-to-run determinism and identical worlds -> identical outputs (the reference's
    race check, src/sim_aba.cu:77-80, tests/test_aba.py:43-53), and the library-noise path: equal
    seeds agree bitwise, different seeds differ."""
    N, H = 64, 3
    qp, qv, pa, steps, W, mean, var, an, rn = _setup(N, H, 12)
    qp[:] = qp[0]
    qv[:] = qv[0]
    an[:] = an[:, :1]
    rn[:] = rn[:, :1]
    outs = []
    for _ in range(2):
        with g1.Env(N, substeps=10, pgs_iters=8, seed=7) as env:
            env.set_state(qp, qv, pa, steps)
            outs.append(_rollout(g1, env, W, mean, var, H, an, rn))
    for f in g1.Trajectory.FIELDS:
        a, b = outs[0][f], outs[1][f]
        assert np.array_equal(a, b), f
        flat = a.reshape(a.shape[0], N, -1) if a.ndim >= 2 else a.reshape(1, N, 1)
        assert np.array_equal(flat, np.broadcast_to(flat[:, :1], flat.shape)), f
    res = []
    for seed in (5, 5, 6):
        with g1.Env(N, substeps=10, pgs_iters=8, seed=seed) as env:
            env.set_state(qp, qv, pa, steps)
            res.append(_rollout(g1, env, W, mean, var, H))
    assert all(np.array_equal(res[0][f], res[1][f]) for f in g1.Trajectory.FIELDS)
    assert not np.array_equal(res[0]["A"], res[2]["A"])


def test_zero_horizon_writes_only_the_bootstrap_value(g1, orc):
    """H = 0 runs no control step and still writes the bootstrap value, as the reference's k_rollout
    does (its loop runs zero times); the state stays as it was."""
    N = 64
    qp, qv, pa, steps, W, mean, var, _, _ = _setup(N, 1, 13)
    import torch
    with g1.Env(N, substeps=10, pgs_iters=8, seed=1) as env:
        env.set_state(qp, qv, pa, steps)
        tr = g1.Trajectory(1, N)
        for t in tr.tensors():
            t.fill_(7.0)
        keep = [_dev(x) for x in (W, mean, var)]
        g1.lib.g1_rollout(env.h, 0, *[g1.dev_ptr(t) for t in (*keep, *tr.tensors())])
        torch.cuda.synchronize()
        st = env.get_state()
        env.bench_phys(0)
        assert env.check() == 0
        st2 = env.get_state()
    out = tr.numpy()
    ref = orc.rollout(qp.copy(), qv.copy(), pa.copy(), steps.copy(), W, mean, var,
                      np.zeros((0, N, 29), np.float32), np.zeros((0, N, 29), np.float32), 0)
    assert all((out[f] == 7.0).all() for f in ("O", "A", "LP", "V", "R", "D"))
    assert np.abs(out["Vlast"] - ref["Vlast"]).max() <= TOL * max(1.0, np.abs(ref["Vlast"]).max())
    for a, b, c in zip(st, st2, (qp, qv, pa, steps)):
        assert np.array_equal(a, c) and np.array_equal(b, c)


def test_reference_driver_call_sequence(g1):
    """The reference driver's call sequence, through this build's own driver (g1.cu_amd/ppo_train.py):
    create -> reset -> g1_rollout into torch buffers -> renormalise -> host-step evaluation; every
    buffer is written in place."""
    import torch
    import ppo_train
    N, H = 256, 16
    with g1.Env(N, substeps=10, pgs_iters=8, seed=1) as env:
        obs0 = env.reset()
        assert obs0.shape == (N, 100) and np.isfinite(obs0).all()
        policy = ppo_train.GaussianPolicy().cuda()
        stats = ppo_train.ObsStats(100, "cuda")
        traj = g1.Trajectory(H, N)
        for t in traj.tensors():
            t.fill_(float("nan"))
        nobs = ppo_train.collect(env, policy, stats, traj)
        for t in traj.tensors():
            assert torch.isfinite(t).all()
        assert torch.isfinite(nobs).all() and float(nobs.abs().max()) <= 10.0
        D = traj.D.cpu().numpy()
        assert set(np.unique(D)) <= {0.0, 1.0}
        assert (traj.O[0, :, 96] == np.float32(0.8)).all() and (traj.O[0, :, 97:] == 0).all()
        ev = ppo_train.evaluate(env, policy, stats, steps=5)
        assert np.isfinite(ev["forward_m"]) and 0 <= ev["fall_rate"] <= 1
        qall = env.qpos_all()
        q0 = np.zeros(36, np.float32)
        g1.lib.g1_env_qpos(env.h, g1.host_ptr(q0))
        assert np.array_equal(q0, qall[0])
        assert env.check() == 0


def test_host_step_matches_oracle(g1, orc):
    """g1_env_step (host buffers) vs the oracle's control step on the same state and actions: done
    flags, rewards and the observations of worlds still running bit for bit (a finished world
    restarts with library noise, which the oracle does not draw)."""
    N = 128
    with g1.Env(N, substeps=10, pgs_iters=8, seed=3) as env:
        obs = env.reset()
        qp, qv, pa, st = env.get_state()
        assert np.array_equal(obs, orc.obs(qp, qv, pa))
        act = np.random.default_rng(4).normal(0, 0.3, (N, 29)).astype(np.float32)
        obs1, rew, done = env.step(act)
    oq, ov, opa, ost = qp.copy(), qv.copy(), pa.copy(), st.copy()
    rr, dd = orc.env_advance(oq, ov, opa, ost, act, np.zeros((N, 29), np.float32), threads=NTHREADS)
    live = dd == 0
    assert np.array_equal(done, dd) and np.array_equal(rew, rr)
    assert np.array_equal(obs1[live], orc.obs(oq, ov, opa)[live])


@pytest.mark.parametrize("path", ["host_step", "rollout"])
def test_velocity_guard_nan_inf_and_clamp(g1, orc, path):
    """The env's velocity guard (src/g1_env.cu:154-160: a non-finite velocity becomes 0, then the
    clamp to +-50) on the GPU, against the oracle bit for bit: worlds start with NaN, +-inf and
    +-1e4 velocities on base and hinge dofs (g1_env_set_state) beside ordinary ones and take one
    control step through the host-step path (k_physics) or a one-step rollout (k_rollout). The
    reference's comparison clamps let NaN through everywhere else, as the kernels do: a NaN hinge
    velocity makes that step's reward NaN and, in the rollout, the world's observation and action
    NaN; the guard leaves every velocity finite and within +-50."""
    import configs
    N = 64
    rng = np.random.default_rng(91)
    qp, qv, pa, steps = configs.reset_states(rng, N)
    qv = rng.normal(0, 0.5, (N, 35)).astype(np.float32)
    bad = {0: (3, np.nan), 1: (20, np.nan), 2: (0, 1e4), 3: (12, -1e4), 4: (30, np.inf), 5: (5, -np.inf),
           6: (7, 60.0), 7: (1, -1e4)}
    for w, (d, v) in bad.items():
        qv[w, d] = v
    act = rng.normal(0, 0.3, (N, 29)).astype(np.float32)
    rn = rng.uniform(-1, 1, (1, N, 29)).astype(np.float32)
    W = configs.policy_init(rng)
    mean, var = np.zeros(100, np.float32), np.ones(100, np.float32)
    with g1.Env(N, substeps=10, pgs_iters=8, seed=4) as env:
        env.set_state(qp, qv, pa, steps)
        if path == "host_step":
            _, rew, done = env.step(act)
            A = act
        else:
            out = _rollout(g1, env, W, mean, var, 1, act[None], rn)
            rew, done, A = out["R"][0], out["D"][0], out["A"][0]
        post = env.get_state()
    if path == "rollout":
        # the policy from the same state: a NaN velocity makes the observation and every action of
        # its world NaN; an infinite or huge one is clamped to +-10 after normalisation
        ref = orc.rollout(*(x.copy() for x in (qp, qv, pa, steps)), W, mean, var, act[None], rn, 1,
                          threads=NTHREADS)
        assert np.array_equal(out["O"][0], ref["O"][0], equal_nan=True)
        assert np.isnan(A[:2]).all() and np.isnan(ref["A"][0][:2]).all() and np.isfinite(A[2:]).all()
        assert relerr_rows(A[2:], ref["A"][0][2:]).max() <= TOL
    # the step's physics driven by the GPU's actions, from the same state; the host step resets
    # finished worlds with the library's own noise (counter 0: no reset or step before it)
    import philox_np
    o = [x.copy() for x in (qp, qv, pa, steps)]
    rst = rn[0] if path == "rollout" else philox_np.uniform_pm1(4, np.arange(N), 0, philox_np.STREAM_RESET)
    rr, dd = orc.env_advance(*o, A, rst, threads=NTHREADS)
    print(f"{path}: rewards of the guarded worlds {rew[:8]}; oracle {rr[:8]}")
    assert np.array_equal(done, dd) and np.array_equal(rew, rr, equal_nan=True)
    for a, b in zip(post, o):
        assert np.array_equal(a, b, equal_nan=a.dtype.kind == "f")
    assert np.isfinite(post.qvel).all() and np.abs(post.qvel).max() <= 50.0
    assert np.isnan(rew[1]) and not np.isnan(rew[8:]).any() and dd[:8].any()


def test_work_queue_matches_small_launch(g1):
    """The physics work queue at scale: a rollout over 8193 worlds (many work items per wave, state
    handed between waves, an odd last pair) gives each of its first 97 worlds bit for bit the
    trajectory those worlds get in a 97-world launch (world 96 then has no partner); the same with
    the fence hand-over."""
    H, N, n = 3, 8193, 97
    qp, qv, pa, steps, W, mean, var, an, rn = _setup(N, H, 21)
    runs = []
    for m, fences in ((N, 0), (n, 0), (N, 1)):
        with g1.Env(m, substeps=10, pgs_iters=8, seed=1) as env:
            env.set_handover(fences)
            env.set_state(qp[:m], qv[:m], pa[:m], steps[:m])
            out = _rollout(g1, env, W, mean, var, H, np.ascontiguousarray(an[:, :m]), np.ascontiguousarray(rn[:, :m]))
            runs.append((out, env.get_state()))
    (big, big_state), (small, small_state), (fen, fen_state) = runs
    for f in g1.Trajectory.FIELDS:
        k = (slice(None), slice(0, n)) if big[f].ndim >= 2 else slice(0, n)
        assert np.array_equal(big[f][k], small[f]), f
        assert np.array_equal(big[f], fen[f]), f
    for b, s, e in zip(big_state, small_state, fen_state):
        assert np.array_equal(b[:n], s) and np.array_equal(b, e)
    assert not np.array_equal(big_state[0], qp)   # the worlds moved


@pytest.mark.parametrize("n", [1, 2, 3])
def test_rollout_of_one_to_three_worlds(g1, n):
    """Ragged smallest sizes: a rollout of n = 1, 2, 3 worlds (one or two pairs, an odd last pair;
    31 of the 32 work queues empty, their blocks drain the one queue of their XCD or exit) gives
    those worlds bit for bit the trajectory they get as the first n worlds of a 64-world launch."""
    H, N = 4, 64
    qp, qv, pa, steps, W, mean, var, an, rn = _setup(N, H, 31)
    runs = []
    for m in (N, n):
        with g1.Env(m, substeps=10, pgs_iters=8, seed=5) as env:
            env.set_state(qp[:m], qv[:m], pa[:m], steps[:m])
            out = _rollout(g1, env, W, mean, var, H, np.ascontiguousarray(an[:, :m]), np.ascontiguousarray(rn[:, :m]))
            runs.append((out, env.get_state()))
    (big, big_state), (small, small_state) = runs
    for f in g1.Trajectory.FIELDS:
        k = (slice(None), slice(0, n)) if big[f].ndim >= 2 else slice(0, n)
        assert np.array_equal(big[f][k], small[f]), f
    for b, s in zip(big_state, small_state):
        assert np.array_equal(b[:n], s)


@pytest.mark.parametrize("N,S,K", [(301, 5, 3), (301, 10, 200)])
def test_work_queue_split_control_steps(g1, N, S, K):
    """K control steps in one physics launch equal K one-step launches bit for bit: S = 5 (items of
    3 and 2 substeps, an odd world count), and S = 10 with K = 200 (at least 8 pair-steps per wave,
    so items of 6 and 4 substeps, against 3, 3, 2, 2 for the one-step launches)."""
    import configs
    qp, qv, pa, steps = configs.reset_states(np.random.default_rng(5), N)
    states = []
    for split in (False, True):
        with g1.Env(N, substeps=S, pgs_iters=8, seed=2) as env:
            env.set_state(qp, qv, pa, steps)
            for _ in range(K if split else 1):
                env.bench_phys(1 if split else K)
            states.append(env.get_state())
    for a, b in zip(*states):
        assert np.array_equal(a, b)
    assert not np.array_equal(states[0][0], qp)


def test_host_step_five_substeps_matches_oracle(g1, orc):
    """g1_env_step with S = 5 (a control step split into work items of 3 and 2 substeps, its reward
    sums carried between items) against the oracle's control step."""
    N, S = 129, 5
    with g1.Env(N, substeps=S, pgs_iters=8, seed=3) as env:
        env.reset()
        qp, qv, pa, st = env.get_state()
        act = np.random.default_rng(6).normal(0, 0.3, (N, 29)).astype(np.float32)
        obs1, rew, done = env.step(act)
    oq, ov, opa, ost = qp.copy(), qv.copy(), pa.copy(), st.copy()
    rr, dd = orc.env_advance(oq, ov, opa, ost, act, np.zeros((N, 29), np.float32), S=S, threads=NTHREADS)
    live = dd == 0
    assert np.array_equal(done, dd) and np.array_equal(rew, rr)
    assert np.array_equal(obs1[live], orc.obs(oq, ov, opa)[live])


def test_reference_trained_policy_walks(g1):
    """End-to-end check of observation, action, physics and reward semantics: the reference's
    trained checkpoint (converted, g1.cu_amd/data) driven through g1_rollout walks forward at about
    its 0.8 m/s command without falling."""
    import torch
    from conftest import ROOT
    tp = np.load(os.path.join(ROOT, "g1.cu_amd", "data", "trained_policy_finish_best.npz"))
    N, H = 1024, 32
    with g1.Env(N, substeps=10, pgs_iters=8, seed=3) as env:
        env.reset()
        W = torch.from_numpy(tp["W"]).cuda()
        mean, var = torch.from_numpy(tp["obs_mean"]).cuda(), torch.from_numpy(tp["obs_var"]).cuda()
        traj = g1.Trajectory(H, N)
        vx, falls = [], []
        for _ in range(4):
            traj.run(env, W, mean, var)
            torch.cuda.synchronize()
            vx.append(traj.O[:, :, 0].mean().item())
            falls.append(traj.D.mean().item())
        assert env.check() == 0
    print(f"trained policy: mean vx per rollout {np.round(vx, 3).tolist()}, done fraction {np.round(falls, 4).tolist()}")
    assert vx[-1] > 0.6 and max(falls[1:]) < 0.005
