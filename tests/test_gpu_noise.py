"""The default noise path: g1_rollout without injected noise, as bench.py and the PPO driver run it.
The library draws its action noise (Philox4x32-10 -> Box-Muller pairs), its auto-reset noise and
g1_env_reset's start noise (Philox -> U(-1, 1)) itself, keyed by the env's seed and counted by
world and control step (reference call sites: src/g1_env.cu:105 reset, :206 auto-reset, :308-318
sampling and log-prob; the reference's curand streams cannot be reproduced, so these are this
build's own streams, restated on the host in tests/philox_np.py).

Each control step runs on the GPU from its own state, and the oracle takes the same pre-step state:
* the noise recovered from the GPU's actions, z = (A - mu) / exp(log_std) with mu the oracle's mean
  action, equals the host stream's normals (the kernel's float32 log/sqrt/sincos against float64:
  a few ulp), and LP = sum(-z^2/2 - log_std - log(2 pi)/2) within 1e-5;
* A, LP, V within 1e-5 of the oracle's rollout fed the host stream as injected noise, O bit for bit;
* the step's physics driven by the GPU's actions with the host's reset stream: qpos, qvel, reward,
  done, counters and every auto-reset state bit for bit;
* g1_env_reset's start states equal stand + 0.02 u bit for bit.
At N=8192 the recovered values are also tested as distributions, independently of the host
restatement: the action noise's moments, Kolmogorov-Smirnov against N(0, 1) and no correlation
within a Box-Muller pair; the reset and start noise against U(-1, 1)."""
import os

import numpy as np
import pytest

import philox_np as P
from conftest import relerr_rows

pytestmark = pytest.mark.gpu

NTHREADS = min(16, os.cpu_count() or 1)
TOL = 1e-5
SEED = 0x2545F4914F6CDD1D   # both Philox key words nonzero


@pytest.fixture(scope="module")
def g1():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import g1env
    return g1env


def _rollout(g1, env, dev, H):
    import torch
    tr = g1.Trajectory(H, env.N)
    tr.run(env, *dev)
    torch.cuda.synchronize()
    assert env.check() == 0
    return tr.numpy()


def _ks_uniform_pm1(u):
    from scipy import stats
    return stats.kstest(np.ravel(u), "uniform", args=(-1.0, 2.0)).statistic


@pytest.mark.timeout(600)
@pytest.mark.parametrize("fused,N", [(True, 8192), (False, 1024)])
def test_library_noise_matches_host_streams(g1, orc, fused, N):
    import torch
    import configs
    import g1_model as gm
    H = 4
    rng = np.random.default_rng(81)
    W = configs.policy_init(rng)
    mean = rng.normal(0, 0.1, 100).astype(np.float32)
    var = rng.uniform(0.5, 2.0, 100).astype(np.float32)
    ls = W[-29:].astype(np.float64)
    dev = [torch.from_numpy(x).cuda() for x in (W, mean, var)]
    stand = gm.qpos_stand.astype(np.float32)
    worlds = np.arange(N)
    with g1.Env(N, substeps=10, pgs_iters=8, seed=SEED) as env:
        assert env.set_fused(fused) == fused
        obs = env.reset()                      # counter 0 -> 1
        st0 = env.get_state()
        u0 = P.uniform_pm1(SEED, worlds, 0, P.STREAM_INIT)
        want = np.tile(stand, (N, 1))
        want[:, 7:] += np.float32(0.02) * u0
        assert np.array_equal(st0.qpos, want)
        assert not st0.qvel.any() and not st0.prev_act.any() and not st0.steps.any()
        assert np.array_equal(obs, orc.obs(st0.qpos, st0.qvel, st0.prev_act))
        steps = st0.steps.copy()
        steps[::2] = 997 + (worlds[::2] // 2) % 3   # timeouts, hence auto-resets, at steps 0, 1, 2
        env.set_state(st0.qpos, st0.qvel, st0.prev_act, steps)
        start = env.get_state()
        zs, us, outs = [], [], []
        for t in range(H):
            pre = env.get_state()
            out = _rollout(g1, env, dev, 1)
            post = env.get_state()
            outs.append(out)
            ctr = 1 + t
            an = P.action_noise(SEED, worlds, ctr)[None]
            rn = P.uniform_pm1(SEED, worlds, ctr, P.STREAM_RESET)[None]
            ref = orc.rollout(*(x.copy() for x in pre), W, mean, var, an, rn, 1, threads=NTHREADS)
            mu = orc.rollout(*(x.copy() for x in pre), W, mean, var, np.zeros_like(an), rn, 1,
                             threads=NTHREADS)["A"][0].astype(np.float64)
            A, LP = out["A"][0], out["LP"][0]
            assert np.array_equal(out["O"][0], ref["O"][0]), t
            e_a = relerr_rows(A, ref["A"][0]).max()
            e_lp = (np.abs(LP - ref["LP"][0]) / np.abs(ref["LP"][0])).max()
            e_v = np.abs(out["V"][0] - ref["V"][0]).max() / max(1.0, np.abs(ref["V"][0]).max())
            z = (A.astype(np.float64) - mu) / np.exp(ls)
            e_z = np.abs(z - an[0]).max()
            lp = (-0.5 * z * z - ls - 0.5 * np.log(2 * np.pi)).sum(1)
            e_lpz = (np.abs(LP - lp) / np.abs(lp)).max()
            o = [x.copy() for x in pre]
            rr, dd = orc.env_advance(*o, A, rn[0], threads=NTHREADS)
            print(f"step {t}: A {e_a:.1e} LP {e_lp:.1e} V {e_v:.1e} |z - host z| {e_z:.1e} LP(z) {e_lpz:.1e} "
                  f"resets {int(dd.sum())}", flush=True)
            assert e_a <= TOL and e_lp <= TOL and e_v <= TOL, t
            assert e_z <= 1e-4 and e_lpz <= TOL, t
            assert np.array_equal(out["D"][0], dd) and np.array_equal(out["R"][0], rr), t
            for a, b in zip(post, o):
                assert np.array_equal(a, b), t
            d = dd > 0
            zs.append(z)
            us.append((post.qpos[d, 7:].astype(np.float64) - stand[7:]) / 0.05)
    n_reset = sum(len(u) for u in us)
    assert n_reset >= N // 2
    # the same steps as one launch from the same start (a new env of the same seed, reset: counter 1)
    with g1.Env(N, substeps=10, pgs_iters=8, seed=SEED) as env:
        assert env.set_fused(fused) == fused
        env.reset()
        env.set_state(*start)
        one = _rollout(g1, env, dev, H)
    for f in ("O", "A", "LP", "V", "R", "D"):
        step_by_step = np.concatenate([q[f] for q in outs], 0)
        assert np.array_equal(one[f].view(np.uint32), step_by_step.view(np.uint32)), f
    if N < 8192:
        return
    from scipy import stats
    z = np.concatenate(zs)
    n = z.size
    ks = stats.kstest(z.ravel(), "norm").statistic
    a, b = z[:, 0:28:2].ravel(), z[:, 1:29:2].ravel()
    c1, c2 = np.corrcoef(a, b)[0, 1], np.corrcoef(a * a, b * b)[0, 1]
    u = np.concatenate(us)
    u_init = (st0.qpos[:, 7:].astype(np.float64) - stand[7:]) / 0.02
    print(f"action noise n={n}: mean {z.mean():.2e} var {z.var():.5f} KS {ks:.2e} (bound {1.95 / np.sqrt(n):.2e}) "
          f"pair corr {c1:.1e} / {c2:.1e}; reset noise n={u.size} KS {_ks_uniform_pm1(u):.2e}; "
          f"start noise n={u_init.size} KS {_ks_uniform_pm1(u_init):.2e}")
    assert abs(z.mean()) < 5 / np.sqrt(n) and abs(z.var() - 1) < 5 * np.sqrt(2 / n)
    assert ks < 1.95 / np.sqrt(n)
    assert abs(c1) < 5 / np.sqrt(a.size) and abs(c2) < 5 / np.sqrt(a.size)
    assert np.abs(u).max() <= 1 + 1e-4 and _ks_uniform_pm1(u) < 1.95 / np.sqrt(u.size)
    assert np.abs(u_init).max() <= 1 + 1e-4 and _ks_uniform_pm1(u_init) < 1.95 / np.sqrt(u_init.size)
