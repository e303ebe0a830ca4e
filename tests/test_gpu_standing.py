"""The standing, continuous-contact regime: the robot reset to its stand pose and held there by zero
actions (the PD target is then the stand keyframe), with most of its 8 foot spheres in contact at
every substep. This regime is the reference's physics-only benchmark (scripts/bench_env_phys.py,
g1_env_bench_phys) and its stability gate (scripts/test_stability.py:15-55)."""
import os

import numpy as np
import pytest

from conftest import relerr_rows

pytestmark = pytest.mark.gpu

NTHREADS = min(16, os.cpu_count() or 1)


@pytest.fixture(scope="module")
def g1():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import g1env
    return g1env


def test_stability_gate(g1):
    """The reference's gate: N=256, S=10, kp=500, 400 zero-action control steps through the host-step
    path: no NaN/inf in observations or rewards, and the mean base linear speed stays bounded
    (< 50). Also: the standing robot does not fall (no world finishes an episode)."""
    N, steps = 256, 400
    with g1.Env(N, substeps=10, pgs_iters=8, seed=0) as env:
        env.reset()
        act = np.zeros((N, 29), np.float32)
        speed, done_any = [], np.zeros(N, bool)
        for t in range(steps):
            obs, rew, done = env.step(act)
            assert np.isfinite(obs).all() and np.isfinite(rew).all(), t
            speed.append(float(np.linalg.norm(obs[:, 0:3], axis=1).mean()))
            done_any |= done.astype(bool)
        z = env.get_state().qpos[:, 2]
    speed = np.array(speed)
    print(f"stability: base |v| start {speed[0]:.4f} mid {speed[steps // 2]:.4f} end {speed[-1]:.4f} "
          f"max {speed.max():.4f}; pelvis z {z.min():.3f}..{z.max():.3f}; worlds done {int(done_any.sum())}")
    assert speed.max() < 50.0
    assert not done_any.any()


def test_bench_phys_matches_oracle_standing(g1, orc):
    """g1_env_bench_phys (zero action, reward/termination/auto-reset included) against the oracle's
    zero-action control step, teacher-forced from the GPU's state before each of 4 control steps:
    qpos, qvel, step counters and previous actions bit for bit (the oracle in the kernel's
    summation association)."""
    N = 1024
    worst = []
    with g1.Env(N, substeps=10, pgs_iters=8, seed=5) as env:
        env.reset()
        for t in range(4):
            pre = env.get_state()
            env.bench_phys(1)
            post = env.get_state()
            oq, ov, opa, ost = (x.copy() for x in pre)
            _, dd = orc.env_advance(oq, ov, opa, ost, np.zeros((N, 29), np.float32),
                                    np.zeros((N, 29), np.float32), threads=NTHREADS)
            assert not dd.any()
            assert np.array_equal(post.steps, ost) and np.array_equal(post.prev_act, opa)
            eq, ev = relerr_rows(post.qpos, oq).max(), relerr_rows(post.qvel, ov).max()
            worst.append((eq, ev))
            print(f"standing step {t}: qpos {eq:.2e} qvel {ev:.2e}")
            assert np.array_equal(post.qpos, oq) and np.array_equal(post.qvel, ov), t
        assert env.check() == 0


def test_standing_contact_histogram(g1):
    """Contact counts of the standing robot over 20 control steps (N=8192): the reference measured
    ncon 6/7/8 in 93% of its contact solves on this benchmark (8: 28%, 7: 38%, 6: 27%;
    DEVLOG.md:546-549). Contact is continuous, so nearly every substep solves contacts."""
    N = 8192
    with g1.Env(N, substeps=10, pgs_iters=8, seed=1) as env:
        env.reset()
        env.bench_phys(5)
        env.ncon_hist(enable=True)
        env.bench_phys(20)
        hist = env.ncon_hist(enable=False)
        assert env.check() == 0
    assert hist.sum() == N * 20 * 10
    contact = hist[1:].sum()
    share = hist[6:9].sum() / contact
    frac = hist / hist.sum()
    print(f"standing ncon histogram {hist.tolist()}; fractions {np.round(frac, 3).tolist()}; "
          f"6/7/8 share of contact substeps {share:.3f}")
    assert contact >= 0.95 * hist.sum()
    assert share >= 0.85
