"""g1_rollout_noalloc (packed policy weights in the library's fixed device array, no allocation in
the call) against g1_rollout_ex on identical states and noise: every trajectory buffer and the
final state bit for bit, on two calls in a row, the second with a smaller input (fewer worlds, a
shorter horizon and a smaller policy, so the array holds a stale, larger packing from the first
call). Each no-alloc call runs on a fresh env and leaves the env's device memory where creation put
it (g1_env_device_bytes), while g1_rollout_ex on a fresh env grows it by its packed policy. A policy
wider than two layers of 256 runs the no-alloc call in the per-step form (the one-launch form's wide
tile needs activation buffers the library allocates), so its g1_rollout_ex comparison takes the
per-step form too."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def g1():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import g1env
    return g1env


def _case(N, H, hidden, seed):
    import configs
    rng = np.random.default_rng(seed)
    qp, qv, pa, st = configs.reset_states(rng, N)
    W = configs.policy_init(rng, hidden=hidden)
    mean = rng.normal(0, 0.1, 100).astype(np.float32)
    var = rng.uniform(0.5, 2.0, 100).astype(np.float32)
    an, rn = configs.rollout_noise(rng, H, N)
    return (qp, qv, pa, st), (W, mean, var, an, rn)


def _run(g1, state, inputs, N, H, hidden, act, noalloc):
    """One rollout on a fresh env; returns the outputs, the final state and the env's device bytes
    before and after the call."""
    import torch
    dev = [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in inputs]
    with g1.Env(N, substeps=10, pgs_iters=8, seed=3) as env:
        env.set_policy(hidden, act)
        narrow = len(hidden) == 2 and max(hidden) <= 256
        env.set_fused(narrow)   # the form g1_rollout_noalloc takes for this shape
        env.set_state(*state)
        traj = g1.Trajectory(H, N)
        ptrs = [g1.dev_ptr(t) for t in (*dev[:3], *traj.tensors(), dev[3], dev[4])]
        before = env.device_bytes()
        if noalloc:
            assert g1.lib.g1_rollout_noalloc(env.h, H, *ptrs) == 0
        else:
            g1.lib.g1_rollout_ex(env.h, H, *ptrs)
        torch.cuda.synchronize()
        after = env.device_bytes()
        assert env.check() == 0
        return traj.numpy(), env.get_state(), (before, after)


def test_noalloc_rollout_matches_allocating_rollout(g1):
    cases = [(96, 3, (512, 512, 256), 1, 71), (40, 2, (256, 256), 0, 72)]   # second: smaller everything
    for N, H, hidden, act, seed in cases:
        state, inputs = _case(N, H, hidden, seed)
        ref, ref_state, (b0, b1) = _run(g1, state, inputs, N, H, hidden, act, noalloc=False)
        got, got_state, (n0, n1) = _run(g1, state, inputs, N, H, hidden, act, noalloc=True)
        assert b1 > b0, (N, b0, b1)          # the allocating form packed into a buffer it allocated
        assert n1 == n0 == b0, (N, n0, n1)   # the no-alloc form allocated nothing
        for f in g1.Trajectory.FIELDS:
            assert np.array_equal(got[f], ref[f]), (N, f)
        for a, b in zip(got_state, ref_state):
            assert np.array_equal(a, b), N
        assert not np.array_equal(got_state.qpos, state[0])   # the worlds moved
