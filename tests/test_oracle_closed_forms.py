"""Pins for the oracle parts that no reference fixture covers, from mathematics and independent
libraries rather than from the oracle's own formulas: M*solveM(x) = x (dense CRBA + numpy),
multi-RHS form == single form, PGS at convergence == brute-force LCP, impedance closed form,
MLP == torch nn.Linear/tanh/ELU, Gaussian log-prob == torch.distributions, observation layout ==
scipy rotations, reward/termination on hand-built cases."""
import itertools

import numpy as np
import pytest

from conftest import relerr_rows


def _states(n, seed=0):
    import configs
    rng = np.random.default_rng(seed)
    qp, qv = configs.perturbed_states(n, rng, joint=0.3, tilt_deg=30)
    return qp, qv, rng


@pytest.mark.parametrize("damped", [False, True])
def test_solve_inverts_dense_mass_matrix(orc, damped):
    qp, _, rng = _states(16)
    x = rng.normal(size=(16, 35))
    Bdt = orc.bdt(np.float64) if damped else None
    y = orc.solve(qp, x, Bdt=Bdt, dtype=np.float64)
    M = orc.mass(qp, dtype=np.float64)
    for i in range(16):
        Mi = M[i] + (np.diag(Bdt) if damped else 0)
        assert np.allclose(Mi @ y[i], x[i], rtol=1e-9, atol=1e-9 * np.abs(x[i]).max())
        assert np.allclose(y[i], np.linalg.solve(Mi, x[i]), rtol=1e-8, atol=1e-10)
        assert np.all(np.linalg.eigvalsh(Mi) > 0)       # SPD


def test_multi_rhs_form_equals_single_form(orc):
    qp, _, rng = _states(32, seed=1)
    x = rng.normal(size=(32, 35)).astype(np.float32)
    a = orc.solve(qp, x, dtype=np.float32, multi=False)
    b = orc.solve(qp, x, dtype=np.float32, multi=True)
    assert relerr_rows(a, b).max() < 1e-6
    assert not np.array_equal(a, b)                        # genuinely different operation order


def test_mass_matrix_planted_error_is_caught(orc):
    """A transposed/dropped term in the factor would break M*y = x: check the identity is sharp."""
    qp, _, rng = _states(2, seed=2)
    x = rng.normal(size=(2, 35))
    y = orc.solve(qp, x, dtype=np.float64)
    M = orc.mass(qp, dtype=np.float64)
    M_bad = M[0].copy(); M_bad[6, 7] *= 1.01; M_bad[7, 6] *= 1.01
    assert not np.allclose(M_bad @ y[0], x[0], rtol=1e-6, atol=1e-8)


def _lcp_bruteforce(A, b):
    """Exact solution of f >= 0, w = A f + b >= 0, f.w = 0 by enumerating active sets."""
    n = len(b)
    for k in range(n + 1):
        for act in itertools.combinations(range(n), k):
            f = np.zeros(n)
            if k:
                idx = list(act)
                f[idx] = np.linalg.solve(A[np.ix_(idx, idx)], -b[idx])
            w = A @ f + b
            if (f >= -1e-12).all() and (w >= -1e-9).all():
                return f
    raise AssertionError("no LCP solution")


@pytest.mark.parametrize("seed", range(5))
def test_pgs_converges_to_lcp_solution(orc, seed):
    rng = np.random.default_rng(seed)
    n = 6
    J = rng.normal(size=(n, 4))
    A = J @ J.T + np.diag(rng.uniform(0.1, 1.0, n))
    b = rng.normal(size=n)
    f = orc.pgs(A, b, iters=5000, dtype=np.float64)
    assert np.allclose(f, _lcp_bruteforce(A, b), atol=1e-8)
    # one sweep from zero equals the hand-computed first Gauss-Seidel pass
    f1 = orc.pgs(A, b, iters=1, dtype=np.float64)
    g = np.zeros(n)
    for i in range(n):
        g[i] = max(0.0, -(b[i] + A[i] @ g - A[i, i] * g[i]) / A[i, i])
    assert np.allclose(f1, g, rtol=1e-14, atol=0)


def test_impedance_closed_form(orc):
    """MuJoCo solimp sigmoid (dmin 0.9, dmax 0.95, width 1e-3, midpoint 0.5, power 2)."""
    assert orc.impedance(0.0) == pytest.approx(0.9)
    assert orc.impedance(-1e-3) == pytest.approx(0.95)
    assert orc.impedance(-5e-3) == pytest.approx(0.95)
    assert orc.impedance(-0.25e-3) == pytest.approx(0.9 + 0.05 * 2 * 0.25 ** 2)
    assert orc.impedance(-0.75e-3) == pytest.approx(0.9 + 0.05 * (1 - 2 * 0.25 ** 2))
    assert orc.impedance(-0.5e-3) == pytest.approx(0.925)   # continuous at the midpoint


@pytest.mark.parametrize("hidden,act", [((256, 256), 0), ((512, 512, 256), 1)])
def test_mlp_matches_torch(orc, hidden, act):
    import torch
    import torch.nn as nn
    import configs
    rng = np.random.default_rng(7)
    W = configs.policy_init(rng, hidden=hidden)
    W[:5] += 0.01  # nonzero biases are covered below
    layers, d, o = [], 100, 0
    for h in hidden:
        lin = nn.Linear(d, h)
        lin.weight.data = torch.from_numpy(W[o:o + h * d].reshape(h, d).copy()); o += h * d
        lin.bias.data = torch.from_numpy(rng.normal(0, 0.1, h).astype(np.float32))
        W[o:o + h] = lin.bias.data.numpy(); o += h
        layers += [lin, nn.Tanh() if act == 0 else nn.ELU()]
        d = h
    mu_l = nn.Linear(d, 29); mu_l.weight.data = torch.from_numpy(W[o:o + 29 * d].reshape(29, d).copy()); o += 29 * d
    mu_l.bias.data = torch.from_numpy(W[o:o + 29].copy()); o += 29
    v_l = nn.Linear(d, 1); v_l.weight.data = torch.from_numpy(W[o:o + d].reshape(1, d).copy()); o += d
    v_l.bias.data = torch.from_numpy(W[o:o + 1].copy()); o += 1
    assert o + 29 == len(W) == orc.policy_params(hidden, act)
    x = rng.normal(0, 2, (64, 100)).astype(np.float32)
    with torch.no_grad():
        z = nn.Sequential(*layers).double()(torch.from_numpy(x).double())
        mu_t = mu_l.double()(z).numpy(); v_t = v_l.double()(z).numpy()[:, 0]
    mu, ls, v = orc.mlp(W, x, hidden=hidden, act=act)
    assert relerr_rows(mu, mu_t).max() < 1e-5
    assert np.abs(v - v_t).max() < 1e-5 * (1 + np.abs(v_t).max())
    assert np.array_equal(ls, np.broadcast_to(W[-29:], ls.shape))


def test_rollout_logprob_and_action_closed_form(orc):
    """A = mu + exp(log_std) n and LP = sum log N(A; mu, exp(log_std)) (torch.distributions)."""
    import torch
    import configs
    rng = np.random.default_rng(8)
    N, H = 16, 1
    qp, qv, pa, st = configs.reset_states(rng, N)
    W = configs.policy_init(rng)
    W[-29:] = rng.uniform(-1, 0, 29).astype(np.float32)
    an, rn = configs.rollout_noise(rng, H, N)
    mean = np.zeros(100, np.float32); var = np.ones(100, np.float32)
    out = orc.rollout(qp.copy(), qv.copy(), pa.copy(), st.copy(), W, mean, var, an, rn, H)
    no = np.clip(out["O"][0], -10, 10)
    mu, ls, v = orc.mlp(W, no)
    assert np.allclose(out["A"][0], mu + np.exp(ls) * an[0], rtol=1e-6, atol=1e-6)
    dist = torch.distributions.Normal(torch.from_numpy(mu).double(), torch.from_numpy(np.exp(ls)).double())
    lp = dist.log_prob(torch.from_numpy(out["A"][0]).double()).sum(-1).numpy()
    assert np.allclose(out["LP"][0], lp, rtol=1e-5, atol=1e-4)
    assert np.allclose(out["V"][0], v, rtol=1e-6, atol=1e-6)


def test_observation_layout(orc):
    from scipy.spatial.transform import Rotation
    qp, qv, rng = _states(8, seed=9)
    pa = rng.normal(size=(8, 29)).astype(np.float32)
    o = orc.obs(qp, qv, pa)
    R = Rotation.from_quat(np.roll(qp[:, 3:7], -1, axis=1)).as_matrix()     # scipy wants (x,y,z,w)
    grav_body = np.einsum("nji,j->ni", R, np.array([0.0, 0.0, -1.0]))          # R^T (0,0,-1)
    assert np.allclose(o[:, 0:6], qv[:, 0:6], atol=1e-6)
    assert np.allclose(o[:, 6:9], grav_body, atol=1e-6)
    assert np.allclose(o[:, 9:38], qp[:, 7:36], atol=1e-6)
    assert np.allclose(o[:, 38:67], qv[:, 6:35], atol=1e-6)
    assert np.array_equal(o[:, 67:96], pa)
    assert np.allclose(o[:, 96:], [0.8, 0, 0, 0])


def _advance(orc, qp, qv, pa, steps, act, noise=None, S=2):
    n = qp.shape[0]
    noise = np.zeros((n, 29), np.float32) if noise is None else noise
    return orc.env_advance(qp, qv, pa, steps, act, noise, S=S)


def test_termination_and_reward_cases(orc):
    """Hand cases of the reward/termination rules (reference: src/g1_env.cu:164-211)."""
    import g1_model as gm
    stand = gm.qpos_stand.astype(np.float32)
    N = 5
    qp = np.tile(stand, (N, 1)); qp[:, 2] += 0.5        # airborne: no contact within 2 substeps
    qv = np.zeros((N, 35), np.float32); pa = np.zeros((N, 29), np.float32)
    steps = np.array([0, 999, 0, 0, 0], np.int32)
    qp[2, 2] = 0.30                                      # fallen: height < 0.45
    qp[3, 0] = 5.2                                       # crossed the finish line upright
    ang = np.deg2rad(70); qp[4, 3:7] = [np.cos(ang / 2), np.sin(ang / 2), 0, 0]   # tilted: up < 0.5
    act = np.zeros((N, 29), np.float32)
    noise = np.full((N, 29), 0.5, np.float32)
    r, d = _advance(orc, qp, qv, pa, steps, act, noise)
    assert list(d) == [0, 1, 1, 1, 1]
    assert r[2] == -5.0 and r[4] == -5.0
    assert r[3] > 50.0                                   # alive reward + finish bonus
    assert 0.0 < r[0] < 2.0
    # finished worlds restart at the stand pose + 0.05 * noise, zero velocity, zero previous action
    for w in (1, 2, 3, 4):
        exp = stand.copy(); exp[7:] += np.float32(0.05) * noise[w]
        assert np.array_equal(qp[w], exp) and not qv[w].any() and not pa[w].any() and steps[w] == 0
    assert steps[0] == 1 and np.array_equal(pa[0], act[0])


def test_action_penalty_and_velocity_guard(orc):
    import g1_model as gm
    stand = gm.qpos_stand.astype(np.float32)
    N = 2
    qp = np.tile(stand, (N, 1)); qp[:, 2] += 0.5
    qv = np.zeros((N, 35), np.float32); pa = np.zeros((N, 29), np.float32)
    steps = np.zeros(N, np.int32)
    act = np.zeros((N, 29), np.float32); act[1, 0] = 1.0    # (a - pa)^2 = 1 -> penalty 0.005
    r, d = _advance(orc, qp, qv, pa, steps, act, S=1)
    assert not d.any()
    # world 1 also gets a different PD torque (energy term), so compare against the penalty bound
    assert r[0] - r[1] > 0.004
    # NaN velocities are zeroed and velocities are clamped to +-50 by the integrator guard
    qp2 = np.tile(stand, (1, 1)); qp2[:, 2] += 0.5
    qv2 = np.zeros((1, 35), np.float32); qv2[0, 10] = np.nan; qv2[0, 12] = 1e4
    _advance(orc, qp2, qv2, np.zeros((1, 29), np.float32), np.zeros(1, np.int32), np.zeros((1, 29), np.float32), S=1)
    assert np.isfinite(qv2).all() and np.abs(qv2).max() <= 50.0


def test_reward_closed_form(orc):
    """The oracle's control-step reward equals the task's reward written out in fp64
    (tests/reward_spec.py, from src/g1_env.cu:164-199) on states where it is known in closed form:
    each case moves one term, so a wrong coefficient, sign, clip or gate fails by >= 1e-2."""
    from reward_spec import crafted_cases, reward_spec
    c = crafted_cases()
    qp, qv, pa, st = c["qp"].copy(), c["qv"].copy(), c["pa"].copy(), c["steps"].copy()
    noise = np.random.default_rng(1).uniform(-1, 1, (len(st), 29)).astype(np.float32)
    r, d = _advance(orc, qp, qv, pa, st, c["act"], noise, S=10)
    # the alive worlds' end state; done worlds are reset, so their reward needs only the flags
    vx_mean = c["qv"][:, 0].astype(np.float64)          # free fall: constant forward speed
    live = d == 0
    r_spec, d_spec = reward_spec(np.where(live[:, None], qp, c["qp"]), np.where(live[:, None], qv, c["qv"]),
                                 vx_mean, c["act"], c["pa"], c["steps"])
    assert list(d.astype(bool)) == list(d_spec), c["names"]
    for w in np.flatnonzero(live):
        assert abs(float(r[w]) - r_spec[w]) <= 1e-6, (c["names"][w], r[w], r_spec[w])
    # done worlds: the falls score exactly -5, the timeout and the finish line score their alive
    # reward (+50 at the line); their end states are reset, so those two are checked against a twin
    # stepped without the done condition (episode step 0; the finish-line twin at x = 4, which
    # changes no term of the alive reward)
    names = c["names"]
    assert r[names.index("fallen (height)")] == -5.0 and r[names.index("fallen (tilt)")] == -5.0
    for nm, bonus in (("timeout", 0.0), ("finish line", 50.0)):
        w = names.index(nm)
        q1, v1, p1 = c["qp"][w:w + 1].copy(), c["qv"][w:w + 1].copy(), c["pa"][w:w + 1].copy()
        s1 = np.zeros(1, np.int32)
        q1[0, 0] = min(q1[0, 0], 4.0)
        r1, d1 = _advance(orc, q1, v1, p1, s1, c["act"][w:w + 1], noise[w:w + 1], S=10)
        assert d1[0] == 0
        rs, _ = reward_spec(q1, v1, vx_mean[w:w + 1], c["act"][w:w + 1], c["pa"][w:w + 1], s1)
        # (r + 50 is rounded to fp32: one ulp of 51.5 is 3.8e-6)
        assert abs(float(r[w]) - (rs[0] + bonus)) <= 1e-6 + float(np.spacing(np.float32(r[w]))), nm
    # every done world restarts at the stand pose + 0.05 * its reset noise
    import g1_model as gm
    for w in np.flatnonzero(~live):
        exp = gm.qpos_stand.astype(np.float32).copy()
        exp[7:] += np.float32(0.05) * noise[w]
        assert np.array_equal(qp[w], exp) and not qv[w].any() and not pa[w].any() and st[w] == 0
