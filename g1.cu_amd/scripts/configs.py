"""Seeded synthetic inputs for the benchmark configurations of the fused-rollout path.

Config 0: 256 single-world states (fp64 CPU reference); config 1: batched smooth dynamics with held
random torques; config 2: foot-contact states with 0..8 penetrating spheres; config 3: the fused
rollout (N=8192, H=32, S=10, MLP 100-256-256 tanh); config 4: the scaled rollout (N=131072, MLP
100-512-512-256 ELU). All draws come from numpy's PCG64 with the seed recorded by the caller.
"""
import numpy as np

import g1_model as gm

NQ, NV, NU = gm.NQ, gm.NV, gm.NU


def _quat_mul(a, b):
    w1, x1, y1, z1 = a[..., 0], a[..., 1], a[..., 2], a[..., 3]
    w2, x2, y2, z2 = b[..., 0], b[..., 1], b[..., 2], b[..., 3]
    return np.stack([w1 * w2 - x1 * x2 - y1 * y2 - z1 * z2, w1 * x2 + x1 * w2 + y1 * z2 - z1 * y2,
                     w1 * y2 - x1 * z2 + y1 * w2 + z1 * x2, w1 * z2 + x1 * y2 - y1 * x2 + z1 * w2], -1)


def perturbed_states(n, rng, joint=0.1, tilt_deg=5.0, qvel_sd=0.5):
    """Stand pose + U(-joint, joint) on the 29 hinges, base tilted by <= tilt_deg about a random
    axis, qvel ~ N(0, qvel_sd) on all 35 dofs (float64)."""
    qpos = np.tile(gm.qpos_stand.astype(np.float64), (n, 1))
    qpos[:, 7:] += rng.uniform(-joint, joint, size=(n, NQ - 7))
    axis = rng.normal(size=(n, 3))
    axis /= np.linalg.norm(axis, axis=1, keepdims=True)
    ang = np.deg2rad(rng.uniform(0.0, tilt_deg, size=n))
    dq = np.concatenate([np.cos(ang / 2)[:, None], axis * np.sin(ang / 2)[:, None]], 1)
    qpos[:, 3:7] = _quat_mul(qpos[:, 3:7], dq)
    qvel = rng.normal(0.0, qvel_sd, size=(n, NV))
    return qpos, qvel


def random_torque(n, rng):
    """tau = U(-1,1) * frc_hi on the actuated dofs 6..34, zero on the free base."""
    tau = np.zeros((n, NV))
    tau[:, 6:] = rng.uniform(-1.0, 1.0, size=(n, NU)) * gm.act_frc_hi.astype(np.float64)
    return tau


def config0(seed=0, n=256):
    rng = np.random.default_rng(seed)
    qpos, qvel = perturbed_states(n, rng)
    return qpos, qvel, random_torque(n, rng)


def _foot_bottoms(qpos, fk):
    """Sphere-bottom heights c_z - r for the 8 foot spheres of each state, via `fk` (a callable
    returning world frames (xpos, xquat, xipos) for a batch of qpos)."""
    xpos, xquat, _ = fk(qpos)
    fb = np.array([7, 7, 7, 7, 13, 13, 13, 13])
    out = np.zeros((qpos.shape[0], 8))
    for s in range(8):
        q = xquat[:, fb[s]]
        v = np.broadcast_to(gm.foot_lpos[s].astype(np.float64), (qpos.shape[0], 3))
        u = q[:, 1:]
        t = 2.0 * np.cross(u, v)
        c = xpos[:, fb[s]] + v + q[:, :1] * t + np.cross(u, t)
        out[:, s] = c[:, 2] - float(gm.foot_radius)
    return out


def config2(fk, seed=2, n=8192):
    """Contact-solve states: joints U(-0.1,0.1), base tilt <= 5 deg, then base z set so that k ~ U{0..8}
    of the lowest sphere bottoms sit below the plane, the k-th lowest by U(0, 5 mm); base linear
    velocity N(0, 0.3) m/s, other dofs N(0, 0.05)."""
    rng = np.random.default_rng(seed)
    qpos, _ = perturbed_states(n, rng)
    qvel = rng.normal(0.0, 0.05, size=(n, NV))
    qvel[:, 0:3] = rng.normal(0.0, 0.3, size=(n, 3))
    k = rng.integers(0, 9, size=n)
    depth = rng.uniform(0.0, 0.005, size=n)
    h = np.sort(_foot_bottoms(qpos, fk), axis=1)
    kth = h[np.arange(n), np.maximum(k - 1, 0)]
    shift = np.where(k == 0, -h[:, 0] + depth + 1e-4, -kth - depth)
    qpos[:, 2] += shift
    return qpos, qvel, k


def policy_init(rng, hidden=(256, 256), log_std=-0.5):
    """Packed policy parameters in torch order W0,b0,..,Wmu,bmu,Wv,bv,log_std with weights
    N(0, 1/fan_in), zero biases, constant log_std."""
    parts = []
    fan = gm.OBS_DIM
    for h in hidden:
        parts += [rng.normal(0.0, 1.0 / np.sqrt(fan), size=(h, fan)).ravel(), np.zeros(h)]
        fan = h
    parts += [rng.normal(0.0, 1.0 / np.sqrt(fan), size=(NU, fan)).ravel(), np.zeros(NU)]
    parts += [rng.normal(0.0, 1.0 / np.sqrt(fan), size=(1, fan)).ravel(), np.zeros(1)]
    parts += [np.full(NU, log_std)]
    return np.concatenate(parts).astype(np.float32)


def rollout_noise(rng, H, N):
    """Pre-generated action noise N(0,1) and reset noise U(-1,1), both [H, N, 29] float32."""
    act = rng.standard_normal(size=(H, N, NU), dtype=np.float32)
    rst = (rng.random(size=(H, N, NU), dtype=np.float32) * 2.0 - 1.0).astype(np.float32)
    return act, rst


def reset_states(rng, N, noise=0.02):
    """k_reset's start distribution: stand pose + noise*U(-1,1) on the actuated joints, zero
    velocity, zero previous action, step counter 0 (reference: src/g1_env.cu:97-111)."""
    qp = np.tile(gm.qpos_stand, (N, 1)).astype(np.float32)
    u = (rng.random(size=(N, NU), dtype=np.float32) * 2.0 - 1.0).astype(np.float32)
    qp[:, 7:] += np.float32(noise) * u
    return qp, np.zeros((N, NV), np.float32), np.zeros((N, NU), np.float32), np.zeros(N, np.int32)


ROLLOUT_CONFIGS = {
    3: dict(N=8192, H=32, S=10, pgs=8, hidden=(256, 256), act=0),
    4: dict(N=131072, H=32, S=10, pgs=8, hidden=(512, 512, 256), act=1),
}
