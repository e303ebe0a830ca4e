"""ctypes binding of libg1env.so plus the actor-critic pieces a PPO driver needs.

Mirrors the reference's scripts/ppo.py interface (G1Env, RunNorm, AC, evaluate, _lib, _fp;
reference scripts/ppo.py:20-125) so a driver written against it runs unchanged on the MI355X
build. torch is imported before the library is loaded so the process uses torch's HIP runtime.
"""
import ctypes
import os
import sys

import numpy as np
import torch
import torch.nn as nn

HERE = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(HERE, "build", "libg1env.so")

if not os.path.exists(LIB):
    raise ImportError(f"{LIB} is missing: build it with `python g1.cu_amd/build.py`")

# ---------------- ctypes env binding (reference: scripts/ppo.py:24-32) ----------------
_lib = ctypes.CDLL(LIB)
_lib.g1_env_create.restype = ctypes.c_void_p
_lib.g1_env_create.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_ulong]
_lib.g1_env_obs_dim.restype = ctypes.c_int
_lib.g1_env_act_dim.restype = ctypes.c_int
_fp = ctypes.POINTER(ctypes.c_float)
_lib.g1_env_reset.argtypes = [ctypes.c_void_p, _fp]
_lib.g1_env_step.argtypes = [ctypes.c_void_p, _fp, _fp, _fp, _fp]
_lib.g1_env_destroy.argtypes = [ctypes.c_void_p]
_lib.g1_rollout.restype = None
_lib.g1_rollout.argtypes = [ctypes.c_void_p, ctypes.c_int] + [ctypes.c_void_p] * 10
_lib.g1_env_bench_phys.restype = None
_lib.g1_env_bench_phys.argtypes = [ctypes.c_void_p, ctypes.c_int]
_lib.g1_env_qpos.argtypes = [ctypes.c_void_p, _fp]
_lib.g1_env_qpos_all.argtypes = [ctypes.c_void_p, _fp]

# additive exports of this build (include/g1env.h)
_lib.g1_rollout_ex.restype = None
_lib.g1_rollout_ex.argtypes = [ctypes.c_void_p, ctypes.c_int] + [ctypes.c_void_p] * 12
_ip = ctypes.POINTER(ctypes.c_int)
_lib.g1_env_set_state.argtypes = [ctypes.c_void_p, _fp, _fp, _fp, _ip]
_lib.g1_env_get_state.argtypes = [ctypes.c_void_p, _fp, _fp, _fp, _ip]
_lib.g1_env_set_policy.restype = ctypes.c_int
_lib.g1_env_set_policy.argtypes = [ctypes.c_void_p, ctypes.c_int, _ip, ctypes.c_int]
_lib.g1_env_policy_params.restype = ctypes.c_long
_lib.g1_env_policy_params.argtypes = [ctypes.c_void_p]
_lib.g1_env_set_contact.argtypes = [ctypes.c_void_p, ctypes.c_float, ctypes.c_int]
_lib.g1_env_ncon_hist.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_ulonglong)]
_lib.g1_env_profile.argtypes = [ctypes.c_void_p, ctypes.c_int]
_lib.g1_env_profile_read.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_double)]
_lib.g1_occupancy_report.restype = None
_lib.g1_probe_qacc.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 3 + [ctypes.c_int] * 3 + [ctypes.c_float] + \
    [ctypes.c_void_p] * 2
_lib.g1_probe_substep.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 3 + [ctypes.c_int] * 2 + [ctypes.c_float] + \
    [ctypes.c_void_p] * 2
_lib.g1_probe_policy.restype = ctypes.c_int
_lib.g1_probe_policy.argtypes = [ctypes.c_int, ctypes.c_int, _ip, ctypes.c_int] + [ctypes.c_void_p] * 4
_lib.g1_probe_philox.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint, ctypes.c_uint]
_lib.g1_probe_divide.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 4
_lib.g1_probe_sincos.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 3
_lib.g1_dynamics_bench.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 3 + [ctypes.c_int] * 5 + [ctypes.c_float] + \
    [ctypes.c_void_p] * 2


def _p(a):
    return a.ctypes.data_as(_fp)


def _dp(t):
    return ctypes.c_void_p(t.data_ptr())


class G1Env:
    """N resident worlds; host-step interface (reference: scripts/ppo.py:39-59)."""

    def __init__(self, n_worlds, substeps=10, pgs_iters=2000, seed=0):
        self.N = n_worlds
        self.obs_dim = _lib.g1_env_obs_dim()
        self.act_dim = _lib.g1_env_act_dim()
        self.h = _lib.g1_env_create(n_worlds, substeps, pgs_iters, seed)
        self._obs = np.zeros((n_worlds, self.obs_dim), np.float32)
        self._rew = np.zeros(n_worlds, np.float32)
        self._done = np.zeros(n_worlds, np.float32)

    def reset(self):
        _lib.g1_env_reset(self.h, _p(self._obs))
        return self._obs.copy()

    def step(self, act):
        act = np.ascontiguousarray(act, np.float32)
        _lib.g1_env_step(self.h, _p(act), _p(self._obs), _p(self._rew), _p(self._done))
        return self._obs.copy(), self._rew.copy(), self._done.copy()

    def close(self):
        _lib.g1_env_destroy(self.h)

    # ---- additive helpers (state access for tests and benchmarks)
    def set_state(self, qp, qv, pa, steps):
        qp = np.ascontiguousarray(qp, np.float32); qv = np.ascontiguousarray(qv, np.float32)
        pa = np.ascontiguousarray(pa, np.float32); st = np.ascontiguousarray(steps, np.int32)
        _lib.g1_env_set_state(self.h, _p(qp), _p(qv), _p(pa), st.ctypes.data_as(_ip))

    def get_state(self):
        qp = np.zeros((self.N, 36), np.float32); qv = np.zeros((self.N, 35), np.float32)
        pa = np.zeros((self.N, 29), np.float32); st = np.zeros(self.N, np.int32)
        _lib.g1_env_get_state(self.h, _p(qp), _p(qv), _p(pa), st.ctypes.data_as(_ip))
        return qp, qv, pa, st

    def set_policy(self, hidden, activation):
        h = np.ascontiguousarray(hidden, np.int32)
        if _lib.g1_env_set_policy(self.h, len(hidden), h.ctypes.data_as(_ip), int(activation)) != 0:
            raise ValueError(f"unsupported policy shape {hidden}/{activation}")

    def set_contact(self, mu, pgs_iters):
        _lib.g1_env_set_contact(self.h, float(mu), int(pgs_iters))

    def ncon_hist(self, enable=True):
        out = (ctypes.c_ulonglong * 9)()
        _lib.g1_env_ncon_hist(self.h, int(enable), out)
        return np.array(out[:], np.int64)


# ---------------- running obs normalizer (reference: scripts/ppo.py:63-81) ----------------
class RunNorm:
    """Running mean/var (parallel Welford merge) of raw observations, clipped normalisation."""

    def __init__(self, dim, dev):
        self.mean = torch.zeros(dim, device=dev)
        self.var = torch.ones(dim, device=dev)
        self.count = 1e-4

    def update(self, x):
        n = x.shape[0]
        batch_mean = x.mean(0)
        batch_var = x.var(0, unbiased=False)
        total = self.count + n
        delta = batch_mean - self.mean
        self.mean += delta * n / total
        m2 = self.var * self.count + batch_var * n + delta ** 2 * self.count * n / total
        self.var = m2 / total
        self.count = total

    def norm(self, x):
        return torch.clamp((x - self.mean) / torch.sqrt(self.var + 1e-8), -10.0, 10.0)


# ---------------- actor-critic (reference: scripts/ppo.py:85-99) ----------------
class AC(nn.Module):
    """Gaussian policy: hidden MLP body, mean head, value head and a state-independent log std.
    Parameter order (body linears, mu, v, log_std) is the packing order of pack_weights."""

    def __init__(self, obs_dim, act_dim, hidden=(256, 256), activation=nn.Tanh):
        super().__init__()
        layers, d = [], obs_dim
        for h in hidden:
            layers += [nn.Linear(d, h), activation()]
            d = h
        self.body = nn.Sequential(*layers)
        self.mu = nn.Linear(d, act_dim)
        self.v = nn.Linear(d, 1)
        self.log_std = nn.Parameter(-0.5 * torch.ones(act_dim))

    def forward(self, x):
        z = self.body(x)
        return self.mu(z), self.log_std.exp(), self.v(z).squeeze(-1)


@torch.no_grad()
def evaluate(env, ac, norm, dev, steps=200):
    """Deterministic (mean-action) evaluation through the host-step path; forward distance from the
    base linear-velocity observation (reference: scripts/ppo.py:102-125)."""
    obs = torch.tensor(env.reset(), device=dev)
    N = env.N
    dt_ctrl = 0.02
    fwd = np.zeros(N); alive_len = np.zeros(N); done_any = np.zeros(N, bool); vx_acc = np.zeros(N)
    for _ in range(steps):
        mu, _, _ = ac(norm.norm(obs))
        no, rw, dn = env.step(mu.cpu().numpy())
        vx = no[:, 0]
        live = ~done_any
        fwd[live] += vx[live] * dt_ctrl
        vx_acc[live] += vx[live]
        alive_len[live] += 1
        done_any |= dn.astype(bool)
        obs = torch.tensor(no, device=dev)
    return dict(fwd_mean=float(fwd.mean()), fwd_max=float(fwd.max()), ep_len_mean=float(alive_len.mean()),
                fall_rate=float(done_any.mean()), vx_mean=float((vx_acc / np.maximum(alive_len, 1)).mean()))


if __name__ == "__main__":
    sys.exit("use ppo_fused.py for training")
