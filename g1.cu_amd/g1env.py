"""Python side of libg1env.so: the ctypes binding of every entry point in include/g1env.h, and a
small handle wrapper used by the tests, the benchmarks and the PPO driver.

The binding of the reference's eleven entry points uses exactly the argtypes the reference's
Python declares for them (scripts/ppo.py:24-32, scripts/ppo_fused.py:27-28), so code written
against the reference's binding and code written against this module drive the same symbols the
same way. torch is imported before the library is loaded: torch ships its own HIP runtime under
the same soname, and loading it first makes the process use one runtime.

The library must be built (python g1.cu_amd/build.py); importing this module without it raises
ImportError. There is no fallback path.
"""
import ctypes
import os
from collections import namedtuple

import numpy as np
import torch  # noqa: F401  (before the library: one HIP runtime per process)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libg1env.so")

NQ, NV, OBS_DIM, ACT_DIM = 36, 35, 100, 29

_c = ctypes
_fp = _c.POINTER(_c.c_float)
_ip = _c.POINTER(_c.c_int)
_vp = _c.c_void_p

# name -> (restype, argtypes). The first block is the reference's surface with the reference
# binding's argtypes; the rest are this build's additive exports.
SIGNATURES = {
    "g1_env_create": (_vp, [_c.c_int, _c.c_int, _c.c_int, _c.c_ulong]),
    "g1_env_reset": (None, [_vp, _fp]),
    "g1_env_step": (None, [_vp, _fp, _fp, _fp, _fp]),
    "g1_rollout": (None, [_vp, _c.c_int] + [_vp] * 10),
    "g1_env_qpos": (None, [_vp, _fp]),
    "g1_env_qpos_all": (None, [_vp, _fp]),
    "g1_env_bench_phys": (None, [_vp, _c.c_int]),
    "g1_occupancy_report": (None, []),
    "g1_env_obs_dim": (_c.c_int, []),
    "g1_env_act_dim": (_c.c_int, []),
    "g1_env_destroy": (None, [_vp]),
    # additive
    "g1_rollout_ex": (None, [_vp, _c.c_int] + [_vp] * 12),
    "g1_rollout_noalloc": (_c.c_int, [_vp, _c.c_int] + [_vp] * 12),
    "g1_env_set_state": (None, [_vp, _fp, _fp, _fp, _ip]),
    "g1_env_get_state": (None, [_vp, _fp, _fp, _fp, _ip]),
    "g1_env_set_policy": (_c.c_int, [_vp, _c.c_int, _ip, _c.c_int]),
    "g1_env_policy_params": (_c.c_long, [_vp]),
    "g1_env_device_bytes": (_c.c_long, [_vp]),
    "g1_env_set_contact": (None, [_vp, _c.c_float, _c.c_int]),
    "g1_env_ncon_hist": (None, [_vp, _c.c_int, _c.POINTER(_c.c_ulonglong)]),
    "g1_env_profile": (None, [_vp, _c.c_int]),
    "g1_env_profile_read": (None, [_vp, _c.POINTER(_c.c_double)]),
    "g1_env_check": (_c.c_int, [_vp]),
    "g1_env_set_handover": (_c.c_int, [_vp, _c.c_int]),
    "g1_env_set_fused": (_c.c_int, [_vp, _c.c_int]),
    "g1_probe_qacc": (None, [_c.c_int, _vp, _vp, _vp, _c.c_int, _c.c_int, _c.c_int, _c.c_float, _vp, _vp]),
    "g1_probe_substep": (None, [_c.c_int, _vp, _vp, _vp, _c.c_int, _c.c_int, _c.c_float, _vp, _vp]),
    "g1_probe_policy": (_c.c_int, [_c.c_int, _c.c_int, _ip, _c.c_int, _vp, _vp, _vp, _vp]),
    "g1_dynamics_bench": (None, [_c.c_int, _vp, _vp, _vp] + [_c.c_int] * 5 + [_c.c_float, _vp, _vp]),
    "g1_probe_divide": (None, [_c.c_int, _vp, _vp, _vp, _vp]),
    "g1_probe_sqrt": (None, [_c.c_int, _vp, _vp]),
    "g1_probe_sincos": (None, [_c.c_int, _vp, _vp, _vp]),
    "g1_probe_sincos_hinge": (None, [_c.c_int, _vp, _vp, _vp]),
    "g1_probe_philox": (None, [_c.c_int, _vp, _vp, _c.c_uint, _c.c_uint]),
}


def _load(path):
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python g1.cu_amd/build.py`")
    handle = _c.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    return handle


lib = _load(LIB_PATH)


def host_ptr(a):
    """float*/int* of a C-contiguous numpy array (checked)."""
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("host array must be C-contiguous")
    return a.ctypes.data_as(_ip if a.dtype == np.int32 else _fp)


def dev_ptr(t):
    """Device address of a contiguous torch tensor (None passes NULL)."""
    if t is None:
        return None
    if not t.is_contiguous():
        raise ValueError("device tensor must be contiguous")
    return _c.c_void_p(t.data_ptr())


State = namedtuple("State", "qpos qvel prev_act steps")


class Env:
    """One library handle: N worlds with S substeps per control step and `pgs` PGS sweeps.

    Host-step use: reset() -> obs, step(actions) -> (obs, reward, done). Device use: run a
    Trajectory. State access (get_state/set_state) and the configuration exports are the additive
    ones of this build."""

    def __init__(self, n_worlds, substeps=10, pgs_iters=8, seed=0):
        self.N, self.S, self.pgs, self.seed = int(n_worlds), int(substeps), int(pgs_iters), int(seed)
        self.h = lib.g1_env_create(self.N, self.S, self.pgs, self.seed)
        self._io = None

    # ---- lifetime
    def close(self):
        if self.h:
            lib.g1_env_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- host-step path
    def _buffers(self):
        if self._io is None:
            self._io = (np.empty((self.N, OBS_DIM), np.float32), np.empty(self.N, np.float32),
                        np.empty(self.N, np.float32))
        return self._io

    def reset(self):
        obs, _, _ = self._buffers()
        lib.g1_env_reset(self.h, host_ptr(obs))
        return obs.copy()

    def step(self, actions):
        obs, rew, done = self._buffers()
        act = np.ascontiguousarray(actions, np.float32).reshape(self.N, ACT_DIM)
        lib.g1_env_step(self.h, host_ptr(act), host_ptr(obs), host_ptr(rew), host_ptr(done))
        return obs.copy(), rew.copy(), done.copy()

    def qpos_all(self):
        out = np.empty((self.N, NQ), np.float32)
        lib.g1_env_qpos_all(self.h, host_ptr(out))
        return out

    def bench_phys(self, K):
        lib.g1_env_bench_phys(self.h, int(K))

    # ---- state access
    def get_state(self):
        st = State(np.empty((self.N, NQ), np.float32), np.empty((self.N, NV), np.float32),
                   np.empty((self.N, ACT_DIM), np.float32), np.empty(self.N, np.int32))
        lib.g1_env_get_state(self.h, *[host_ptr(a) for a in st])
        return st

    def set_state(self, qpos, qvel, prev_act, steps):
        arrs = [np.ascontiguousarray(qpos, np.float32).reshape(self.N, NQ),
                np.ascontiguousarray(qvel, np.float32).reshape(self.N, NV),
                np.ascontiguousarray(prev_act, np.float32).reshape(self.N, ACT_DIM),
                np.ascontiguousarray(steps, np.int32).reshape(self.N)]
        lib.g1_env_set_state(self.h, *[host_ptr(a) for a in arrs])

    # ---- configuration
    def set_policy(self, hidden, activation):
        hid = np.ascontiguousarray(hidden, np.int32)
        if lib.g1_env_set_policy(self.h, len(hid), host_ptr(hid), int(activation)) != 0:
            raise ValueError(f"unsupported policy shape {tuple(hidden)} / activation {activation}")

    def policy_params(self):
        return int(lib.g1_env_policy_params(self.h))

    def set_contact(self, mu, pgs_iters):
        lib.g1_env_set_contact(self.h, float(mu), int(pgs_iters))

    def set_handover(self, fences):
        if lib.g1_env_set_handover(self.h, int(fences)) != 0:
            raise RuntimeError("hand-over mode unavailable on this placement")

    def set_fused(self, on):
        """One persistent launch per rollout (True, the default) or per-step launches (False).
        Returns whether the one-launch form applies to the current policy shape."""
        rc = lib.g1_env_set_fused(self.h, int(bool(on)))
        if rc < 0:
            raise ValueError("invalid rollout form")
        return bool(on) and rc == 0

    def ncon_hist(self, enable=True):
        out = (_c.c_ulonglong * 9)()
        lib.g1_env_ncon_hist(self.h, int(enable), out)
        return np.array(out[:], np.int64)

    def device_bytes(self):
        """Device memory the handle holds (state, queue and staging buffers, packed policies)."""
        return int(lib.g1_env_device_bytes(self.h))

    def check(self):
        """Synchronise and return the work queue's error word (0: none)."""
        return int(lib.g1_env_check(self.h))

    def profile(self, enable):
        lib.g1_env_profile(self.h, int(enable))

    def profile_read(self):
        out = (_c.c_double * 4)()
        lib.g1_env_profile_read(self.h, out)
        return dict(physics_ms=out[0], physics_launches=int(out[1]), policy_ms=out[2], policy_launches=int(out[3]))


class Trajectory:
    """Caller-owned device buffers of one fused rollout, in the ABI's layouts: O [H,N,100] raw
    observations, A [H,N,29] actions, LP/V/R/D [H,N], Vlast [N]."""

    FIELDS = ("O", "A", "LP", "V", "R", "D", "Vlast")

    def __init__(self, H, N, device="cuda"):
        self.H, self.N = int(H), int(N)
        z = lambda *shape: torch.zeros(*shape, device=device, dtype=torch.float32)
        self.O, self.A = z(H, N, OBS_DIM), z(H, N, ACT_DIM)
        self.LP, self.V, self.R, self.D = z(H, N), z(H, N), z(H, N), z(H, N)
        self.Vlast = z(N)

    def tensors(self):
        return [getattr(self, f) for f in self.FIELDS]

    def run(self, env, W, mean, var, act_noise=None, reset_noise=None):
        """Enqueue one fused rollout of H control steps on the null stream (asynchronous).
        W/mean/var and the optional pre-generated noise [H,N,29] are contiguous fp32 device
        tensors; without noise the library's own random streams are used (g1_rollout)."""
        if env.N != self.N:
            raise ValueError("trajectory and env differ in N")
        args = [dev_ptr(t) for t in (W, mean, var, *self.tensors())]
        if act_noise is None and reset_noise is None:
            lib.g1_rollout(env.h, self.H, *args)
        else:
            lib.g1_rollout_ex(env.h, self.H, *args, dev_ptr(act_noise), dev_ptr(reset_noise))

    def numpy(self):
        return {f: getattr(self, f).cpu().numpy() for f in self.FIELDS}
