"""ctypes front-end of the CPU oracle (oracle/libg1oracle.so). TEST INFRASTRUCTURE ONLY.

Importable only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, where it is the
checker. The product path (g1.cu_amd/, libg1env.so) never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libg1oracle.so")

NQ, NV, NBODY, ACT, OBS = 36, 35, 31, 29, 100
MU_MODEL = 0.6

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_c = ctypes


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load():
    if not os.path.exists(LIB):
        build()
    lib = ctypes.CDLL(LIB)
    for suf, fp, real in (("f", _f32p, _c.c_float), ("d", _f64p, _c.c_double)):
        getattr(lib, f"orc_fk_{suf}").argtypes = [_c.c_int, fp, fp, fp, fp]
        getattr(lib, f"orc_bias_{suf}").argtypes = [_c.c_int, fp, fp, fp, fp]
        getattr(lib, f"orc_mass_{suf}").argtypes = [_c.c_int, fp, fp]
        getattr(lib, f"orc_solve_{suf}").argtypes = [_c.c_int, fp, _c.c_void_p, fp, fp, _c.c_int]
        getattr(lib, f"orc_qacc_{suf}").argtypes = [_c.c_int, fp, fp, fp, _c.c_void_p, _c.c_int, real, fp,
                                                    _c.c_void_p, _c.c_int, _c.c_int]
        getattr(lib, f"orc_substep_{suf}").argtypes = [_c.c_int, fp, fp, fp, _c.c_int, real, _c.c_void_p,
                                                       _c.c_void_p, _c.c_int]
        getattr(lib, f"orc_dyn_{suf}").argtypes = [_c.c_int, fp, fp, fp] + [_c.c_int] * 5 + [real, _c.c_void_p,
                                                    _c.c_void_p, _c.c_int]
        getattr(lib, f"orc_pgs_{suf}").argtypes = [_c.c_int, fp, fp, fp, _c.c_int]
        getattr(lib, f"orc_impedance_{suf}").argtypes = [real]
        getattr(lib, f"orc_impedance_{suf}").restype = real
        getattr(lib, f"orc_bdt_{suf}").argtypes = [fp]
        getattr(lib, f"orc_smooth_traj_{suf}").argtypes = [fp, fp, _c.c_int, fp, fp]
        getattr(lib, f"orc_implicit_traj_{suf}").argtypes = [fp, fp, fp, fp, _c.c_int, fp, fp]
    lib.orc_fk_recursive_f.argtypes = [_c.c_int, _f32p, _f32p, _f32p, _f32p]
    lib.orc_set_reference_order.argtypes = [_c.c_int]
    lib.orc_qacc_debug_f.argtypes = [_f32p, _f32p, _f32p, _c.c_void_p, _c.c_int, _c.c_float] + [_f32p] * 7
    lib.orc_qacc_debug_f.restype = _c.c_int
    lib.orc_obs_f.argtypes = [_c.c_int, _f32p, _f32p, _f32p, _f32p]
    lib.orc_sincos_f.argtypes = [_c.c_long, _f32p, _f32p, _f32p]
    lib.orc_policy_params.argtypes = [_c.c_int, _i32p, _c.c_int]
    lib.orc_policy_params.restype = _c.c_long
    lib.orc_mlp_f.argtypes = [_c.c_int, _c.c_int, _i32p, _c.c_int, _f32p, _f32p, _f32p, _f32p, _f32p]
    lib.orc_env_advance_f.argtypes = [_c.c_int, _f32p, _f32p, _f32p, _i32p, _f32p, _f32p, _c.c_int, _c.c_int,
                                      _c.c_float, _f32p, _f32p, _c.c_int]
    lib.orc_rollout_f.argtypes = ([_c.c_int] * 4 + [_c.c_float] + [_f32p] * 3 + [_i32p] + [_f32p] +
                                  [_c.c_int, _i32p, _c.c_int] + [_f32p] * 11 + [_c.c_void_p, _c.c_int])
    return lib


_lib = None
_flib = None

COUNT_KEYS = ("add", "mul", "fma", "div", "sqrt", "cmp", "trans")


def flops_lib():
    """The operation-counting instantiation of the oracle (oracle/libg1flops.so)."""
    global _flib
    if _flib is None:
        path = os.path.join(HERE, "libg1flops.so")
        if not os.path.exists(path):
            build()
        _flib = ctypes.CDLL(path)
        _flib.flc_substep.argtypes = [_f32p, _f32p, _f32p, _c.c_int, _c.c_float, _c.c_int,
                                      np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")]
        _flib.flc_substep.restype = _c.c_int
        _flib.flc_step_overhead.argtypes = [_c.c_int, np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")]
    return _flib


def flops_of(counts):
    """Floating-point operations of an operation count: add/sub, mul, div and sqrt one each, a fused
    multiply-add two; comparisons and transcendental calls are reported apart."""
    return counts["add"] + counts["mul"] + 2 * counts["fma"] + counts["div"] + counts["sqrt"]


def count_substep(qpos, qvel, target, pgs=8, mu=MU_MODEL, ref_order=True):
    """Operation counts of one env substep of one world (the reference's association by default).
    Returns (ncon, dict of counts)."""
    out = np.zeros(7)
    nc = flops_lib().flc_substep(_arr(qpos, np.float32), _arr(qvel, np.float32), _arr(target, np.float32), int(pgs),
                                 float(mu), int(ref_order), out)
    return nc, dict(zip(COUNT_KEYS, out.astype(np.int64).tolist()))


def count_step_overhead(ref_order=True):
    """Operation counts of a control step's work outside its substeps (targets, reward, termination)."""
    out = np.zeros(7)
    flops_lib().flc_step_overhead(int(ref_order), out)
    return dict(zip(COUNT_KEYS, out.astype(np.int64).tolist()))


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _dt(dtype):
    return "f" if np.dtype(dtype) == np.float32 else "d"


def _arr(x, dtype):
    return np.ascontiguousarray(x, dtype=dtype)


def set_reference_order(on):
    """Associate the contact basis solves, the PGS row sums and the reward's energy and
    action-penalty totals as the reference's serial loops do (on), or as the GPU kernel does (off,
    the default). Same algorithm; the results differ at rounding level."""
    lib().orc_set_reference_order(int(bool(on)))


class reference_order:
    """Context manager: the oracle in the reference's association inside the block."""

    def __enter__(self):
        set_reference_order(True)

    def __exit__(self, *exc):
        set_reference_order(False)


def bdt(dtype=np.float32):
    """Implicit-damping diagonal dt*kd on the actuated dofs (reference: src/g1_env.cu:137-139)."""
    out = np.zeros(NV, dtype)
    getattr(lib(), f"orc_bdt_{_dt(dtype)}")(out)
    return out


def fk(qpos, dtype=np.float64):
    q = _arr(np.atleast_2d(qpos), dtype)
    n = q.shape[0]
    xp = np.zeros((n, NBODY, 3), dtype); xq = np.zeros((n, NBODY, 4), dtype); xi = np.zeros((n, NBODY, 3), dtype)
    getattr(lib(), f"orc_fk_{_dt(dtype)}")(n, q, xp, xq, xi)
    return xp, xq, xi


def fk_recursive(qpos):
    """fp32 forward kinematics by the reference's root -> leaf recursion (src/dynamics.cuh:47-88),
    the association check of fk's ancestor doubling."""
    q = _arr(np.atleast_2d(qpos), np.float32)
    n = q.shape[0]
    xp = np.zeros((n, NBODY, 3), np.float32); xq = np.zeros((n, NBODY, 4), np.float32)
    xi = np.zeros((n, NBODY, 3), np.float32)
    lib().orc_fk_recursive_f(n, q, xp, xq, xi)
    return xp, xq, xi


def bias(qpos, qvel, dtype=np.float64):
    q = _arr(np.atleast_2d(qpos), dtype); v = _arr(np.atleast_2d(qvel), dtype)
    n = q.shape[0]
    S = np.zeros((n, NV, 6), dtype); b = np.zeros((n, NV), dtype)
    getattr(lib(), f"orc_bias_{_dt(dtype)}")(n, q, v, S, b)
    return S, b


def mass(qpos, dtype=np.float64):
    q = _arr(np.atleast_2d(qpos), dtype)
    n = q.shape[0]
    Mo = np.zeros((n, NV, NV), dtype)
    getattr(lib(), f"orc_mass_{_dt(dtype)}")(n, q, Mo)
    return Mo


def solve(qpos, x, Bdt=None, multi=False, dtype=np.float64):
    q = _arr(np.atleast_2d(qpos), dtype); xx = _arr(np.atleast_2d(x), dtype)
    n = q.shape[0]
    y = np.zeros((n, NV), dtype)
    B = None if Bdt is None else _arr(Bdt, dtype)
    getattr(lib(), f"orc_solve_{_dt(dtype)}")(n, q, None if B is None else B.ctypes.data, xx, y, int(multi))
    return y


def qacc(qpos, qvel, tau=None, Bdt=None, pgs=8, mu=MU_MODEL, dtype=np.float32, threads=1, contact=True):
    q = _arr(np.atleast_2d(qpos), dtype); v = _arr(np.atleast_2d(qvel), dtype)
    n = q.shape[0]
    t = np.zeros((n, NV), dtype) if tau is None else _arr(np.atleast_2d(tau), dtype)
    B = None if Bdt is None else _arr(Bdt, dtype)
    out = np.zeros((n, NV), dtype); nc = np.zeros(n, np.int32)
    getattr(lib(), f"orc_qacc_{_dt(dtype)}")(n, q, v, t, None if B is None else B.ctypes.data, pgs, mu, out,
                                             nc.ctypes.data, threads, int(contact))
    return out, nc


def substep(qpos, qvel, target, pgs=8, mu=MU_MODEL, dtype=np.float32, threads=1):
    """One substep in place on copies; returns (qpos', qvel', qacc, ncon)."""
    q = _arr(np.atleast_2d(qpos), dtype).copy(); v = _arr(np.atleast_2d(qvel), dtype).copy()
    tg = _arr(np.atleast_2d(target), dtype)
    n = q.shape[0]
    qa = np.zeros((n, NV), dtype); nc = np.zeros(n, np.int32)
    getattr(lib(), f"orc_substep_{_dt(dtype)}")(n, q, v, tg, pgs, mu, qa.ctypes.data, nc.ctypes.data, threads)
    return q, v, qa, nc


def dynamics(qpos, qvel, tau, nsub=1, contact=False, damped=False, guard=False, pgs=8, mu=MU_MODEL, dtype=np.float32,
             threads=1):
    """nsub tau-driven substeps on copies; returns (qpos', qvel', qacc of the last substep, ncon)."""
    q = _arr(np.atleast_2d(qpos), dtype).copy(); v = _arr(np.atleast_2d(qvel), dtype).copy()
    t = _arr(np.atleast_2d(tau), dtype)
    n = q.shape[0]
    qa = np.zeros((n, NV), dtype); nc = np.zeros(n, np.int32)
    getattr(lib(), f"orc_dyn_{_dt(dtype)}")(n, q, v, t, nsub, int(contact), int(damped), int(guard), pgs, mu, qa.ctypes.data,
                                            nc.ctypes.data, threads)
    return q, v, qa, nc


def qacc_debug(qpos, qvel, tau=None, Bdt=None, pgs=8, mu=MU_MODEL):
    q = _arr(qpos, np.float32); v = _arr(qvel, np.float32)
    t = np.zeros(NV, np.float32) if tau is None else _arr(tau, np.float32)
    B = None if Bdt is None else _arr(Bdt, np.float32)
    qa = np.zeros(NV, np.float32); A = np.zeros(32 * 32, np.float32)
    b, f, R, aref = (np.zeros(32, np.float32) for _ in range(4))
    qs = np.zeros(NV, np.float32)
    nc = lib().orc_qacc_debug_f(q, v, t, None if B is None else B.ctypes.data, pgs, mu, qa, A, b, f, R, aref, qs)
    ne = 4 * nc
    return dict(ncon=nc, qacc=qa, A=A[:ne * ne].reshape(ne, ne), b=b[:ne], f=f[:ne], R=R[:ne], aref=aref[:ne],
                qacc_smooth=qs)


def smooth_traj(qpos0, qvel0, nsteps, dtype=np.float64):
    """Smooth multibody trajectory (no actuation/contact), semi-implicit Euler."""
    q0 = _arr(qpos0, dtype); v0 = _arr(qvel0, dtype)
    qo = np.zeros((nsteps + 1, NQ), dtype); vo = np.zeros((nsteps + 1, NV), dtype)
    getattr(lib(), f"orc_smooth_traj_{_dt(dtype)}")(q0, v0, nsteps, qo, vo)
    return qo, vo


def implicit_traj(qpos0, qvel0, Bdt, targets, dtype=np.float64):
    """Implicit-PD trajectory (contacts ignored) with per-step targets [nsteps, 29]."""
    q0 = _arr(qpos0, dtype); v0 = _arr(qvel0, dtype); B = _arr(Bdt, dtype); tg = _arr(targets, dtype)
    n = tg.shape[0]
    qo = np.zeros((n + 1, NQ), dtype); vo = np.zeros((n + 1, NV), dtype)
    getattr(lib(), f"orc_implicit_traj_{_dt(dtype)}")(q0, v0, B, tg, n, qo, vo)
    return qo, vo


def pgs(A, b, iters, dtype=np.float64):
    A = _arr(A, dtype); b = _arr(b, dtype)
    f = np.zeros_like(b)
    getattr(lib(), f"orc_pgs_{_dt(dtype)}")(b.shape[0], A, b, f, iters)
    return f


def impedance(pos, dtype=np.float64):
    return getattr(lib(), f"orc_impedance_{_dt(dtype)}")(pos)


def sincos(x):
    """sin and cos of float32 values as the oracle evaluates them: fp64 libm, rounded once."""
    x = _arr(np.ravel(x), np.float32)
    sn, cs = np.zeros_like(x), np.zeros_like(x)
    lib().orc_sincos_f(x.size, x, sn, cs)
    return sn, cs


def obs(qp, qv, pa):
    qp = _arr(np.atleast_2d(qp), np.float32); qv = _arr(np.atleast_2d(qv), np.float32)
    pa = _arr(np.atleast_2d(pa), np.float32)
    out = np.zeros((qp.shape[0], OBS), np.float32)
    lib().orc_obs_f(qp.shape[0], qp, qv, pa, out)
    return out


def policy_params(hidden=(256, 256), act=0):
    h = np.asarray(hidden, np.int32)
    return int(lib().orc_policy_params(len(hidden), h, act))


def mlp(W, x, hidden=(256, 256), act=0):
    x = _arr(np.atleast_2d(x), np.float32); W = _arr(W, np.float32)
    n = x.shape[0]
    mu = np.zeros((n, ACT), np.float32); ls = np.zeros((n, ACT), np.float32); v = np.zeros(n, np.float32)
    lib().orc_mlp_f(n, len(hidden), np.asarray(hidden, np.int32), act, W, x, mu, ls, v)
    return mu, ls, v


def env_advance(qp, qv, pa, steps, act, reset_noise, S=10, pgs=8, mu=MU_MODEL, threads=1):
    """One control step for a batch; arrays are updated IN PLACE. Returns (rew, done)."""
    n = qp.shape[0]
    rew = np.zeros(n, np.float32); done = np.zeros(n, np.float32)
    lib().orc_env_advance_f(n, qp, qv, pa, steps, _arr(act, np.float32), _arr(reset_noise, np.float32), S, pgs, mu,
                            rew, done, threads)
    return rew, done


def rollout(qp, qv, pa, steps, W, mean, var, act_noise, reset_noise, H, S=10, pgs=8, mu=MU_MODEL,
            hidden=(256, 256), act=0, threads=1, hist=False):
    """Fused rollout with pre-generated noise; state arrays updated IN PLACE."""
    N = qp.shape[0]
    O = np.zeros((H, N, OBS), np.float32); A = np.zeros((H, N, ACT), np.float32)
    LP, V, R, D = (np.zeros((H, N), np.float32) for _ in range(4))
    Vlast = np.zeros(N, np.float32)
    h = np.zeros(9, np.int32)
    lib().orc_rollout_f(N, H, S, pgs, mu, qp, qv, pa, steps, _arr(W, np.float32), len(hidden),
                        np.asarray(hidden, np.int32), act, _arr(mean, np.float32), _arr(var, np.float32),
                        _arr(act_noise, np.float32), _arr(reset_noise, np.float32), O, A, LP, V, R, D, Vlast,
                        h.ctypes.data, threads)
    out = dict(O=O, A=A, LP=LP, V=V, R=R, D=D, Vlast=Vlast)
    if hist:
        out["ncon_hist"] = h
    return out
