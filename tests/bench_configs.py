"""Measurements of the benchmark configurations other than the headline rollout, GPU and CPU side by
side (the headline config-3 rollout is bench.py's; config 4 is `bench.py --config 4`).

    python tests/bench_configs.py [--cpu-threads T] [--skip-cpu]

A measurement harness beside the test suite (it checks the GPU against the CPU oracle), not part of
the library.

config 0  qacc of 256 perturbed single-world states (no contact, plain factor): fp64 CPU oracle time
          per state (1 thread) and the GPU's fp32 relerr against it.
config 1  N=8192 smooth dynamics (no contact, plain factor, semi-implicit Euler with the env's
          velocity guard: full-range random torques make the unconstrained robot's explicit Euler
          diverge within ~50 substeps), 1000 substeps with tau resampled every 10: GPU substeps/s;
          free-run drift of 1000 substeps against the fp32 CPU oracle on 64 worlds; CPU oracle
          world-substeps/s (1 thread and T threads).
config 2  N=8192 contact solve on config-2 states (0..8 penetrating spheres, mu=1.0, pgs=8): GPU
          qacc evaluations/s with the realised contact histogram, relerr against the fp32 oracle;
          CPU oracle evaluations/s.
config 3/4 CPU oracle rollout world-substeps/s at N=1024 (the GPU numbers come from bench.py).
standing  the physics-only bench of the reference (scripts/bench_env_phys.py: g1_env_bench_phys
          after g1_env_reset, zero action, S=10, pgs=8) at N=8192 and 16384: substeps/s and the
          contact-count histogram of the standing robot (continuous foot contact).
Prints one JSON object per line.
"""
import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, os.path.join(ROOT, "g1.cu_amd", "scripts"))
sys.path.insert(0, os.path.join(ROOT, "g1.cu_amd"))

import numpy as np  # noqa: E402


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    oracle.build()
    return oracle


def relerr_rows(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return np.linalg.norm(a - b, axis=-1) / np.maximum(np.linalg.norm(b, axis=-1), 1e-30)


def timed(fn, min_s=0.0):
    t0 = time.perf_counter(); fn(); dt = time.perf_counter() - t0
    return dt


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--cpu-threads", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--skip-cpu", action="store_true")
    args = ap.parse_args()
    import torch
    import configs
    import g1env
    orc = _oracle()
    T = args.cpu_threads
    dev = "cuda"
    out = lambda d: print(json.dumps(d), flush=True)

    # ---------------- config 0
    qp, qv, tau = configs.config0()
    t64 = timed(lambda: orc.qacc(qp, qv, tau=tau, pgs=0, dtype=np.float64, contact=False, threads=1))
    ref64, _ = orc.qacc(qp, qv, tau=tau, pgs=0, dtype=np.float64, contact=False)
    q = torch.from_numpy(qp.astype(np.float32)).to(dev); v = torch.from_numpy(qv.astype(np.float32)).to(dev)
    t = torch.from_numpy(tau.astype(np.float32)).to(dev)
    qa = torch.zeros(len(qp), 35, device=dev); nc = torch.zeros(len(qp), dtype=torch.int32, device=dev)
    g1env.lib.g1_probe_qacc(len(qp), g1env.dev_ptr(q), g1env.dev_ptr(v), g1env.dev_ptr(t), 0, 0, 0, 0.6, g1env.dev_ptr(qa), g1env.dev_ptr(nc))
    torch.cuda.synchronize()
    out(dict(config=0, cpu_fp64_us_per_state=t64 / len(qp) * 1e6, cpu_threads=1,
             gpu_fp32_vs_fp64_worst_relerr=float(relerr_rows(qa.cpu().numpy(), ref64).max())))

    # ---------------- config 1
    N, SUB, HOLD = 8192, 1000, 10
    rng = np.random.default_rng(1)
    qp, qv, _ = configs.config0(seed=11, n=N)
    taus = [configs.random_torque(N, rng).astype(np.float32) for _ in range(SUB // HOLD)]
    dq = torch.from_numpy(qp.astype(np.float32)).to(dev); dv = torch.from_numpy(qv.astype(np.float32)).to(dev)
    dts = [torch.from_numpy(x).to(dev) for x in taus]
    qa = torch.zeros(N, 35, device=dev); nc = torch.zeros(N, dtype=torch.int32, device=dev)

    def run_c1(dq_, dv_, n):
        for k in range(SUB // HOLD):
            g1env.lib.g1_dynamics_bench(n, g1env.dev_ptr(dq_), g1env.dev_ptr(dv_), g1env.dev_ptr(dts[k][:n]), HOLD, 0, 0, 1, 8, 0.6,
                                       g1env.dev_ptr(qa), g1env.dev_ptr(nc))
    run_c1(dq.clone(), dv.clone(), N); torch.cuda.synchronize()   # warm-up
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(); run_c1(dq, dv, N); e1.record(); torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    # free-run drift vs the fp32 oracle on 64 worlds
    n64 = 64
    gq = torch.from_numpy(qp[:n64].astype(np.float32)).to(dev); gv = torch.from_numpy(qv[:n64].astype(np.float32)).to(dev)
    run_c1(gq, gv, n64); torch.cuda.synchronize()
    oq, ov = qp[:n64].astype(np.float32), qv[:n64].astype(np.float32)
    for k in range(SUB // HOLD):
        oq, ov, _, _ = orc.dynamics(oq, ov, taus[k][:n64], nsub=HOLD, guard=True, threads=T)
    drift_q = relerr_rows(gq.cpu().numpy(), oq); drift_v = relerr_rows(gv.cpu().numpy(), ov)
    rec = dict(config=1, N=N, substeps=SUB, gpu_ms=ms, gpu_substeps_per_s=N * SUB / (ms * 1e-3),
               drift_1000_substeps_64_worlds=dict(qpos_median=float(np.median(drift_q)), qpos_worst=float(drift_q.max()),
                                                  qvel_median=float(np.median(drift_v)), qvel_worst=float(drift_v.max())))
    if not args.skip_cpu:
        for thr, n in ((1, 256), (T, 1024)):
            qq, vv = qp[:n].astype(np.float32), qv[:n].astype(np.float32)
            dt1 = timed(lambda: orc.dynamics(qq, vv, taus[0][:n], nsub=100, guard=True, threads=thr))
            rec[f"cpu_{thr}thr_world_substeps_per_s"] = n * 100 / dt1
    out(rec)

    # ---------------- config 2
    qp2, qv2, k2 = configs.config2(lambda x: orc.fk(x, dtype=np.float64), n=N)
    q = torch.from_numpy(qp2.astype(np.float32)).to(dev); v = torch.from_numpy(qv2.astype(np.float32)).to(dev)
    t0 = torch.zeros(N, 35, device=dev)
    qa = torch.zeros(N, 35, device=dev); nc = torch.zeros(N, dtype=torch.int32, device=dev)
    call = lambda: g1env.lib.g1_probe_qacc(N, g1env.dev_ptr(q), g1env.dev_ptr(v), g1env.dev_ptr(t0), 0, 1, 8, 1.0, g1env.dev_ptr(qa), g1env.dev_ptr(nc))
    call(); torch.cuda.synchronize()
    reps = 50
    e0.record()
    for _ in range(reps):
        call()
    e1.record(); torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    ref, rnc = orc.qacc(qp2, qv2, pgs=8, mu=1.0, threads=T)
    rel = relerr_rows(qa.cpu().numpy(), ref)
    rec = dict(config=2, N=N, mu=1.0, pgs=8, gpu_ms_per_solve_batch=ms, gpu_solves_per_s=N / (ms * 1e-3),
               ncon_hist=np.bincount(nc.cpu().numpy(), minlength=9).tolist(),
               gpu_vs_fp32_oracle_worst_relerr=float(rel.max()), ncon_equal=bool((nc.cpu().numpy() == rnc).all()))
    if not args.skip_cpu:
        for thr, n in ((1, 512), (T, 4096)):
            dt2 = timed(lambda: orc.qacc(qp2[:n], qv2[:n], pgs=8, mu=1.0, threads=thr))
            rec[f"cpu_{thr}thr_solves_per_s"] = n / dt2
    out(rec)

    # ---------------- config 3 through the host-step path: H control steps of g1_env_step with host
    # numpy buffers (the reference's non-fused loop, scripts/ppo.py evaluate / DEVLOG's host-loop rollout)
    N3, H3 = 8192, 32
    env = g1env.Env(N3, substeps=10, pgs_iters=8, seed=1)
    env.reset()
    acts = np.random.default_rng(2).normal(0, 0.5, (H3, N3, 29)).astype(np.float32)
    for t in range(4):
        env.step(acts[t])
    t0 = time.perf_counter()
    for t in range(H3):
        env.step(acts[t])
    dt_h = time.perf_counter() - t0
    env.close()
    out(dict(config="3-host-step", N=N3, H=H3, ms_per_rollout=dt_h * 1e3, ms_per_step=dt_h * 1e3 / H3,
             substeps_per_s=N3 * H3 * 10 / dt_h))

    # ---------------- standing regime: physics-only bench after reset with zero action (reference
    # scripts/bench_env_phys.py: 5 warm-up control steps, then K = 50 timed)
    for n_st in (8192, 16384):
        with g1env.Env(n_st, substeps=10, pgs_iters=8, seed=1) as env:
            env.reset()
            env.bench_phys(5)
            env.ncon_hist(enable=True)
            t0 = time.perf_counter()
            env.bench_phys(50)
            dt_s = time.perf_counter() - t0
            hist = env.ncon_hist(enable=False)
            assert env.check() == 0
        contact = hist[1:].sum()
        out(dict(config="standing-physics", N=n_st, K=50, S=10, ms=dt_s * 1e3,
                 substeps_per_s=n_st * 50 * 10 / dt_s, ncon_hist=hist.tolist(),
                 share_ncon_6_7_8_of_contact_substeps=float(hist[6:9].sum() / max(contact, 1)),
                 mean_ncon=float((hist * np.arange(9)).sum() / max(hist.sum(), 1))))

    # ---------------- configs 3 and 4: CPU oracle rollout rate (GPU: bench.py)
    if not args.skip_cpu:
        for cfgid in (3, 4):
            cfg = configs.ROLLOUT_CONFIGS[cfgid]
            rng = np.random.default_rng(5)
            n, H = 1024, 4
            qp3, qv3, pa3, st3 = configs.reset_states(rng, n)
            W = configs.policy_init(rng, hidden=cfg["hidden"])
            an, rn = configs.rollout_noise(rng, H, n)
            mean = np.zeros(100, np.float32); var = np.ones(100, np.float32)
            rec = dict(config=cfgid, cpu_sample=f"oracle rollout, {n} worlds x {H} control steps x {cfg['S']} substeps")
            for thr in (1, T):
                a = [x.copy() for x in (qp3, qv3, pa3, st3)]
                dt3 = timed(lambda: orc.rollout(*a, W, mean, var, an, rn, H, S=cfg["S"], pgs=cfg["pgs"],
                                                hidden=cfg["hidden"], act=cfg["act"], threads=thr))
                rec[f"cpu_{thr}thr_world_substeps_per_s"] = n * H * cfg["S"] / dt3
            out(rec)
    import platform
    cpu = "unknown"
    try:
        cpu = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except Exception:
        pass
    out(dict(host_cpu=cpu, nproc=os.cpu_count(), threads_used=T, python=platform.python_version()))


if __name__ == "__main__":
    main()
