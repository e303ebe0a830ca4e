"""Benchmark of the fused rollout on one MI355X: the BASELINE metric (physics substeps/s and ms per
fused rollout, N=8192, H=32, S=10, pgs=8, MLP 100-256-256 tanh), with the physics kernel's
roofline fraction and the CPU oracle timed on this host beside it.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3|4] [--no-cpu]

A "step" is one fused rollout (one g1_rollout call: H control steps x S substeps for all N worlds)
with the policy weights and frozen statistics already resident in HBM. Prints ONE JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "g1.cu_amd", "scripts"))
sys.path.insert(0, os.path.join(ROOT, "g1.cu_amd"))

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0            # MI355X published HBM3E bandwidth
RTX3090_SUBSTEPS_PER_S = 4.96e6  # reference's published fused-rollout number (N=8192, H=32, S=10)
# HBM bytes per k_physics dispatch at config 3 from rocprofv3 FETCH_SIZE / WRITE_SIZE, each scaled
# by the same counter on a copy of known size (profiles/k_physics_config3_pmc.md)
PHYS_TRAFFIC_BYTES = {3: 16.04e6}


def bytes_per_world_substep(c, p):
    """Algorithmic bytes of one world-substep with c contacts and p PGS sweeps: every per-world
    intermediate of the reference algorithm written once and read once in fp32, the PGS matrix
    read once per sweep (B_ws(c) = 4 [2 (3244 + 1390 c + 35 [c>0]) + 16 c^2 (1 + p)])."""
    return 4.0 * (2.0 * (3244 + 1390 * c + 35 * (c > 0)) + 16.0 * c * c * (1 + p))


def cpu_baseline(cfg, threads, seed=0):
    """The CPU oracle's rollout (fp32, OpenMP over worlds) on a bounded sample of the workload."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    import configs
    oracle.build()
    rng = np.random.default_rng(seed)
    n = min(8192, cfg["N"])   # config 3 whole (~25 core-seconds); config 4 as its first 8192 worlds
    H, S = cfg["H"], cfg["S"]
    qp, qv, pa, st = configs.reset_states(rng, n)
    W = configs.policy_init(rng, hidden=cfg["hidden"])
    an, rn = configs.rollout_noise(rng, H, n)
    mean = np.zeros(100, np.float32); var = np.ones(100, np.float32)
    t0 = time.perf_counter()
    oracle.rollout(qp, qv, pa, st, W, mean, var, an, rn, H, S=S, pgs=cfg["pgs"], hidden=cfg["hidden"],
                   act=cfg["act"], threads=threads)
    dt = time.perf_counter() - t0
    return dict(value=n * H * S / dt, unit="substeps/s", cores=threads, kind="port",
                sample=f"oracle rollout of {n} worlds x {H} control steps x {S} substeps "
                       f"({n * H * S} world-substeps, {dt:.1f} s wall on {threads} threads)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=3, choices=[3, 4])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--policy", choices=["random", "trained"], default="random",
                    help="random-init weights (the configuration's definition) or the reference's trained "
                         "checkpoint (g1.cu_amd/data/trained_policy_finish_best.npz: walking contact mix)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the rollout shards worlds across GPUs with no exchange, "
              "and this build runs on single-GPU boxes only (--gpus 1).", file=sys.stderr)
        sys.exit(2)

    import torch
    import configs
    import g1env
    cfg = configs.ROLLOUT_CONFIGS[args.config]
    N, H, S, pgs = cfg["N"], cfg["H"], cfg["S"], cfg["pgs"]
    rng = np.random.default_rng(1234)
    env = g1env.Env(N, substeps=S, pgs_iters=pgs, seed=1)
    env.set_policy(cfg["hidden"], cfg["act"])
    env.reset()
    if args.policy == "trained":
        if args.config != 3:
            sys.exit("the trained checkpoint has the config-3 policy shape (100-256-256 tanh)")
        tp = np.load(os.path.join(ROOT, "g1.cu_amd", "data", "trained_policy_finish_best.npz"))
        W = torch.from_numpy(tp["W"]).cuda()
        mean = torch.from_numpy(tp["obs_mean"]).cuda(); var = torch.from_numpy(tp["obs_var"]).cuda()
    else:
        W = torch.from_numpy(configs.policy_init(rng, hidden=cfg["hidden"])).cuda()
        mean = torch.zeros(100, device="cuda"); var = torch.ones(100, device="cuda")
    traj = g1env.Trajectory(H, N)

    def rollout():
        traj.run(env, W, mean, var)

    for _ in range(args.warmup):
        rollout()
    torch.cuda.synchronize()
    env.ncon_hist(enable=True)
    env.profile(1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        rollout()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    pr = env.profile_read()
    env.profile(0)
    hist = env.ncon_hist(enable=False)
    if env.check() != 0:
        sys.exit("physics work queue error: results undefined")
    ms_rollout = wall * 1e3 / args.steps
    substeps_per_s = N * H * S / (wall / args.steps)

    phys_ms, phys_n, pol_ms = pr["physics_ms"], pr["physics_launches"], pr["policy_ms"]
    nsub = hist.sum()
    bytes_total = sum(int(hist[c]) * bytes_per_world_substep(c, pgs) for c in range(9))
    launches = phys_n
    bytes_per_launch = bytes_total / max(launches, 1)
    avg_launch_s = phys_ms / max(launches, 1) * 1e-3
    achieved = bytes_per_launch / avg_launch_s / 1e9
    cbar = float((hist * np.arange(9)).sum() / max(nsub, 1))
    policy_flops = 2 * N * (H + 1) * sum(a * b for a, b in zip((100,) + tuple(cfg["hidden"]),
                                                                 tuple(cfg["hidden"]) + (30,)))
    out = {
        "metric": "physics substeps/sec + ms per fused rollout (N=8192, H=32, 10 substeps) on 1 GPU",
        "value": substeps_per_s,
        "unit": "substeps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_rollout,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": substeps_per_s / RTX3090_SUBSTEPS_PER_S if args.config == 3 else None,
        "dtype": "fp32",
        "data": ("synthetic (stand-pose resets, random-init policy N(0,1/fan_in), library Philox noise)"
                 if args.policy == "random" else
                 "stand-pose resets, the reference's trained policy (models/ppo_ckpt/finish_best.pt, converted) "
                 "with its frozen obs statistics, library Philox noise"),
        "config": {"workload": f"config{args.config}{' (trained policy)' if args.policy == 'trained' else ''}: "
                               f"fused rollout N={N} H={H} S={S} pgs={pgs} "
                               f"policy 100-{'-'.join(map(str, cfg['hidden']))} {'tanh' if cfg['act'] == 0 else 'ELU'}",
                   "N": N, "H": H, "substeps": S, "pgs": pgs, "ms_per_rollout": ms_rollout},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": PHYS_TRAFFIC_BYTES.get(args.config),
                     "kernel": "k_physics", "avg_launch_ms": phys_ms / max(launches, 1),
                     "algorithmic_bytes_per_launch": bytes_per_launch, "mean_ncon": cbar},
        "phases": {"physics_ms_per_rollout": phys_ms / args.steps, "policy_ms_per_rollout": pol_ms / args.steps,
                   "policy_tflops": policy_flops / (pol_ms / args.steps * 1e-3) / 1e12 if pol_ms > 0 else None,
                   "ncon_hist": hist.tolist()},
    }
    env.close()
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        out["cpu_baseline"] = cpu_baseline(cfg, threads)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
