"""Benchmark of the fused rollout on one MI355X: the BASELINE metric (physics substeps/s and ms per
fused rollout, N=8192, H=32, S=10, pgs=8, MLP 100-256-256 tanh), with the dominant kernel's
roofline and the CPU oracle timed on this host beside it.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3|4] [--no-cpu] [--no-counters]

A "step" is one fused rollout (one g1_rollout call: H control steps x S substeps for all N worlds)
with the policy weights and frozen statistics already resident in HBM. Prints ONE JSON line.

The dominant kernel is k_rollout (the whole rollout in one launch: physics work items and the
policy of 16-world tiles; config 4's three-layer policy runs on the wide tile), or k_physics with
--per-step (the policy and physics launched once per control step). The physics
runs out of registers and LDS and is bound by VALU issue, so `achieved` is the launch's algorithmic
FLOP rate: the reference algorithm's floating-point operations per world-substep by contact count
(g1.cu_amd/roofline.py, counted by an instrumented oracle) summed over the launch's measured contact
histogram, plus (k_rollout) the policy MLP's multiply-adds, divided by the average launch time from
HIP events on the kernel's stream; `peak` is the MI355X fp32 figure. Hardware
counters come from rocprofv3 passes over a one-rollout run of this script, started as child
processes before this process touches the GPU: HBM traffic per dispatch (FETCH_SIZE and
WRITE_SIZE, each scaled by what the counter reads for a copy of known size in the same run),
VALU busy and lane utilisation, LDS utilisation, bank-conflict share and LDS bytes moved. The working-set unit of
the reference algorithm (bytes of every per-world intermediate written and read once) is reported
beside it as `hbm_proxy`: a workload measure, not an HBM ceiling.
"""
import argparse
import csv
import glob
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "g1.cu_amd", "scripts"))
sys.path.insert(0, os.path.join(ROOT, "g1.cu_amd"))

import numpy as np  # noqa: E402

import roofline as rf  # noqa: E402

RTX3090_SUBSTEPS_PER_S = 4.96e6  # reference's published fused-rollout number (N=8192, H=32, S=10)
COPY_MIB = 1024                  # copy of known size that calibrates FETCH_SIZE / WRITE_SIZE
COUNTER_PASSES = (
    ("fetch", ["FETCH_SIZE"]),
    ("write", ["WRITE_SIZE"]),
    ("sq", ["VALUBusy", "VALUUtilization", "LdsUtil", "LDSBankConflict", "SQ_INSTS_VALU", "SQ_INSTS_LDS",
            "SQ_WAVES"]),
    # LDS bytes moved: instruction size x active lanes, in 64-byte units
    ("lds", ["SQ_INSTS_LDS_LOAD_BANDWIDTH", "SQ_INSTS_LDS_STORE_BANDWIDTH"]),
)


def cpu_model():
    """The host CPU's model name (lscpu's "Model name"), from /proc/cpuinfo."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, threads, seed=0):
    """The CPU oracle's rollout (fp32) on a bounded sample of the workload, on `threads` host
    threads (OpenMP over worlds) and on one thread (a sixteenth of the sample)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    import configs
    oracle.build()
    H, S = cfg["H"], cfg["S"]

    def run(n, nthreads):
        rng = np.random.default_rng(seed)
        qp, qv, pa, st = configs.reset_states(rng, n)
        W = configs.policy_init(rng, hidden=cfg["hidden"])
        an, rn = configs.rollout_noise(rng, H, n)
        mean = np.zeros(100, np.float32)
        var = np.ones(100, np.float32)
        t0 = time.perf_counter()
        oracle.rollout(qp, qv, pa, st, W, mean, var, an, rn, H, S=S, pgs=cfg["pgs"], hidden=cfg["hidden"],
                       act=cfg["act"], threads=nthreads)
        return time.perf_counter() - t0

    n = min(8192, cfg["N"])   # config 3 whole (~25 core-seconds); config 4 as its first 8192 worlds
    dt = run(n, threads)
    n1 = n // 16
    dt1 = run(n1, 1)
    return dict(value=n * H * S / dt, unit="substeps/s", cores=threads, kind="port",
                cpu_model=cpu_model(), nproc=os.cpu_count(),
                sample=f"oracle rollout of {n} worlds x {H} control steps x {S} substeps "
                       f"({n * H * S} world-substeps, {dt:.1f} s wall on {threads} threads)",
                single_thread={"value": n1 * H * S / dt1, "unit": "substeps/s", "cores": 1,
                               "sample": f"the first {n1} worlds of the same rollout ({n1 * H * S} "
                                         f"world-substeps, {dt1:.1f} s on one thread)"})


def measure_copy_bandwidth(mib=COPY_MIB, reps=10):
    """BW_meas: device-to-device copy of `mib` MiB timed with HIP events (read + write bytes per
    second), the box's measured HBM stream bandwidth."""
    import torch
    n = mib * (1 << 20) // 4
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del a, b
    torch.cuda.empty_cache()
    return 2.0 * mib * (1 << 20) / (ms * 1e-3) / 1e9


# ---------------------------------------------------------------- hardware counters (rocprofv3)
STANDING_N, STANDING_K = 8192, 50   # standing regime: worlds, control steps per bench_phys call (the reference's K)


def counter_child(config, workload="rollout", per_step=False):
    """The profiled program: one copy of COPY_MIB MiB (the calibration dispatch), then one warm-up
    and one timed rollout of the configuration (in the library's default rollout form), or for the
    standing workload two physics-only bench calls of STANDING_K control steps after a reset."""
    import torch
    import configs
    import g1env
    n = COPY_MIB * (1 << 20) // 4
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b
    if workload == "standing":
        with g1env.Env(STANDING_N, substeps=10, pgs_iters=8, seed=1) as env:
            env.reset()
            for _ in range(2):
                env.bench_phys(STANDING_K)
            assert env.check() == 0
        return
    cfg = configs.ROLLOUT_CONFIGS[config]
    N, H = cfg["N"], cfg["H"]
    W = torch.from_numpy(configs.policy_init(np.random.default_rng(1234), hidden=cfg["hidden"])).cuda()
    mean, var = torch.zeros(100, device="cuda"), torch.ones(100, device="cuda")
    with g1env.Env(N, substeps=cfg["S"], pgs_iters=cfg["pgs"], seed=1) as env:
        env.set_policy(cfg["hidden"], cfg["act"])
        env.set_fused(not per_step)
        env.reset()
        traj = g1env.Trajectory(H, N)
        for _ in range(2):
            traj.run(env, W, mean, var)
        torch.cuda.synchronize()
        assert env.check() == 0


def _read_counters(outdir):
    rows = []
    for path in glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True):
        with open(path, newline="") as f:
            rows += list(csv.DictReader(f))
    return rows


def measure_counters(config, kernel, timeout_s=150, workload="rollout", per_step=False):
    """Runs the counter passes on child processes; returns per-dispatch averages for `kernel` and
    the calibration copy, or None with the reason."""
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None, "rocprofv3 not found"
    res = {"physics": {}, "copy": {}}
    env = dict(os.environ, TMPDIR="/tmp")
    for name, counters in COUNTER_PASSES:
        outdir = tempfile.mkdtemp(prefix=f"g1bench_{name}_", dir="/tmp")
        cmd = [exe, "--pmc", *counters, "--output-format", "csv", "-d", outdir, "-o", "p", "--",
               sys.executable, os.path.abspath(__file__), "--counter-child", "--config", str(config),
               "--workload", workload] + (["--per-step"] if per_step else [])
        try:
            p = subprocess.run(cmd, cwd="/tmp", env=env, timeout=timeout_s, capture_output=True, text=True)
        except subprocess.TimeoutExpired:
            return None, f"counter pass {name} timed out"
        rows = _read_counters(outdir)
        shutil.rmtree(outdir, ignore_errors=True)
        print(f"bench: counter pass {name} done (exit {p.returncode}, {len(rows)} rows)", file=sys.stderr, flush=True)
        if not rows:
            return None, f"counter pass {name}: no output (exit {p.returncode}): {p.stderr[-300:]}"
        for r in rows:
            kname, cname, val = r["Kernel_Name"], r["Counter_Name"], float(r["Counter_Value"])
            key = "physics" if kernel in kname else ("copy" if "copyBuffer" in kname else None)
            if key is None:
                continue
            res[key].setdefault(cname, []).append(val)
    phys = {k: float(np.mean(v)) for k, v in res["physics"].items()}
    copy = {k: float(np.max(v)) for k, v in res["copy"].items()}
    need = {"FETCH_SIZE", "WRITE_SIZE"}
    if not need <= set(phys) or not need <= set(copy):
        return None, "counter passes did not report the physics or copy dispatches"
    kib = COPY_MIB * 1024.0
    scale_f, scale_w = kib / copy["FETCH_SIZE"], kib / copy["WRITE_SIZE"]
    phys["fetch_bytes"], phys["write_bytes"] = phys["FETCH_SIZE"] * scale_f * 1024.0, phys["WRITE_SIZE"] * scale_w * 1024.0
    phys["traffic_bytes"] = phys["fetch_bytes"] + phys["write_bytes"]
    phys["fetch_scale"], phys["write_scale"] = scale_f, scale_w
    phys["dispatches"] = len(res["physics"]["FETCH_SIZE"])
    return phys, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=3, choices=[3, 4])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-counters", action="store_true", help="skip the rocprofv3 counter passes")
    ap.add_argument("--counter-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--per-step", action="store_true",
                    help="launch the policy and the physics once per control step instead of one k_rollout")
    ap.add_argument("--workload", choices=["rollout", "standing"], default="rollout",
                    help="rollout: the fused rollout of --config (the headline); standing: the reference's "
                         "physics-only bench (scripts/bench_env_phys.py: reset, zero action, g1_env_bench_phys) "
                         "at N=8192, a step being one call of 50 control steps")
    ap.add_argument("--policy", choices=["random", "trained"], default="random",
                    help="random-init weights (the configuration's definition) or the reference's trained "
                         "checkpoint (g1.cu_amd/data/trained_policy_finish_best.npz: walking contact mix)")
    args = ap.parse_args()
    if args.counter_child:
        counter_child(args.config, args.workload, args.per_step)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: the rollout shards worlds across GPUs with no exchange, "
              "and this build runs on single-GPU boxes only (--gpus 1).", file=sys.stderr)
        sys.exit(2)

    if args.workload == "standing":
        standing_main(args)
        return
    import configs
    cfg = configs.ROLLOUT_CONFIGS[args.config]
    # the library runs a two-hidden-layer policy of at most 256 units as one launch (k_rollout)
    # every accepted policy shape runs as one launch (k_rollout) unless --per-step asks for the
    # policy and physics launches per control step
    one_launch = not args.per_step
    kernel = "k_rollout" if one_launch else "k_physics"
    # counter passes first, while this process has not touched the GPU
    counters, counter_note = ((None, "skipped (--no-counters)") if args.no_counters
                              else measure_counters(args.config, kernel, per_step=args.per_step))

    import torch
    import g1env
    N, H, S, pgs = cfg["N"], cfg["H"], cfg["S"], cfg["pgs"]
    rng = np.random.default_rng(1234)
    env = g1env.Env(N, substeps=S, pgs_iters=pgs, seed=1)
    env.set_policy(cfg["hidden"], cfg["act"])
    if env.set_fused(one_launch) != one_launch:
        sys.exit("rollout form differs from the one this script expects")
    env.reset()
    if args.policy == "trained":
        if args.config != 3:
            sys.exit("the trained checkpoint has the config-3 policy shape (100-256-256 tanh)")
        tp = np.load(os.path.join(ROOT, "g1.cu_amd", "data", "trained_policy_finish_best.npz"))
        W = torch.from_numpy(tp["W"]).cuda()
        mean = torch.from_numpy(tp["obs_mean"]).cuda()
        var = torch.from_numpy(tp["obs_var"]).cuda()
    else:
        W = torch.from_numpy(configs.policy_init(rng, hidden=cfg["hidden"])).cuda()
        mean = torch.zeros(100, device="cuda")
        var = torch.ones(100, device="cuda")
    traj = g1env.Trajectory(H, N)

    for _ in range(args.warmup):
        traj.run(env, W, mean, var)
    torch.cuda.synchronize()
    env.ncon_hist(enable=True)
    env.profile(1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        traj.run(env, W, mean, var)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    pr = env.profile_read()
    env.profile(0)
    hist = env.ncon_hist(enable=False)
    if env.check() != 0:
        sys.exit("physics work queue error: results undefined")
    env.close()
    ms_rollout = wall * 1e3 / args.steps
    substeps_per_s = N * H * S / (wall / args.steps)

    bw_meas = measure_copy_bandwidth()
    # Compulsory HBM bytes of one rollout: the trajectory written once (O [H,N,100], A [H,N,29],
    # LP/V/R/D [H,N], Vlast [N]), the env state read and written once (qpos 36, qvel 35, previous
    # action 29, step and noise counters), the policy (weights and biases, obs mean and variance) read
    # once; library noise, so no noise arrays.
    n_weights = sum(i * o + o for i, o in zip((100,) + tuple(cfg["hidden"]), tuple(cfg["hidden"]) + (30,)))
    compulsory = 4.0 * (N * H * (g1env.OBS_DIM + g1env.ACT_DIM + 4) + N + 2 * N * (g1env.NQ + g1env.NV + g1env.ACT_DIM + 2)
                        + n_weights + 200)
    launches = max(pr["physics_launches"], 1)
    avg_launch_s = pr["physics_ms"] / launches * 1e-3
    bytes_total, flops_total = rf.physics_work(hist, pgs, control_steps_worlds=N * H * args.steps)
    phys_flops_launch, bytes_launch = flops_total / launches, bytes_total / launches
    cbar = float((hist * np.arange(9)).sum() / max(hist.sum(), 1))
    # policy MLP multiply-adds per rollout: H steps plus the bootstrap value (fp32, MFMA)
    pol_flops = 2 * N * (H + 1) * sum(a * b for a, b in zip((100,) + tuple(cfg["hidden"]), tuple(cfg["hidden"]) + (30,)))
    mlp_flops_launch = pol_flops * args.steps / launches if one_launch else 0.0
    flops_launch = phys_flops_launch + mlp_flops_launch
    achieved_tf = flops_launch / avg_launch_s / 1e12
    pol_ms = pr["policy_ms"] / args.steps
    pol_tf = pol_flops / (pol_ms * 1e-3) / 1e12 if pol_ms > 0 else None

    roof = {"bound": "valu", "achieved": achieved_tf, "peak": rf.FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": achieved_tf / rf.FP32_PEAK_TFLOPS,
            "traffic": counters["traffic_bytes"] if counters else None,
            "kernel": kernel, "avg_launch_ms": avg_launch_s * 1e3, "algorithmic_flops_per_launch": flops_launch,
            "physics_flops_per_launch": phys_flops_launch, "mlp_flops_per_launch": mlp_flops_launch,
            "mean_ncon": cbar, "frac_of_unpacked_fp32": achieved_tf / rf.FP32_UNPACKED_TFLOPS,
            "bw_meas_gbs": bw_meas,
            "hbm_proxy": {"unit": "GB/s", "achieved": bytes_launch / avg_launch_s / 1e9, "peak": rf.HBM_PEAK_GBS,
                          "frac": bytes_launch / avg_launch_s / 1e9 / rf.HBM_PEAK_GBS,
                          "frac_of_bw_meas": bytes_launch / avg_launch_s / 1e9 / bw_meas,
                          "algorithmic_bytes_per_launch": bytes_launch,
                          "note": "reference-algorithm working set per world-substep, written and read once; "
                                  "held in registers and LDS, not HBM"}}
    if counters:
        valu = counters.get("SQ_INSTS_VALU")
        roof["counters"] = {
            "source": f"rocprofv3 --pmc, one-rollout run of this script ({counters['dispatches']} {kernel} dispatches)",
            "hbm_bytes_per_dispatch": counters["traffic_bytes"],
            "hbm_read_bytes_per_dispatch": counters["fetch_bytes"],
            "hbm_write_bytes_per_dispatch": counters["write_bytes"],
            "hbm_compulsory_bytes": compulsory,
            "hbm_over_compulsory": counters["traffic_bytes"] / compulsory,
            "hbm_gbs": counters["traffic_bytes"] / avg_launch_s / 1e9,
            "hbm_frac_of_bw_meas": counters["traffic_bytes"] / avg_launch_s / 1e9 / bw_meas,
            "fetch_write_scale": [counters["fetch_scale"], counters["write_scale"]],
            "valu_busy_frac": counters.get("VALUBusy", float("nan")) / 100.0,
            "valu_lane_utilization": counters.get("VALUUtilization", float("nan")) / 100.0,
            "valu_insts_per_dispatch": valu,
            "valu_issue_frac": valu / (rf.VALU_ISSUE_PEAK * avg_launch_s) if valu else None,
            "physics_flops_per_valu_lane_slot": phys_flops_launch / (valu * 64) if valu else None,
            "lds_util_frac": counters.get("LdsUtil", float("nan")) / 100.0,
            "lds_bank_conflict_frac": counters.get("LDSBankConflict", float("nan")) / 100.0,
            "lds_insts_per_dispatch": counters.get("SQ_INSTS_LDS")}
        lds_ld, lds_st = counters.get("SQ_INSTS_LDS_LOAD_BANDWIDTH"), counters.get("SQ_INSTS_LDS_STORE_BANDWIDTH")
        if lds_ld is not None and lds_st is not None:
            lds_bytes = (lds_ld + lds_st) * 64.0
            roof["counters"].update({
                "lds_bytes_per_dispatch": lds_bytes, "lds_load_bytes_per_dispatch": lds_ld * 64.0,
                "lds_gbs": lds_bytes / avg_launch_s / 1e9, "lds_peak_gbs": rf.LDS_PEAK_GBS,
                "lds_frac": lds_bytes / avg_launch_s / 1e9 / rf.LDS_PEAK_GBS})
    else:
        roof["counters"] = {"note": counter_note}

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
        "roofline": roof,
        "phases": ({"rollout_launch_ms": pr["physics_ms"] / args.steps,
                    "note": "physics and policy share one k_rollout launch per rollout"} if one_launch else
                   {"physics_ms_per_rollout": pr["physics_ms"] / args.steps, "policy_ms_per_rollout": pol_ms,
                    "policy_tflops": pol_tf,
                    "policy_mfma_frac": pol_tf / rf.FP32_PEAK_TFLOPS if pol_tf else None}),
        "ncon_hist": hist.tolist(),
    }
    print(f"bench: {args.steps} rollouts timed, {ms_rollout:.3f} ms each", file=sys.stderr, flush=True)
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        out["cpu_baseline"] = cpu_baseline(cfg, threads)
    print(json.dumps(out), flush=True)


def counter_summary(counters, kernel, avg_launch_s, phys_flops_launch, bw_meas):
    """The counter block of the JSON line (per dispatch of `kernel`)."""
    valu = counters.get("SQ_INSTS_VALU")
    out = {
        "source": f"rocprofv3 --pmc, one run of this script's counter child ({counters['dispatches']} {kernel} dispatches)",
        "hbm_bytes_per_dispatch": counters["traffic_bytes"],
        "hbm_read_bytes_per_dispatch": counters["fetch_bytes"],
        "hbm_write_bytes_per_dispatch": counters["write_bytes"],
        "hbm_gbs": counters["traffic_bytes"] / avg_launch_s / 1e9,
        "hbm_frac_of_bw_meas": counters["traffic_bytes"] / avg_launch_s / 1e9 / bw_meas,
        "fetch_write_scale": [counters["fetch_scale"], counters["write_scale"]],
        "valu_busy_frac": counters.get("VALUBusy", float("nan")) / 100.0,
        "valu_lane_utilization": counters.get("VALUUtilization", float("nan")) / 100.0,
        "valu_insts_per_dispatch": valu,
        "valu_issue_frac": valu / (rf.VALU_ISSUE_PEAK * avg_launch_s) if valu else None,
        "physics_flops_per_valu_lane_slot": phys_flops_launch / (valu * 64) if valu else None,
        "lds_util_frac": counters.get("LdsUtil", float("nan")) / 100.0,
        "lds_bank_conflict_frac": counters.get("LDSBankConflict", float("nan")) / 100.0,
        "lds_insts_per_dispatch": counters.get("SQ_INSTS_LDS")}
    lds_ld, lds_st = counters.get("SQ_INSTS_LDS_LOAD_BANDWIDTH"), counters.get("SQ_INSTS_LDS_STORE_BANDWIDTH")
    if lds_ld is not None and lds_st is not None:
        lds_bytes = (lds_ld + lds_st) * 64.0
        out.update({"lds_bytes_per_dispatch": lds_bytes, "lds_gbs": lds_bytes / avg_launch_s / 1e9,
                    "lds_frac": lds_bytes / avg_launch_s / 1e9 / rf.LDS_PEAK_GBS})
    return out


def standing_main(args):
    """The reference's physics-only benchmark (scripts/bench_env_phys.py:15-24 -> g1_env_bench_phys,
    k_phys_bench, src/g1_env.cu:343-359): N=8192 worlds reset to the stand pose, zero action, the
    physics of STANDING_K control steps per call (continuous foot contact, 6-8 contacts per world in
    most substeps). One JSON line like the rollout's, for k_physics."""
    counters, note = ((None, "skipped (--no-counters)") if args.no_counters
                      else measure_counters(3, "k_physics", workload="standing"))
    import torch
    import g1env
    N, K, S, pgs = STANDING_N, STANDING_K, 10, 8
    env = g1env.Env(N, substeps=S, pgs_iters=pgs, seed=1)
    env.reset()
    for _ in range(args.warmup):
        env.bench_phys(K)
    env.ncon_hist(enable=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        env.bench_phys(K)   # blocks: one k_physics launch of K control steps
    wall = time.perf_counter() - t0
    hist = env.ncon_hist(enable=False)
    if env.check() != 0:
        sys.exit("physics work queue error: results undefined")
    env.close()
    launch_s = wall / args.steps
    bw_meas = measure_copy_bandwidth()
    _, flops_total = rf.physics_work(hist, pgs, control_steps_worlds=N * K * args.steps)
    flops_launch = flops_total / args.steps
    achieved = flops_launch / launch_s / 1e12
    roof = {"bound": "valu", "achieved": achieved, "peak": rf.FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": achieved / rf.FP32_PEAK_TFLOPS, "traffic": counters["traffic_bytes"] if counters else None,
            "kernel": "k_physics", "avg_launch_ms": launch_s * 1e3, "algorithmic_flops_per_launch": flops_launch,
            "mean_ncon": float((hist * np.arange(9)).sum() / max(hist.sum(), 1)),
            "frac_of_unpacked_fp32": achieved / rf.FP32_UNPACKED_TFLOPS, "bw_meas_gbs": bw_meas,
            "counters": (counter_summary(counters, "k_physics", launch_s, flops_launch, bw_meas) if counters
                         else {"note": note})}
    out = {"metric": "physics substeps/sec, standing regime (reference scripts/bench_env_phys.py), N=8192, 1 GPU",
           "value": N * K * S / launch_s, "unit": "substeps/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": launch_s * 1e3, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "fp32",
           "data": "stand-pose resets (library Philox noise), zero action",
           "config": {"workload": f"standing: g1_env_bench_phys N={N} K={K} S={S} pgs={pgs}", "N": N, "K": K,
                      "substeps": S, "pgs": pgs},
           "roofline": roof, "ncon_hist": hist.tolist()}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
