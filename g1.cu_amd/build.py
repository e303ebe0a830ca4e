"""Build libg1env.so for gfx950 in-tree (g1.cu_amd/build/libg1env.so).

    python g1.cu_amd/build.py

The library lands where the reference's Python looks for it relative to its scripts folder
(<root>/build/libg1env.so, reference scripts/ppo.py:20-24), with <root> = g1.cu_amd.
"""
import json
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "build")
OUT = os.path.join(OUT_DIR, "libg1env.so")
ARCH = os.environ.get("G1_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # no packed-FP32 VALU forms (v_pk_*_f32): some of their forms have produced silently wrong
    # results on this GPU pool; hipcc's host pass warns that it does not know the feature
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # code-object v5 loads under both the ROCm 7.2 runtime and torch's bundled HIP 7.0 runtime
    "-mcode-object-version=5",
    # no a*b+c -> fma contraction: the physics then performs the oracle's IEEE operation sequence.
    # With contraction, two valid fp32 evaluations of the same algorithm differ by up to 1.8e-5 on
    # penetrating-contact states (8 unconverged PGS sweeps amplify rounding), above the 1e-5 gate.
    "-ffp-contract=off",
    "-Wno-pass-failed",
]


# translation units and their own flags: both are scheduled for instruction-level parallelism with
# LLVM's max-ilp machine scheduler. k_physics and k_policy since the physics lost its force
# broadcast and select cascades (config 4 rollout 185.4 -> 183.5 ms; with the older physics the
# same flag had made it 3% slower); the iterative ILP scheduler measured 2.5% slower and the default
# 2.1% slower in the standing regime. The one-launch rollout kernel had max-ilp from its first version
# (config 3 12.83 -> 12.77 ms), then for a while the iterative ILP scheduler (9.358 -> 9.320 ms),
# and with the physics' current LDS layouts max-ilp again: config 3 8.36 -> 8.25 ms, config 4 151.7
# -> 151.0 ms same-box (the default scheduler and max-memory-clause: 8.36).
ILP_FIRST = ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]
# k_rollout's policy tiles keep their MFMA accumulators in VGPRs: the physics items need ~230
# VGPRs, which the policy path does not use at the same time, while accumulators in AGPRs add to
# that count (the wide tile's 8 groups of accumulators took 48 AGPRs: 278 registers, one wave per SIMD)
MFMA_VGPR = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
SOURCES = (
    ("g1env.hip", ILP_FIRST),
    ("rollout_kernel.hip", ILP_FIRST + MFMA_VGPR),
)


# the compiler's per-kernel resource report (-Rpass-analysis=kernel-resource-usage), kept beside the
# library: the persistent kernels are sized for two waves per SIMD (k_rollout sits at the 256-VGPR
# edge of that occupancy, and one wave per SIMD runs it ~70% slower), which tests/test_abi_exports.py
# checks from this file
RESOURCES = os.path.join(OUT_DIR, "resource_usage.json")
_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]|"
                     r"VGPRs Spill|LDS Size \[bytes/block\]):\s+(\S+)")


def _parse_resources(text, table):
    fn = None
    for m in _REMARK.finditer(text):
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            fn = val
            table[fn] = {}
        elif fn is not None:
            table[fn][key.split(" [")[0]] = int(val)


def build(verbose=False):
    os.makedirs(OUT_DIR, exist_ok=True)
    objs = []
    resources = {}
    for name, extra in SOURCES:
        obj = os.path.join(OUT_DIR, os.path.splitext(name)[0] + ".o")
        cmd = ["hipcc", *FLAGS, *extra, "-Rpass-analysis=kernel-resource-usage", "-c",
               os.path.join(HERE, "csrc", name), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        p = subprocess.run(cmd, capture_output=True, text=True)
        if p.returncode != 0 or verbose:
            sys.stderr.write(p.stdout + p.stderr)
        if p.returncode != 0:
            raise subprocess.CalledProcessError(p.returncode, cmd)
        _parse_resources(p.stderr, resources)
        objs.append(obj)
    cmd = ["hipcc", f"--offload-arch={ARCH}", "-fPIC", "-shared", *objs, "-o", OUT + ".tmp"]
    subprocess.run(cmd, check=True)
    for obj in objs:
        os.remove(obj)
    os.replace(OUT + ".tmp", OUT)
    with open(RESOURCES, "w") as f:
        json.dump(resources, f, indent=1, sort_keys=True)
    for fn, r in resources.items():
        if ("k_rollout" in fn or "k_physics" in fn) and (r.get("Occupancy", 0) < 2 or r.get("ScratchSize", 0)):
            sys.stderr.write(f"WARNING: {fn}: {r} (the persistent kernels are sized for 2 waves/SIMD, no scratch)\n")
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
