"""Algorithmic work units of the physics and the MI355X peaks they are priced against, used by
bench.py and tests/bench_configs.py.

Two units per world-substep with c foot contacts and p PGS sweeps:

* bytes_per_world_substep: every per-world intermediate of the reference algorithm written once
  and read once in fp32, with the PGS matrix read once per sweep:
  B_ws(c) = 4 [2 (3244 + 1390 c + 35 [c>0]) + 16 c^2 (1 + p)]. The physics keeps this working
  set in registers and LDS, so it is a workload measure, not an HBM ceiling: the kernel's real
  HBM traffic is state in and out, measured separately.
* flops_per_world_substep: floating-point operations of one substep of the reference algorithm
  (FK, PD torque, RNE bias, damped factor, smooth and contact solves, PGS, Euler, integration).
  add, sub, mul, div and sqrt count one, a fused multiply-add two; the 60 transcendental calls
  (sin/cos of the hinge angles and the base rotation, the impedance pow) and the comparisons are
  left out. The table comes from the CPU oracle instantiated on an operation-counting scalar, in
  the reference's summation association (oracle/flop_count.cpp). tests/test_flop_table.py
  regenerates it and checks these constants. Within one contact count, data-dependent branches
  (the impedance sigmoid's two sides, torque and velocity clamps) add up to 0.05%; the table holds
  the smallest count over sampled contact states.
"""

# MI355X published peaks
HBM_PEAK_GBS = 8000.0          # HBM3E
FP32_PEAK_TFLOPS = 157.3       # dense fp32, vector and matrix (the vector figure counts packed FP32)
FP32_UNPACKED_TFLOPS = 78.65   # 256 CUs x 128 fp32 FMA-flops/clock x 2.4 GHz (no packed-FP32 ops)
CUS, PEAK_CLOCK_GHZ = 256, 2.4
VALU_ISSUE_PEAK = CUS * PEAK_CLOCK_GHZ * 1e9   # wave64 VALU instructions per second (1 per CU per clock)
LDS_BYTES_PER_CLK_CU = 128     # LDS data path per CU per clock (CDNA3/CDNA4 ISA figure)
LDS_PEAK_GBS = CUS * LDS_BYTES_PER_CLK_CU * PEAK_CLOCK_GHZ   # 78,643 GB/s

PGS_TABLE = 8
FLOPS_P8 = (35939, 43859, 52598, 62205, 72680, 84023, 96234, 109313, 123260)   # c = 0..8 at p = 8
STEP_OVERHEAD_FLOPS = 230   # per world and control step outside the substeps (targets, reward)


def bytes_per_world_substep(c, p):
    return 4.0 * (2.0 * (3244 + 1390 * c + 35 * (c > 0)) + 16.0 * c * c * (1 + p))


def flops_per_world_substep(c, p):
    """Table value at p = 8, moved by (p - 8) PGS sweeps of n = 4c rows: a sweep costs n (n + 1)
    fused multiply-adds, n divisions and n sign clamps, 2 n^2 + 3 n flops."""
    n = 4 * c
    return FLOPS_P8[c] + (p - PGS_TABLE) * (2 * n * n + 3 * n)


def physics_work(hist, p, control_steps_worlds=0):
    """(algorithmic bytes, algorithmic flops) of a contact-count histogram hist[0..8] of
    world-substeps, plus the per-control-step flops of control_steps_worlds world-steps."""
    b = sum(int(hist[c]) * bytes_per_world_substep(c, p) for c in range(9))
    f = sum(int(hist[c]) * flops_per_world_substep(c, p) for c in range(9))
    return b, f + control_steps_worlds * STEP_OVERHEAD_FLOPS
