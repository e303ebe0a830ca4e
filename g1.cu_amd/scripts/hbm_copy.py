"""Plain device-to-device copy of a known size on the GPU: the HBM stream-copy bandwidth of the box
and the reference dispatch for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE counters (the copy
reads and writes exactly --mib MiB per dispatch).

    python g1.cu_amd/scripts/hbm_copy.py [--mib 1024] [--reps 10]
"""
import argparse

import torch


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=1024)
    ap.add_argument("--reps", type=int, default=10)
    args = ap.parse_args()
    n = args.mib * (1 << 20) // 4
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.reps):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.reps
    print(f"copy {args.mib} MiB: {ms:.3f} ms per dispatch, {2 * args.mib * (1 << 20) / (ms * 1e-3) / 1e9:.1f} GB/s "
          f"(read + write)", flush=True)


if __name__ == "__main__":
    main()
