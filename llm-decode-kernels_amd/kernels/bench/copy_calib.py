"""Calibration workload for rocprofv3 byte counters: copies a 64 MiB device buffer into another
`--reps` times (torch's device-to-device copy kernel). Each copy reads and writes exactly
64 MiB = 65536 KiB, so FETCH_SIZE and WRITE_SIZE per dispatch divided by 65536 give the factor
that turns those counters into HBM bytes on this GPU.

    rocprofv3 --pmc FETCH_SIZE -- python3 -m kernels.bench.copy_calib
"""

from __future__ import annotations

import argparse

import torch

NBYTES = 64 * 2**20


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=8)
    args = ap.parse_args()
    a = torch.randint(0, 255, (NBYTES,), dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(args.reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(f"copied {NBYTES} bytes x {args.reps}")


if __name__ == "__main__":
    main()
