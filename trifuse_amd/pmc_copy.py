"""Copy kernel of known size, for calibrating HBM byte counters.

    python -m trifuse_amd.pmc_copy [--mib 1024] [--reps 5]

Runs `reps` device-to-device copies of `mib` MiB with torch on cuda:0. Under
`rocprofv3 --pmc FETCH_SIZE` (or WRITE_SIZE) each copy dispatch reads and
writes exactly mib MiB, so counter / (mib * 1024) is the counter's scale in
KiB per KiB moved.
"""
import argparse

import torch


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--mib", type=int, default=1024)
    p.add_argument("--reps", type=int, default=5)
    a = p.parse_args()
    n = a.mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(a.reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {a.mib} MiB x {a.reps}")


if __name__ == "__main__":
    main()
