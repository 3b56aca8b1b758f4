"""Timing of the exact lm_head verify over both weight formats, at the Maple vocabulary.

    python -m momij_amd.headbench [--vocab 151936] [--hidden 2048] [--rows 1,8,17] [--calls 50]

Synthetic device-resident inputs: an fp16 head ~ N(0, 0.02) and a 4-bit gs64 head (uniform
codes, scale ~ U(0.001, 0.004), bias = -7.5 scale), hidden rows ~ N(0, 1).  For each format and
row count it prints the mean wall time per call over `--calls` back-to-back argmax calls (head
kernel + partial fold) and the algorithmic bytes per call over that time.  Run it under
`rocprofv3 --kernel-trace --stats` for per-kernel durations.
"""
from __future__ import annotations

import argparse
import time


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--vocab", type=int, default=151936)
    ap.add_argument("--hidden", type=int, default=2048)
    ap.add_argument("--rows", default="1,8,17")
    ap.add_argument("--calls", type=int, default=50)
    a = ap.parse_args()
    import torch

    from momij_amd.ops import Context

    ctx = Context(0)
    V, K = a.vocab, a.hidden
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    w16 = (torch.randn((V, K), generator=g, device="cuda") * 0.02).half()
    w4 = torch.randint(-(2**31), 2**31 - 1, (V, K // 8), generator=g, device="cuda",
                       dtype=torch.int64).to(torch.int32)
    s4 = (torch.rand((V, K // 64), generator=g, device="cuda") * 0.003 + 0.001).half()
    b4 = (-7.5 * s4.float()).half()
    for kind in ("fp16", "q4"):
        for M in [int(m) for m in a.rows.split(",")]:
            x = torch.randn((M, K), generator=g, device="cuda").half()
            am = torch.empty(M, dtype=torch.int32, device="cuda")
            if kind == "fp16":
                def call():
                    ctx.lm_head_verify(x, w16, M, K, V, am)
                nbytes = V * K * 2
            else:
                def call():
                    ctx.lm_head_verify_q4(x, w4, s4, b4, M, K, V, am)
                nbytes = V * K // 2 + V * (K // 64) * 4
            for _ in range(5):
                call()
            ctx.sync()
            t = time.perf_counter()
            for _ in range(a.calls):
                call()
            ctx.sync()
            dt = (time.perf_counter() - t) / a.calls
            print(f"{kind:5s} V={V} K={K} rows={M:2d}: {dt * 1e6:7.1f} us/call, "
                  f"{nbytes / dt / 1e9:6.0f} GB/s of {nbytes / 1e6:.1f} MB", flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
