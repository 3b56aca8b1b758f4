"""HBM rates of the single-row kernels with their weights rotated through more memory than the
last-level cache holds, so that every call streams its weights from HBM.

    python -m momij_amd.hbmbench [--case qmv,moe1,head4,head16] [--gib 1.0] [--reps 3]

Cases (synthetic device-resident weights, the 2-bit draws of the workloads: codes uniform,
scale ~ U(0.005, 0.02), bias = -1.5 scale; hidden rows ~ N(0, 1)):

  qmv     one-row 2-bit GEMV, W [5632 x 2048] group 64 through mj_gather_qmm2 (M = 1, one
          expert): 3,619,840 algorithmic bytes a call (codes 2,883,584 + scales and biases
          720,896 + x 4,096 + y 11,264).
  moe1    the MoE block for one token through mj_moe_block: router fp16 [64 x 2048], 64
          experts of up||gate [2048 x 2048] and down [2048 x 1024], top-8, group 64.  Per call
          8 experts x 1,966,080 B + router 262,144 B + activations.
  head4   the Maple 4-bit lm_head [151936 x 2048] group 64, one row: 175,030,272 B a call.
  head16  the fp16 lm_head [151936 x 2048], one row: 622,329,856 B a call.

Each case holds ceil(gib / bytes of one set) independent weight sets (at least 2) and calls them
in turn, `--reps` rounds (at least 10 for the heads, which have few sets), after one untimed
round.  The script prints the sets, calls and the
algorithmic bytes per call; the kernel durations come from running it under
`rocprofv3 --kernel-trace --stats` (GB/s = algorithmic bytes per call / summed mean duration of
the case's kernels).
"""
from __future__ import annotations

import argparse
import math

QMV_N, H, E, I, TOPK, GS, V = 5632, 2048, 64, 1024, 8, 64, 151936


def qmv_bytes() -> int:
    return QMV_N * H // 4 + 2 * QMV_N * (H // GS) * 2 + H * 2 + QMV_N * 2


def expert_bytes() -> int:
    up = 2 * I * (H // 4 + 2 * (H // GS) * 2)
    dn = H * (I // 4 + 2 * (I // GS) * 2)
    return up + dn


def moe1_bytes() -> int:
    return TOPK * expert_bytes() + E * H * 2 + 2 * H * 2


def head4_bytes() -> int:
    return V * H // 2 + V * (H // 64) * 4


def head16_bytes() -> int:
    return V * H * 2


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--case", default="qmv,moe1,head4,head16")
    ap.add_argument("--gib", type=float, default=1.0)
    ap.add_argument("--reps", type=int, default=3, help="timed rounds (heads: at least 10)")
    args = ap.parse_args()

    import torch

    from . import synth
    from .ops import Context

    ctx = Context(0)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    x = synth.torch_normal(gen, (1, H))
    target = args.gib * (1 << 30)

    def nsets(one_set: int) -> int:
        return max(2, math.ceil(target / one_set))

    def run(name, calls, per_call):
        torch.cuda.synchronize()  # the weight sets were drawn on torch's stream
        for c in calls:  # untimed round
            c()
        ctx.sync()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = args.reps if len(calls) > 8 else max(args.reps, 10)
        ev0.record(ctx.stream)
        for _ in range(reps):
            for c in calls:
                c()
        ev1.record(ctx.stream)
        ctx.sync()
        n = reps * len(calls)
        us = ev0.elapsed_time(ev1) * 1e3 / n
        print(f"{name}: {len(calls)} sets, {n} timed calls, {per_call} algorithmic B/call, "
              f"{us:.2f} us/call between events (launch gaps included), "
              f"{per_call / us / 1e3:.0f} GB/s", flush=True)

    for case in args.case.split(","):
        if case == "qmv":
            n = nsets(qmv_bytes())
            sets = [synth.torch_qweight(gen, (1,), QMV_N, H, GS) for _ in range(n)]
            inds = torch.zeros(1, dtype=torch.int32, device="cuda")
            y = torch.empty((1, QMV_N), dtype=torch.float16, device="cuda")
            calls = [(lambda w=w, s=s, b=b: ctx.gather_qmm2(x, w, s, b, inds, y, 1, 1, H, QMV_N,
                                                             GS)) for w, s, b in sets]
            run("qmv 5632x2048 gs64", calls, qmv_bytes())
        elif case == "moe1":
            per_set = E * expert_bytes() + E * H * 2
            n = nsets(per_set)
            sets = []
            for _ in range(n):
                ugw, ugs, ugb = synth.torch_qweight(gen, (E,), 2 * I, H, GS)
                dw, ds, db = synth.torch_qweight(gen, (E,), H, I, GS)
                sets.append(dict(router_w=synth.torch_normal(gen, (E, H), 0.02),
                                 up_gate_w=ugw, up_gate_s=ugs, up_gate_b=ugb,
                                 down_w=dw, down_s=ds, down_b=db,
                                 E=E, top_k=TOPK, H=H, I=I, gs=GS, eps=1e-6))
            y = torch.empty((1, H), dtype=torch.float16, device="cuda")
            calls = [(lambda mw=mw: ctx.moe_block(mw, x, y, 1, 0)) for mw in sets]
            run("moe1 E=64 top-8 I=1024", calls, moe1_bytes())
        elif case == "head4":
            n = nsets(head4_bytes())
            sets = []
            for _ in range(n):
                w4 = torch.randint(-(2**31), 2**31 - 1, (V, H // 8), generator=gen,
                                   device="cuda", dtype=torch.int64).to(torch.int32)
                s4 = (torch.rand((V, H // 64), generator=gen, device="cuda") * 0.003
                      + 0.001).half()
                sets.append((w4, s4, (-7.5 * s4.float()).half()))
            am = torch.empty(1, dtype=torch.int32, device="cuda")
            calls = [(lambda w=w, s=s, b=b: ctx.lm_head_verify_q4(x, w, s, b, 1, H, V, am))
                     for w, s, b in sets]
            run("head4 151936x2048", calls, head4_bytes())
        elif case == "head16":
            n = nsets(head16_bytes())
            sets = [synth.torch_normal(gen, (V, H), 0.02) for _ in range(n)]
            am = torch.empty(1, dtype=torch.int32, device="cuda")
            calls = [(lambda w=w: ctx.lm_head_verify(x, w, 1, H, V, am)) for w in sets]
            run("head16 151936x2048", calls, head16_bytes())
        else:
            raise SystemExit(f"unknown case {case}")
        del sets, calls
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    ctx.close()


if __name__ == "__main__":
    main()
