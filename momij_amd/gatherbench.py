"""Expert gathers over row-alpha weights: the fold kernels against the group-scale kernels on
the same arrays and the same routing.

    python -m momij_amd.gatherbench [--experts 64] [--inter 1024] [--rows 9] [--sets 8] [--reps 20]

Synthetic device-resident MoE weights (hidden 2048, top-8, 2-bit gs64, random codes) in row-alpha
form: alpha = a row's first group scale, every group scale alpha, every bias -alpha.  `--sets`
independent weight sets (each about 96 MB at the defaults) are called in turn, so that the
weights stream from HBM rather than from the last-level cache; each set is run with alpha given
(fold kernels) and without it (group-scale kernels), with identical routing.  Run it under
`rocprofv3 --kernel-trace --stats`: the fold kernels are `k_gather5<..., true>` (last template
argument), the group-scale ones `k_gather5<..., false>`.
"""
from __future__ import annotations

import argparse


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--experts", type=int, default=64)
    ap.add_argument("--inter", type=int, default=1024)
    ap.add_argument("--rows", type=int, default=9)
    ap.add_argument("--sets", type=int, default=8)
    ap.add_argument("--reps", type=int, default=20)
    args = ap.parse_args()

    import numpy as np
    import torch

    from . import synth
    from .ops import Context

    ctx = Context(0)
    rng = np.random.default_rng(1)
    H, E, I, M = 2048, args.experts, args.inter, args.rows
    sets = []
    for _ in range(args.sets):
        mw = synth.moe_weights(rng, E, H, I, 64)
        for p in ("up_gate", "down"):
            alpha = np.ascontiguousarray(mw[p + "_s"][..., 0])
            mw[p + "_s"] = np.ascontiguousarray(np.repeat(alpha[..., None],
                                                          mw[p + "_s"].shape[-1], -1))
            mw[p + "_b"] = (-mw[p + "_s"]).astype(np.float16)
            mw[p + "_alpha"] = alpha
        sets.append({k: (torch.from_numpy(v.view(np.int32) if v.dtype == np.uint32 else v)
                         .to("cuda") if isinstance(v, np.ndarray) else v)
                     for k, v in mw.items()})
    x = torch.from_numpy(synth.normal_f16(rng, (M, H))).to("cuda")
    y = torch.empty_like(x)
    for _ in range(args.reps):
        for w in sets:
            ctx.moe_block(w, x, y, M, 3)
        for w in sets:
            ctx.moe_block({k: v for k, v in w.items() if not k.endswith("_alpha")}, x, y, M, 3)
    ctx.sync()
    print(f"done: {args.reps} x {args.sets} sets x 2 forms, E={E} I={I} rows={M}", flush=True)


if __name__ == "__main__":
    main()
