#!/usr/bin/env python3
"""Verify-step benchmark on one MI355X.

Workload (the verify step of a 24-layer Maple-like 2-bit MoE): hidden 2048, 16 query / 4 KV
heads of 128, sliding window 1024, RoPE base 1e6 on 64 dims, 64 experts top-8 with
intermediate 1024, 2-bit affine experts and projections (group 64), fp16 lm_head [151936 x
2048], RMSNorm eps 1e-6; random-init weights, a 2048-token seeded prompt prefilled into the KV
cache.  One step = one verify pass over [y] + K=8 chain draft rows (the first 5 draft tokens
are the target's greedy continuation, the other 3 random), device-side greedy acceptance and KV
commit, one host wait.  Reported value = accepted tokens (accepted + bonus) per second.
The 16-node depth-6 draft tree is measured the same way and reported under "tree".

roofline: the dominant kernel is the bucketed up||gate expert gather; algorithmic bytes per
launch = routed unique experts x 1,310,720 B (2-bit codes + fp16 scales/biases of 2048 x 2048)
+ activations, divided by its launch time from HIP events on the model stream.
cpu_baseline: the CPU oracle (C restatement, OpenMP) on a bounded sample of the same step --
2 of the 24 layers plus the full lm_head for the 9 verify rows, scaled to 24 layers.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
TREE16 = [-1, 0, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 10, 11, 12, 13, 14]
METRIC = "verify-step tokens/s (K=8, 1 GPU) + 2-bit gather-qmm HBM GB/s vs peak"
TIMER_HOLD_MS = 0.020  # length of the calibration hold the library brackets (MJ_KERNEL_TIMER)
UP_KERNEL = "void k_gather5<8, 64, 2, 8, 2, true, false, true>"  # up||gate gather, fused routing
MOE_KERNEL = "void k_moe_fused<64, false, 16>"  # up||gate then down in one launch (<= 16 rows)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def greedy_continuation(eng, y, n):
    L0 = eng.offset
    out, t = [], y
    for _ in range(n):
        t = eng.step_chain_feeds([t])[0]
        out.append(t)
    eng.rewind(L0)
    return out


def tree_draft(cont, vocab, rng, depth_hit=4):
    toks = [int(t) for t in rng.integers(0, vocab, len(TREE16) - 1)]
    depth = [0] * len(TREE16)
    for r in range(1, len(TREE16)):
        depth[r] = depth[TREE16[r]] + 1
    path = [0]
    while True:
        kids = [c for c in range(1, len(TREE16)) if TREE16[c] == path[-1]]
        if not kids:
            break
        path.append(kids[0])
    for d, r in enumerate(path[1:1 + depth_hit]):
        toks[r - 1] = cont[d]
    for r in range(1, len(TREE16)):
        if r not in path[1:1 + depth_hit] and toks[r - 1] == cont[depth[r] - 1]:
            toks[r - 1] = (toks[r - 1] + 1) % vocab
    return toks


def timed_steps(eng, y, draft, parents, L0, steps, warmup):
    import torch

    for _ in range(warmup):
        eng.rewind(L0)
        eng.verify_greedy(y, draft, parents)
    torch.cuda.synchronize()
    toks, dev_ms = 0, 0.0
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.rewind(L0)
        acc, _ = eng.verify_greedy(y, draft, parents)
        toks += acc + 1
        dev_ms += eng.last_pass_ms()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return toks, dt, dev_ms / steps, acc


def timed_sampled(eng, y, draft, L0, steps, warmup, **opts):
    """Sampled verify passes (T = 0.7, uniform draft q, fresh Philox counter each step); with
    `opts` the LogitsProcessor options go through mj_verify_sampled_ex."""
    import torch

    def one(i):
        eng.rewind(L0)
        if opts:
            return eng.verify_sampled_ex(y, draft, 1, 7, i, 0.7, **opts)
        return eng.verify_sampled(y, draft, 0.7, 1, 7, i)

    for i in range(warmup):
        one(i)
    torch.cuda.synchronize()
    toks, dev_ms = 0, 0.0
    t0 = time.perf_counter()
    for i in range(steps):
        acc, _ = one(warmup + i)
        toks += acc + 1
        dev_ms += eng.last_pass_ms()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return {"tokens_per_s": round(toks / dt, 3), "ms_per_step": round(dt / steps * 1e3, 4),
            "device_ms_per_step": round(dev_ms / steps, 4),
            "mean_tokens_per_step": round(toks / steps, 3)}


def expert_bytes(cfg, inds_layers, M):
    """Algorithmic bytes of one up||gate and one down launch per layer (unique experts once)."""
    H, I, gs, k = cfg.H, cfg.I, cfg.gs, cfg.top_k
    up_w = 2 * I * (H // 16 * 4 + 2 * (H // gs) * 2)
    dn_w = H * (I // 16 * 4 + 2 * (I // gs) * 2)
    up, dn, uniq = [], [], []
    for l in range(cfg.n_layers):
        eu = len(np.unique(inds_layers[l, :M]))
        uniq.append(eu)
        act = M * k * I * 2 + M * k * (I // 64) * 8
        xin = M * H * 2 + M * (H // 64) * 8
        up.append(eu * up_w + xin + act)
        dn.append(eu * dn_w + act + M * k * H * 2)
    return np.array(up), np.array(dn), np.array(uniq)


def kernel_profile(eng, cfg, y, draft, parents, L0, steps):
    """Per-kernel-class times of eager verify passes of (draft, parents) from HIP events, less
    the timer's own cost, and the HBM rates of the expert gathers and the head from the pass's
    own routing (unique experts per layer counted once)."""
    import torch

    M = len(draft) + 1
    icap = torch.empty((cfg.n_layers, 64, cfg.top_k), dtype=torch.int32, device="cuda")
    eng.rewind(L0)
    eng.set_capture(inds=icap)
    eng.verify_greedy(y, draft, parents)
    eng.set_capture()
    inds = icap.cpu().numpy()
    up_b, dn_b, uniq = expert_bytes(cfg, inds, M)
    eng.profile(True)
    for _ in range(steps):
        eng.rewind(L0)
        eng.verify_greedy(y, draft, parents)
    km = eng.kernel_ms()
    eng.profile(False)
    # each bracketed time is kernel + timer cost; brackets around a 20 us wall-clock hold in
    # the same passes give that cost, which is taken off every launch
    ev_ms, ev_n = km.pop("timer")
    ev_each = max(ev_ms / max(ev_n, 1) - TIMER_HOLD_MS, 0.0)
    km = {name: (ms - n * ev_each, n) for name, (ms, n) in km.items() if n > 0}
    hd_ms, hd_n = km["lm_head"]
    head_bytes = cfg.vocab * cfg.H * 2 + M * cfg.H * 2
    hd_gbs = head_bytes * hd_n / (hd_ms * 1e-3) / 1e9
    kernels = {name: dict(ms_per_launch=round(ms / max(n, 1), 5), launches=n)
               for name, (ms, n) in km.items()}
    rates = {}  # GB/s of the expert classes that ran, from the pass's own routing
    for name, b in (("expert_up", up_b), ("expert_down", dn_b), ("expert_moe", up_b + dn_b)):
        if name in km:
            ms, n = km[name]
            rates[name] = b.sum() * steps / (ms * 1e-3) / 1e9
            kernels[name]["GBps"] = round(rates[name], 1)
            kernels[name]["bytes_per_launch"] = int(b.mean())
    kernels["lm_head"]["GBps"] = round(hd_gbs, 1)
    kernels["lm_head"]["bytes_per_launch"] = int(head_bytes)
    # the dominant expert kernel: the fused launch where it ran, else the up||gate gather
    fused = "expert_moe" in km
    g = "expert_moe" if fused else "expert_up"
    return dict(kernels=kernels, rates=rates, hd_gbs=hd_gbs, g_gbs=rates[g], g_ms=km[g][0],
                g_n=km[g][1], g_b=(up_b + dn_b) if fused else up_b, fused=fused,
                timer_ms=ev_each, uniq=uniq)


def cpu_baseline(eng, cfg, weights, y, draft, L0, reps=5):
    """Oracle restatement timed on the host: layers 0-1 of the verify pass (from the GPU's own
    layer inputs and KV cache) + the full fp16 lm_head for the 9 rows; scaled to 24 layers.
    Median of `reps` timings with one OpenMP thread and with every core of the process."""
    import torch

    from oracle import oracle as orc

    orc.build()
    layers, embed, fnorm, head = weights
    M = len(draft) + 1
    hcap = torch.empty((cfg.n_layers + 1, 64, cfg.H), dtype=torch.float16, device="cuda")
    eng.rewind(L0)
    kv0 = []
    for l in range(2):
        k, _ = eng.kv(l)
        n = 2 * cfg.n_kv_heads * cfg.kv_capacity * 128
        buf = np.empty(n, np.float16)
        eng.ctx.check(eng.lib.mj_d2h(eng.ctx.h, buf.ctypes.data, k, n * 2))
        kv0.append(buf.reshape(2, cfg.n_kv_heads, cfg.kv_capacity, 128))
    eng.set_capture(h=hcap)
    acc, _ = eng.verify_greedy(y, draft)
    eng.set_capture()
    hc = hcap.cpu().numpy()

    def hw(d):
        return {kk: (v.detach().cpu().numpy().view(np.uint32) if v.dtype == torch.int32 else
                     v.detach().cpu().numpy()) if hasattr(v, "detach") else v
                for kk, v in d.items()}

    lw = [dict(attn=hw(layers[l]["attn"]), moe=hw(layers[l]["moe"])) for l in range(2)]
    head_h = head.cpu().numpy()
    fn = fnorm.cpu().numpy()
    par = np.array(list(range(-1, M - 1)), np.int32)

    def sample():
        """One timing of the bounded sample: (layers 0-1 seconds, lm_head seconds)."""
        t0 = time.perf_counter()
        for l in range(2):
            orc.layer_forward(cfg.attn_cfg(), lw[l], hc[l, :M], kv0[l][0], kv0[l][1], L0, par)
        t1 = time.perf_counter()
        xf = orc.rms_norm(hc[cfg.n_layers, :M], fn, cfg.eps)
        orc.argmax_rows(orc.lm_head_logits(xf, head_h))
        return t1 - t0, time.perf_counter() - t1

    all_threads = int(os.environ.get("OMP_NUM_THREADS", 0)) or len(os.sched_getaffinity(0))
    res = {}
    for threads in (1, all_threads):
        orc.set_threads(threads)
        runs = [sample() for _ in range(reps)]
        step = sorted(tl / 2 * cfg.n_layers + th for tl, th in runs)
        res[threads] = (step[len(step) // 2], runs)
        log(f"cpu baseline, {threads} thread(s): step s {['%.3f' % x for x in step]}")
    orc.set_threads(all_threads)
    med, runs = res[all_threads]
    med1, runs1 = res[1]
    tl, th = sorted(runs, key=lambda r: r[0] / 2 * cfg.n_layers + r[1])[len(runs) // 2]
    return dict(value=round((acc + 1) / med, 4), unit="tokens/s", cores=all_threads, kind="port",
                single_thread=dict(value=round((acc + 1) / med1, 4), cores=1),
                statistic=f"median of {reps}", cpu_model=cpu_model(),
                sample=(f"oracle verify pass, layers 0-1 of 24 ({tl:.3f} s, teacher-forced from "
                        f"the GPU layer inputs) + fp16 lm_head over 9 rows ({th:.3f} s), scaled "
                        f"to 24 layers: {med:.3f} s/step at {all_threads} threads, {med1:.3f} "
                        f"s/step at 1 thread, {acc + 1} tokens/step"))


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--copy-calib-mb", type=int, default=0,
                    help="end with one plain device copy of this many MiB (a known-size "
                         "reference for HBM counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X only (asked for --gpus {args.gpus}); the verify "
              "step here runs on a single GPU (expert / vocabulary sharding is a design, not "
              "built)", file=sys.stderr)
        sys.exit(2)

    import torch

    from momij_amd.engine import MapleLikeConfig, VerifyEngine, random_model
    from momij_amd.ops import Context

    ctx = Context(0)
    cfg = MapleLikeConfig()
    t0 = time.perf_counter()
    weights = random_model(cfg, seed=args.seed)
    torch.cuda.synchronize()
    eng = VerifyEngine(ctx, cfg, *weights)
    log(f"model ready in {time.perf_counter() - t0:.1f}s")
    rng = np.random.default_rng(args.seed)
    prompt = rng.integers(0, cfg.vocab, 2048).tolist()
    t0 = time.perf_counter()
    y = eng.prefill(prompt, chunk=64)
    log(f"prefill 2048 tokens in {time.perf_counter() - t0:.2f}s, offset {eng.offset}")
    cont = greedy_continuation(eng, y, 8)
    draft = cont[:5] + [int(t) for t in rng.integers(0, cfg.vocab, 3)]
    for i in range(5, 8):
        if draft[i] == cont[i]:
            draft[i] = (draft[i] + 1) % cfg.vocab
    L0 = eng.offset

    # headline: chain K=8, graphs on
    toks, dt, dev_ms, acc = timed_steps(eng, y, draft, None, L0, args.steps, args.warmup)
    value = toks / dt
    log(f"chain K=8: {value:.1f} tok/s, {dt / args.steps * 1e3:.3f} ms/step wall, "
        f"{dev_ms:.3f} ms/step device, accepted {acc}")
    # tree
    tdraft = tree_draft(cont, cfg.vocab, rng)
    ttoks, tdt, tdev, tacc = timed_steps(eng, y, tdraft, TREE16, L0, args.steps, args.warmup)
    log(f"tree16: {ttoks / tdt:.1f} tok/s, {tdt / args.steps * 1e3:.3f} ms/step, accepted {tacc}")
    # sampled verify of the same chain: plain softmax, then top-p 0.9 with repetition 1.1,
    # presence 0.1 and frequency 0.1 over the prompt's token counts
    sampled = timed_sampled(eng, y, draft, L0, args.steps, args.warmup)
    htok, hcnt = np.unique(np.asarray(prompt, np.int32), return_counts=True)
    hist = (htok.astype(np.int32), hcnt.astype(np.int32))  # ascending tokens, counts
    sampled_opts = timed_sampled(eng, y, draft, L0, args.steps, args.warmup, top_p=0.9, rep=1.1,
                                 pres=0.1, freq=0.1, hist=hist)
    log(f"sampled: {sampled}; top-p + penalties: {sampled_opts}")

    # per-kernel times from HIP events (eager passes) and the routing of the pass: the K=8
    # chain (the headline) and the 16-node tree (config 4's own pass, 17 rows)
    prof_steps = max(5, min(args.steps, 20))
    kp = kernel_profile(eng, cfg, y, draft, None, L0, prof_steps)
    kt = kernel_profile(eng, cfg, y, tdraft, TREE16, L0, prof_steps)
    kernels, g_gbs, g_ms, g_n, ev_each, g_b, uniq = (
        kp["kernels"], kp["g_gbs"], kp["g_ms"], kp["g_n"], kp["timer_ms"], kp["g_b"],
        kp["uniq"])
    g_kernel = MOE_KERNEL if kp["fused"] else UP_KERNEL
    g_label = ("expert up||gate gather + SwiGLU, then down gather, one launch" if kp["fused"]
               else "expert up||gate gather + SwiGLU")
    M = len(draft) + 1
    log(f"experts {', '.join(f'{k} {v:.0f} GB/s' for k, v in kp['rates'].items())}, head "
        f"{kp['hd_gbs']:.0f} GB/s, unique experts/layer {uniq.mean():.1f}")
    log(f"tree16 (17 rows): experts {', '.join(f'{k} {v:.0f} GB/s' for k, v in kt['rates'].items())}, "
        f"head {kt['hd_gbs']:.0f} GB/s, unique experts/layer {kt['uniq'].mean():.1f}")

    # HBM bytes per launch of the same kernel, from the FETCH_SIZE / WRITE_SIZE collections
    # summarised under profiles/ (counter runs cannot share a process with this timing)
    traffic, tpath = None, os.path.join(
        ROOT, "profiles",
        "expert_moe_fused_k8_traffic.json" if kp["fused"] else "expert_up_gather_k8_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            t = json.load(f)
        if t.get("kernel") == g_kernel and t.get("rows") == M:
            traffic = t["traffic_bytes_per_launch"]

    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(eng, cfg, weights, y, draft, L0)
            log(f"cpu baseline {cpu}")
        except Exception as e:  # the CPU leg is reported, never required
            log(f"cpu baseline skipped: {e!r}")

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded random-init weights, 2048-token random prompt)",
        "config": {
            "workload": "24-layer Maple-like 2-bit MoE verify step, K=8 chain draft "
                        "(5 accepted + bonus), 2048-token prompt, window 1024",
            "layers": cfg.n_layers, "hidden": cfg.H, "experts": cfg.E, "top_k": cfg.top_k,
            "moe_intermediate": cfg.I, "group_size": cfg.gs, "vocab": cfg.vocab,
            "verify_rows": M, "accepted": acc, "device_ms_per_step": round(dev_ms, 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": g_label + " (" + g_kernel + ")",
            "achieved": round(g_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(g_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": int(g_b.mean()),
            "ms_per_launch": round(g_ms / max(g_n, 1), 5),
            "timer_ms_per_launch": round(ev_each, 5),
        },
        "cpu_baseline": cpu,
        "tree": {"tokens_per_s": round(ttoks / tdt, 3), "ms_per_step": round(tdt / args.steps * 1e3, 4),
                 "accepted": tacc, "rows": len(TREE16), "device_ms_per_step": round(tdev, 4),
                 "kernels": kt["kernels"],
                 "unique_experts_per_layer": round(float(kt["uniq"].mean()), 2)},
        "sampled": dict(sampled, temperature=0.7, q="uniform 1/V"),
        "sampled_top_p_penalties": dict(sampled_opts, temperature=0.7, top_p=0.9,
                                        repetition=1.1, presence=0.1, frequency=0.1),
        "kernels": kernels,
        "unique_experts_per_layer": round(float(uniq.mean()), 2),
    }
    print(json.dumps(line), flush=True)
    if args.copy_calib_mb > 0:
        n = args.copy_calib_mb << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: {n} bytes")
    eng.close()
    ctx.close()


if __name__ == "__main__":
    main()
