"""Teacher-forced parity of a captured verify pass against the oracle (test infrastructure).

A pass run with mj_model_set_capture_ex leaves every block boundary on the device: each
layer's input h, its attention output, the normed MoE input, the router logits and routing,
the layer output, the K/V rows appended, and the head input and logits.  Each block is re-run
by the oracle from exactly the inputs the device used, so the only differences left are the
two implementations' own rounding:

  * router logits: |gpu - oracle| <= fp32_bound (a first-order bound on both fp32 sums);
  * top-k of the device's own logits through the oracle's rule == the device's routing, exactly;
  * top-k of the oracle's logits == the device's routing, except rows whose k / k+1 logit gap
    is inside the two sums' bound (a tie the fp32 rounding decides; reported);
  * head argmax == the oracle's argmax of the same head input, except where the oracle's
    best and the device's pick differ by less than the bound;
  * float outputs within the verify step's tolerance (2e-2 relative to the norm, 1e-2 abs).
"""
from __future__ import annotations

import numpy as np

from tests.gpu_util import assert_close, host

EPS32 = 2.0 ** -24


def fp32_dot_bound(w, x, depth):
    """|fl(sum_k w x) - exact| <= depth * 2^-24 * sum_k |w x| (first order), for every pair of
    rows of w [N][K] and x [M][K]; returns [M][N]."""
    aw = np.abs(np.asarray(w, np.float64))
    ax = np.abs(np.asarray(x, np.float64))
    return depth * EPS32 * (ax @ aw.T)


def router_depth(H):
    """Rounding depth of one router logit: the device's lane partials (16 dot2 steps) and its
    6-level shuffle tree, the oracle's 32 lane sums of H/32 terms and its 5-level tree."""
    return (16 + 6) + (H // 32 + 5) + 2


def head_depth(K):
    """Rounding depth of one lm_head logit: the device's MFMA chains (K/32 products per lane
    position, two K halves, per-MFMA 32-term sums) and the oracle's double sum rounded once."""
    return K // 16 + 64 + 1


def host_layer(lw: dict) -> dict:
    """A layer's device weights as host arrays (int32 device views become uint32)."""
    def h(v):
        if not hasattr(v, "detach"):
            return v
        a = v.detach().cpu().numpy()
        return a.view(np.uint32) if a.dtype == np.int32 else a

    return {"attn": {k: h(v) for k, v in lw["attn"].items()},
            "moe": {k: h(v) for k, v in lw["moe"].items()}}


def check_routing(orc, W, xn, gpu_logits, gpu_inds, k, what):
    """Router logits within the fp32 bound, the top-k rule exact; returns rows decided by a
    rounding-level tie."""
    ref = orc.router_logits(W, xn)
    bound = fp32_dot_bound(W, xn, router_depth(xn.shape[1]))
    err = np.abs(gpu_logits.astype(np.float64) - ref)
    assert (err <= bound).all(), (what, "router logits", float((err / bound).max()))
    own, _ = orc.route_topk(gpu_logits, k)
    assert (own == gpu_inds).all(), (what, "top-k of the device logits", own, gpu_inds)
    ri, _ = orc.route_topk(ref, k)
    ties = []
    for r in range(len(gpu_inds)):
        if (ri[r] == gpu_inds[r]).all():
            continue
        s = np.sort(ref[r])[::-1]
        gap = s[k - 1] - s[k]
        b2 = 2 * np.sort(bound[r])[::-1][: k + 1].max()
        assert gap <= b2, (what, r, "routing differs outside the rounding bound", ri[r],
                           gpu_inds[r], gap, b2)
        print(f"[{what}] row {r}: routing decided by a rounding-level tie (gap {gap:.2e} <= "
              f"{b2:.2e})", flush=True)
        ties.append(r)
    return ties


def check_head(orc, head_in, gpu_argmax, what, w_head=None, q4=None, banned=None):
    """Oracle logits of the device's own head input (fp16 head w_head [V][K], or q4 = (w, s, b)
    of the 4-bit head); the argmax must equal the device's unless the oracle's best and the
    device's pick are within the rounding bound.  Returns (oracle argmax, oracle logits)."""
    from momij_amd import synth

    if q4 is not None:
        ref = orc.lm_head_q4_logits(head_in, *q4)

        def rows(ids):
            return synth.dequant4(q4[0][ids], q4[1][ids], q4[2][ids])
    else:
        ref = orc.lm_head_logits(head_in, w_head)

        def rows(ids):
            return w_head[ids]
    idx, best, _ = orc.argmax_rows(ref, banned)
    K = head_in.shape[1]
    for r, (g, o) in enumerate(zip(gpu_argmax, idx)):
        if g == o:
            continue
        b = fp32_dot_bound(rows([g, o]), head_in[r:r + 1], head_depth(K))[0]
        gap = best[r] - ref[r, g]
        assert gap <= b.sum() + EPS32 * abs(best[r]), (what, r, g, o, gap, b)
        print(f"[{what}] row {r}: argmax tie within the bound ({g} vs {o}, gap {gap:.2e})",
              flush=True)
    return idx, ref


def capture_pass(eng, fn, logits=True):
    """Run fn() with every block boundary of its passes captured; returns (fn(), host copies).
    The capture keeps the last pass's values."""
    bufs = eng.capture_buffers(logits=logits)
    eng.set_capture_ex(**bufs)
    try:
        out = fn()
    finally:
        eng.set_capture_ex()
    return out, {k: host(v) for k, v in bufs.items()}


def check_layer(orc, cfg, l, lw_host, cap, M, kv_before, L, parents):
    """One layer of a captured pass re-run by the oracle from the device's inputs.
    cap: host copies of the capture buffers; kv_before: (k, v) host caches before the pass."""
    par = np.asarray(parents, np.int32)
    acfg = cfg.attn_cfg(l)
    h_in = cap["h"][l, :M]
    h_mid, kc, vc = orc.attn_block(acfg, lw_host["attn"], h_in, kv_before[0], kv_before[1], L,
                                   par)
    assert_close(cap["attn_out"][l, :M], h_mid, what=f"layer {l} attention out")
    # the appended rows (before any commit)
    C = acfg["C"]
    slots = [(L + r) % C for r in range(M)]
    assert_close(cap["kv_rows"][l, 0, :, :M], kc[:, slots], what=f"layer {l} K rows")
    assert_close(cap["kv_rows"][l, 1, :, :M], vc[:, slots], what=f"layer {l} V rows")
    mw = lw_host["moe"]
    xn = orc.rms_norm(cap["attn_out"][l, :M], mw["norm_w"], cfg.eps)
    assert_close(cap["moe_in"][l, :M], xn, what=f"layer {l} moe norm")
    ties = check_routing(orc, mw["router_w"], cap["moe_in"][l, :M],
                         cap["router_logits"][l, :M], cap["inds"][l, :M], cfg.top_k,
                         f"layer {l}")
    h_out, ri, _ = orc.moe_block(mw, cap["attn_out"][l, :M], prenorm=True, residual=True)
    keep = [r for r in range(M) if r not in ties]
    assert_close(cap["h"][l + 1, keep], h_out[keep], what=f"layer {l} out")
    return ties
