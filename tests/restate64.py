"""float64 numpy restatement of the verify step's composite blocks (test infrastructure).

An independent second statement of what the reference computes, used to pin the CPU oracle's
composites (MoE block, attention block, layer, score-weighted residual).  Arithmetic is float64
and vectorised; values are rounded to fp16 exactly where the reference's kernels store `half`
(the rounding points are part of the semantics):

  MoE block (encodeMoEBlock, SeedlessMetal.swift:576-609; MapleMoE.swift:58-80)
    xn   = half(rms(x) * w)                          maple_rms_norm 2496-2526
    l    = W_router xn          (not rounded)        maple_batched_gemv 2574-2595
    top-k by logit, lowest index on ties, softmax gates renormalised over the k
                                                     maple_route_top8 2720-2791
    ug   = half(deq(up||gate)[e] xn)   rows 0..I-1 up, I..2I-1 gate (WeightStore.swift:81-90)
    act  = half(silu(min(gate, 7)) * clamp(up, -7, 7))   maple_clamped_swiglu 2435-2450
    d    = half(deq(down)[e] act)
    y    = half(x + half(sum_k d_k score_k))         maple_score_resid 2474-2493

  Attention block (encodeAttnBlock 926-1005 + the input norm of encodeLayerBlock 1008-1048)
    xa   = half(rms(h) * w);  qkv = half(deq(qkv) xa)   q rows, k rows, v rows (WeightStore 66-79)
    q, k = half(rope(rms_head(.) * w_qk))   non-traditional half split on the first rope_dim
           dims at position L + depth(r)           maple_qk_norm_rope 2794-2847
    v    = the raw v rows (no norm)
    K/V appended at slot (L + r) % C                maple_write_kv_pair 2871-2901
    o    = half(softmax(q k^T / sqrt(D)) v) over the row's window and its tree ancestors
                                                   maple_sdpa_d128 2919-2997, AttentionMasks 10-27
    h    = half(h + half(deq(o_proj) o))            gqmm2_rows_fold_add 3488-3543

Nothing here calls the oracle.
"""
from __future__ import annotations

import math

import numpy as np

from momij_amd import synth


def f16(x) -> np.ndarray:
    """Round to fp16 and return float64 (IEEE round to nearest even, via numpy)."""
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def rms(x, w, eps) -> np.ndarray:
    x = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return f16(x * inv * np.asarray(w, np.float64))


def route(logits, k):
    """Top-k by logit (lowest index on ties), softmax gates renormalised over the k."""
    logits = np.asarray(logits, np.float64)
    M, E = logits.shape
    inds = np.zeros((M, k), np.int64)
    scores = np.zeros((M, k))
    for m in range(M):
        order = sorted(range(E), key=lambda e: (-logits[m, e], e))[:k]
        g = np.exp(logits[m] - logits[m].max())
        g /= g.sum()
        inds[m] = order
        scores[m] = g[order] / g[order].sum()
    return inds, scores


def topk_gap(logits, k):
    """Gap between the k-th and (k+1)-th largest logit of each row (routing robustness)."""
    s = -np.sort(-np.asarray(logits, np.float64), axis=1)
    return s[:, k - 1] - s[:, k]


def moe_block(mw: dict, x, prenorm=True, residual=True, swap_up_gate=False, skip_norm_up=False,
              inds=None):
    """Returns (y fp16-valued float64 [M][H], inds, scores, logits).  swap_up_gate /
    skip_norm_up plant known mistakes (negative controls); inds forces the routing."""
    x = np.asarray(x, np.float64)
    M, H = x.shape
    E, k, I, gs = mw["E"], mw["top_k"], mw["I"], mw["gs"]
    xn = rms(x, mw["norm_w"], mw["eps"]) if prenorm else f16(x)
    logits = xn @ np.asarray(mw["router_w"], np.float64).T
    ri, sc = route(logits, k)
    if inds is not None:
        ri = np.asarray(inds, np.int64)
    ug_w = synth.dequant(mw["up_gate_w"], mw["up_gate_s"], mw["up_gate_b"], gs)
    dn_w = synth.dequant(mw["down_w"], mw["down_s"], mw["down_b"], gs)
    up_in = f16(x) if skip_norm_up else xn
    acc = np.zeros((M, H))
    for m in range(M):
        for j in range(k):
            e = ri[m, j]
            ug = f16(ug_w[e] @ up_in[m])
            up, gate = (ug[I:], ug[:I]) if swap_up_gate else (ug[:I], ug[I:])
            g = np.minimum(gate, 7.0)
            act = f16(g / (1.0 + np.exp(-g)) * np.clip(up, -7.0, 7.0))
            d = f16(dn_w[e] @ act)
            acc[m] += d * float(np.float32(sc[m, j]))
    y = f16(x + f16(acc)) if residual else f16(acc)
    return y, ri, sc, logits


def score_resid(down, scores, h):
    """h = half(h + half(sum_k down_k * score_k)); down [M*k][H], scores [M][k]."""
    M, k = scores.shape
    d = np.asarray(down, np.float64).reshape(M, k, -1)
    acc = np.einsum("mkh,mk->mh", d, np.asarray(scores, np.float64))
    return f16(np.asarray(h, np.float64) + f16(acc))


def tree_of(parents, M):
    par = list(range(-1, M - 1)) if parents is None else [int(p) for p in parents]
    depth = [0] * M
    anc = np.eye(M, dtype=bool)
    for r in range(1, M):
        depth[r] = depth[par[r]] + 1
        anc[r] |= anc[par[r]]
    return par, depth, anc


def rope_heads(x, w, pos, rope_dim, base, eps):
    """Per-head RMSNorm * w then the half-split RoPE of the first rope_dim dims; x [nh][D]."""
    x = np.asarray(x, np.float64)
    D = x.shape[-1]
    v = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * np.asarray(w, np.float64)
    if rope_dim > 0:
        half = rope_dim // 2
        inv = np.asarray(np.float32(base) ** (-np.arange(half, dtype=np.float32) / np.float32(half)),
                         np.float64)
        th = float(pos) * inv
        a, b = v[:, :half].copy(), v[:, half:rope_dim].copy()
        v[:, :half] = a * np.cos(th) - b * np.sin(th)
        v[:, half:rope_dim] = b * np.cos(th) + a * np.sin(th)
    return f16(v)


def attn_block(cfg: dict, aw: dict, h, kcache, vcache, L, parents, norm_v=False):
    """Returns (h_out, kcache, vcache) as float64 arrays of fp16 values.  norm_v plants the
    mistake of passing V through the k-norm (negative control)."""
    H, nQ, nKV, D = cfg["H"], cfg["nQ"], cfg["nKV"], cfg["D"]
    C, W, gs = cfg["C"], cfg["window"], cfg["gs"]
    h = np.asarray(h, np.float64)
    M = h.shape[0]
    kc = np.array(kcache, np.float64)
    vc = np.array(vcache, np.float64)
    par, depth, anc = tree_of(parents, M)
    xa = rms(h, aw["norm_w"], cfg["eps"])
    qkv = f16(xa @ synth.dequant(aw["qkv_w"], aw["qkv_s"], aw["qkv_b"], gs).T)
    q = np.zeros((M, nQ, D))
    for r in range(M):
        pos = L + depth[r]
        heads = qkv[r, :nQ * D].reshape(nQ, D)
        q[r] = rope_heads(heads, aw["q_norm_w"], pos, cfg["rope_dim"], cfg["rope_base"], cfg["eps"])
        kh = qkv[r, nQ * D:(nQ + nKV) * D].reshape(nKV, D)
        vh = qkv[r, (nQ + nKV) * D:].reshape(nKV, D)
        slot = (L + r) % C
        kc[:, slot] = rope_heads(kh, aw["k_norm_w"], pos, cfg["rope_dim"], cfg["rope_base"],
                                 cfg["eps"])
        vc[:, slot] = rope_heads(vh, aw["k_norm_w"], pos, 0, 1.0, cfg["eps"]) if norm_v else vh
    o = np.zeros((M, nQ * D))
    gqa = nQ // nKV
    for r in range(M):
        P = L + depth[r]
        lo = max(0, P - W + 1) if W > 0 else 0
        slots = [p % C for p in range(lo, L)] + [(L + a) % C for a in range(M)
                                                 if anc[r, a] and L + depth[a] >= lo]
        for hh in range(nQ):
            g = hh // gqa
            s = kc[g, slots] @ q[r, hh] / math.sqrt(D)
            p = np.exp(s - s.max())
            o[r, hh * D:(hh + 1) * D] = p @ vc[g, slots] / p.sum()
    o = f16(o)
    proj = f16(o @ synth.dequant(aw["o_w"], aw["o_s"], aw["o_b"], gs).T)
    return f16(h + proj), kc, vc

