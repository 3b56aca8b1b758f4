"""ctypes binding of the CPU oracle (libmomij_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the parity reference or the timed CPU baseline, never as the thing
measured or shipped.  The product (momij_amd / libmomij_hip.so) never imports this module.

fp16 arrays are numpy float16; everything else is float32 / int32 / int64 / uint32.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmomij_oracle.so")

_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, seconds)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", HERE], check=True)
    return LIB_PATH


def _p(a, ct):
    return a.ctypes.data_as(C.POINTER(ct)) if a is not None else None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        L = _lib
        L.or_h2f.restype = C.c_float
        L.or_h2f.argtypes = [C.c_uint16]
        L.or_f2h.restype = C.c_uint16
        L.or_f2h.argtypes = [C.c_float]
        L.or_canon_expf.restype = C.c_float
        L.or_canon_expf.argtypes = [C.c_float]
        L.or_canon_sum.restype = C.c_float
        L.or_canon_walk.restype = C.c_int
        L.or_canon_walk.argtypes = [C.c_void_p, C.c_int, C.c_float]
        L.or_u01_from_u32.restype = C.c_float
        L.or_splitmix64_next.restype = C.c_uint64
        L.or_accept_greedy.restype = C.c_int
        L.or_accept_sampled.restype = C.c_int
        L.or_accept_sampled.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_float,
                                        C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
        L.or_set_threads.argtypes = [C.c_int]
        L.or_max_threads.restype = C.c_int
        L.or_accept_sampled_ex.restype = C.c_int
        L.or_accept_sampled_ex.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_float,
                                           C.c_float, C.c_float, C.c_float, C.c_float,
                                           C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                           C.c_void_p, C.c_void_p]
        L.or_penalize_row.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int,
                                      C.c_void_p, C.c_int, C.c_float, C.c_float, C.c_float]
        L.or_nucleus_sample.restype = C.c_int
        L.or_nucleus_sample.argtypes = [C.c_void_p, C.c_int, C.c_float, C.c_float, C.c_float]
        L.or_try_accept.restype = C.c_int
        L.or_try_accept.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_float,
                                    C.c_float, C.c_void_p, C.c_void_p]
        L.or_walk_draft.restype = C.c_int
        L.or_walk_draft.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int,
                                    C.c_float, C.c_void_p, C.c_void_p]
        L.or_verify_uniforms.argtypes = [C.c_uint64, C.c_uint64, C.c_int, C.c_void_p]
        vp, i = C.c_void_p, C.c_int
        L.or_h2f_array.argtypes = [vp, vp, C.c_size_t]
        L.or_f2h_array.argtypes = [vp, vp, C.c_size_t]
        L.or_qmm2.argtypes = [vp] * 6 + [i] * 6
        L.or_clamped_swiglu.argtypes = [vp, vp, i, i]
        L.or_score_reduce.argtypes = [vp, vp, vp, i, i, i]
        L.or_score_resid.argtypes = [vp, vp, vp, i, i, i]
        L.or_router_logits.argtypes = [vp, vp, vp, i, i, i]
        L.or_route_topk.argtypes = [vp, vp, vp, i, i, i]
        L.or_moe_block.argtypes = [vp, vp, vp, i, i, vp, vp]
        L.or_layer_forward.argtypes = [vp, vp, vp, vp, vp, vp, C.c_int64, vp, i, vp, vp]
        L.or_attn_block.argtypes = [vp, vp, vp, vp, vp, vp, C.c_int64, vp, i]
        L.or_kv_commit.argtypes = [vp, vp, i, C.c_int64, i, C.c_int64, vp, i]
        L.or_lm_head_logits.argtypes = [vp, vp, vp, i, i, i]
        L.or_lm_head_q4_logits.argtypes = [vp, vp, vp, vp, vp, i, i, i]
        L.or_argmax_rows.argtypes = [vp, i, i, vp, i, vp, vp, vp]
        L.or_accept_greedy.argtypes = [vp, vp, vp, i, vp, vp]
        L.or_philox4x32_10.argtypes = [vp, vp, vp]
        L.or_splitmix64_next.argtypes = [vp]
        L.or_canon_sum.argtypes = [vp, i]
        L.or_rms_norm.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_float]
        L.or_rope_inv_freq.argtypes = [C.c_void_p, C.c_int, C.c_float]
        L.or_qk_norm_rope.argtypes = [C.c_void_p] * 7 + [C.c_int] * 5 + [C.c_float]
        L.or_attention.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64,
                                   C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                   C.c_void_p]
    return _lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def f2h(x) -> np.ndarray:
    """fp32 -> fp16 bit patterns (uint16) via the oracle's own conversion."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f2h_array(x.ctypes.data, out.ctypes.data, C.c_size_t(x.size))
    return out


def h2f(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_h2f_array(h.ctypes.data, out.ctypes.data, C.c_size_t(h.size))
    return out


def qmm2(x, w, scales, biases, inds, M, ktop, K, N, gs, lhs_per_expert=False):
    """gqmm2_rows semantics: y [M*ktop, N] fp16."""
    x = _c(x, np.float16)
    w = _c(w, np.uint32)
    s = _c(scales, np.float16)
    b = _c(biases, np.float16)
    inds = _c(inds, np.int32)
    y = np.empty((M * ktop, N), np.float16)
    lib().or_qmm2(x.ctypes.data, w.ctypes.data, s.ctypes.data, b.ctypes.data, inds.ctypes.data,
                  y.ctypes.data, M, ktop, K, N, gs, int(lhs_per_expert))
    return y


def clamped_swiglu(ug, rows, I):
    ug = _c(ug, np.float16)
    act = np.empty((rows, I), np.float16)
    lib().or_clamped_swiglu(ug.ctypes.data, act.ctypes.data, rows, I)
    return act


def score_reduce(down, scores, M, ktop, H):
    down = _c(down, np.float16)
    scores = _c(scores, np.float32)
    y = np.empty((M, H), np.float16)
    lib().or_score_reduce(down.ctypes.data, scores.ctypes.data, y.ctypes.data, M, ktop, H)
    return y


def score_resid(down, scores, h):
    """h + combine of the expert rows (two fp16 roundings); down [M*k][H], scores [M][k]."""
    scores = _c(scores, np.float32)
    M, k = scores.shape
    down = _c(down, np.float16)
    out = np.array(h, dtype=np.float16, copy=True, order="C")
    lib().or_score_resid(down.ctypes.data, scores.ctypes.data, out.ctypes.data, M, k,
                         out.shape[1])
    return out


def set_threads(n: int):
    """OpenMP threads of the oracle's parallel loops."""
    lib().or_set_threads(int(n))


def max_threads() -> int:
    return int(lib().or_max_threads())


def rms_norm(x, w, eps):
    x = _c(x, np.float16)
    w = _c(w, np.float16)
    M, H = x.shape
    out = np.empty_like(x)
    lib().or_rms_norm(x.ctypes.data, w.ctypes.data, out.ctypes.data, M, H, C.c_float(eps))
    return out


def router_logits(W, x):
    W = _c(W, np.float16)
    x = _c(x, np.float16)
    E, H = W.shape
    M = x.shape[0]
    out = np.empty((M, E), np.float32)
    lib().or_router_logits(W.ctypes.data, x.ctypes.data, out.ctypes.data, M, E, H)
    return out


def route_topk(logits, k):
    logits = _c(logits, np.float32)
    M, E = logits.shape
    inds = np.empty((M, k), np.int32)
    scores = np.empty((M, k), np.float32)
    lib().or_route_topk(logits.ctypes.data, inds.ctypes.data, scores.ctypes.data, M, E, k)
    return inds, scores


class _MoeW(C.Structure):
    _fields_ = [("norm_w", C.c_void_p), ("router_w", C.c_void_p), ("up_gate_w", C.c_void_p),
                ("up_gate_s", C.c_void_p), ("up_gate_b", C.c_void_p), ("down_w", C.c_void_p),
                ("down_s", C.c_void_p), ("down_b", C.c_void_p), ("E", C.c_int), ("top_k", C.c_int),
                ("H", C.c_int), ("I", C.c_int), ("gs", C.c_int), ("eps", C.c_float)]


class _AttnW(C.Structure):
    _fields_ = [("norm_w", C.c_void_p), ("qkv_w", C.c_void_p), ("qkv_s", C.c_void_p),
                ("qkv_b", C.c_void_p), ("q_norm_w", C.c_void_p), ("k_norm_w", C.c_void_p),
                ("o_w", C.c_void_p), ("o_s", C.c_void_p), ("o_b", C.c_void_p)]


class _Cfg(C.Structure):
    _fields_ = [("H", C.c_int), ("nQ", C.c_int), ("nKV", C.c_int), ("D", C.c_int),
                ("rope_dim", C.c_int), ("window", C.c_int), ("gs", C.c_int),
                ("rope_base", C.c_float), ("eps", C.c_float), ("C", C.c_int64)]


class _LayerW(C.Structure):
    _fields_ = [("attn", _AttnW), ("moe", _MoeW)]


def _moe_struct(mw: dict, keep: list):
    def ptr(name, dt):
        if mw.get(name) is None:
            return None
        a = _c(mw[name], dt)
        keep.append(a)
        return a.ctypes.data

    return _MoeW(ptr("norm_w", np.float16), ptr("router_w", np.float16),
                 ptr("up_gate_w", np.uint32), ptr("up_gate_s", np.float16),
                 ptr("up_gate_b", np.float16), ptr("down_w", np.uint32),
                 ptr("down_s", np.float16), ptr("down_b", np.float16), mw["E"], mw["top_k"],
                 mw["H"], mw["I"], mw["gs"], mw["eps"])


def _attn_struct(aw: dict, keep: list):
    def ptr(name, dt):
        a = _c(aw[name], dt)
        keep.append(a)
        return a.ctypes.data

    return _AttnW(ptr("norm_w", np.float16), ptr("qkv_w", np.uint32), ptr("qkv_s", np.float16),
                  ptr("qkv_b", np.float16), ptr("q_norm_w", np.float16),
                  ptr("k_norm_w", np.float16), ptr("o_w", np.uint32), ptr("o_s", np.float16),
                  ptr("o_b", np.float16))


def moe_block(mw: dict, x, prenorm=False, residual=False):
    """MoE block; mw keys: router_w, up_gate_{w,s,b}, down_{w,s,b}, norm_w, E, top_k, H, I, gs, eps."""
    keep = []
    st = _moe_struct(mw, keep)
    x = _c(x, np.float16)
    M = x.shape[0]
    y = np.empty_like(x)
    inds = np.empty((M, mw["top_k"]), np.int32)
    scores = np.empty((M, mw["top_k"]), np.float32)
    flags = (1 if prenorm else 0) | (2 if residual else 0)
    lib().or_moe_block(C.byref(st), x.ctypes.data, y.ctypes.data, M, flags, inds.ctypes.data,
                       scores.ctypes.data)
    return y, inds, scores


def rope_inv_freq(rope_dim, base):
    out = np.empty(max(rope_dim // 2, 1), np.float32)
    lib().or_rope_inv_freq(out.ctypes.data, rope_dim, C.c_float(base))
    return out


def qk_norm_rope(qkv, q_norm_w, k_norm_w, inv_freq, pos, nQ, nKV, D, rope_dim, eps):
    qkv = _c(qkv, np.float16)
    M = qkv.shape[0]
    pos = _c(pos, np.int64)
    qn = _c(q_norm_w, np.float16)
    kn = _c(k_norm_w, np.float16)
    inv = _c(inv_freq, np.float32)
    qo = np.empty((M, nQ, D), np.float16)
    ko = np.empty((M, nKV, D), np.float16)
    lib().or_qk_norm_rope(qkv.ctypes.data, qn.ctypes.data, kn.ctypes.data, inv.ctypes.data,
                          pos.ctypes.data, qo.ctypes.data, ko.ctypes.data, M, nQ, nKV, D,
                          rope_dim, C.c_float(eps))
    return qo, ko


def attention(q, kcache, vcache, C_slots, L, parents, window):
    q = _c(q, np.float16)
    M, nQ, D = q.shape
    kc = _c(kcache, np.float16)
    vc = _c(vcache, np.float16)
    nKV = kc.shape[0]
    par = None if parents is None else _c(parents, np.int32)
    out = np.empty((M, nQ * D), np.float16)
    lib().or_attention(q.ctypes.data, kc.ctypes.data, vc.ctypes.data, C_slots, L,
                       None if par is None else par.ctypes.data, M, nQ, nKV, D, window,
                       out.ctypes.data)
    return out


def make_cfg(cfg: dict) -> _Cfg:
    return _Cfg(cfg["H"], cfg["nQ"], cfg["nKV"], cfg["D"], cfg["rope_dim"], cfg["window"],
                cfg["gs"], cfg["rope_base"], cfg["eps"], cfg["C"])


def attn_block(cfg: dict, aw: dict, h, kcache, vcache, L, parents):
    """Attention block with residual on copies; returns (h_out, kcache, vcache)."""
    keep = []
    st = _attn_struct(aw, keep)
    c = make_cfg(cfg)
    inv = rope_inv_freq(cfg["rope_dim"], cfg["rope_base"])
    h = np.array(h, dtype=np.float16, copy=True, order="C")
    kc = np.array(kcache, dtype=np.float16, copy=True, order="C")
    vc = np.array(vcache, dtype=np.float16, copy=True, order="C")
    par = _c(parents, np.int32)
    lib().or_attn_block(C.byref(c), C.byref(st), inv.ctypes.data, h.ctypes.data, kc.ctypes.data,
                        vc.ctypes.data, C.c_int64(L), par.ctypes.data, h.shape[0])
    return h, kc, vc


def layer_forward(cfg: dict, lw: dict, h, kcache, vcache, L, parents):
    """One decoder layer in place on copies; returns (h_out, kcache, vcache, inds, scores)."""
    keep = []
    st = _LayerW(_attn_struct(lw["attn"], keep), _moe_struct(lw["moe"], keep))
    c = make_cfg(cfg)
    inv = rope_inv_freq(cfg["rope_dim"], cfg["rope_base"])
    h = np.array(h, dtype=np.float16, copy=True, order="C")
    kc = np.array(kcache, dtype=np.float16, copy=True, order="C")
    vc = np.array(vcache, dtype=np.float16, copy=True, order="C")
    M = h.shape[0]
    par = _c(parents, np.int32)
    k = lw["moe"]["top_k"]
    inds = np.empty((M, k), np.int32)
    scores = np.empty((M, k), np.float32)
    lib().or_layer_forward(C.byref(c), C.byref(st), inv.ctypes.data, h.ctypes.data,
                           kc.ctypes.data, vc.ctypes.data, C.c_int64(L), par.ctypes.data, M,
                           inds.ctypes.data, scores.ctypes.data)
    return h, kc, vc, inds, scores


def kv_commit(kcache, vcache, L, path):
    """Accepted tree path moved into consecutive positions; caches [nKV][C][D], returns copies."""
    kc = np.array(kcache, dtype=np.float16, copy=True, order="C")
    vc = np.array(vcache, dtype=np.float16, copy=True, order="C")
    nKV, Cs, D = kc.shape
    p = _c(path, np.int32)
    lib().or_kv_commit(kc.ctypes.data, vc.ctypes.data, nKV, C.c_int64(Cs), D, C.c_int64(L),
                       p.ctypes.data, len(p))
    return kc, vc


def lm_head_logits(x, w):
    x = _c(x, np.float16)
    w = _c(w, np.float16)
    M, K = x.shape
    V = w.shape[0]
    out = np.empty((M, V), np.float32)
    lib().or_lm_head_logits(x.ctypes.data, w.ctypes.data, out.ctypes.data, M, K, V)
    return out


def lm_head_q4_logits(x, w, scales, biases):
    """The Maple 4-bit head (group size 64): w uint32 [V][K/8], scales / biases fp16 [V][K/64]."""
    x = _c(x, np.float16)
    w = _c(w, np.uint32)
    s = _c(scales, np.float16)
    b = _c(biases, np.float16)
    M, K = x.shape
    V = w.shape[0]
    assert w.shape == (V, K // 8) and s.shape == (V, K // 64) and b.shape == (V, K // 64)
    out = np.empty((M, V), np.float32)
    lib().or_lm_head_q4_logits(x.ctypes.data, w.ctypes.data, s.ctypes.data, b.ctypes.data,
                               out.ctypes.data, M, K, V)
    return out


def argmax_rows(logits, banned=None):
    logits = _c(logits, np.float32)
    M, V = logits.shape
    b = _c(banned if banned is not None else np.zeros(0), np.int32)
    idx = np.empty(M, np.int32)
    best = np.empty(M, np.float32)
    second = np.empty(M, np.float32)
    lib().or_argmax_rows(logits.ctypes.data, M, V, b.ctypes.data, b.size, idx.ctypes.data,
                         best.ctypes.data, second.ctypes.data)
    return idx, best, second


def accept_greedy(tokens, parents, argmax):
    tokens = _c(tokens, np.int32)
    argmax = _c(argmax, np.int32)
    n = tokens.size
    par = None if parents is None else _c(parents, np.int32)
    path = np.empty(n, np.int32)
    emit = np.empty(n, np.int32)
    acc = lib().or_accept_greedy(tokens.ctypes.data, None if par is None else par.ctypes.data,
                                 argmax.ctypes.data, n, path.ctypes.data, emit.ctypes.data)
    return acc, path[: acc + 1].copy(), emit[: acc + 1].copy()


def philox4x32_10(ctr, key):
    c = _c(ctr, np.uint32)
    k = _c(key, np.uint32)
    out = np.empty(4, np.uint32)
    lib().or_philox4x32_10(c.ctypes.data, k.ctypes.data, out.ctypes.data)
    return out


def verify_uniforms(seed, counter, rows):
    u = np.empty((rows, 2), np.float32)
    lib().or_verify_uniforms(C.c_uint64(seed), C.c_uint64(counter), rows, u.ctypes.data)
    return u


def splitmix64(seed, n):
    st = C.c_uint64(seed)
    return [lib().or_splitmix64_next(C.byref(st)) for _ in range(n)]


def canon_expf(x: float) -> float:
    return lib().or_canon_expf(C.c_float(x))


def canon_expf_array(x):
    f = lib().or_canon_expf
    return np.array([f(C.c_float(float(v))) for v in np.asarray(x, np.float32)], np.float32)


def canon_sum(v):
    v = _c(v, np.float32)
    return lib().or_canon_sum(C.c_void_p(v.ctypes.data), C.c_int(v.size))


def canon_walk(v, t):
    v = _c(v, np.float32)
    return lib().or_canon_walk(v.ctypes.data, v.size, C.c_float(t))


def accept_sampled(logits, draft, temperature, q_mode, uniforms, q_point=None):
    logits = _c(logits, np.float32)
    rows, V = logits.shape
    d = _c(draft, np.int32)
    u = _c(uniforms, np.float32)
    qp = None if q_point is None else _c(q_point, np.float32)
    tok = np.zeros(1, np.int32)
    acc = lib().or_accept_sampled(logits.ctypes.data, rows, V, d.ctypes.data,
                                  C.c_float(temperature), q_mode,
                                  None if qp is None else qp.ctypes.data, u.ctypes.data,
                                  tok.ctypes.data)
    return acc, int(tok[0])


def penalize_row(logits, hist_tok=(), hist_cnt=(), extra=(), rep=1.0, pres=0.0, freq=0.0):
    """LogitsProcessor.prepare over one full row (a copy is returned)."""
    l = np.array(logits, np.float32, copy=True)
    ht = _c(np.asarray(hist_tok, np.int32), np.int32)
    hc = _c(np.asarray(hist_cnt, np.int32), np.int32)
    ex = _c(np.asarray(extra, np.int32), np.int32)
    lib().or_penalize_row(l.ctypes.data, l.size, ht.ctypes.data, hc.ctypes.data, ht.size,
                          ex.ctypes.data, ex.size, C.c_float(rep), C.c_float(pres),
                          C.c_float(freq))
    return l


def nucleus_sample(e, Z, top_p, u):
    e = _c(e, np.float32)
    return lib().or_nucleus_sample(e.ctypes.data, e.size, C.c_float(Z), C.c_float(top_p),
                                   C.c_float(u))


def accept_sampled_ex(logits, draft, temperature, q_mode, uniforms, q_point=None, top_p=1.0,
                      rep=1.0, pres=0.0, freq=0.0, hist_tok=(), hist_cnt=()):
    logits = _c(logits, np.float32)
    rows, V = logits.shape
    d = _c(draft, np.int32)
    u = _c(uniforms, np.float32)
    qp = None if q_point is None else _c(q_point, np.float32)
    ht = _c(np.asarray(hist_tok, np.int32), np.int32)
    hc = _c(np.asarray(hist_cnt, np.int32), np.int32)
    tok = np.zeros(1, np.int32)
    acc = lib().or_accept_sampled_ex(logits.ctypes.data, rows, V, d.ctypes.data,
                                     C.c_float(temperature), C.c_float(top_p), C.c_float(rep),
                                     C.c_float(pres), C.c_float(freq), ht.ctypes.data,
                                     hc.ctypes.data, ht.size, q_mode,
                                     None if qp is None else qp.ctypes.data, u.ctypes.data,
                                     tok.ctypes.data)
    return acc, int(tok[0])


def try_accept(draft_token, ids, logits, temperature, draft_q, rng_state):
    ids = _c(ids, np.int32)
    lg = _c(logits, np.float32)
    st = C.c_uint64(rng_state)
    tok = np.zeros(1, np.int32)
    ok = lib().or_try_accept(draft_token, ids.ctypes.data, lg.ctypes.data, ids.size,
                             C.c_float(temperature), C.c_float(draft_q), C.byref(st),
                             tok.ctypes.data)
    return bool(ok), int(tok[0]), st.value


def walk_draft(draft, rows_ids, rows_logits, temperature, rng_state):
    d = _c(draft, np.int32)
    ids = _c(rows_ids, np.int32)
    lg = _c(rows_logits, np.float32)
    st = C.c_uint64(rng_state)
    nxt = np.zeros(1, np.int32)
    acc = lib().or_walk_draft(d.ctypes.data, d.size, ids.ctypes.data, lg.ctypes.data,
                              ids.shape[1], C.c_float(temperature), C.byref(st), nxt.ctypes.data)
    return acc, int(nxt[0])
