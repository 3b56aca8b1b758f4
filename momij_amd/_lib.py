"""ctypes binding of libmomij_hip.so (the C ABI declared in include/momij_hip.h).

The library is built in-tree by momij_amd.build (or __graft_entry__.build()).  Loading fails
loudly when it is missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmomij_hip.so")

MJ_OK = 0
STATUS = {0: "MJ_OK", 1: "MJ_NO_DEVICE", 2: "MJ_NOT_READY", 3: "MJ_UNSUPPORTED_SHAPE",
          4: "MJ_INVALID_ARG", 5: "MJ_ABORTED", 6: "MJ_HIP_ERROR", 7: "MJ_CAPACITY",
          8: "MJ_OUT_OF_MEMORY"}
MJ_MAX_ROWS = 64
MJ_MOE_NOALLOC_BYTES = 8 << 20
MJ_EPI_STORE, MJ_EPI_ADD = 0, 1
MJ_MOE_PRENORM, MJ_MOE_RESIDUAL = 1, 2
MJ_Q_POINT, MJ_Q_UNIFORM = 0, 1


class MomijError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS.get(status, status)}: {msg}")
        self.status = status


vp = C.c_void_p
i32 = C.c_int
f32 = C.c_float
i64 = C.c_int64
u64 = C.c_uint64


class MoeWeights(C.Structure):
    _fields_ = [("norm_w", vp), ("router_w", vp), ("up_gate_w", vp), ("up_gate_s", vp),
                ("up_gate_b", vp), ("down_w", vp), ("down_s", vp), ("down_b", vp),
                ("E", i32), ("top_k", i32), ("H", i32), ("I", i32), ("gs", i32), ("eps", f32),
                ("up_gate_alpha", vp), ("down_alpha", vp)]


class AttnWeights(C.Structure):
    _fields_ = [("norm_w", vp), ("qkv_w", vp), ("qkv_s", vp), ("qkv_b", vp), ("q_norm_w", vp),
                ("k_norm_w", vp), ("o_w", vp), ("o_s", vp), ("o_b", vp)]


class AttnConfig(C.Structure):
    _fields_ = [("H", i32), ("n_heads", i32), ("n_kv_heads", i32), ("head_dim", i32),
                ("rope_dim", i32), ("rope_base", f32), ("eps", f32), ("window", i32),
                ("kv_capacity", i64), ("gs", i32)]


class ModelConfig(C.Structure):
    _fields_ = [("n_layers", i32), ("H", i32), ("n_heads", i32), ("n_kv_heads", i32),
                ("head_dim", i32), ("rope_dim", i32), ("rope_base", f32), ("eps", f32),
                ("window", i32), ("kv_capacity", i64), ("E", i32), ("top_k", i32), ("I", i32),
                ("gs", i32), ("vocab", i32), ("layer_window", vp), ("layer_rope_dim", vp),
                ("head_bits", i32), ("lm_head_scales", vp), ("lm_head_biases", vp)]


class LayerWeights(C.Structure):
    _fields_ = [("attn", AttnWeights), ("moe", MoeWeights)]


class Sampling(C.Structure):
    _fields_ = [("temperature", f32), ("top_p", f32), ("repetition_penalty", f32),
                ("presence_penalty", f32), ("frequency_penalty", f32), ("hist_tokens", vp),
                ("hist_counts", vp), ("n_hist", i32)]


MJ_MAX_HIST = 65536


def sampling(temperature, top_p=1.0, rep=1.0, pres=0.0, freq=0.0, hist=None):
    """mj_sampling for the given options.  hist: the seen set and counts, either a dict
    {token: count} or a pair of int32 numpy arrays (tokens, counts) used in place (ascending
    tokens spare the library a sort).  Returns (struct, keep-alive objects)."""
    if isinstance(hist, tuple):
        import numpy as np

        ht = np.ascontiguousarray(hist[0], dtype=np.int32)
        hc = np.ascontiguousarray(hist[1], dtype=np.int32)
        if ht.shape != hc.shape or ht.ndim != 1:
            raise ValueError("hist arrays must be two 1-D arrays of one length")
        n = int(ht.shape[0])
        sp = Sampling(float(temperature), float(top_p), float(rep), float(pres), float(freq),
                      ht.ctypes.data if n else None, hc.ctypes.data if n else None, n)
        return sp, (ht, hc)
    toks = list(hist.keys()) if hist else []
    ht = (C.c_int32 * max(len(toks), 1))(*[int(t) for t in toks])
    hc = (C.c_int32 * max(len(toks), 1))(*[int(hist[t]) for t in toks])
    sp = Sampling(float(temperature), float(top_p), float(rep), float(pres), float(freq),
                  C.cast(ht, C.c_void_p) if toks else None,
                  C.cast(hc, C.c_void_p) if toks else None, len(toks))
    return sp, (ht, hc)


class Capture(C.Structure):
    _fields_ = [("h", vp), ("inds", vp), ("logits", vp), ("attn_out", vp), ("moe_in", vp),
                ("router_logits", vp), ("head_in", vp), ("kv_rows", vp)]


_SIGS = {
    "mj_abi_version": (i32, []),
    "mj_status_str": (C.c_char_p, [i32]),
    "mj_init": (i32, [i32, C.POINTER(vp)]),
    "mj_destroy": (i32, [vp]),
    "mj_last_error": (C.c_char_p, [vp]),
    "mj_set_stream": (i32, [vp, vp]),
    "mj_get_stream": (vp, [vp]),
    "mj_set_abort": (i32, [vp, i32]),
    "mj_set_wait_limit": (i32, [vp, i32]),
    "mj_sync": (i32, [vp]),
    "mj_alloc": (i32, [vp, C.c_size_t, C.POINTER(vp)]),
    "mj_free": (i32, [vp, vp]),
    "mj_h2d": (i32, [vp, vp, vp, C.c_size_t]),
    "mj_d2h": (i32, [vp, vp, vp, C.c_size_t]),
    "mj_gather_qmm2": (i32, [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32]),
    "mj_moe_block": (i32, [vp, C.POINTER(MoeWeights), vp, vp, i32, i32, vp, vp]),
    "mj_moe_block_noalloc": (i32, [vp, C.POINTER(MoeWeights), vp, vp, i32, i32, vp, vp]),
    "mj_attn_block": (i32, [vp, C.POINTER(AttnConfig), C.POINTER(AttnWeights), vp, vp, vp, i64,
                            vp, i32]),
    "mj_lm_head_verify": (i32, [vp, vp, vp, i32, i32, i32, vp, i32, f32, vp, vp, vp, vp]),
    "mj_lm_head_verify_q4": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, i32, f32, vp, vp,
                                   vp, vp]),
    "mj_suffix_index_create": (i32, [i32, C.POINTER(vp)]),
    "mj_suffix_index_destroy": (i32, [vp]),
    "mj_suffix_index_clear": (i32, [vp]),
    "mj_suffix_index_tokens": (i64, [vp]),
    "mj_suffix_index_insert": (i32, [vp, vp, i32]),
    "mj_suffix_index_draft": (i32, [vp, vp, i32, i32, C.c_double, vp, vp, vp]),
    "mj_suffix_max_spec": (i32, [i32, i32, C.c_double]),
    "mj_suffix_best_draft": (i32, [vp, vp, vp, i32, i32, C.c_double, vp, vp, vp]),
    "mj_suffix_index_q_along": (i32, [vp, vp, i32, vp, i32, vp]),
    "mj_suffix_draft_pld": (i32, [vp, i32, i32, i32, i32, vp, vp]),
    "mj_tree_draft": (i32, [vp, i32, i32, vp, vp, C.c_double, i32, vp, vp]),
    "mj_adaptive_draft_k": (i32, [C.c_double, i32]),
    "mj_recycle_index_create": (i32, [i32, C.POINTER(vp)]),
    "mj_recycle_index_destroy": (i32, [vp]),
    "mj_recycle_index_clear": (i32, [vp]),
    "mj_recycle_index_observe": (i32, [vp, i32, vp, i32]),
    "mj_recycle_index_draft": (i32, [vp, i32, i32, vp, vp]),
    "mj_recycle_index_entries": (i32, [vp]),
    "mj_accept_greedy": (i32, [vp, vp, vp, vp, i32, vp]),
    "mj_accept_sampled": (i32, [vp, vp, i32, i32, vp, f32, i32, vp, u64, u64, vp]),
    "mj_accept_sampled_ex": (i32, [vp, vp, i32, i32, vp, C.POINTER(Sampling), i32, vp, u64, u64,
                                   vp]),
    "mj_model_create": (i32, [vp, C.POINTER(ModelConfig), vp, vp, vp, vp, C.POINTER(vp)]),
    "mj_model_destroy": (i32, [vp]),
    "mj_model_offset": (i64, [vp]),
    "mj_model_rewind": (i32, [vp, i64]),
    "mj_model_kv": (i32, [vp, i32, C.POINTER(vp), C.POINTER(vp)]),
    "mj_prefill": (i32, [vp, vp, i32, i32, vp]),
    "mj_step_chain_feeds": (i32, [vp, vp, i32, vp]),
    "mj_verify_greedy": (i32, [vp, i32, vp, i32, vp, vp, vp]),
    "mj_verify_sampled": (i32, [vp, i32, vp, i32, f32, i32, vp, u64, u64, vp, vp]),
    "mj_verify_sampled_ex": (i32, [vp, i32, vp, i32, C.POINTER(Sampling), i32, vp, u64, u64, vp,
                                   vp]),
    "mj_model_set_capture": (i32, [vp, vp, vp, vp]),
    "mj_model_set_capture_ex": (i32, [vp, C.POINTER(Capture)]),
    "mj_model_set_graphs": (i32, [vp, i32]),
    "mj_model_last_pass_ms": (f32, [vp]),
    "mj_selftest_mfma": (i32, [vp, vp, vp, vp]),
    "mj_model_profile": (i32, [vp, i32]),
    "mj_model_kernel_ms": (f32, [vp, i32, C.POINTER(i64)]),
}

_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m momij_amd.build` (or "
                "__graft_entry__.build()) first -- there is no fallback path")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def header_symbols() -> list[str]:
    """Function names declared in include/momij_hip.h."""
    import re

    hdr = os.path.join(os.path.dirname(HERE), "include", "momij_hip.h")
    text = open(hdr).read()
    return sorted(set(re.findall(r"^\s*(?:[\w\s\*]+?)\b(mj_\w+)\s*\(", text, flags=re.M)))
