"""Python face of the C ABI over torch device tensors.

torch provides device memory and a stream (plumbing only); every computation runs in
libmomij_hip.so.  A Context owns an mj_ctx bound to its own torch stream; call
`torch.cuda.synchronize()` (or run torch work inside `with torch.cuda.stream(ctx.stream)`)
before handing freshly written tensors to it, and `ctx.sync()` before reading results.
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from ._lib import AttnConfig, AttnWeights, LayerWeights, MoeWeights, ModelConfig, MomijError


def ptr(t) -> int | None:
    """Device pointer of a torch tensor (None passes a NULL)."""
    if t is None:
        return None
    return t.data_ptr()


class Context:
    def __init__(self, device: int = 0):
        import torch

        self.lib = _lib.load()
        h = C.c_void_p()
        st = self.lib.mj_init(device, C.byref(h))
        if st != 0:
            raise MomijError(st, f"mj_init(device={device}) failed")
        self.h = h
        self.device = device
        self.stream = torch.cuda.Stream(device=device)
        self.check(self.lib.mj_set_stream(self.h, self.stream.cuda_stream))

    def close(self):
        if self.h:
            self.lib.mj_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, st: int):
        if st != 0:
            msg = self.lib.mj_last_error(self.h)
            raise MomijError(st, msg.decode() if msg else "")

    def sync(self):
        self.check(self.lib.mj_sync(self.h))

    def set_abort(self, flag: bool):
        self.check(self.lib.mj_set_abort(self.h, int(flag)))

    def set_wait_limit(self, polls: int):
        """Bound of the fused MoE launch's waits for its up product, in re-stagings of a
        down item's act rows."""
        self.check(self.lib.mj_set_wait_limit(self.h, int(polls)))

    # ---------------------------------------------------------------- ops
    def gather_qmm2(self, x, w, scales, biases, inds, y, M, ktop, K, N, gs, lhs_per_expert=False,
                    epilogue=_lib.MJ_EPI_STORE):
        self.check(self.lib.mj_gather_qmm2(self.h, ptr(x), ptr(w), ptr(scales), ptr(biases),
                                           ptr(inds), ptr(y), M, ktop, K, N, gs,
                                           int(lhs_per_expert), epilogue))

    @staticmethod
    def moe_struct(mw: dict) -> MoeWeights:
        return MoeWeights(ptr(mw.get("norm_w")), ptr(mw["router_w"]), ptr(mw["up_gate_w"]),
                          ptr(mw["up_gate_s"]), ptr(mw["up_gate_b"]), ptr(mw["down_w"]),
                          ptr(mw["down_s"]), ptr(mw["down_b"]), mw["E"], mw["top_k"], mw["H"],
                          mw["I"], mw["gs"], mw["eps"], ptr(mw.get("up_gate_alpha")),
                          ptr(mw.get("down_alpha")))

    def moe_block(self, mw: dict, x, y, M, flags=0, inds=None, scores=None):
        st = self.moe_struct(mw)
        self.check(self.lib.mj_moe_block(self.h, C.byref(st), ptr(x), ptr(y), M, flags, ptr(inds),
                                         ptr(scores)))

    def moe_block_noalloc(self, mw: dict, x, y, M, flags=0, inds=None, scores=None):
        """mj_moe_block over the library's static per-GPU scratch (no device allocation)."""
        st = self.moe_struct(mw)
        self.check(self.lib.mj_moe_block_noalloc(self.h, C.byref(st), ptr(x), ptr(y), M, flags,
                                                 ptr(inds), ptr(scores)))

    @staticmethod
    def attn_struct(aw: dict) -> AttnWeights:
        return AttnWeights(ptr(aw["norm_w"]), ptr(aw["qkv_w"]), ptr(aw["qkv_s"]), ptr(aw["qkv_b"]),
                           ptr(aw["q_norm_w"]), ptr(aw["k_norm_w"]), ptr(aw["o_w"]),
                           ptr(aw["o_s"]), ptr(aw["o_b"]))

    @staticmethod
    def attn_config(cfg: dict) -> AttnConfig:
        return AttnConfig(cfg["H"], cfg["nQ"], cfg["nKV"], cfg["D"], cfg["rope_dim"],
                          cfg["rope_base"], cfg["eps"], cfg["window"], cfg["C"], cfg["gs"])

    def attn_block(self, cfg: dict, aw: dict, h, kcache, vcache, L: int, parents, M: int):
        c = self.attn_config(cfg)
        w = self.attn_struct(aw)
        par = None
        if parents is not None:
            par = (C.c_int32 * M)(*[int(p) for p in parents])
        self.check(self.lib.mj_attn_block(self.h, C.byref(c), C.byref(w), ptr(h), ptr(kcache),
                                          ptr(vcache), L, par, M))

    def lm_head_verify(self, x, w, M, K, V, out_argmax, out_max=None, out_logits=None,
                       banned=None, n_banned=0, temperature=1.0, out_lse=None):
        self.check(self.lib.mj_lm_head_verify(self.h, ptr(x), ptr(w), M, K, V, ptr(banned),
                                              n_banned, float(temperature), ptr(out_argmax),
                                              ptr(out_max), ptr(out_lse), ptr(out_logits)))

    def lm_head_verify_q4(self, x, w, scales, biases, M, K, V, out_argmax, out_max=None,
                          out_logits=None, banned=None, n_banned=0, group_size=64,
                          temperature=1.0, out_lse=None):
        self.check(self.lib.mj_lm_head_verify_q4(self.h, ptr(x), ptr(w), ptr(scales),
                                                 ptr(biases), M, K, V, group_size, ptr(banned),
                                                 n_banned, float(temperature), ptr(out_argmax),
                                                 ptr(out_max), ptr(out_lse), ptr(out_logits)))

    def accept_greedy(self, tokens, parents, argmax, n_rows, out):
        par = None
        if parents is not None:
            par = (C.c_int32 * n_rows)(*[int(p) for p in parents])
        self.check(self.lib.mj_accept_greedy(self.h, ptr(tokens), par, ptr(argmax), n_rows,
                                             ptr(out)))

    def accept_sampled(self, logits, rows, V, draft, temperature, q_mode, seed, counter, out,
                       q_point=None):
        self.check(self.lib.mj_accept_sampled(self.h, ptr(logits), rows, V, ptr(draft),
                                              temperature, q_mode, ptr(q_point), seed, counter,
                                              ptr(out)))

    def accept_sampled_ex(self, logits, rows, V, draft, q_mode, seed, counter, out,
                          temperature, top_p=1.0, rep=1.0, pres=0.0, freq=0.0, hist=None,
                          q_point=None):
        """mj_accept_sampled_ex: LogitsProcessor options; hist {token: count}."""
        sp, keep = _lib.sampling(temperature, top_p, rep, pres, freq, hist)
        self.check(self.lib.mj_accept_sampled_ex(self.h, ptr(logits), rows, V, ptr(draft),
                                                 C.byref(sp), q_mode, ptr(q_point), seed,
                                                 counter, ptr(out)))

    def selftest_mfma(self, A, B, D):
        self.check(self.lib.mj_selftest_mfma(self.h, ptr(A), ptr(B), ptr(D)))
