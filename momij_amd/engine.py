"""VerifyEngine: the resident verify stack through the C ABI (mirrors SeedlessDecodeEngine's
decode/verify surface: prefillPrompt, stepChainFeeds, verifyDraftChain, verifyDraftSampled --
SeedlessDecodeEngine.swift:194-228, 516-545, 1541-1603).

Weights are caller-owned torch device tensors in the MLX layout; the engine keeps them alive.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

from . import _lib
from ._lib import LayerWeights, ModelConfig, MomijError
from .ops import Context, ptr


@dataclass
class MapleLikeConfig:
    n_layers: int = 24
    H: int = 2048
    n_heads: int = 16
    n_kv_heads: int = 4
    head_dim: int = 128
    rope_dim: int = 64
    rope_base: float = 1e6
    eps: float = 1e-6
    window: int = 1024
    kv_capacity: int = 1024 + 64
    E: int = 64
    top_k: int = 8
    I: int = 1024
    gs: int = 64
    vocab: int = 151936
    # Maple's layer mix: per-layer sliding window (0 = full attention) and rope dims (0 = NoPE);
    # None = every layer takes window / rope_dim
    layer_window: list | None = None
    layer_rope_dim: list | None = None
    # 16: fp16 lm_head [V][H]; 4: the checkpoint's 4-bit gs64 head
    head_bits: int = 16

    def to_c(self, lm_head_scales=None, lm_head_biases=None) -> ModelConfig:
        c = ModelConfig(self.n_layers, self.H, self.n_heads, self.n_kv_heads, self.head_dim,
                        self.rope_dim, self.rope_base, self.eps, self.window, self.kv_capacity,
                        self.E, self.top_k, self.I, self.gs, self.vocab)
        self._arrays = []
        if self.layer_window is not None:
            a = (C.c_int32 * self.n_layers)(*[int(v) for v in self.layer_window])
            self._arrays.append(a)
            c.layer_window = C.cast(a, C.c_void_p)
        if self.layer_rope_dim is not None:
            a = (C.c_int32 * self.n_layers)(*[int(v) for v in self.layer_rope_dim])
            self._arrays.append(a)
            c.layer_rope_dim = C.cast(a, C.c_void_p)
        c.head_bits = self.head_bits
        c.lm_head_scales = ptr(lm_head_scales)
        c.lm_head_biases = ptr(lm_head_biases)
        return c

    def layer_window_of(self, l: int) -> int:
        return self.window if self.layer_window is None else int(self.layer_window[l])

    def layer_rope_of(self, l: int) -> int:
        return self.rope_dim if self.layer_rope_dim is None else int(self.layer_rope_dim[l])

    def attn_cfg(self, layer: int | None = None) -> dict:
        """Attention configuration of one layer (or of the uniform stack)."""
        win = self.window if layer is None else self.layer_window_of(layer)
        rd = self.rope_dim if layer is None else self.layer_rope_of(layer)
        return dict(H=self.H, nQ=self.n_heads, nKV=self.n_kv_heads, D=self.head_dim,
                    rope_dim=rd, rope_base=self.rope_base, eps=self.eps, window=win,
                    C=self.kv_capacity, gs=self.gs)

    @staticmethod
    def maple_layer_mix(n_layers: int, window: int, rope_dim: int, layer_types=None):
        """Per-layer (windows, rope dims) of MapleConfig.isSliding (MapleConfig.swift:145-148)
        and SeedlessAttn.swift:81-83: layer l slides (window, partial RoPE) when
        layer_types[l] == "sliding_attention", or, without layer_types, when (l + 1) % 4 != 0;
        the others are full attention without RoPE."""
        wins, ropes = [], []
        for l in range(n_layers):
            if layer_types is not None and l < len(layer_types):
                sliding = layer_types[l] == "sliding_attention"
            else:
                sliding = (l + 1) % 4 != 0
            wins.append(window if sliding else 0)
            ropes.append(rope_dim if sliding else 0)
        return wins, ropes


class VerifyEngine:
    def __init__(self, ctx: Context, cfg: MapleLikeConfig, layers: list, embed, final_norm_w,
                 lm_head, lm_head_scales=None, lm_head_biases=None):
        self.ctx = ctx
        self.cfg = cfg
        self.lib = ctx.lib
        self._keep = (layers, embed, final_norm_w, lm_head, lm_head_scales, lm_head_biases)
        arr = (LayerWeights * cfg.n_layers)()
        for i, lw in enumerate(layers):
            arr[i].attn = Context.attn_struct(lw["attn"])
            arr[i].moe = Context.moe_struct(lw["moe"])
        self._arr = arr
        # per-call argument buffers, filled in place (building ctypes arrays every call costs
        # more host time than the call itself)
        self._rows = (C.c_int32 * _lib.MJ_MAX_ROWS)()
        self._par = (C.c_int32 * _lib.MJ_MAX_ROWS)()
        self._out = (C.c_int32 * _lib.MJ_MAX_ROWS)()
        self._acc, self._tok = C.c_int32(), C.c_int32()
        h = C.c_void_p()
        c = cfg.to_c(lm_head_scales, lm_head_biases)
        ctx.check(self.lib.mj_model_create(ctx.h, C.byref(c), C.cast(arr, C.c_void_p), ptr(embed),
                                           ptr(final_norm_w), ptr(lm_head), C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            self.lib.mj_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------------ state
    @property
    def offset(self) -> int:
        return int(self.lib.mj_model_offset(self.h))

    def rewind(self, offset: int):
        self.ctx.check(self.lib.mj_model_rewind(self.h, offset))

    def kv(self, layer: int):
        k, v = C.c_void_p(), C.c_void_p()
        self.ctx.check(self.lib.mj_model_kv(self.h, layer, C.byref(k), C.byref(v)))
        return k.value, v.value

    def set_graphs(self, enable: bool):
        self.ctx.check(self.lib.mj_model_set_graphs(self.h, int(enable)))

    def set_capture(self, h=None, inds=None, logits=None):
        self.ctx.check(self.lib.mj_model_set_capture(self.h, ptr(h), ptr(inds), ptr(logits)))

    def set_capture_ex(self, **bufs):
        """Capture every block boundary (mj_capture field names: h, inds, logits, attn_out,
        moe_in, router_logits, head_in, kv_rows); no arguments switches capture off."""
        cap = _lib.Capture(*[ptr(bufs.get(f)) for f, _ in _lib.Capture._fields_])
        self._capture = bufs  # the device buffers outlive the capture
        self.ctx.check(self.lib.mj_model_set_capture_ex(self.h, C.byref(cap)))

    def capture_buffers(self, logits: bool = True) -> dict:
        """Device buffers for set_capture_ex at this configuration (torch tensors; the row
        stride is MJ_MAX_ROWS)."""
        import torch

        c, R = self.cfg, _lib.MJ_MAX_ROWS
        f16 = dict(dtype=torch.float16, device="cuda")
        out = dict(h=torch.zeros((c.n_layers + 1, R, c.H), **f16),
                   inds=torch.zeros((c.n_layers, R, c.top_k), dtype=torch.int32, device="cuda"),
                   attn_out=torch.zeros((c.n_layers, R, c.H), **f16),
                   moe_in=torch.zeros((c.n_layers, R, c.H), **f16),
                   router_logits=torch.zeros((c.n_layers, R, c.E), dtype=torch.float32,
                                             device="cuda"),
                   head_in=torch.zeros((R, c.H), **f16),
                   kv_rows=torch.zeros((c.n_layers, 2, c.n_kv_heads, R, c.head_dim), **f16))
        if logits:
            out["logits"] = torch.zeros((R, c.vocab), dtype=torch.float32, device="cuda")
        return out

    def last_pass_ms(self) -> float:
        return float(self.lib.mj_model_last_pass_ms(self.h))

    KERNEL_CLASSES = ("expert_up", "expert_down", "lm_head", "attention", "dense", "timer",
                      "expert_moe")

    def profile(self, enable: bool):
        self.ctx.check(self.lib.mj_model_profile(self.h, int(enable)))

    def kernel_ms(self) -> dict:
        out = {}
        for i, name in enumerate(self.KERNEL_CLASSES):
            n = C.c_int64()
            ms = self.lib.mj_model_kernel_ms(self.h, i, C.byref(n))
            out[name] = (float(ms), int(n.value))
        return out

    # ------------------------------------------------------------------ passes
    def prefill(self, tokens, chunk: int = 64) -> int:
        toks = (C.c_int32 * len(tokens))(*[int(t) for t in tokens])
        nxt = C.c_int32()
        self.ctx.check(self.lib.mj_prefill(self.h, toks, len(tokens), chunk, C.byref(nxt)))
        return nxt.value

    def step_chain_feeds(self, feeds) -> list[int]:
        M = len(feeds)
        f = (C.c_int32 * M)(*[int(t) for t in feeds])
        ev = (C.c_int32 * M)()
        self.ctx.check(self.lib.mj_step_chain_feeds(self.h, f, M, ev))
        return list(ev)

    def _draft_args(self, draft, parents=None):
        n = len(draft)
        if n + 1 > _lib.MJ_MAX_ROWS:  # the library's own refusal (MJ_INVALID_ARG)
            raise MomijError(4, f"draft of {n} nodes exceeds {_lib.MJ_MAX_ROWS - 1}")
        self._rows[:n] = [int(t) for t in draft]
        par = None
        if parents is not None:
            assert len(parents) == n + 1
            self._par[: n + 1] = [int(p) for p in parents]
            par = self._par
        return n, par

    def verify_greedy(self, y: int, draft, parents=None) -> tuple[int, list[int]]:
        n, par = self._draft_args(draft, parents)
        self.ctx.check(self.lib.mj_verify_greedy(self.h, int(y), self._rows, n, par,
                                                 C.byref(self._acc), self._out))
        acc = self._acc.value
        return acc, list(self._out[: acc + 1])

    def verify_sampled(self, y: int, draft, temperature: float, q_mode: int, seed: int,
                       counter: int, q_point=None) -> tuple[int, int]:
        n, _ = self._draft_args(draft)
        qp = None if q_point is None else (C.c_float * max(n, 1))(*[float(q) for q in q_point])
        self.ctx.check(self.lib.mj_verify_sampled(self.h, int(y), self._rows, n, temperature,
                                                  q_mode, qp, seed, counter, C.byref(self._acc),
                                                  C.byref(self._tok)))
        return self._acc.value, self._tok.value

    def verify_sampled_ex(self, y: int, draft, q_mode: int, seed: int, counter: int,
                          temperature: float, top_p=1.0, rep=1.0, pres=0.0, freq=0.0,
                          hist=None, q_point=None) -> tuple[int, int]:
        """mj_verify_sampled_ex: LogitsProcessor options; hist {token: count} or a pair of
        int32 arrays (tokens, counts)."""
        n, _ = self._draft_args(draft)
        qp = None if q_point is None else (C.c_float * max(n, 1))(*[float(q) for q in q_point])
        sp, keep = _lib.sampling(temperature, top_p, rep, pres, freq, hist)
        self.ctx.check(self.lib.mj_verify_sampled_ex(self.h, int(y), self._rows, n, C.byref(sp),
                                                     q_mode, qp, seed, counter,
                                                     C.byref(self._acc), C.byref(self._tok)))
        return self._acc.value, self._tok.value


def random_model(cfg: MapleLikeConfig, seed: int = 0, device: str = "cuda",
                 embed_std: float = 1.0):
    """Random-init weights of the configuration on the device (same distributions as the
    2-bit workloads); returns (layers, embed, final_norm_w, lm_head).

    The embedding is ~N(0, embed_std), by default N(0, 1) like the activations of the
    single-layer workloads: token identity then dominates the residual stream, so the rows of a
    verify pass route independently (about 45 of 64 experts per layer at 9 rows).  With a small
    embedding (0.02) the random layers' attention output, common to all rows, dominates after
    two layers and every row picks the same ~9 experts, which understates expert traffic."""
    import torch

    from . import synth

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    H, D, nQ, nKV = cfg.H, cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    layers = []
    for _ in range(cfg.n_layers):
        qw, qs, qb = synth.torch_qweight(gen, (), (nQ + 2 * nKV) * D, H, cfg.gs, device)
        ow, os_, ob = synth.torch_qweight(gen, (), H, nQ * D, cfg.gs, device)
        ugw, ugs, ugb = synth.torch_qweight(gen, (cfg.E,), 2 * cfg.I, H, cfg.gs, device)
        dw, ds, db = synth.torch_qweight(gen, (cfg.E,), H, cfg.I, cfg.gs, device)

        def norm_w(n):
            return (1.0 + 0.1 * torch.randn(n, generator=gen, device=device)).half()

        attn = dict(norm_w=norm_w(H), qkv_w=qw, qkv_s=qs, qkv_b=qb, q_norm_w=norm_w(D),
                    k_norm_w=norm_w(D), o_w=ow, o_s=os_, o_b=ob)
        moe = dict(norm_w=norm_w(H), router_w=synth.torch_normal(gen, (cfg.E, H), 0.02, device),
                   up_gate_w=ugw, up_gate_s=ugs, up_gate_b=ugb, down_w=dw, down_s=ds, down_b=db,
                   E=cfg.E, top_k=cfg.top_k, H=H, I=cfg.I, gs=cfg.gs, eps=cfg.eps)
        layers.append(dict(attn=attn, moe=moe))
    embed = synth.torch_normal(gen, (cfg.vocab, H), embed_std, device)
    final_norm = (1.0 + 0.1 * torch.randn(H, generator=gen, device=device)).half()
    lm_head = synth.torch_normal(gen, (cfg.vocab, H), 0.02, device)
    return layers, embed, final_norm, lm_head
