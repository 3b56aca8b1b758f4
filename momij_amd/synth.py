"""Seeded synthetic inputs with the distributions of the verify-step workloads.

2-bit affine weights in MLX layout: codes uniform in {0..3}, 16 per uint32 word, LSB first
(code k of a row in bits [2(k%16), 2(k%16)+1] of word k/16); one fp16 scale and one fp16 bias
per group of `gs` inputs, scale ~ U(0.005, 0.02) and bias = fp16(-1.5 * scale).  Activations
~ N(0, 1) fp16, router / lm_head / embedding weights ~ N(0, 0.02) fp16.

numpy generators serve the small CPU-checkable cases; the torch generators fill device memory
for the full-size workloads (same distributions, not the same bits as numpy).
"""
from __future__ import annotations

import numpy as np


def pack_codes(codes: np.ndarray) -> np.ndarray:
    """codes [..., K] in {0..3} -> uint32 words [..., K/16], LSB-first."""
    codes = np.asarray(codes, np.uint32)
    K = codes.shape[-1]
    assert K % 16 == 0
    c = codes.reshape(codes.shape[:-1] + (K // 16, 16))
    shifts = (2 * np.arange(16, dtype=np.uint32))
    return np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint32)


def unpack_codes(words: np.ndarray) -> np.ndarray:
    words = np.asarray(words, np.uint32)
    shifts = (2 * np.arange(16, dtype=np.uint32))
    c = (words[..., None] >> shifts) & np.uint32(3)
    return c.reshape(words.shape[:-1] + (words.shape[-1] * 16,)).astype(np.uint8)


def qweight(rng: np.random.Generator, lead: tuple, N: int, K: int, gs: int):
    """Random 2-bit affine weight: (w uint32 [*lead, N, K/16], s fp16, b fp16 [*lead, N, K/gs])."""
    w = rng.integers(0, 2**32, size=lead + (N, K // 16), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(0.005, 0.02, size=lead + (N, K // gs)).astype(np.float16)
    b = (-1.5 * s.astype(np.float32)).astype(np.float16)
    return w, s, b


def dequant(w, s, b, gs: int) -> np.ndarray:
    """float64 dense weight [..., N, K] = s * q + b."""
    q = unpack_codes(w).astype(np.float64)
    K = q.shape[-1]
    sg = np.repeat(s.astype(np.float64), gs, axis=-1)[..., :K]
    bg = np.repeat(b.astype(np.float64), gs, axis=-1)[..., :K]
    return sg * q + bg


def qweight4(rng: np.random.Generator, V: int, K: int, scale=(0.001, 0.004)):
    """Random 4-bit affine weight of the Maple head, group size 64: (w uint32 [V, K/8] with 8
    codes a word, LSB first; s, b fp16 [V, K/64]; b = -7.5 s centres the codes)."""
    w = rng.integers(0, 2**32, size=(V, K // 8), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(scale[0], scale[1], size=(V, K // 64)).astype(np.float16)
    b = (-7.5 * s.astype(np.float32)).astype(np.float16)
    return w, s, b


def dequant4(w, s, b) -> np.ndarray:
    """float64 dense 4-bit weight [V, K] = s * q + b (group size 64)."""
    V = w.shape[0]
    q = ((w[..., :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15).reshape(V, -1)
    sg = np.repeat(s.astype(np.float64), 64, axis=-1)
    bg = np.repeat(b.astype(np.float64), 64, axis=-1)
    return sg * q.astype(np.float64) + bg


def normal_f16(rng: np.random.Generator, shape, std=1.0) -> np.ndarray:
    return (rng.standard_normal(shape) * std).astype(np.float16)


def moe_weights(rng: np.random.Generator, E: int, H: int, I: int, gs: int, eps=1e-6, top_k=8):
    ugw, ugs, ugb = qweight(rng, (E,), 2 * I, H, gs)
    dw, ds, db = qweight(rng, (E,), H, I, gs)
    return dict(
        norm_w=(1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16),
        router_w=normal_f16(rng, (E, H), 0.02),
        up_gate_w=ugw, up_gate_s=ugs, up_gate_b=ugb,
        down_w=dw, down_s=ds, down_b=db,
        E=E, top_k=top_k, H=H, I=I, gs=gs, eps=eps,
    )


def attn_weights(rng: np.random.Generator, H: int, nQ: int, nKV: int, D: int, gs: int):
    qkvN = (nQ + 2 * nKV) * D
    qw, qs, qb = qweight(rng, (), qkvN, H, gs)
    ow, os_, ob = qweight(rng, (), H, nQ * D, gs)
    return dict(
        norm_w=(1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16),
        qkv_w=qw, qkv_s=qs, qkv_b=qb,
        q_norm_w=(1.0 + 0.1 * rng.standard_normal(D)).astype(np.float16),
        k_norm_w=(1.0 + 0.1 * rng.standard_normal(D)).astype(np.float16),
        o_w=ow, o_s=os_, o_b=ob,
    )


# ---------------------------------------------------------------------------------------
# torch (device) generators for the full-size workloads
# ---------------------------------------------------------------------------------------
def torch_qweight(gen, lead: tuple, N: int, K: int, gs: int, device="cuda"):
    import torch

    w = torch.randint(-(2**31), 2**31 - 1, lead + (N, K // 16), generator=gen, device=device,
                      dtype=torch.int64).to(torch.int32)
    s = (torch.rand(lead + (N, K // gs), generator=gen, device=device) * 0.015 + 0.005).half()
    b = (-1.5 * s.float()).half()
    return w, s, b


def torch_normal(gen, shape, std=1.0, device="cuda"):
    import torch

    return (torch.randn(shape, generator=gen, device=device) * std).half()
