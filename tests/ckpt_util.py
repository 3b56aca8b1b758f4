"""A synthetic MLX Maple checkpoint on disk, in the naming and layout the reference loads
(WeightStore.swift:9-92, SeedlessAttn.swift:85-105, SeedlessDecodeEngine.swift:111-123):
separate q/k/v and up/gate projections (the loader concatenates them), a row_alpha in place of
the scales and biases of layer 0's q_proj, bf16 float tensors, a 4-bit gs64 word embedding and
lm_head, two safetensors shards and their index.  Returns the arrays written, for checks."""
from __future__ import annotations

import json
import os

import numpy as np


def write_maple_checkpoint(d: str, *, n_layers=4, H=2048, nQ=16, nKV=4, D=128, E=16, top_k=4,
                           I=1024, gs=64, vocab=2048, window=48, layer_types=None, seed=0,
                           embed_scale=(0.05, 0.2), defaults_config=False):
    """defaults_config: write a config.json holding only the layer count and vocabulary, so
    every other field takes MapleConfig's defaults (MapleConfig.swift:5-49: hidden 2048, 16 / 4
    heads of 128, 256 experts top-8, intermediate 512, group size 128, window 512, rope theta
    1e4, partial rotary 0.5, 4-bit gs64 head); the arrays must then have those shapes."""
    import torch
    from safetensors.torch import save_file

    rng = np.random.default_rng(seed)

    def bf16(a):
        return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)

    def codes(*shape):
        return torch.from_numpy(rng.integers(0, 2**32, size=shape, dtype=np.uint64)
                                .astype(np.uint32).view(np.int32)).view(torch.uint32)

    def q2(lead, N, K):  # 2-bit weight, its scales and biases
        s = rng.uniform(0.005, 0.02, size=lead + (N, K // gs))
        return codes(*lead, N, K // 16), bf16(s), bf16(-1.5 * s)

    def norm(n):
        return bf16(1.0 + 0.1 * rng.standard_normal(n))

    arrays = {}
    for l in range(n_layers):
        p, at, mo = f"model.layers.{l}", f"model.layers.{l}.self_attn", \
            f"model.layers.{l}.mlp.switch_mlp"
        arrays[f"{p}.input_layernorm.weight"] = norm(H)
        arrays[f"{p}.post_attention_layernorm.weight"] = norm(H)
        for name, n in (("q", nQ * D), ("k", nKV * D), ("v", nKV * D)):
            w, s, b = q2((), n, H)
            arrays[f"{at}.{name}_proj.weight"] = w
            if l == 0 and name == "q":
                arrays[f"{at}.q_proj.row_alpha"] = bf16(rng.uniform(0.005, 0.02, size=n))
            else:
                arrays[f"{at}.{name}_proj.scales"] = s
                arrays[f"{at}.{name}_proj.biases"] = b
        w, s, b = q2((), H, nQ * D)
        arrays[f"{at}.o_proj.weight"], arrays[f"{at}.o_proj.scales"], \
            arrays[f"{at}.o_proj.biases"] = w, s, b
        arrays[f"{at}.q_norm.weight"] = norm(D)
        arrays[f"{at}.k_norm.weight"] = norm(D)
        arrays[f"{p}.mlp.gate.weight"] = bf16(0.02 * rng.standard_normal((E, H)))
        for name, (N, K) in (("up", (I, H)), ("gate", (I, H)), ("down", (H, I))):
            w, s, b = q2((E,), N, K)
            arrays[f"{mo}.{name}_proj.weight"] = w
            if l == 1:  # row-alpha experts
                arrays[f"{mo}.{name}_proj.row_alpha"] = bf16(rng.uniform(0.005, 0.02,
                                                                         size=(E, N)))
            else:
                arrays[f"{mo}.{name}_proj.scales"], arrays[f"{mo}.{name}_proj.biases"] = s, b
    es = rng.uniform(*embed_scale, size=(vocab, H // 64))
    arrays["model.word_embeddings.weight"] = codes(vocab, H // 8)
    arrays["model.word_embeddings.scales"] = bf16(es)
    arrays["model.word_embeddings.biases"] = bf16(-7.5 * es)
    arrays["model.norm.weight"] = norm(H)
    hs = rng.uniform(0.001, 0.004, size=(vocab, H // 64))
    arrays["lm_head.weight"] = codes(vocab, H // 8)
    arrays["lm_head.scales"] = bf16(hs)
    arrays["lm_head.biases"] = bf16(-7.5 * hs)

    os.makedirs(d, exist_ok=True)
    names = sorted(arrays)
    shards = {"model-00001-of-00002.safetensors": names[: len(names) // 2],
              "model-00002-of-00002.safetensors": names[len(names) // 2:]}
    wmap = {}
    for fn, ks in shards.items():
        save_file({k: arrays[k].contiguous() for k in ks}, os.path.join(d, fn))
        wmap.update({k: fn for k in ks})
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wmap}, f)
    if defaults_config:
        with open(os.path.join(d, "config.json"), "w") as f:
            json.dump(dict(model_type="maple", num_hidden_layers=n_layers, vocab_size=vocab), f)
        return arrays
    cj = dict(model_type="maple", hidden_size=H, num_hidden_layers=n_layers,
              num_attention_heads=nQ, num_key_value_heads=nKV, head_dim=D, vocab_size=vocab,
              num_experts=E, num_experts_per_tok=top_k, moe_intermediate_size=I,
              rms_norm_eps=1e-6, rope_theta=1e6, sliding_window=window,
              partial_rotary_factor=0.5,
              quantization=dict(group_size=gs, bits=2, lm_head=dict(bits=4, group_size=64)))
    if layer_types is not None:
        cj["layer_types"] = layer_types
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(cj, f)
    return arrays
