"""MLX Maple checkpoints for VerifyEngine: config.json, safetensors shards and the sanitize step.

Follows WeightStore (WeightStore.swift:9-92) and the engine's weight lookups
(SeedlessAttn.swift:85-105, SeedlessDecodeEngine.swift:111-123):

  * every shard named by `model.safetensors.index.json` is loaded; bf16 arrays become fp16
    (`metalF16`, 28-30), integer code arrays are kept as they are;
  * `<p>.row_alpha` [..., N] replaces `<p>.scales` / `<p>.biases` of the 2-bit weight
    `<p>.weight` [..., N, K/16]: scales = alpha repeated over the K / group_size groups,
    biases = -scales (47-63); alpha itself is kept as `<p>.alpha`, and the experts' copy goes
    to the MoE block, whose batched kernels then fold it (one alpha a row, no group loads);
  * q_proj, k_proj, v_proj concatenate along the output rows into qkv_proj, and the experts'
    up_proj, gate_proj along their rows into up_gate_proj, up first (66-90);
  * the 4-bit gs64 word embedding is dequantised once into an fp16 table
    (SeedlessDecodeEngine.swift:111-117); the lm_head stays 4-bit for mj_lm_head_verify_q4
    (headBits, MapleConfig.swift:141);
  * the layer mix (sliding layers with partial RoPE, full-attention NoPE layers) comes from
    `layer_types`, or every 4th layer full (MapleConfig.swift:143-148, SeedlessAttn.swift:81-83).

    cfg, weights = load_maple(model_dir)            # host tensors, sanitized
    eng = VerifyEngine(ctx, cfg, *weights.device())  # resident stack on cuda:0
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass

from .engine import MapleLikeConfig


def read_config(model_dir: str) -> dict:
    with open(os.path.join(model_dir, "config.json")) as f:
        return json.load(f)


def maple_config(cj: dict, max_context: int = 4096) -> MapleLikeConfig:
    """MapleLikeConfig of a Maple config.json (MapleConfig.swift:5-49, 139-148 defaults).  The
    KV ring holds max_context positions plus one pass of rows, enough for the full-attention
    layers; sliding layers use the same ring."""
    q = cj.get("quantization") or {}
    head_dim = int(cj.get("head_dim", 128))
    n_layers = int(cj.get("num_hidden_layers", 24))
    window = int(cj.get("sliding_window", 512))
    rope_dim = int(head_dim * float(cj.get("partial_rotary_factor", 0.5)))
    wins, ropes = MapleLikeConfig.maple_layer_mix(n_layers, window, rope_dim,
                                                  cj.get("layer_types") or None)
    head = q.get("lm_head") or {}
    return MapleLikeConfig(
        n_layers=n_layers, H=int(cj.get("hidden_size", 2048)),
        n_heads=int(cj.get("num_attention_heads", 16)),
        n_kv_heads=int(cj.get("num_key_value_heads", 4)), head_dim=head_dim, rope_dim=rope_dim,
        rope_base=float(cj.get("rope_theta", 10000.0)), eps=float(cj.get("rms_norm_eps", 1e-6)),
        window=window, kv_capacity=max(max_context, window) + 64,
        E=int(cj.get("num_experts", 256)), top_k=int(cj.get("num_experts_per_tok", 8)),
        I=int(cj.get("moe_intermediate_size", 512)), gs=int(q.get("group_size", 128)),
        vocab=int(cj.get("vocab_size", 151936)), layer_window=wins, layer_rope_dim=ropes,
        head_bits=int(head.get("bits", 4)))


def load_arrays(model_dir: str) -> dict:
    """Every tensor of the checkpoint's shards (CPU torch tensors); bf16 -> fp16."""
    import torch
    from safetensors.torch import load_file

    with open(os.path.join(model_dir, "model.safetensors.index.json")) as f:
        wmap = json.load(f).get("weight_map", {})
    out = {}
    for shard in sorted(set(wmap.values())):
        for k, v in load_file(os.path.join(model_dir, shard)).items():
            out[k] = v.to(torch.float16) if v.dtype == torch.bfloat16 else v
    return out


def sanitize(arrays: dict, n_layers: int, group_size: int) -> dict:
    """row_alpha expansion and the qkv / up||gate concatenations (WeightStore.swift:47-91)."""
    import torch

    for key in sorted(k for k in arrays if k.endswith(".row_alpha")):
        alpha = arrays.pop(key)
        prefix = key[: -len(".row_alpha")]
        packed = arrays.get(prefix + ".weight")
        if packed is None:
            continue
        n_groups = packed.shape[-1] * 16 // group_size  # 16 2-bit codes a word
        scales = (alpha.unsqueeze(-1) * torch.ones(n_groups, dtype=alpha.dtype)).contiguous()
        arrays[prefix + ".scales"] = scales
        arrays[prefix + ".biases"] = scales * -1
        arrays[prefix + ".alpha"] = alpha.contiguous()
    for l in range(n_layers):
        attn = f"model.layers.{l}.self_attn"
        for sfx in ("weight", "scales", "biases"):
            parts = [f"{attn}.{p}_proj.{sfx}" for p in ("q", "k", "v")]
            if all(p in arrays for p in parts):
                arrays[f"{attn}.qkv_proj.{sfx}"] = torch.cat([arrays.pop(p) for p in parts], 0)
        mlp = f"model.layers.{l}.mlp.switch_mlp"
        for sfx in ("weight", "scales", "biases", "alpha"):
            up, gate = f"{mlp}.up_proj.{sfx}", f"{mlp}.gate_proj.{sfx}"
            if up in arrays and gate in arrays:
                arrays[f"{mlp}.up_gate_proj.{sfx}"] = torch.cat([arrays.pop(up),
                                                                 arrays.pop(gate)], 1)
    return arrays


def dequant4(w, s, b, group_size: int = 64, rows_per_chunk: int = 8192):
    """fp16 table [V][K] of a 4-bit affine weight [V][K/8] (8 codes a uint32 word, LSB first):
    q * s + b in fp32, rounded once to fp16; done in row chunks to bound the fp32 temporaries."""
    import torch

    wi = w.view(torch.int32) if w.dtype != torch.int32 else w
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    V = wi.shape[0]
    out = torch.empty((V, wi.shape[1] * 8), dtype=torch.float16)
    for r0 in range(0, V, rows_per_chunk):
        r1 = min(V, r0 + rows_per_chunk)
        q = ((wi[r0:r1].unsqueeze(-1) >> shifts) & 15).reshape(r1 - r0, -1).float()
        sg = s[r0:r1].float().repeat_interleave(group_size, dim=-1)
        bg = b[r0:r1].float().repeat_interleave(group_size, dim=-1)
        out[r0:r1] = (q * sg + bg).to(torch.float16)
    return out


def _codes(t):
    """uint32 code arrays as int32 tensors (the device kernels read the bits)."""
    import torch

    return t.view(torch.int32) if t.dtype == torch.uint32 else t


@dataclass
class MapleWeights:
    layers: list
    embed: object
    final_norm: object
    lm_head: object
    lm_head_scales: object
    lm_head_biases: object

    def device(self, device: str = "cuda"):
        """(layers, embed, final_norm, lm_head, lm_head_scales, lm_head_biases) on the device,
        in VerifyEngine's argument order."""
        def mv(x):
            return x.to(device).contiguous() if hasattr(x, "to") else x
        layers = [{part: {k: mv(v) for k, v in lw[part].items()} for part in ("attn", "moe")}
                  for lw in self.layers]
        return (layers, mv(self.embed), mv(self.final_norm), mv(self.lm_head),
                mv(self.lm_head_scales), mv(self.lm_head_biases))


def load_maple(model_dir: str, max_context: int = 4096):
    """(MapleLikeConfig, MapleWeights) of an MLX Maple checkpoint directory."""
    cj = read_config(model_dir)
    cfg = maple_config(cj, max_context)
    a = sanitize(load_arrays(model_dir), cfg.n_layers, cfg.gs)

    def req(name):
        if name not in a:
            raise KeyError(f"missing weight: {name}")
        return a[name]

    layers = []
    for l in range(cfg.n_layers):
        p, at, mo = f"model.layers.{l}", f"model.layers.{l}.self_attn", \
            f"model.layers.{l}.mlp.switch_mlp"
        attn = dict(norm_w=req(f"{p}.input_layernorm.weight"),
                    qkv_w=_codes(req(f"{at}.qkv_proj.weight")),
                    qkv_s=req(f"{at}.qkv_proj.scales"), qkv_b=req(f"{at}.qkv_proj.biases"),
                    q_norm_w=req(f"{at}.q_norm.weight"), k_norm_w=req(f"{at}.k_norm.weight"),
                    o_w=_codes(req(f"{at}.o_proj.weight")), o_s=req(f"{at}.o_proj.scales"),
                    o_b=req(f"{at}.o_proj.biases"))
        moe = dict(norm_w=req(f"{p}.post_attention_layernorm.weight"),
                   router_w=req(f"{p}.mlp.gate.weight"),
                   up_gate_w=_codes(req(f"{mo}.up_gate_proj.weight")),
                   up_gate_s=req(f"{mo}.up_gate_proj.scales"),
                   up_gate_b=req(f"{mo}.up_gate_proj.biases"),
                   down_w=_codes(req(f"{mo}.down_proj.weight")),
                   down_s=req(f"{mo}.down_proj.scales"), down_b=req(f"{mo}.down_proj.biases"),
                   up_gate_alpha=a.get(f"{mo}.up_gate_proj.alpha"),
                   down_alpha=a.get(f"{mo}.down_proj.alpha"),
                   E=cfg.E, top_k=cfg.top_k, H=cfg.H, I=cfg.I, gs=cfg.gs, eps=cfg.eps)
        layers.append(dict(attn=attn, moe=moe))
    embed = dequant4(req("model.word_embeddings.weight"), req("model.word_embeddings.scales"),
                     req("model.word_embeddings.biases"), 64)
    w = MapleWeights(layers=layers, embed=embed, final_norm=req("model.norm.weight"),
                     lm_head=_codes(req("lm_head.weight")), lm_head_scales=a.get("lm_head.scales"),
                     lm_head_biases=a.get("lm_head.biases"))
    if cfg.head_bits != 4:
        w.lm_head = req("lm_head.weight")
    return cfg, w
