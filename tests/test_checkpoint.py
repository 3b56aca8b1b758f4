"""The MLX Maple checkpoint loader (momij_amd/checkpoint.py) against the rules of WeightStore
(WeightStore.swift:47-91) and MapleConfig (MapleConfig.swift:139-148), restated independently
here in numpy over a synthetic checkpoint written in the reference's naming (tests/ckpt_util.py).
"""
import numpy as np
import pytest

from tests.ckpt_util import write_maple_checkpoint


def _np(t):
    import torch

    if t.dtype == torch.uint32:
        t = t.view(torch.int32)
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.numpy()


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    from momij_amd.checkpoint import load_maple

    d = str(tmp_path_factory.mktemp("maple"))
    arrays = write_maple_checkpoint(d, n_layers=8, H=128, nQ=2, nKV=1, D=32, E=3, top_k=2, I=64,
                                    gs=64, vocab=40, window=16, seed=3)
    cfg, w = load_maple(d, max_context=256)
    return arrays, cfg, w


def test_config_and_layer_mix(ckpt):
    _, cfg, _ = ckpt
    assert (cfg.H, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim) == (128, 8, 2, 1, 32)
    assert (cfg.E, cfg.top_k, cfg.I, cfg.gs, cfg.vocab, cfg.head_bits) == (3, 2, 64, 64, 40, 4)
    assert cfg.rope_dim == 16 and cfg.window == 16 and cfg.kv_capacity == 256 + 64
    # without layer_types every 4th layer is full attention without RoPE
    assert cfg.layer_window == [16, 16, 16, 0, 16, 16, 16, 0]
    assert cfg.layer_rope_dim == [16, 16, 16, 0, 16, 16, 16, 0]


def test_layer_types_rule():
    from momij_amd.engine import MapleLikeConfig

    types = ["full_attention", "sliding_attention", "sliding_attention"]
    wins, ropes = MapleLikeConfig.maple_layer_mix(5, 512, 64, types)
    # listed layers follow layer_types; layers past the list fall back to the every-4th rule
    assert wins == [0, 512, 512, 0, 512] and ropes == [0, 64, 64, 0, 64]


def test_qkv_and_up_gate_concatenation(ckpt):
    arrays, _, w = ckpt
    for l in (0, 5):
        at = f"model.layers.{l}.self_attn"
        want = np.concatenate([_np(arrays[f"{at}.{p}_proj.weight"]) for p in "qkv"], 0)
        assert (_np(w.layers[l]["attn"]["qkv_w"]) == want).all()
        mo = f"model.layers.{l}.mlp.switch_mlp"
        for sfx, key in (("weight", "up_gate_w"), ("scales", "up_gate_s"),
                         ("biases", "up_gate_b")):
            want = np.concatenate([_np(arrays[f"{mo}.up_proj.{sfx}"]),
                                   _np(arrays[f"{mo}.gate_proj.{sfx}"])], 1)
            got = _np(w.layers[l]["moe"][key])
            assert got.shape == want.shape and (got.astype(np.float64)
                                                == want.astype(np.float64)).all()


def test_row_alpha_expansion(ckpt):
    arrays, cfg, w = ckpt
    at = "model.layers.0.self_attn"
    alpha = _np(arrays[f"{at}.q_proj.row_alpha"]).astype(np.float16)  # bf16 -> fp16, exact
    nq = alpha.shape[0]
    groups = cfg.H // cfg.gs
    s = _np(w.layers[0]["attn"]["qkv_s"])
    b = _np(w.layers[0]["attn"]["qkv_b"])
    assert s.dtype == np.float16 and s.shape == (nq + 2 * 32, groups)
    assert (s[:nq] == np.repeat(alpha[:, None], groups, 1)).all()
    assert (b[:nq] == -s[:nq]).all()
    # k and v keep their own scales after the alpha-expanded q rows
    assert (s[nq:nq + 32] == _np(arrays[f"{at}.k_proj.scales"]).astype(np.float16)).all()


def test_float_tensors_become_fp16(ckpt):
    arrays, _, w = ckpt
    nw = w.layers[2]["attn"]["norm_w"]
    assert str(nw.dtype) == "torch.float16"
    assert (_np(nw) == _np(arrays["model.layers.2.input_layernorm.weight"]).astype(np.float16)).all()
    assert str(w.lm_head_scales.dtype) == "torch.float16"


def test_embedding_dequantised(ckpt):
    arrays, cfg, w = ckpt
    words = _np(arrays["model.word_embeddings.weight"]).view(np.uint32)
    q = ((words[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15).reshape(cfg.vocab, -1)
    s = np.repeat(_np(arrays["model.word_embeddings.scales"]).astype(np.float16)
                  .astype(np.float64), 64, 1)
    b = np.repeat(_np(arrays["model.word_embeddings.biases"]).astype(np.float16)
                  .astype(np.float64), 64, 1)
    want = (q * s + b).astype(np.float16)
    got = _np(w.embed)
    assert got.shape == (cfg.vocab, cfg.H)
    # the loader rounds q*s + b from fp32 once; float64 then fp16 agrees to an ulp
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert (diff <= np.abs(want.astype(np.float64)) * 2.0**-10 + 2.0**-24).all()


def test_missing_weight_is_an_error(tmp_path):
    import os

    from momij_amd.checkpoint import load_maple

    d = str(tmp_path / "broken")
    write_maple_checkpoint(d, n_layers=1, H=128, nQ=2, nKV=1, D=32, E=3, top_k=2, I=64, vocab=8)
    import json

    idx = json.load(open(os.path.join(d, "model.safetensors.index.json")))
    del idx["weight_map"]["model.norm.weight"]  # its shard still holds it: drop from both
    json.dump(idx, open(os.path.join(d, "model.safetensors.index.json"), "w"))
    from safetensors.torch import load_file, save_file

    for fn in set(idx["weight_map"].values()):
        t = load_file(os.path.join(d, fn))
        t.pop("model.norm.weight", None)
        save_file(t, os.path.join(d, fn))
    with pytest.raises(KeyError):
        load_maple(d)


def test_expert_row_alpha_kept_for_the_fold(ckpt):
    """Row-alpha experts keep alpha (up || gate along the rows) beside the expanded scales, and
    the loader hands it to the MoE block; other layers pass none."""
    _, cfg, w = ckpt
    m1, m0 = w.layers[1]["moe"], w.layers[0]["moe"]
    a_ug, a_dn = _np(m1["up_gate_alpha"]), _np(m1["down_alpha"])
    assert a_ug.shape == (cfg.E, 2 * cfg.I) and a_dn.shape == (cfg.E, cfg.H)
    s_ug = _np(m1["up_gate_s"])
    assert (s_ug == a_ug[..., None]).all() and (_np(m1["up_gate_b"]) == -s_ug).all()
    assert (_np(m1["down_s"]) == a_dn[..., None]).all()
    assert m0["up_gate_alpha"] is None and m0["down_alpha"] is None
