"""GPU parity of a Maple checkpoint end to end: the MLX safetensors layout loaded and sanitized
by momij_amd/checkpoint.py, Maple's layer mix (sliding layers with partial RoPE, every 4th layer
full attention without RoPE) and its 4-bit gs64 lm_head inside the resident model.

A synthetic 4-layer checkpoint at the real layer shapes (hidden 2048, 16/4 heads of 128,
16 experts top-4, intermediate 1024, gs 64, vocabulary 2048, window 48; tests/ckpt_util.py) is
prefilled with 100 tokens and verified with an 8-token chain draft.  Every block of the verify
pass is re-run by the oracle from the inputs the device used (its own window / RoPE per layer,
the 4-bit head; tests/teacher.py): routing and head argmax exact up to ties inside the computed
fp32 bound, accepted length and emitted tokens equal to the oracle's acceptance; the oracle's
free-running replay of the prompt and the pass stays within tolerance of the device's head input.
"""
import numpy as np
import pytest

from tests.ckpt_util import write_maple_checkpoint
from tests.gpu_util import assert_close
from tests.teacher import capture_pass, check_head, check_layer

pytestmark = pytest.mark.gpu

# Drift check, not the parity bar: absolute bound of the free-running comparisons, where the
# oracle replays every pass on its own caches so both sides' rounding accumulates over the
# layers (8 fp16 ulps at magnitude 4).  Parity itself is the teacher-forced block checks
# (check_layer / check_head), which keep the 1e-2 absolute and 2e-2 relative-to-norm bar.
DRIFT_ABS = 3.2e-2


@pytest.fixture(scope="module")
def maple(tmp_path_factory):
    import torch

    from momij_amd.checkpoint import load_maple
    from momij_amd.engine import VerifyEngine
    from momij_amd.ops import Context

    d = str(tmp_path_factory.mktemp("maple_gpu"))
    write_maple_checkpoint(d, n_layers=4, E=16, top_k=4, vocab=2048, window=48, seed=11)
    cfg, w = load_maple(d, max_context=192)
    assert cfg.layer_window == [48, 48, 48, 0] and cfg.layer_rope_dim == [64, 64, 64, 0]
    ctx = Context(0)
    dev = w.device()
    torch.cuda.synchronize()
    eng = VerifyEngine(ctx, cfg, *dev)

    def h(t):
        a = t.detach().cpu().numpy()
        return a.view(np.uint32) if a.dtype == np.int32 else a

    host = dict(layers=[{part: {k: (h(v) if hasattr(v, "detach") else v)
                                for k, v in lw[part].items()} for part in ("attn", "moe")}
                        for lw in w.layers],
                embed=h(w.embed), fnorm=h(w.final_norm), head=h(w.lm_head),
                head_s=h(w.lm_head_scales), head_b=h(w.lm_head_biases))
    yield dict(ctx=ctx, cfg=cfg, eng=eng, w=host, dev=dev)
    eng.close()
    ctx.close()


class OracleMaple:
    def __init__(self, orc, cfg, w):
        self.orc, self.cfg, self.w = orc, cfg, w
        C = cfg.kv_capacity
        self.kc = [np.zeros((cfg.n_kv_heads, C, 128), np.float16) for _ in range(cfg.n_layers)]
        self.vc = [np.zeros((cfg.n_kv_heads, C, 128), np.float16) for _ in range(cfg.n_layers)]
        self.L = 0

    def rows(self, tokens, parents):
        h = self.w["embed"][np.asarray(tokens)]
        for l in range(self.cfg.n_layers):
            h, self.kc[l], self.vc[l], _, _ = self.orc.layer_forward(
                self.cfg.attn_cfg(l), self.w["layers"][l], h, self.kc[l], self.vc[l], self.L,
                np.asarray(parents, np.int32))
        return self.orc.rms_norm(h, self.w["fnorm"], self.cfg.eps)  # the head input

    def prefill(self, tokens, chunk=64):
        for i in range(0, len(tokens), chunk):
            t = tokens[i:i + chunk]
            self.rows(t, list(range(-1, len(t) - 1)))
            self.L += len(t)


def _host_kv(eng, layer):
    k, _ = eng.kv(layer)
    cfg = eng.cfg
    n = 2 * cfg.n_kv_heads * cfg.kv_capacity * 128
    out = np.empty(n, np.float16)
    eng.ctx.check(eng.lib.mj_d2h(eng.ctx.h, out.ctypes.data, k, n * 2))
    return out.reshape(2, cfg.n_kv_heads, cfg.kv_capacity, 128)


def test_maple_checkpoint_prefill_and_verify(maple, orc):
    eng, cfg, w = maple["eng"], maple["cfg"], maple["w"]
    q4 = (w["head"], w["head_s"], w["head_b"])
    print("case: maple checkpoint, 4 layers (layer 3 full NoPE), 4-bit head", flush=True)
    rng = np.random.default_rng(2)
    prompt = rng.integers(0, cfg.vocab, 100).tolist()
    eng.rewind(0)
    y, cap = capture_pass(eng, lambda: eng.prefill(prompt, chunk=64))
    am, _ = check_head(orc, cap["head_in"][35:36], [y], "prefill", q4=q4)
    assert am[0] == y
    om = OracleMaple(orc, cfg, w)
    om.prefill(prompt[:-1])
    xf = om.rows(prompt[-1:], [-1])
    om.L += 1
    assert_close(cap["head_in"][35:36], xf, abs_tol=DRIFT_ABS,
                 what="prefill head input (free-running)")
    L0 = eng.offset
    cont, t = [], y
    for _ in range(8):
        t = eng.step_chain_feeds([t])[0]
        cont.append(t)
    eng.rewind(L0)
    draft = cont[:5] + [int(v) for v in rng.integers(0, cfg.vocab, 3)]
    for i in range(5, 8):
        if draft[i] == cont[i]:
            draft[i] = (draft[i] + 1) % cfg.vocab
    kv0 = [_host_kv(eng, l) for l in range(cfg.n_layers)]
    (acc, toks), cap = capture_pass(eng, lambda: eng.verify_greedy(y, draft))
    assert acc == 5 and toks == cont[:6], (acc, toks, cont)
    parents = list(range(-1, 8))
    for l in range(cfg.n_layers):
        check_layer(orc, cfg, l, w["layers"][l], cap, 9, (kv0[l][0], kv0[l][1]), L0, parents)
    gpu_am = orc.argmax_rows(cap["logits"][:9])[0]
    am, _ = check_head(orc, cap["head_in"][:9], gpu_am, "verify", q4=q4)
    oacc, _, oemit = orc.accept_greedy([y] + draft, None, am)
    assert oacc == acc and list(oemit) == toks
    # the free-running replay accumulates both sides' rounding over 4 layers and 109 positions:
    # the relative bar holds, single elements of magnitude ~4 may drift by a few fp16 ulps
    xf = om.rows([y] + draft, parents)
    assert_close(cap["head_in"][:9], xf, abs_tol=DRIFT_ABS, what="verify head input (free-running)")


def test_full_attention_capacity_guard(maple):
    from momij_amd._lib import MomijError

    eng, cfg = maple["eng"], maple["cfg"]
    print("case: full-attention layer past its KV capacity", flush=True)
    eng.rewind(0)
    y = eng.prefill(list(range(1, cfg.kv_capacity - 3)), chunk=64)
    # 9 more rows do not fit the full-attention layer's ring: refused before any kernel runs
    with pytest.raises(MomijError):
        eng.verify_greedy(y, [2, 3, 4, 5, 6, 7, 8, 9])
    eng.rewind(0)


def test_row_alpha_alignment_checked_at_model_create(maple):
    """A row-alpha array that is not 16-byte aligned is refused by mj_model_create (the expert
    kernels load it 16 bytes at a time), before any kernel runs."""
    import torch

    from momij_amd._lib import MomijError
    from momij_amd.engine import VerifyEngine

    print("case: misaligned row-alpha array at model create", flush=True)
    layers, *rest = maple["dev"]
    bad = [{part: dict(lw[part]) for part in ("attn", "moe")} for lw in layers]
    a = bad[1]["moe"]["down_alpha"]
    assert a is not None
    buf = torch.empty(a.numel() + 8, dtype=torch.float16, device="cuda")
    bad[1]["moe"]["down_alpha"] = buf[1:1 + a.numel()].view_as(a)
    with pytest.raises(MomijError):
        VerifyEngine(maple["ctx"], maple["cfg"], bad, *rest)


def test_layer_expert_shape_checked_at_model_create(maple):
    """A layer whose expert shape differs from the model configuration (the pass scratch is
    sized from the configuration) is refused by mj_model_create before any kernel runs."""
    from momij_amd._lib import MomijError
    from momij_amd.engine import VerifyEngine

    print("case: layer expert shape differs from the model configuration", flush=True)
    layers, *rest = maple["dev"]
    for field, value in (("I", 2048), ("E", 8), ("top_k", 2), ("gs", 128)):
        bad = [{part: dict(lw[part]) for part in ("attn", "moe")} for lw in layers]
        bad[2]["moe"][field] = value
        with pytest.raises(MomijError) as ei:
            VerifyEngine(maple["ctx"], maple["cfg"], bad, *rest)
        assert ei.value.status == 4 and "layer 2" in str(ei.value), field


@pytest.fixture(scope="module")
def maple_real(tmp_path_factory):
    """A 4-layer checkpoint at Maple's own shapes, loaded from a config.json that leaves every
    architecture field at MapleConfig's defaults: 256 experts top-8, intermediate 512, group
    size 128, window 512, rope theta 1e4 on 64 dims, the 4-bit gs64 head (vocabulary 2048)."""
    import torch

    from momij_amd.checkpoint import load_maple
    from momij_amd.engine import VerifyEngine
    from momij_amd.ops import Context

    d = str(tmp_path_factory.mktemp("maple_real"))
    write_maple_checkpoint(d, n_layers=4, E=256, top_k=8, I=512, gs=128, vocab=2048, window=512,
                           seed=21, defaults_config=True)
    cfg, w = load_maple(d, max_context=256)
    assert (cfg.E, cfg.top_k, cfg.I, cfg.gs, cfg.window, cfg.rope_dim, cfg.head_bits) == \
        (256, 8, 512, 128, 512, 64, 4)
    assert cfg.rope_base == 1e4 and cfg.layer_window == [512, 512, 512, 0]
    ctx = Context(0)
    dev = w.device()
    torch.cuda.synchronize()
    eng = VerifyEngine(ctx, cfg, *dev)

    def h(t):
        a = t.detach().cpu().numpy()
        return a.view(np.uint32) if a.dtype == np.int32 else a

    host = dict(layers=[{part: {k: (h(v) if hasattr(v, "detach") else v)
                                for k, v in lw[part].items()} for part in ("attn", "moe")}
                        for lw in w.layers],
                embed=h(w.embed), fnorm=h(w.final_norm), head=h(w.lm_head),
                head_s=h(w.lm_head_scales), head_b=h(w.lm_head_biases))
    yield dict(ctx=ctx, cfg=cfg, eng=eng, w=host)
    eng.close()
    ctx.close()


def test_maple_real_shape_prefill_and_verify(maple_real, orc):
    """Maple's own expert shape end to end: prefill, an 8-token chain verify and a 16-node tree
    verify, each block re-run by the oracle from the device's inputs (tests/teacher.py)."""
    eng, cfg, w = maple_real["eng"], maple_real["cfg"], maple_real["w"]
    q4 = (w["head"], w["head_s"], w["head_b"])
    print("case: maple defaults, E=256 top-8 I=512 gs=128 window 512, 4 layers", flush=True)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, cfg.vocab, 150).tolist()
    eng.rewind(0)
    y, cap = capture_pass(eng, lambda: eng.prefill(prompt, chunk=64))
    M_last = 150 - 128
    am, _ = check_head(orc, cap["head_in"][M_last - 1:M_last], [y], "prefill", q4=q4)
    assert am[0] == y
    L0 = eng.offset
    cont, t = [], y
    for _ in range(8):
        t = eng.step_chain_feeds([t])[0]
        cont.append(t)
    eng.rewind(L0)
    draft = cont[:5] + [int(v) for v in rng.integers(0, cfg.vocab, 3)]
    for i in range(5, 8):
        if draft[i] == cont[i]:
            draft[i] = (draft[i] + 1) % cfg.vocab
    for parents, toks, want in ((None, draft, 5),
                                (TREE16, _tree_draft(cont, cfg.vocab, rng), 4)):
        eng.rewind(L0)
        M = len(toks) + 1
        par = list(range(-1, M - 1)) if parents is None else parents
        kv0 = [_host_kv(eng, l) for l in range(cfg.n_layers)]
        (acc, out), cap = capture_pass(eng, lambda: eng.verify_greedy(y, toks, parents))
        assert acc == want and out == cont[:want + 1], (acc, out, cont)
        for l in range(cfg.n_layers):
            check_layer(orc, cfg, l, w["layers"][l], cap, M, (kv0[l][0], kv0[l][1]), L0, par)
        gpu_am = orc.argmax_rows(cap["logits"][:M])[0]
        am, _ = check_head(orc, cap["head_in"][:M], gpu_am, "verify", q4=q4)
        oacc, _, oemit = orc.accept_greedy([y] + toks, parents, am)
        assert oacc == acc and list(oemit) == out
    eng.rewind(L0)


TREE16 = [-1, 0, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 10, 11, 12, 13, 14]


def _tree_draft(cont, vocab, rng):
    """TREE16 tokens whose first-child path (0-1-4-10-12) carries the continuation."""
    toks = [int(t) for t in rng.integers(0, vocab, len(TREE16) - 1)]
    depth = [0] * len(TREE16)
    for r in range(1, len(TREE16)):
        depth[r] = depth[TREE16[r]] + 1
    path = [1, 4, 10, 12]
    for d, r in enumerate(path):
        toks[r - 1] = cont[d]
    for r in range(1, len(TREE16)):
        if r not in path and toks[r - 1] == cont[depth[r] - 1]:
            toks[r - 1] = (toks[r - 1] + 1) % vocab
    return toks
