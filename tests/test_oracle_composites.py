"""Pins of the oracle's composite blocks against an independent float64 restatement.

or_moe_block, or_attn_block, or_layer_forward, or_score_resid and or_kv_commit are compared
with tests/restate64.py (numpy float64, vectorised, rounded to fp16 only where the reference's
kernels store half) or with invariants that do not restate them:
  * the composite outputs agree with the float64 statement within a few fp16 ulps, the routing
    exactly (rows whose top-k gap is below 1e-4 would be reported, none occurs at these seeds);
  * planted mistakes -- up and gate swapped, the up gather fed the un-normed row, V passed
    through the k-norm -- move the float64 statement far outside that band, so the comparison
    can tell each of them from the oracle;
  * the residual's two roundings (half(h + half(acc)), SeedlessMetal.swift:2474-2493) by a case
    where one rounding would give a different fp16 value;
  * or_layer_forward is bit for bit or_attn_block followed by or_moe_block;
  * or_kv_commit: a tree verify followed by the commit of its accepted path leaves the cache a
    chain verify of that path leaves, bit for bit (layer by layer through the oracle's own
    attention), and a chain path is the identity.
"""
import numpy as np
import pytest

from momij_amd import synth
from tests import restate64 as r64


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _ulps(a, b, floor=0.0):
    """|a - b| in fp16 ulps of max(|b|, floor) (values are fp16-representable); the floor keeps
    values that cancel to near zero from counting their tiny ulp."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    mag = np.maximum(np.abs(b), max(floor, 2.0 ** -14))
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 10)
    return np.abs(a - b) / ulp


# float64 statement vs the fp32 oracle: a handful of fp16 ulps where an fp32 sum lands on the
# other side of a rounding boundary, propagated through the block
COMPOSITE_REL = 2e-3
PLANTED_REL = 5e-2


def _moe_case(rng, gs, E=16, k=4, M=5, H=512, I=256):
    mw = synth.moe_weights(rng, E, H, I, gs, top_k=k)
    x = synth.normal_f16(rng, (M, H))
    return mw, x


@pytest.mark.parametrize("gs", [64, 128])
def test_moe_block_vs_float64(orc, gs):
    rng = np.random.default_rng(100 + gs)
    mw, x = _moe_case(rng, gs)
    y, inds, scores = orc.moe_block(mw, x, prenorm=True, residual=True)
    ref, ri, rs, lg = r64.moe_block(mw, x)
    assert (r64.topk_gap(lg, mw["top_k"]) > 1e-4).all()
    assert (inds == ri).all(), (inds, ri)
    assert np.allclose(scores, rs, rtol=1e-5, atol=1e-6)
    rel = _rel(y, ref)
    u = _ulps(y, ref)
    print(f"moe gs={gs}: rel {rel:.2e}, max ulps {u.max()}, equal {np.mean(u == 0):.3f}")
    assert rel < COMPOSITE_REL and (u == 0).mean() > 0.9


def test_moe_block_no_residual_no_prenorm(orc):
    rng = np.random.default_rng(7)
    mw, x = _moe_case(rng, 64, E=8, k=2, M=3)
    y, inds, _ = orc.moe_block(mw, x, prenorm=False, residual=False)
    ref, ri, _, lg = r64.moe_block(mw, x, prenorm=False, residual=False)
    assert (r64.topk_gap(lg, 2) > 1e-4).all() and (inds == ri).all()
    assert _rel(y, ref) < COMPOSITE_REL


@pytest.mark.parametrize("mistake", ["swap_up_gate", "skip_norm_up"])
def test_moe_block_planted_mistakes_are_caught(orc, mistake):
    rng = np.random.default_rng(101)
    mw, x = _moe_case(rng, 64)
    y, inds, _ = orc.moe_block(mw, x, prenorm=True, residual=False)
    ok, _, _, _ = r64.moe_block(mw, x, residual=False, inds=inds)
    bad, _, _, _ = r64.moe_block(mw, x, residual=False, inds=inds, **{mistake: True})
    assert _rel(y, ok) < COMPOSITE_REL
    assert _rel(y, bad) > PLANTED_REL, mistake


def test_score_resid_rounds_twice(orc):
    """half(h + half(acc)): acc = 0.50024 rounds to 0.5, and 1024 + 0.5 ties to even (1024);
    a single rounding of 1024.50024 would give 1025."""
    H = 16
    h = np.full((1, H), 1024.0, np.float16)
    down = np.ones((1, H), np.float16)
    sc = np.array([[0.50024]], np.float32)
    got = orc.score_resid(down, sc, h)
    assert (got == np.float16(1024.0)).all(), got
    assert (r64.score_resid(down, sc, h) == 1024.0).all()
    # and at random values the float64 statement agrees with the oracle
    rng = np.random.default_rng(8)
    M, k, H = 4, 8, 256
    down = synth.normal_f16(rng, (M * k, H))
    sc = rng.dirichlet(np.ones(k), M).astype(np.float32)
    h = synth.normal_f16(rng, (M, H), 2.0)
    u = _ulps(orc.score_resid(down, sc, h), r64.score_resid(down, sc, h))
    assert u.max() <= 1 and (u == 0).mean() > 0.99


def _attn_case(rng, window, rope_dim=64):
    cfg = dict(H=512, nQ=4, nKV=2, D=128, rope_dim=rope_dim, rope_base=1e6, eps=1e-6,
               window=window, C=100, gs=64)
    aw = synth.attn_weights(rng, cfg["H"], cfg["nQ"], cfg["nKV"], cfg["D"], cfg["gs"])
    kc = synth.normal_f16(rng, (cfg["nKV"], cfg["C"], cfg["D"]))
    vc = synth.normal_f16(rng, (cfg["nKV"], cfg["C"], cfg["D"]))
    return cfg, aw, kc, vc


@pytest.mark.parametrize("shape,window,L", [("chain", 32, 60), ("tree", 32, 150),
                                           ("tree", 0, 40), ("chain", 48, 7)])
def test_attn_block_vs_float64(orc, shape, window, L):
    rng = np.random.default_rng(200 + L + window)
    cfg, aw, kc, vc = _attn_case(rng, window, rope_dim=64 if window else 0)
    parents = (list(range(-1, 7)) if shape == "chain"
               else [-1, 0, 0, 0, 1, 1, 2, 4, 4, 7, 9])
    M = len(parents)
    h = synth.normal_f16(rng, (M, cfg["H"]), 2.0)
    par = np.array(parents, np.int32)
    ho, ko, vo = orc.attn_block(cfg, aw, h, kc, vc, L, par)
    rh, rk, rv = r64.attn_block(cfg, aw, h, kc, vc, L, parents)
    slots = [(L + r) % cfg["C"] for r in range(M)]
    # k rows are unit-RMS per head (norm, then rotation mixes pairs): ulps of 1.0 below that
    uk = _ulps(ko[:, slots], rk[:, slots], floor=1.0)
    uv = _ulps(vo[:, slots], rv[:, slots], floor=0.25)
    rel = _rel(ho, rh)
    print(f"attn {shape} W={window} L={L}: rel {rel:.2e}, k rel {_rel(ko[:, slots], rk[:, slots]):.2e}"
          f" ulps {uk.max()} eq {(uk == 0).mean():.3f}, v ulps {uv.max()} eq {(uv == 0).mean():.3f}")
    assert rel < COMPOSITE_REL
    assert _rel(ko[:, slots], rk[:, slots]) < COMPOSITE_REL and uk.max() <= 4
    # v is the projection itself: its bias term uses the reference's half-precision 4-sums of
    # the input (ld16_b2, SeedlessMetal.swift:2145-2156), which the float64 statement does not
    assert _rel(vo[:, slots], rv[:, slots]) < COMPOSITE_REL and uv.max() <= 4
    other = np.ones(cfg["C"], bool)
    other[slots] = False
    assert (ko[:, other] == kc[:, other]).all() and (vo[:, other] == vc[:, other]).all()


def test_attn_block_planted_v_norm_is_caught(orc):
    rng = np.random.default_rng(300)
    cfg, aw, kc, vc = _attn_case(rng, 32)
    M, L = 6, 4  # a short prefix: the pass's own V rows carry most of the attention weight
    h = synth.normal_f16(rng, (M, cfg["H"]), 2.0)
    par = np.arange(-1, M - 1, dtype=np.int32)
    ho, _, _ = orc.attn_block(cfg, aw, h, kc, vc, L, par)
    bad, _, _ = r64.attn_block(cfg, aw, h, kc, vc, L, list(par), norm_v=True)
    ok, _, _ = r64.attn_block(cfg, aw, h, kc, vc, L, list(par))
    hd = h.astype(np.float64)
    upd = ho.astype(np.float64) - hd  # the block's contribution on top of the residual
    print("v-norm control:", _rel(upd, ok - hd), _rel(upd, bad - hd))
    assert _rel(upd, ok - hd) < 10 * COMPOSITE_REL
    assert _rel(upd, bad - hd) > 4 * PLANTED_REL


def _layer_case(rng):
    cfg, aw, kc, vc = _attn_case(rng, 32)
    mw = synth.moe_weights(rng, 8, cfg["H"], 256, cfg["gs"], top_k=2)
    return cfg, dict(attn=aw, moe=mw), kc, vc


def test_layer_forward_is_attn_then_moe(orc):
    rng = np.random.default_rng(400)
    cfg, lw, kc, vc = _layer_case(rng)
    M, L = 5, 70
    h = synth.normal_f16(rng, (M, cfg["H"]), 2.0)
    par = np.arange(-1, M - 1, dtype=np.int32)
    ho, ko, vo, inds, _ = orc.layer_forward(cfg, lw, h, kc, vc, L, par)
    ha, ka, va = orc.attn_block(cfg, lw["attn"], h, kc, vc, L, par)
    hm, im, _ = orc.moe_block(lw["moe"], ha, prenorm=True, residual=True)
    assert (ho.view(np.uint16) == hm.view(np.uint16)).all()
    assert (ko.view(np.uint16) == ka.view(np.uint16)).all() and (inds == im).all()
    # and the whole layer against the float64 statement
    rh, _, _ = r64.attn_block(cfg, lw["attn"], h, kc, vc, L, list(par))
    ry, ri, _, lg = r64.moe_block(lw["moe"], rh)
    assert (r64.topk_gap(lg, 2) > 1e-4).all() and (inds == ri).all()
    assert _rel(ho, ry) < COMPOSITE_REL


def test_kv_commit_tree_equals_chain(orc):
    """Two layers: verify a draft tree on copies of the cache, commit the accepted path; verify
    the path alone as a chain on other copies.  The committed rows are identical bit for bit
    (each path row attends the committed window plus its ancestors, which is the chain prefix),
    and a second pass after each reads identical caches."""
    rng = np.random.default_rng(500)
    cfg, lw0, kc0, vc0 = _layer_case(rng)
    _, lw1, kc1, vc1 = _layer_case(rng)
    layers, caches = [lw0, lw1], [(kc0, vc0), (kc1, vc1)]
    L = 93  # ring wraps for the rows past slot 99
    tree = [-1, 0, 0, 1, 1, 2, 4, 4, 7]
    path = [0, 1, 4, 7, 8]  # depth 0..4 along the tree
    M = len(tree)
    x = synth.normal_f16(rng, (M, cfg["H"]), 2.0)

    def run(rows_x, parents, kv):
        h = rows_x
        out = []
        for l, lw in enumerate(layers):
            h, k, v, _, _ = orc.layer_forward(cfg, lw, h, kv[l][0], kv[l][1], L,
                                              np.array(parents, np.int32))
            out.append((k, v))
        return h, out

    ht, kv_tree = run(x, tree, caches)
    committed = [orc.kv_commit(k, v, L, path) for k, v in kv_tree]
    hc, kv_chain = run(x[path], list(range(-1, len(path) - 1)), caches)
    assert (ht[path].view(np.uint16) == hc.view(np.uint16)).all()
    slots = [(L + i) % cfg["C"] for i in range(len(path))]
    for (kt, vt), (kc, vc) in zip(committed, kv_chain):
        assert (kt[:, slots].view(np.uint16) == kc[:, slots].view(np.uint16)).all()
        assert (vt[:, slots].view(np.uint16) == vc[:, slots].view(np.uint16)).all()
    # the next pass (a 3-row chain at L + 5) reads the same committed prefix either way
    nxt = synth.normal_f16(rng, (3, cfg["H"]), 2.0)
    L2 = L + len(path)
    for (kt, vt), (kc, vc), lw in zip(committed, kv_chain, layers):
        a = orc.attn_block(cfg, lw["attn"], nxt, kt, vt, L2, np.arange(-1, 2, dtype=np.int32))[0]
        b = orc.attn_block(cfg, lw["attn"], nxt, kc, vc, L2, np.arange(-1, 2, dtype=np.int32))[0]
        assert (a.view(np.uint16) == b.view(np.uint16)).all()
    # a chain path is the identity
    k0, v0 = kv_tree[0]
    ki, vi = orc.kv_commit(k0, v0, L, list(range(4)))
    assert (ki.view(np.uint16) == k0.view(np.uint16)).all()
    assert (vi.view(np.uint16) == v0.view(np.uint16)).all()
