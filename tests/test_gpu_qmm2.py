"""GPU parity: 2-bit gather-qmm (GEMV and bucketed MFMA GEMM) and the MoE block vs the oracle.

Float outputs: relative-to-norm 2e-2 and absolute 1e-2 (the verify-step bar).  Expert indices
are compared bit for bit.
"""
import numpy as np
import pytest

from momij_amd import synth
from tests.gpu_util import assert_close, dev, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch

    from momij_amd.ops import Context

    assert torch.cuda.is_available()
    c = Context(0)
    yield c
    c.close()


def _run(ctx, fn):
    import torch

    torch.cuda.synchronize()
    fn()
    ctx.sync()


def test_mfma_operand_layout(ctx):
    import torch

    rng = np.random.default_rng(0)
    A = rng.integers(-4, 5, (16, 32)).astype(np.float16)
    B = rng.integers(-4, 5, (32, 16)).astype(np.float16)
    D = torch.zeros((16, 16), dtype=torch.float32, device="cuda")
    dA, dB = dev(A), dev(B)
    _run(ctx, lambda: ctx.selftest_mfma(dA, dB, D))
    ref = A.astype(np.float64) @ B.astype(np.float64)
    assert (host(D) == ref).all()


def test_qmv2_gemv_config0(ctx, orc):
    """Single-token 2-bit GEMV: W [5632 x 2048], gs 64, x ~ N(0,1)."""
    import torch

    print("case: qmv2 cfg0 N=5632 K=2048 gs=64", flush=True)
    rng = np.random.default_rng(100)
    N, K, gs = 5632, 2048, 64
    w, s, b = synth.qweight(rng, (1,), N, K, gs)
    x = synth.normal_f16(rng, (1, K))
    inds = np.zeros(1, np.int32)
    ref = orc.qmm2(x, w, s, b, inds, 1, 1, K, N, gs)
    y = torch.empty((1, N), dtype=torch.float16, device="cuda")
    dx, dw, ds, db, di = dev(x), dev(w), dev(s), dev(b), dev(inds)
    _run(ctx, lambda: ctx.gather_qmm2(dx, dw, ds, db, di, y, 1, 1, K, N, gs))
    rel, mx = assert_close(host(y), ref, what="cfg0")
    assert rel < 2e-3  # fp16 output rounding level
    # float64 closed form as a second restatement
    dense = synth.dequant(w[0], s[0], b[0], gs)
    ref64 = dense @ x[0].astype(np.float64)
    assert_close(host(y)[0], ref64, what="cfg0 vs f64")


@pytest.mark.parametrize("case", ["up_gs64", "down_lhs", "gs128", "dense_add", "prefill_rows",
                                  "down_k512_gs128", "down_k512_gs64", "qmv_k512"])
def test_gather_rows(ctx, orc, case):
    import torch

    print(f"case: gather {case}", flush=True)
    rng = np.random.default_rng(hash(case) % 1000)
    E, M, ktop, K, N, gs, lhs, epi = 16, 9, 8, 2048, 256, 64, False, 0
    if case == "down_lhs":
        K, lhs = 1024, True
    elif case == "gs128":
        gs = 128
    elif case == "dense_add":
        E, ktop, N, epi = 1, 1, 512, 1
    elif case == "prefill_rows":
        M, ktop, E = 40, 2, 4  # more rows per expert than one MFMA row group holds
    elif case.startswith("down_k512"):  # Maple's down projection: K = I = 512
        K, N, lhs, gs = 512, 2048, True, (64 if case.endswith("gs64") else 128)
    elif case == "qmv_k512":  # one row: the GEMV kernel at K = 512
        E, M, ktop, K, N, gs = 4, 1, 1, 512, 2048, 128
    w, s, b = synth.qweight(rng, (E,), N, K, gs)
    x = synth.normal_f16(rng, (M * ktop if lhs else M, K))
    inds = np.stack([rng.permutation(E)[:ktop] for _ in range(M)]).reshape(-1).astype(np.int32)
    y0 = synth.normal_f16(rng, (M * ktop, N))
    ref = orc.qmm2(x, w, s, b, inds, M, ktop, K, N, gs, lhs)
    if epi == 1:
        ref = (y0.astype(np.float32) + ref.astype(np.float32)).astype(np.float16)
    y = dev(y0)
    dx, dw, ds, db, di = dev(x), dev(w), dev(s), dev(b), dev(inds)
    _run(ctx, lambda: ctx.gather_qmm2(dx, dw, ds, db, di, y, M, ktop, K, N, gs, lhs, epi))
    rel, _ = assert_close(host(y), ref, what=case)
    assert rel < 3e-3


def _moe_data(rng, E, H, I, gs):
    return synth.moe_weights(rng, E, H, I, gs)


def _moe_dev(mw):
    d = {k: (dev(v) if isinstance(v, np.ndarray) else v) for k, v in mw.items()}
    return d


@pytest.mark.parametrize("M,flags", [(1, 0), (8, 0), (8, 3), (1, 3), (9, 3), (16, 3), (17, 3),
                                     (32, 3), (33, 3)])
def test_moe_block(ctx, orc, M, flags):
    """Config 1 (M=1) and the K=8 verify rows of config 2 (M=8), and the pre-norm+residual form
    used inside a layer: routing bit-exact, outputs within tolerance.  Up to 16 rows the up ||
    gate product ranks the router logits itself (M = 16: two rows on every wave); 17 rows take
    the separate top-k launch."""
    import torch

    print(f"case: moe M={M} flags={flags}", flush=True)
    rng = np.random.default_rng(200 + M + flags)
    E, H, I, gs, k = 64, 2048, 1024, 64, 8
    mw = _moe_data(rng, E, H, I, gs)
    x = synth.normal_f16(rng, (M, H))
    ref_y, ref_i, ref_s = orc.moe_block(mw, x, prenorm=bool(flags & 1), residual=bool(flags & 2))
    dmw = _moe_dev(mw)
    dx = dev(x)
    y = torch.empty_like(dx)
    inds = torch.empty((M, k), dtype=torch.int32, device="cuda")
    scores = torch.empty((M, k), dtype=torch.float32, device="cuda")
    _run(ctx, lambda: ctx.moe_block(dmw, dx, y, M, flags, inds, scores))
    gi = host(inds)
    assert (gi == ref_i).all(), (gi, ref_i)
    assert np.allclose(host(scores), ref_s, rtol=1e-4, atol=1e-5)
    rel, _ = assert_close(host(y), ref_y, what=f"moe M={M}")
    assert rel < 5e-3


@pytest.mark.parametrize("M", [1, 9, 16, 17, 32])
def test_moe_fused_routing_equals_separate_topk(ctx, M):
    """Passes of at most 32 rows rank the router logits in the fused MoE launch's prologue
    (every block builds the slot records in LDS; four rows a wave past 16) and run both expert
    products in that one launch; 33 rows take the separate top-k, up and down launches.  A
    row's routing and output do not depend on the other rows of its pass, so an M-row pass
    equals the first M rows of a 33-row pass bit for bit: expert ids, weights and outputs."""
    import torch

    print(f"case: moe fused routing M={M} vs 33 rows", flush=True)
    rng = np.random.default_rng(500 + M)
    E, H, I, gs, k = 64, 2048, 1024, 64, 8
    mw = _moe_data(rng, E, H, I, gs)
    dmw = _moe_dev(mw)
    x = synth.normal_f16(rng, (33, H))

    def run(rows):
        dx = dev(np.ascontiguousarray(x[:rows]))
        y = torch.empty_like(dx)
        inds = torch.empty((rows, k), dtype=torch.int32, device="cuda")
        scores = torch.empty((rows, k), dtype=torch.float32, device="cuda")
        _run(ctx, lambda: ctx.moe_block(dmw, dx, y, rows, 3, inds, scores))
        return host(y), host(inds), host(scores)

    y33, i33, s33 = run(33)
    ym, im, sm = run(M)
    assert (im == i33[:M]).all()
    assert (sm.view(np.uint32) == s33[:M].view(np.uint32)).all()
    diff = ym.view(np.uint16) != y33[:M].view(np.uint16)
    assert not diff.any(), f"rows differing: {np.nonzero(diff.any(axis=1))[0].tolist()}"


def _row_alpha(mw):
    """Row-alpha form of the expert weights (WeightStore.swift:47-63): alpha = the row's first
    group scale, scales = alpha in every group, biases = -alpha."""
    for p in ("up_gate", "down"):
        alpha = np.ascontiguousarray(mw[p + "_s"][..., 0])
        mw[p + "_s"] = np.ascontiguousarray(np.repeat(alpha[..., None], mw[p + "_s"].shape[-1], -1))
        mw[p + "_b"] = (-mw[p + "_s"]).astype(np.float16)
        mw[p + "_alpha"] = alpha
    return mw


@pytest.mark.parametrize("E,I,gs,M", [(64, 1024, 64, 8), (16, 1024, 128, 9),
                                      (128, 1024, 128, 17), (128, 2048, 64, 8),
                                      (64, 1024, 64, 1), (64, 1024, 128, 64),
                                      (256, 512, 128, 9), (64, 512, 64, 17)])
def test_moe_block_row_alpha(ctx, orc, E, I, gs, M):
    """Row-alpha experts: the fold kernels (one alpha per row) against the oracle on the
    expanded scales / biases, and against the group-scale kernels on the same arrays --
    persistent slot records (E <= 64) and per-expert lists (E = 128), both K widths of down,
    one row (the same tile kernels as a verify pass) up to 64 rows."""
    import torch

    print(f"case: moe row-alpha E={E} I={I} gs={gs} M={M}", flush=True)
    rng = np.random.default_rng(900 + E + I + gs + M)
    H, k = 2048, 8
    mw = _row_alpha(synth.moe_weights(rng, E, H, I, gs))
    x = synth.normal_f16(rng, (M, H))
    ref_y, ref_i, _ = orc.moe_block(mw, x, prenorm=True, residual=True)
    dmw = _moe_dev(mw)
    dx = dev(x)
    outs = []
    for use_alpha in (True, False):
        w = dict(dmw) if use_alpha else {k2: v for k2, v in dmw.items() if not k2.endswith("_alpha")}
        y = torch.empty_like(dx)
        inds = torch.empty((M, k), dtype=torch.int32, device="cuda")
        _run(ctx, lambda: ctx.moe_block(w, dx, y, M, 3, inds, None))
        assert (host(inds) == ref_i).all()
        outs.append(host(y))
    rel, _ = assert_close(outs[0], ref_y, what="row-alpha fold vs oracle")
    assert rel < 5e-3
    rel2, _ = assert_close(outs[0], outs[1], what="row-alpha fold vs group scales")
    assert rel2 < 2e-3


@pytest.mark.parametrize("E,I,gs,M", [(256, 512, 128, 1), (256, 512, 128, 9),
                                      (256, 512, 128, 17), (64, 512, 64, 9),
                                      (64, 1536, 64, 9)])
def test_moe_block_maple_expert_shape(ctx, orc, E, I, gs, M):
    """Maple's real experts (MapleConfig.swift:5-23, 139-148): 256 experts top-8, intermediate
    512, group size 128 -- the down projection runs K = 512 (four 128-groups a row), one row
    through the same tile kernels as a verify pass.  I = 1536 has no tile kernel for its down
    projection and takes the GEMV (one row) or bucketed general path.  Routing bit-exact,
    outputs within tolerance of the oracle."""
    import torch

    print(f"case: moe maple shape E={E} I={I} gs={gs} M={M}", flush=True)
    rng = np.random.default_rng(700 + E + I + gs + M)
    H, k = 2048, 8
    mw = synth.moe_weights(rng, E, H, I, gs, top_k=k)
    x = synth.normal_f16(rng, (M, H))
    ref_y, ref_i, ref_s = orc.moe_block(mw, x, prenorm=True, residual=True)
    dmw = _moe_dev(mw)
    dx = dev(x)
    y = torch.empty_like(dx)
    inds = torch.empty((M, k), dtype=torch.int32, device="cuda")
    scores = torch.empty((M, k), dtype=torch.float32, device="cuda")
    _run(ctx, lambda: ctx.moe_block(dmw, dx, y, M, 3, inds, scores))
    assert (host(inds) == ref_i).all()
    assert np.allclose(host(scores), ref_s, rtol=1e-4, atol=1e-5)
    rel, _ = assert_close(host(y), ref_y, what=f"moe E={E} I={I} gs={gs} M={M}")
    assert rel < 5e-3


def test_moe_block_row_alpha_alignment(ctx):
    import torch

    from momij_amd._lib import MomijError

    rng = np.random.default_rng(5)
    mw = _moe_dev(_row_alpha(synth.moe_weights(rng, 16, 2048, 1024, 64)))
    buf = torch.empty(mw["down_alpha"].numel() + 8, dtype=torch.float16, device="cuda")
    mw["down_alpha"] = buf[1:1 + mw["down_alpha"].numel()]  # 2-byte offset
    dx = dev(synth.normal_f16(rng, (4, 2048)))
    with pytest.raises(MomijError):
        ctx.moe_block(mw, dx, torch.empty_like(dx), 4, 3)


@pytest.mark.parametrize("M", [9, 20, 40])
def test_moe_block_all_rows_on_each_expert(ctx, orc, M):
    """8 experts with top-8: every row picks every expert, so each expert's gather serves all M
    rows -- more than one pass of staged rows (9 per pass) for M = 20 and 40."""
    import torch

    print(f"case: moe all experts M={M}", flush=True)
    rng = np.random.default_rng(300 + M)
    E, H, I, gs, k = 8, 2048, 1024, 64, 8
    mw = synth.moe_weights(rng, E, H, I, gs, top_k=k)
    x = synth.normal_f16(rng, (M, H))
    ref_y, ref_i, ref_s = orc.moe_block(mw, x, prenorm=True, residual=True)
    dmw = _moe_dev(mw)
    dx = dev(x)
    y = torch.empty_like(dx)
    inds = torch.empty((M, k), dtype=torch.int32, device="cuda")
    scores = torch.empty((M, k), dtype=torch.float32, device="cuda")
    _run(ctx, lambda: ctx.moe_block(dmw, dx, y, M, 3, inds, scores))
    assert (host(inds) == ref_i).all()
    assert np.allclose(host(scores), ref_s, rtol=1e-4, atol=1e-5)
    rel, _ = assert_close(host(y), ref_y, what=f"moe all experts M={M}")
    assert rel < 5e-3


@pytest.mark.parametrize("E,I,M", [(64, 1024, 9), (64, 1024, 64), (128, 1024, 17), (40, 1024, 5),
                                   (64, 1024, 27)])
def test_moe_routing_ties(ctx, orc, E, I, M):
    """Router rows repeated in pairs, so every logit is tied with another expert's: the lower
    index has to rank first, exactly as in the oracle (ties reach the exact comparison rule of
    the top-k; E = 128 takes the several-experts-per-lane path)."""
    import torch

    print(f"case: moe routing ties E={E} I={I} M={M}", flush=True)
    rng = np.random.default_rng(400 + E + M)
    H, gs, k = 2048, 64, 8
    mw = synth.moe_weights(rng, E, H, I, gs, top_k=k)
    mw["router_w"][1::2] = mw["router_w"][0::2]
    x = synth.normal_f16(rng, (M, H))
    ref_y, ref_i, ref_s = orc.moe_block(mw, x, prenorm=True, residual=True)
    assert (ref_i[:, 0] % 2 == 0).all() and (ref_i[:, 1] == ref_i[:, 0] + 1).all()
    dmw = _moe_dev(mw)
    dx = dev(x)
    y = torch.empty_like(dx)
    inds = torch.empty((M, k), dtype=torch.int32, device="cuda")
    scores = torch.empty((M, k), dtype=torch.float32, device="cuda")
    _run(ctx, lambda: ctx.moe_block(dmw, dx, y, M, 3, inds, scores))
    assert (host(inds) == ref_i).all()
    assert np.allclose(host(scores), ref_s, rtol=1e-4, atol=1e-5)
    rel, _ = assert_close(host(y), ref_y, what=f"moe ties E={E} M={M}")
    assert rel < 5e-3


def test_abort_word_skips_work(ctx):
    import torch

    from momij_amd._lib import MomijError

    rng = np.random.default_rng(5)
    N, K, gs = 512, 2048, 64
    w, s, b = synth.qweight(rng, (1,), N, K, gs)
    x = synth.normal_f16(rng, (1, K))
    y = torch.full((1, N), 7.0, dtype=torch.float16, device="cuda")
    dx, dw, ds, db = dev(x), dev(w), dev(s), dev(b)
    di = dev(np.zeros(1, np.int32))
    torch.cuda.synchronize()
    ctx.set_abort(True)
    ctx.gather_qmm2(dx, dw, ds, db, di, y, 1, 1, K, N, gs)
    with pytest.raises(MomijError) as e:
        ctx.sync()
    assert e.value.status == 5
    ctx.set_abort(False)
    ctx.sync()
    assert (host(y) == 7.0).all()


def test_shape_guards(ctx):
    import torch

    from momij_amd._lib import MomijError

    t = torch.zeros(16, dtype=torch.int32, device="cuda")
    with pytest.raises(MomijError) as e:
        ctx.gather_qmm2(t, t, t, t, t, t, 1, 1, 1000, 64, 64)
    assert e.value.status == 3
    with pytest.raises(MomijError) as e:
        ctx.gather_qmm2(t, t, t, t, t, t, 1, 1, 1024, 64, 96)
    assert e.value.status == 3
