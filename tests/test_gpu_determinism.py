"""Allocation-churn determinism (ContaminationProbeTests.swift:43-131; the reference once read
past an index buffer, docs/findings-evprtr-serve-default-fix-2026-09-13.md:60-92, so results
depended on what the heap held next to it).

Two contexts and two models over the same weights -- model B's weights are copies at other
addresses, made after freed buffers full of NaN were handed back to the allocator, and the
contexts' scratch arenas are grown to different sizes by op-level calls in between -- run the
same prefill (ring-wrapping the window), chain verify, 16-node tree verify and a chain after
the tree commit.  Every block boundary the capture exposes (layer inputs, routing, attention
and MoE inputs, router logits, head input, head logits, the pass's K/V rows), the accepted
tokens and the whole KV cache must be identical bit for bit; graph-replayed passes of the same
inputs agree with the eager ones.  Any read of memory a kernel does not own would show up as a
difference between the two allocation histories.
"""
import numpy as np
import pytest

from tests.gpu_util import host

pytestmark = pytest.mark.gpu

TREE16 = [-1, 0, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 10, 11, 12, 13, 14]


def _nan_churn(torch, sizes):
    """Allocate, fill with NaN bit patterns, free, and hand the memory back to the driver."""
    bufs = [torch.full((n,), float("nan"), dtype=torch.float16, device="cuda") for n in sizes]
    torch.cuda.synchronize()
    del bufs
    torch.cuda.empty_cache()


def _clone_tree(obj):
    import torch

    if isinstance(obj, torch.Tensor):
        return obj.clone()
    if isinstance(obj, dict):
        return {k: _clone_tree(v) for k, v in obj.items()}
    if isinstance(obj, list):
        return [_clone_tree(v) for v in obj]
    return obj


def _kv_all(eng):
    out = []
    cfg = eng.cfg
    n = 2 * cfg.n_kv_heads * cfg.kv_capacity * 128
    for l in range(cfg.n_layers):
        k, _ = eng.kv(l)
        buf = np.empty(n, np.uint16)
        eng.ctx.check(eng.lib.mj_d2h(eng.ctx.h, buf.ctypes.data, k, n * 2))
        out.append(buf)
    return np.concatenate(out)


def _bits(t):
    a = host(t)
    return a.view(np.uint16) if a.dtype == np.float16 else a.view(np.uint32)


def _run(eng, prompt, drafts, capture):
    """Eager passes with every boundary captured; returns the records and the final cache."""
    rec = []
    eng.set_graphs(False)
    eng.rewind(0)
    y = eng.prefill(prompt)
    rec.append(("prefill", y))
    for name, draft, parents in drafts:
        for b in capture.values():
            b.zero_()
        eng.set_capture_ex(**capture)
        acc, toks = eng.verify_greedy(y, draft, parents)
        eng.set_capture_ex()
        rec.append((name, acc, tuple(toks), eng.offset))
        for k in sorted(capture):
            rec.append((name, k, _bits(capture[k]).tobytes()))
        y = toks[-1]
    return rec, _kv_all(eng)


def _run_graphs(eng, prompt, drafts):
    eng.set_graphs(True)
    eng.rewind(0)
    y = eng.prefill(prompt)
    out = [y]
    for _, draft, parents in drafts:
        acc, toks = eng.verify_greedy(y, draft, parents)
        out.append((acc, tuple(toks), eng.offset))
        y = toks[-1]
    return out, _kv_all(eng)


def test_allocation_churn_determinism():
    import torch

    from momij_amd.engine import MapleLikeConfig, VerifyEngine, random_model
    from momij_amd.ops import Context

    # the real layer shapes (64 experts top-8, intermediate 1024, 16/4 heads), three layers, a
    # window of 128 in a ring of 192 slots, a vocabulary of 8192
    cfg = MapleLikeConfig(n_layers=3, window=128, kv_capacity=128 + 64, vocab=8192)
    rng = np.random.default_rng(17)
    prompt = rng.integers(0, cfg.vocab, 300).tolist()

    ctx_a = Context(0)
    layers, embed, fnorm, head = random_model(cfg, seed=23)
    torch.cuda.synchronize()
    eng_a = VerifyEngine(ctx_a, cfg, layers, embed, fnorm, head)

    _nan_churn(torch, [1 << 20, 3 << 22, 5 << 18, 1 << 24])
    spacer = torch.full((7 << 20,), float("nan"), dtype=torch.float16, device="cuda")
    w_b = _clone_tree((layers, embed, fnorm, head))
    ctx_b = Context(0)
    # grow B's op-level scratch arena through a large MoE block call (A's stays small)
    from momij_amd import synth

    mw = synth.moe_weights(np.random.default_rng(1), 64, cfg.H, cfg.I, cfg.gs, top_k=8)
    dmw = {k: (torch.from_numpy(v.view(np.int32) if v.dtype == np.uint32 else v).cuda()
               if isinstance(v, np.ndarray) else v) for k, v in mw.items()}
    xm = torch.randn((40, cfg.H), device="cuda").half()
    ym = torch.empty_like(xm)
    im = torch.empty((40, 8), dtype=torch.int32, device="cuda")
    sm = torch.empty((40, 8), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx_b.moe_block(dmw, xm, ym, 40, 3, im, sm)
    ctx_b.sync()
    _nan_churn(torch, [3 << 21, 1 << 23])
    eng_b = VerifyEngine(ctx_b, cfg, *w_b)
    del spacer

    cont_draft = [int(t) for t in rng.integers(0, cfg.vocab, 8)]
    tree_draft = [int(t) for t in rng.integers(0, cfg.vocab, 16)]
    drafts = [("chain", cont_draft, None), ("tree", tree_draft, TREE16),
              ("chain2", cont_draft[::-1], None)]
    # the greedy continuation as the first chain's leading drafts, so something is accepted
    eng_a.set_graphs(False)
    eng_a.rewind(0)
    y0 = eng_a.prefill(prompt)
    t = y0
    for i in range(4):
        t = eng_a.step_chain_feeds([t])[0]
        cont_draft[i] = t
    drafts[0] = ("chain", cont_draft, None)

    cap_a = eng_a.capture_buffers()
    cap_b = eng_b.capture_buffers()
    rec_a, kv_a = _run(eng_a, prompt, drafts, cap_a)
    rec_b, kv_b = _run(eng_b, prompt, drafts, cap_b)
    print("passes", [r for r in rec_a if len(r) == 4], flush=True)
    assert [r for r in rec_a if len(r) == 4][0][1] >= 4  # the chain accepted its greedy prefix
    for ra, rb in zip(rec_a, rec_b):
        assert ra == rb, (ra[:2], "differs between the two allocation histories")
    assert (kv_a == kv_b).all()

    # interleaved graph replays: A, B, A again
    ga, gkv_a = _run_graphs(eng_a, prompt, drafts)
    gb, gkv_b = _run_graphs(eng_b, prompt, drafts)
    ga2, gkv_a2 = _run_graphs(eng_a, prompt, drafts)
    eager = [rec_a[0][1]] + [(r[1], r[2], r[3]) for r in rec_a if len(r) == 4]
    assert ga == gb == ga2 == eager, (ga, gb, ga2, eager)
    assert (gkv_a == kv_a).all() and (gkv_b == kv_a).all() and (gkv_a2 == kv_a).all()
    eng_a.close()
    eng_b.close()
    ctx_a.close()
    ctx_b.close()
