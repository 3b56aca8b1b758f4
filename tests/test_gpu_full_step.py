"""GPU parity of the full verify step at its own size.

The 24-layer Maple-like 2-bit MoE of the benchmark (hidden 2048, 16 / 4 heads of 128, window
1024 with RoPE base 1e6 on 64 dims, 64 experts top-8 with intermediate 1024, gs 64, fp16
lm_head 151936 x 2048; random-init, seed 2024) with a 2048-token prompt prefilled, so the KV
ring (1088 slots) has wrapped.  Two passes as the benchmark runs them, and the pass after a
tree commit (verifyDraftChain, SeedlessDecodeEngine.swift:1574-1603):

  * a K = 8 chain draft whose first 5 tokens are the greedy continuation (accept 5 + bonus);
  * the 16-node depth-6 draft tree whose first-child path carries 4 continuation tokens;
  * a K = 8 chain pass from the committed tree path.

Every pass is captured at each block boundary (mj_model_set_capture_ex) and checked against
the oracle from the inputs the device used (tests/teacher.py): the routing of all 24 layers
through the router logits' fp32 bound and the exact top-k rule; layers 0, 8, 16 and 23 re-run
whole (attention from the device's KV cache, appended K/V rows, MoE output); the head argmax of
every row against the oracle's logits of the same head input; the accepted length and tokens
against the oracle's acceptance over its own argmax; the tree commit bit for bit against
or_kv_commit over the rows the pass appended.
"""
import numpy as np
import pytest

from tests.gpu_util import host
from tests.teacher import capture_pass, check_head, check_layer, check_routing, host_layer

pytestmark = pytest.mark.gpu

LAYERS = (0, 8, 16, 23)
TREE16 = [-1, 0, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 10, 11, 12, 13, 14]


def _kv(eng, layer):
    k, _ = eng.kv(layer)
    cfg = eng.cfg
    n = 2 * cfg.n_kv_heads * cfg.kv_capacity * 128
    out = np.empty(n, np.float16)
    eng.ctx.check(eng.lib.mj_d2h(eng.ctx.h, out.ctypes.data, k, n * 2))
    return out.reshape(2, cfg.n_kv_heads, cfg.kv_capacity, 128)


def _greedy(eng, y, n):
    L0 = eng.offset
    out, t = [], y
    for _ in range(n):
        t = eng.step_chain_feeds([t])[0]
        out.append(t)
    eng.rewind(L0)
    return out


@pytest.fixture(scope="module")
def full():
    import torch

    from momij_amd.engine import MapleLikeConfig, VerifyEngine, random_model
    from momij_amd.ops import Context

    print("case: full step, 24 layers, E=64 top-8, V=151936, 2048-token prompt", flush=True)
    ctx = Context(0)
    cfg = MapleLikeConfig()
    layers, embed, fnorm, head = random_model(cfg, seed=2024)
    torch.cuda.synchronize()
    eng = VerifyEngine(ctx, cfg, layers, embed, fnorm, head)
    rng = np.random.default_rng(2024)
    prompt = rng.integers(0, cfg.vocab, 2048).tolist()
    y = eng.prefill(prompt, chunk=64)
    assert eng.offset == 2048
    w = dict(layers={l: host_layer(layers[l]) for l in LAYERS},
             routers=[host(layers[l]["moe"]["router_w"]) for l in range(cfg.n_layers)],
             head=host(head))
    yield dict(ctx=ctx, cfg=cfg, eng=eng, y=y, rng=rng, w=w, cont=_greedy(eng, y, 8),
               prompt=prompt)
    eng.close()
    ctx.close()


def _check(orc, f, cap, M, kv0, L, parents, what):
    cfg, w = f["cfg"], f["w"]
    for l in range(cfg.n_layers):
        check_routing(orc, w["routers"][l], cap["moe_in"][l, :M], cap["router_logits"][l, :M],
                      cap["inds"][l, :M], cfg.top_k, f"{what} layer {l}")
    for l in LAYERS:
        check_layer(orc, cfg, l, w["layers"][l], cap, M, (kv0[l][0], kv0[l][1]), L, parents)
    gpu_am = orc.argmax_rows(cap["logits"][:M])[0]
    am, _ = check_head(orc, cap["head_in"][:M], gpu_am, what, w_head=w["head"])
    return am


def test_full_chain_k8(full, orc):
    eng, cfg, y, cont = full["eng"], full["cfg"], full["y"], full["cont"]
    print("case: full step, K=8 chain verify", flush=True)
    rng = np.random.default_rng(11)
    draft = cont[:5] + [int(t) for t in rng.integers(0, cfg.vocab, 3)]
    for i in range(5, 8):
        if draft[i] == cont[i]:
            draft[i] = (draft[i] + 1) % cfg.vocab
    L0 = eng.offset
    kv0 = {l: _kv(eng, l) for l in LAYERS}
    (acc, toks), cap = capture_pass(eng, lambda: eng.verify_greedy(y, draft))
    eng.rewind(L0)
    assert acc == 5 and toks == cont[:6], (acc, toks, cont)
    am = _check(orc, full, cap, 9, kv0, L0, list(range(-1, 8)), "chain")
    oacc, _, oemit = orc.accept_greedy([y] + draft, None, am)
    assert oacc == acc and list(oemit) == toks


def test_full_chain_rows_bitwise_equal_one_row_steps(full):
    """At full size: the 9 rows of a K = 8 chain pass give bit for bit the head input and
    logits of nine one-row steps at the same positions (chain evals == sequential,
    RealTextParityTests.swift:96-111, here on the bits rather than the tokens)."""
    eng, cfg, y, cont = full["eng"], full["cfg"], full["y"], full["cont"]
    print("case: full step, chain rows == one-row steps, bitwise", flush=True)
    L0 = eng.offset
    feeds = [y] + cont[:4] + [int(t) for t in np.random.default_rng(13).integers(0, cfg.vocab, 4)]
    head, logits = [], []
    for t in feeds:
        _, cap = capture_pass(eng, lambda: eng.step_chain_feeds([t]))
        head.append(cap["head_in"][0].copy())
        logits.append(cap["logits"][0].copy())
    eng.rewind(L0)
    _, cap = capture_pass(eng, lambda: eng.step_chain_feeds(feeds))
    eng.rewind(L0)
    M = len(feeds)
    assert (cap["head_in"][:M].view(np.uint16) == np.stack(head).view(np.uint16)).all()
    assert (cap["logits"][:M].view(np.uint32) == np.stack(logits).view(np.uint32)).all()


def test_full_tree16_commit_and_next_pass(full, orc):
    eng, cfg, y, cont = full["eng"], full["cfg"], full["y"], full["cont"]
    print("case: full step, 16-node tree verify, commit, next chain pass", flush=True)
    rng = np.random.default_rng(12)
    toks = [int(t) for t in rng.integers(0, cfg.vocab, len(TREE16) - 1)]
    depth = [0] * len(TREE16)
    for r in range(1, len(TREE16)):
        depth[r] = depth[TREE16[r]] + 1
    path = [0, 1, 4, 10, 12]  # first children down to depth 4
    for d, r in enumerate(path[1:]):
        toks[r - 1] = cont[d]
    for r in range(1, len(TREE16)):
        if r not in path and toks[r - 1] == cont[depth[r] - 1]:
            toks[r - 1] = (toks[r - 1] + 1) % cfg.vocab
    L0 = eng.offset
    C = cfg.kv_capacity
    kv0 = [_kv(eng, l) for l in range(cfg.n_layers)]
    (acc, out), cap = capture_pass(eng, lambda: eng.verify_greedy(y, toks, TREE16))
    assert acc == 4 and out == cont[:5], (acc, out, cont)
    assert eng.offset == L0 + 5
    am = _check(orc, full, cap, len(TREE16), kv0, L0, TREE16, "tree")
    oacc, opath, oemit = orc.accept_greedy([y] + toks, TREE16, am)
    assert oacc == acc and list(oemit) == out and list(opath) == path
    # the commit of every layer, bit for bit
    kv1 = [_kv(eng, l) for l in range(cfg.n_layers)]
    for l in range(cfg.n_layers):
        pre = kv0[l].copy()
        for r in range(len(TREE16)):
            pre[:, :, (L0 + r) % C] = cap["kv_rows"][l, :, :, r]
        k_ref, v_ref = orc.kv_commit(pre[0], pre[1], L0, path)
        assert (kv1[l][0].view(np.uint16) == k_ref.view(np.uint16)).all(), l
        assert (kv1[l][1].view(np.uint16) == v_ref.view(np.uint16)).all(), l
    # the next chain pass reads the committed cache; the oracle re-runs it from that cache
    y2 = out[-1]
    cont2 = _greedy(eng, y2, 8)
    draft = cont2[:3] + [int(t) for t in rng.integers(0, cfg.vocab, 5)]
    for i in range(3, 8):
        if draft[i] == cont2[i]:
            draft[i] = (draft[i] + 1) % cfg.vocab
    L1 = eng.offset
    (acc2, toks2), cap = capture_pass(eng, lambda: eng.verify_greedy(y2, draft))
    assert acc2 == 3 and toks2 == cont2[:4], (acc2, toks2, cont2)
    am = _check(orc, full, cap, 9, {l: kv1[l] for l in LAYERS}, L1, list(range(-1, 8)),
                "after commit")
    oacc, _, oemit = orc.accept_greedy([y2] + draft, None, am)
    assert oacc == acc2 and list(oemit) == toks2
    eng.rewind(L0)


def test_abort_from_another_thread_during_prefill(full):
    """stopBuf from a cancelling thread (SeedlessMetal.swift:60, 69-70): a second host thread
    sets the abort word while mj_prefill of the 2048-token prompt runs (32 chunks of 64 rows).
    The call returns MJ_ABORTED with no HIP error and the offset at a whole chunk before the
    end; every kernel of the pass in flight exits normally (the next calls succeed); after the
    word is cleared a prefill from the start gives the same next token and greedy continuation
    as the uninterrupted one."""
    import threading
    import time

    from momij_amd._lib import MomijError

    ctx, eng = full["ctx"], full["eng"]
    eng.rewind(0)
    t0 = time.perf_counter()
    y = eng.prefill(full["prompt"], chunk=64)
    t_full = time.perf_counter() - t0
    assert y == full["y"]
    eng.rewind(0)
    delay = max(0.2 * t_full, 0.002)
    timer = threading.Timer(delay, lambda: ctx.set_abort(True))
    timer.start()
    try:
        with pytest.raises(MomijError) as e:
            eng.prefill(full["prompt"], chunk=64)
    finally:
        timer.join()
    print(f"prefill {t_full * 1e3:.1f} ms, abort after {delay * 1e3:.1f} ms: offset "
          f"{eng.offset}", flush=True)
    assert e.value.status == 5, e.value
    assert eng.offset % 64 == 0 and eng.offset < 2048
    # still set: the next call queues nothing and reports the abort
    with pytest.raises(MomijError) as e2:
        eng.step_chain_feeds([y])
    assert e2.value.status == 5
    ctx.set_abort(False)
    ctx.sync()
    eng.rewind(0)
    assert eng.prefill(full["prompt"], chunk=64) == full["y"]
    assert eng.offset == 2048
    assert _greedy(eng, full["y"], 3) == full["cont"][:3]
