"""GPU parity of the whole verify step through the model (C ABI mj_model_* / mj_verify_*).

A 2-layer Maple-like model (same layer shapes as the full one, fewer experts and a small
vocabulary and window so the oracle can replay everything) is checked end to end:
  * prefill + chain verify: every block of the pass re-run by the oracle from the inputs the
    device used (tests/teacher.py: routing exact up to ties inside the computed fp32 bound,
    head argmax exact up to the same kind of bound, floats within tolerance), the accepted
    length and tokens equal to the oracle's acceptance over its own argmax, and the oracle's
    free-running replay of the whole prompt within tolerance of the device's head input;
  * the M-row verify equals sequential single-token steps (MomijCoreTests M-row == sequential);
  * a 16-node draft tree, greedy acceptance along the longest matching path, and the KV
    compaction of the accepted path checked bit for bit against or_kv_commit over the rows the
    pass appended (and the next pass sees the same cache as after a chain);
  * sampled verification over the exact head (bit-exact vs the oracle on the pass's logits);
  * graph replays equal eager passes, replay after replay;
  * per-layer teacher forcing of a tree pass.
"""
import numpy as np
import pytest

from tests.gpu_util import assert_close, draft_q_values, host
from tests.teacher import capture_pass, check_head, check_layer

pytestmark = pytest.mark.gpu

# Drift check, not the parity bar: absolute bound of the free-running comparisons, where the
# oracle replays every pass on its own caches so both sides' rounding accumulates over the
# layers (8 fp16 ulps at magnitude 4).  Parity itself is the teacher-forced block checks
# (check_layer / check_head), which keep the 1e-2 absolute and 2e-2 relative-to-norm bar.
DRIFT_ABS = 3.2e-2

# 16 draft nodes, depth 6: 3 at depth 1, 2 under each, 2 under the first depth-2 node, then
# 1-chains (3+6+2+2+2+1); row 0 is the fed token.
TREE16 = [-1, 0, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 10, 11, 12, 13, 14]


def small_cfg():
    from momij_amd.engine import MapleLikeConfig

    return MapleLikeConfig(n_layers=2, window=48, kv_capacity=48 + 64, E=16, top_k=4,
                           vocab=2048)


@pytest.fixture(scope="module")
def model():
    import torch

    from momij_amd.engine import VerifyEngine, random_model
    from momij_amd.ops import Context

    ctx = Context(0)
    cfg = small_cfg()
    layers, embed, fnorm, head = random_model(cfg, seed=7)
    torch.cuda.synchronize()
    eng = VerifyEngine(ctx, cfg, layers, embed, fnorm, head)

    def h(t):
        a = t.detach().cpu().numpy()
        return a.view(np.uint32) if a.dtype == np.int32 else a

    host_w = dict(layers=[{"attn": {k: h(v) for k, v in lw["attn"].items()},
                           "moe": {k: (h(v) if hasattr(v, "detach") else v)
                                   for k, v in lw["moe"].items()}} for lw in layers],
                  embed=h(embed), fnorm=h(fnorm), head=h(head))
    yield dict(ctx=ctx, cfg=cfg, eng=eng, w=host_w)
    eng.close()
    ctx.close()


class OracleModel:
    """The oracle replaying the model on its own KV caches."""

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
                self.cfg.attn_cfg(), self.w["layers"][l], h, self.kc[l], self.vc[l], self.L,
                np.asarray(parents, np.int32))
        return self.orc.rms_norm(h, self.w["fnorm"], self.cfg.eps)  # the head input

    def prefill(self, tokens, chunk=64):
        for i in range(0, len(tokens), chunk):
            t = tokens[i:i + chunk]
            self.rows(t, list(range(-1, len(t) - 1)))
            self.L += len(t)


def greedy_continuation(eng, y, n):
    """n greedy tokens after y by single-token steps, then rewind."""
    L0 = eng.offset
    out, t = [], y
    for _ in range(n):
        t = eng.step_chain_feeds([t])[0]
        out.append(t)
    eng.rewind(L0)
    return out


def kv_all(eng):
    return [host_kv(eng, l) for l in range(eng.cfg.n_layers)]


def check_pass(orc, model, cap, M, kv0, L, parents, what):
    """Teacher-forced layers and head of a captured pass; returns the oracle argmax rows."""
    cfg, w = model["cfg"], model["w"]
    for l in range(cfg.n_layers):
        check_layer(orc, cfg, l, w["layers"][l], cap, M, (kv0[l][0], kv0[l][1]), L, parents)
    am, _ = check_head(orc, cap["head_in"][:M], cap_argmax(orc, cap, M), what,
                       w_head=w["head"])
    return am


def cap_argmax(orc, cap, M):
    """The device's argmax rows, read back from its captured logits (lowest id on ties)."""
    return orc.argmax_rows(cap["logits"][:M])[0]


def test_prefill_and_chain_verify_vs_oracle(model, orc):
    eng, cfg = model["eng"], model["cfg"]
    print("case: 2-layer model, 100-token prefill + K=8 chain verify", flush=True)
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, cfg.vocab, 100).tolist()
    eng.rewind(0)
    y, cap = capture_pass(eng, lambda: eng.prefill(prompt, chunk=64))
    Mlast = 100 - 64
    am, _ = check_head(orc, cap["head_in"][Mlast - 1:Mlast], [y], "prefill", w_head=model["w"]["head"])
    assert am[0] == y
    # the oracle's free-running replay of the whole prompt (its own caches) ends at the same
    # head input within tolerance
    om = OracleModel(orc, cfg, model["w"])
    om.prefill(prompt[:-1])
    xf = om.rows(prompt[-1:], [-1])
    om.L += 1
    assert_close(cap["head_in"][Mlast - 1:Mlast], xf, abs_tol=DRIFT_ABS,
                 what="prefill head input (free-running)")
    cont = greedy_continuation(eng, y, 8)
    draft = cont[:5] + [int(t) for t in rng.integers(0, cfg.vocab, 3)]
    for i in range(5, 8):
        if draft[i] == cont[i]:
            draft[i] = (draft[i] + 1) % cfg.vocab
    L0 = eng.offset
    kv0 = kv_all(eng)
    (acc, toks), cap = capture_pass(eng, lambda: eng.verify_greedy(y, draft))
    assert acc == 5 and toks == cont[:6], (acc, toks, cont)
    assert eng.offset == L0 + 6
    am = check_pass(orc, model, cap, 9, kv0, L0, list(range(-1, 8)), "verify")
    oacc, _, oemit = orc.accept_greedy([y] + draft, None, am)
    assert oacc == acc and list(oemit) == toks
    # and the oracle's own pass on its own caches stays within tolerance of the device's
    xf = om.rows([y] + draft, list(range(-1, 8)))
    assert_close(cap["head_in"][:9], xf, abs_tol=DRIFT_ABS,
                 what="verify head input (free-running)")


def test_mrow_verify_equals_sequential(model):
    eng = model["eng"]
    rng = np.random.default_rng(2)
    eng.rewind(0)
    y = eng.prefill(rng.integers(0, model["cfg"].vocab, 70).tolist())
    cont = greedy_continuation(eng, y, 9)
    acc, toks = eng.verify_greedy(y, cont[:8])
    assert acc == 8 and toks == cont[:9]


def test_chain_rows_bitwise_equal_one_row_steps(model):
    """Every row of a chain pass computes bit for bit what a one-row step at its position
    computes: head input and head logits compared as bits over a 9-row pass and nine one-row
    steps from the same cache.  Speculative verification is then lossless by construction
    (the reference checks the tokens: RealTextParityTests.swift:96-111)."""
    eng = model["eng"]
    rng = np.random.default_rng(21)
    eng.rewind(0)
    y = eng.prefill(rng.integers(0, model["cfg"].vocab, 75).tolist())
    L0 = eng.offset
    feeds = [y] + [int(t) for t in rng.integers(0, model["cfg"].vocab, 8)]
    head, logits = [], []
    for t in feeds:
        _, cap = capture_pass(eng, lambda: eng.step_chain_feeds([t]))
        head.append(cap["head_in"][0].copy())
        logits.append(cap["logits"][0].copy())
    eng.rewind(L0)
    _, cap = capture_pass(eng, lambda: eng.step_chain_feeds(feeds))
    M = len(feeds)
    assert (cap["head_in"][:M].view(np.uint16) == np.stack(head).view(np.uint16)).all()
    assert (cap["logits"][:M].view(np.uint32) == np.stack(logits).view(np.uint32)).all()


def test_tree_verify_and_compaction(model, orc):
    eng, cfg = model["eng"], model["cfg"]
    print("case: 2-layer model, 16-node tree verify + KV commit", flush=True)
    rng = np.random.default_rng(3)
    eng.rewind(0)
    prompt = rng.integers(0, cfg.vocab, 80).tolist()
    y = eng.prefill(prompt)
    L0 = eng.offset
    cont = greedy_continuation(eng, y, 6)
    toks, path = tree_tokens(cont, cfg.vocab, rng)
    kv0 = kv_all(eng)
    (acc, out), cap = capture_pass(eng, lambda: eng.verify_greedy(y, toks, TREE16))
    assert acc == 4 and out == cont[:5], (acc, out, cont)
    assert eng.offset == L0 + 5
    # acceptance over the oracle's argmax of the device's head input, on the tree
    am = check_pass(orc, model, cap, len(TREE16), kv0, L0, TREE16, "tree verify")
    oacc, opath, oemit = orc.accept_greedy([y] + toks, TREE16, am)
    assert oacc == acc and list(oemit) == out and list(opath) == path[:acc + 1]
    # the commit, bit for bit: the cache before the commit (the pass's appended rows at slots
    # (L0 + r) % C over the cache before the pass) run through or_kv_commit
    C = cfg.kv_capacity
    kv1 = kv_all(eng)
    for l in range(cfg.n_layers):
        pre = kv0[l].copy()
        for r in range(len(TREE16)):
            pre[:, :, (L0 + r) % C] = cap["kv_rows"][l, :, :, r]
        k_ref, v_ref = orc.kv_commit(pre[0], pre[1], L0, list(opath))
        assert (kv1[l][0].view(np.uint16) == k_ref.view(np.uint16)).all(), l
        assert (kv1[l][1].view(np.uint16) == v_ref.view(np.uint16)).all(), l
    # after compaction the cache equals the one a chain verify of the accepted path leaves
    k_tree = kv1
    eng.rewind(L0)
    acc2, out2 = eng.verify_greedy(y, cont[:4] + [(cont[4] + 1) % cfg.vocab])
    assert acc2 == 4 and out2 == out
    k_chain = kv_all(eng)
    slots = [(L0 + i) % C for i in range(5)]
    for l in range(cfg.n_layers):
        assert_close(k_tree[l][:, :, slots], k_chain[l][:, :, slots], what=f"kv layer {l}")


def tree_tokens(cont, vocab, rng):
    """Draft tokens of TREE16 whose first-child path carries the first four tokens of the
    continuation (no other node matches by accident); returns (tokens, first-child path)."""
    toks = [int(t) for t in rng.integers(0, vocab, len(TREE16) - 1)]
    depth = [0] * len(TREE16)
    for r in range(1, len(TREE16)):
        depth[r] = depth[TREE16[r]] + 1
    path = [0]
    while True:
        kids = [c for c in range(1, len(TREE16)) if TREE16[c] == path[-1]]
        if not kids:
            break
        path.append(kids[0])
    for d, r in enumerate(path[1:5]):
        toks[r - 1] = cont[d]
    for r in range(1, len(TREE16)):
        if r not in path[1:5] and toks[r - 1] == cont[depth[r] - 1]:
            toks[r - 1] = (toks[r - 1] + 1) % vocab
    return toks, path


def host_kv(eng, layer):
    """Layer cache [2][n_kv][C][128] copied to host through the C ABI."""
    k, _ = eng.kv(layer)
    cfg = eng.cfg
    n = 2 * cfg.n_kv_heads * cfg.kv_capacity * 128
    out = np.empty(n, np.float16)
    eng.ctx.check(eng.lib.mj_d2h(eng.ctx.h, out.ctypes.data, k, n * 2))
    return out.reshape(2, cfg.n_kv_heads, cfg.kv_capacity, 128)


@pytest.mark.parametrize("q_mode", [0, 1])
def test_sampled_verify_bit_exact(model, orc, q_mode):
    import torch

    eng, cfg = model["eng"], model["cfg"]
    rng = np.random.default_rng(4 + q_mode)
    eng.rewind(0)
    y = eng.prefill(rng.integers(0, cfg.vocab, 60).tolist())
    cont = greedy_continuation(eng, y, 8)
    L0 = eng.offset
    cap = torch.empty((64, cfg.vocab), dtype=torch.float32, device="cuda")
    hist = {}
    for trial in range(6):
        eng.rewind(L0)
        draft = cont[:4] + [int(t) for t in rng.integers(0, cfg.vocab, 4)]
        eng.set_capture(logits=cap)
        acc, tok = eng.verify_sampled(y, draft, 0.7, q_mode, seed=99, counter=trial)
        eng.set_capture()
        lg = host(cap)[:9]
        u = orc.verify_uniforms(99, trial, 9)
        ref = orc.accept_sampled(lg, np.array(draft, np.int32), 0.7, q_mode, u)
        assert (acc, tok) == ref, (trial, acc, tok, ref)
        assert eng.offset == L0 + acc + 1
        hist[acc] = hist.get(acc, 0) + 1
    print("sampled accepted histogram", hist, flush=True)


@pytest.mark.parametrize("q_mode", [0, 1])
def test_sampled_verify_ex_bit_exact(model, orc, q_mode):
    """mj_verify_sampled_ex (penalties with a history, nucleus) through the model: the eager
    pass's decision equals the oracle's on the pass's own logits, and a graph-replayed pass of
    the same inputs decides the same, replay after replay."""
    import torch

    eng, cfg = model["eng"], model["cfg"]
    rng = np.random.default_rng(40 + q_mode)
    eng.rewind(0)
    y = eng.prefill(rng.integers(0, cfg.vocab, 60).tolist())
    cont = greedy_continuation(eng, y, 8)
    L0 = eng.offset
    cap = torch.empty((64, cfg.vocab), dtype=torch.float32, device="cuda")
    opts = [dict(top_p=0.8, rep=1.2, pres=0.3, freq=0.2), dict(top_p=0.3),
            dict(rep=1.4, freq=0.5)]
    for trial in range(6):
        o = opts[trial % 3]
        hist = {int(t): int(c) for t, c in zip(rng.integers(0, cfg.vocab, 30),
                                                 rng.integers(1, 3, 30))}
        hist[int(cont[0])] = 2
        draft = cont[:4] + [int(t) for t in rng.integers(0, cfg.vocab, 4)]
        eng.rewind(L0)
        eng.set_capture(logits=cap)
        acc, tok = eng.verify_sampled_ex(y, draft, q_mode, 123, trial, 0.7, hist=hist, **o)
        eng.set_capture()
        lg = host(cap)[:9]
        u = orc.verify_uniforms(123, trial, 9)
        ht = np.array(list(hist.keys()), np.int32)
        hc = np.array([hist[t] for t in ht.tolist()], np.int32)
        ref = orc.accept_sampled_ex(lg, np.array(draft, np.int32), 0.7, q_mode, u,
                                    hist_tok=ht, hist_cnt=hc, **o)
        assert (acc, tok) == ref, (trial, o, acc, tok, ref)
        order = np.argsort(ht)
        for hh in (hist, (ht[order], hc[order])):  # graph replays: dict, then sorted arrays
            eng.rewind(L0)
            assert eng.verify_sampled_ex(y, draft, q_mode, 123, trial, 0.7, hist=hh,
                                         **o) == (acc, tok)


@pytest.mark.parametrize("ex", [False, True])
def test_sampled_verify_point_q_bit_exact(model, orc, ex):
    """mj_verify_sampled(_ex) with a host array q_point of draft densities: from a suffix index
    over the prompt (qAlong, the draftQ of verifyDraftSampled, SeedlessDecodeEngine.swift:
    1530-1559) on even trials, from the mixed generator (0, 1e-6, count ratios, q near p) on odd
    ones.  Decisions bit for bit against the oracle on the pass's own logits; a graph replay of
    the same inputs decides the same."""
    import torch

    from momij_amd.drafts import SuffixDraftIndex

    eng, cfg = model["eng"], model["cfg"]
    rng = np.random.default_rng(70 + ex)
    eng.rewind(0)
    prompt = rng.integers(0, cfg.vocab, 60).tolist()
    y = eng.prefill(prompt)
    cont = greedy_continuation(eng, y, 8)
    L0 = eng.offset
    cap = torch.empty((64, cfg.vocab), dtype=torch.float32, device="cuda")
    idx = SuffixDraftIndex(16)
    # the prompt and continuations that share its last five tokens and leave the greedy path
    # after 2, 1, 1 and 0 tokens: qAlong from that five-token context gives count ratios
    # (4/5, 1/2, 1/2, then 1 along the prompt's own path)
    idx.insert(prompt + [y] + cont)
    tail = prompt[-4:] + [y]
    for pre in (cont[:2], cont[:1], cont[:1], []):
        idx.insert(tail + pre + [int(t) for t in rng.integers(0, cfg.vocab, 3)])
    ctx_hist = [(prompt[-5] + 1) % cfg.vocab] + tail  # longest matched suffix: the five tokens
    o = dict(top_p=0.7, rep=1.2, pres=0.3, freq=0.2) if ex else {}
    hist = {int(t): 1 for t in prompt[-20:]} if ex else None
    seen = {}
    for trial in range(8):
        draft = cont[:5] + [int(t) for t in rng.integers(0, cfg.vocab, 3)]
        eng.rewind(L0)
        if trial % 2 == 0:
            qp = np.array(idx.q_along(ctx_hist, draft), np.float32)
            assert (qp[:3] < 1).all(), qp
        else:
            eng.set_capture(logits=cap)
            eng.verify_greedy(y, draft)  # this pass's logits, to place q near p
            eng.set_capture()
            eng.rewind(L0)
            qp = draft_q_values(rng, host(cap)[:8], draft, 0.7)
        eng.set_capture(logits=cap)
        if ex:
            acc, tok = eng.verify_sampled_ex(y, draft, 0, 321, trial, 0.7, hist=hist, q_point=qp,
                                             **o)
        else:
            acc, tok = eng.verify_sampled(y, draft, 0.7, 0, seed=321, counter=trial, q_point=qp)
        eng.set_capture()
        lg = host(cap)[:9]
        u = orc.verify_uniforms(321, trial, 9)
        if ex:
            ht = np.array(list(hist.keys()), np.int32)
            hc = np.array([hist[t] for t in ht.tolist()], np.int32)
            ref = orc.accept_sampled_ex(lg, np.array(draft, np.int32), 0.7, 0, u, q_point=qp,
                                        hist_tok=ht, hist_cnt=hc, **o)
        else:
            ref = orc.accept_sampled(lg, np.array(draft, np.int32), 0.7, 0, u, q_point=qp)
        assert (acc, tok) == ref, (trial, qp.tolist(), acc, tok, ref)
        assert eng.offset == L0 + acc + 1
        eng.rewind(L0)
        if ex:
            again = eng.verify_sampled_ex(y, draft, 0, 321, trial, 0.7, hist=hist, q_point=qp, **o)
        else:
            again = eng.verify_sampled(y, draft, 0.7, 0, seed=321, counter=trial, q_point=qp)
        assert again == (acc, tok), (trial, again, acc, tok)
        seen[acc] = seen.get(acc, 0) + 1
    print("sampled (point q) accepted histogram", ex, seen, flush=True)
    assert len(seen) >= 2


def test_graph_replays_equal_eager(model):
    eng, cfg = model["eng"], model["cfg"]
    rng = np.random.default_rng(5)
    eng.rewind(0)
    y = eng.prefill(rng.integers(0, cfg.vocab, 50).tolist())
    L0 = eng.offset
    draft = [int(t) for t in rng.integers(0, cfg.vocab, 8)]
    results = []
    for graphs in (False, True, True, True):
        eng.set_graphs(graphs)
        eng.rewind(L0)
        results.append(eng.verify_greedy(y, draft))
        eng.rewind(L0)
        eng.step_chain_feeds([y])  # eager-ish work between replays
    eng.set_graphs(True)
    assert all(r == results[0] for r in results), results


def test_fused_moe_wait_bound_reported(model):
    """The fused MoE launch's waits for its up product: one that runs out its bound is reported
    by the synchronising call (MJ_HIP_ERROR) and the report is cleared.  With no re-staging
    allowed, a pass either finds every down item's act rows complete at its first check, and
    then equals the normal pass, or fails with that report; the normal pass after it is
    unaffected."""
    from momij_amd._lib import MomijError

    eng, cfg, ctx = model["eng"], model["cfg"], model["ctx"]
    print("case: 9-row chain verify, fused MoE waits bounded to 0 polls", flush=True)
    rng = np.random.default_rng(8)
    eng.rewind(0)
    y = eng.prefill(rng.integers(0, cfg.vocab, 40).tolist())
    L0 = eng.offset
    draft = [int(t) for t in rng.integers(0, cfg.vocab, 8)]
    eng.set_graphs(False)
    faults = 0
    try:
        eng.rewind(L0)
        want = eng.verify_greedy(y, draft)
        ctx.set_wait_limit(0)
        for _ in range(4):
            eng.rewind(L0)
            try:
                got = eng.verify_greedy(y, draft)
            except MomijError as e:
                assert e.status == 6 and "fused MoE" in str(e), e
                faults += 1
            else:
                assert got == want
    finally:
        ctx.set_wait_limit(1 << 17)
        eng.set_graphs(True)
    eng.rewind(L0)
    assert eng.verify_greedy(y, draft) == want
    print("passes with a reported wait", faults, "of 4", flush=True)


def test_teacher_forced_layers(model, orc):
    """Each layer of a tree verify pass re-run by the oracle from the device's own block inputs
    and KV cache (a random draft: acceptance mostly 0, so every row is exercised)."""
    eng, cfg = model["eng"], model["cfg"]
    print("case: 2-layer model, teacher-forced random tree pass", flush=True)
    rng = np.random.default_rng(6)
    eng.rewind(0)
    y = eng.prefill(rng.integers(0, cfg.vocab, 90).tolist())
    L0 = eng.offset
    kv0 = kv_all(eng)
    M = len(TREE16)
    draft = [int(t) for t in rng.integers(0, cfg.vocab, M - 1)]
    (acc, out), cap = capture_pass(eng, lambda: eng.verify_greedy(y, draft, TREE16))
    am = check_pass(orc, model, cap, M, kv0, L0, TREE16, "random tree")
    oacc, _, oemit = orc.accept_greedy([y] + draft, TREE16, am)
    assert oacc == acc and list(oemit) == out
