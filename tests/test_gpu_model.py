"""GPU parity of the whole verify step through the model (C ABI mj_model_* / mj_verify_*).

A 2-layer Maple-like model (same layer shapes as the full one, fewer experts and a small
vocabulary and window so the oracle can replay everything) is checked end to end:
  * prefill + chain verify against the oracle's own prefill + pass (argmax rows, accepted
    length, emitted tokens bit for bit; any differing argmax must be a numerical near-tie);
  * the M-row verify equals sequential single-token steps (MomijCoreTests M-row == sequential);
  * a 16-node draft tree, greedy acceptance along the longest matching path, and the KV
    compaction of the accepted path (the next pass sees the same cache as after a chain);
  * sampled verification over the exact head (bit-exact vs the oracle on the pass's logits);
  * graph replays equal eager passes, replay after replay;
  * per-layer teacher forcing: routing bit-exact and hidden states within tolerance.
"""
import numpy as np
import pytest

from tests.gpu_util import assert_close, host

pytestmark = pytest.mark.gpu

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
        xf = self.orc.rms_norm(h, self.w["fnorm"], self.cfg.eps)
        logits = self.orc.lm_head_logits(xf, self.w["head"])
        return logits

    def prefill(self, tokens, chunk=64):
        for i in range(0, len(tokens), chunk):
            t = tokens[i:i + chunk]
            self.rows(t, list(range(-1, len(t) - 1)))
            self.L += len(t)


def _argmax_match(orc, gpu_am, logits, what):
    idx, best, second = orc.argmax_rows(logits)
    for r, (g, o) in enumerate(zip(gpu_am, idx)):
        if g != o:
            near = (best[r] - logits[r, g]) <= 1e-3 * max(1.0, abs(best[r]))
            assert near, (what, r, g, o, best[r], logits[r, g])
            print(f"[{what}] row {r}: near-tie argmax {g} vs {o}", flush=True)
    return idx


def greedy_continuation(eng, y, n):
    """n greedy tokens after y by single-token steps, then rewind."""
    L0 = eng.offset
    out, t = [], y
    for _ in range(n):
        t = eng.step_chain_feeds([t])[0]
        out.append(t)
    eng.rewind(L0)
    return out


def test_prefill_and_chain_verify_vs_oracle(model, orc):
    eng, cfg = model["eng"], model["cfg"]
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, cfg.vocab, 100).tolist()
    eng.rewind(0)
    y = eng.prefill(prompt, chunk=64)
    om = OracleModel(orc, cfg, model["w"])
    om.prefill(prompt[:-1])
    lg = om.rows(prompt[-1:], [-1])
    om.L += 1
    assert _argmax_match(orc, [y], lg, "prefill")[0] == y
    cont = greedy_continuation(eng, y, 8)
    draft = cont[:5] + [int(t) for t in rng.integers(0, cfg.vocab, 3)]
    for i in range(5, 8):
        if draft[i] == cont[i]:
            draft[i] = (draft[i] + 1) % cfg.vocab
    L0 = eng.offset
    acc, toks = eng.verify_greedy(y, draft)
    assert acc == 5 and toks == cont[:6], (acc, toks, cont)
    assert eng.offset == L0 + 6
    # oracle: same pass on its own caches
    lg = om.rows([y] + draft, list(range(-1, 8)))
    am = _argmax_match(orc, [*cont[:5], cont[5]], lg[:6], "verify")
    oacc, _, oemit = orc.accept_greedy([y] + draft, None, am.tolist() + [0] * 3)
    assert oacc == acc and list(oemit) == toks


def test_mrow_verify_equals_sequential(model):
    eng = model["eng"]
    rng = np.random.default_rng(2)
    eng.rewind(0)
    y = eng.prefill(rng.integers(0, model["cfg"].vocab, 70).tolist())
    cont = greedy_continuation(eng, y, 9)
    acc, toks = eng.verify_greedy(y, cont[:8])
    assert acc == 8 and toks == cont[:9]


def test_tree_verify_and_compaction(model, orc):
    eng, cfg = model["eng"], model["cfg"]
    rng = np.random.default_rng(3)
    eng.rewind(0)
    prompt = rng.integers(0, cfg.vocab, 80).tolist()
    y = eng.prefill(prompt)
    L0 = eng.offset
    cont = greedy_continuation(eng, y, 6)
    # the path along first children (0-1-4-10-12-14-16) carries the target continuation
    toks = [int(t) for t in rng.integers(0, cfg.vocab, len(TREE16) - 1)]
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
    for r in range(1, len(TREE16)):  # no other node matches by accident
        if r not in path[1:5] and toks[r - 1] == cont[depth[r] - 1]:
            toks[r - 1] = (toks[r - 1] + 1) % cfg.vocab
    acc, out = eng.verify_greedy(y, toks, TREE16)
    assert acc == 4 and out == cont[:5], (acc, out, cont)
    assert eng.offset == L0 + 5
    # after compaction the cache equals the one a chain verify of the accepted path leaves
    k_tree = [host_kv(eng, l) for l in range(cfg.n_layers)]
    eng.rewind(L0)
    acc2, out2 = eng.verify_greedy(y, cont[:4] + [(cont[4] + 1) % cfg.vocab])
    assert acc2 == 4 and out2 == out
    k_chain = [host_kv(eng, l) for l in range(cfg.n_layers)]
    C = cfg.kv_capacity
    slots = [(L0 + i) % C for i in range(5)]
    for l in range(cfg.n_layers):
        assert_close(k_tree[l][:, :, slots], k_chain[l][:, :, slots], what=f"kv layer {l}")


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


def test_teacher_forced_layers(model, orc):
    """Each layer of a tree verify pass re-run by the oracle from the GPU's own input hidden
    states and KV cache: routing bit-exact (unless a numerical tie), outputs within tolerance."""
    import torch

    eng, cfg, w = model["eng"], model["cfg"], model["w"]
    rng = np.random.default_rng(6)
    eng.rewind(0)
    y = eng.prefill(rng.integers(0, cfg.vocab, 90).tolist())
    L0 = eng.offset
    kv0 = [host_kv(eng, l) for l in range(cfg.n_layers)]
    M = len(TREE16)
    hcap = torch.empty((cfg.n_layers + 1, 64, cfg.H), dtype=torch.float16, device="cuda")
    icap = torch.empty((cfg.n_layers, 64, cfg.top_k), dtype=torch.int32, device="cuda")
    draft = [int(t) for t in rng.integers(0, cfg.vocab, M - 1)]
    eng.set_capture(h=hcap, inds=icap)
    eng.verify_greedy(y, draft, TREE16)
    eng.set_capture()
    hc, ic = host(hcap), host(icap)
    par = np.array(TREE16, np.int32)
    for l in range(cfg.n_layers):
        lw = w["layers"][l]
        h_in = hc[l, :M]
        h_mid, _, _ = orc.attn_block(cfg.attn_cfg(), lw["attn"], h_in, kv0[l][0], kv0[l][1], L0,
                                     par)
        xn = orc.rms_norm(h_mid, lw["moe"]["norm_w"], cfg.eps)
        lg = orc.router_logits(lw["moe"]["router_w"], xn)
        ref_i, _ = orc.route_topk(lg, cfg.top_k)
        for r in range(M):
            if sorted(ic[l, r]) != sorted(ref_i[r]):
                srt = np.sort(lg[r])[::-1]
                gap = srt[cfg.top_k - 1] - srt[cfg.top_k]
                assert gap < 1e-3, (l, r, ic[l, r], ref_i[r], gap)
                print(f"layer {l} row {r}: routing near-tie gap {gap:.2e}", flush=True)
        h_out, _, _ = orc.moe_block(lw["moe"], h_mid, prenorm=True, residual=True)
        assert_close(hc[l + 1, :M], h_out, what=f"layer {l} h")
