"""GPU parity: exact fp16 lm_head verify (argmax, logits) and greedy / sampled acceptance.

Config 3: lm_head fp16 [151936 x 2048] ~ N(0, 0.02), hidden fp16 [8 x 2048] ~ N(0, 1); drafts:
the first 5 equal the target argmax, the rest random; sampled acceptance at T = 0.7 with
Philox uniforms and a uniform (or point-mass) draft q.  Argmax ids, accepted lengths and
emitted tokens are compared bit for bit; for the argmax the oracle's top-1/top-2 margin is
checked to exceed the fp32 accumulation error bound, so the match is not luck.
"""
import numpy as np
import pytest

from tests.gpu_util import assert_close, dev, draft_q_values, host

pytestmark = pytest.mark.gpu

V, K, M = 151936, 2048, 8


@pytest.fixture(scope="module")
def ctx():
    from momij_amd.ops import Context

    c = Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def head_case(ctx, orc):
    import torch

    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    w = (torch.randn((V, K), generator=gen, device="cuda") * 0.02).half()
    x = torch.randn((M, K), generator=gen, device="cuda").half()
    logits = torch.empty((M, V), dtype=torch.float32, device="cuda")
    am = torch.empty(M, dtype=torch.int32, device="cuda")
    mx = torch.empty(M, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.lm_head_verify(x, w, M, K, V, am, mx, logits)
    ctx.sync()
    wh, xh = host(w), host(x)
    ref = orc.lm_head_logits(xh, wh)
    return dict(w=w, x=x, logits=logits, am=host(am), mx=host(mx), ref=ref, wh=wh, xh=xh)


def test_lm_head_config3(head_case, orc):
    c = head_case
    ref = c["ref"]
    idx, best, second = orc.argmax_rows(ref)
    # rounding bound of an fp32 sum of 2048 products (8 sqrt(K) eps sum|w x|) at the top-2
    top2 = np.argsort(-ref, axis=1)[:, :2]
    absdot = np.array([[np.abs(c["wh"][v].astype(np.float64) * c["xh"][m]).sum()
                        for v in top2[m]] for m in range(M)])
    bound = 8 * np.sqrt(K) * 2.0 ** -24 * absdot.max(1)
    print("margins", (best - second).tolist(), "bound", bound.tolist(), flush=True)
    assert ((best - second) > bound).all()
    assert (c["am"] == idx).all(), (c["am"], idx)
    got = host(c["logits"])
    assert_close(got, ref, rel_tol=1e-5, abs_tol=1e-4, what="cfg3 logits")
    assert (c["mx"] == got.max(1)).all()


# log-sum-exp bar: the fp32 running sums see at most a few hundred roundings (per-lane strip
# sums, then lane, wave and block merges), 2e-5 relative in the worst case, i.e. 2e-5 absolute
# in the logarithm; plus the logits' own rounding (1e-6 relative, |logit / T| < 10)
LSE_TOL = 3e-5


def _lse64(logits, T, banned=()):
    z = logits.astype(np.float64) / T
    if len(banned):
        z[:, list(banned)] = -np.inf
    mx = z.max(1, keepdims=True)
    return (mx[:, 0] + np.log(np.exp(z - mx).sum(1)))


def test_lm_head_logsumexp_config3(ctx, head_case):
    """Per-row ln sum exp(logit / T) from the head pass (LogitsProcessor.probabilities'
    normaliser, LogitsProcessor.swift:168-189) at T = 0.7, with the two largest ids of every
    row banned so that the banned filter moves the result by ~1e-3 (well past the tolerance).
    Checked against a float64 log-sum-exp of the oracle's logits and of the kernel's own;
    argmax and row max must not change when the sum is requested."""
    import torch

    c = head_case
    T = 0.7
    ref = c["ref"]
    top2 = np.argsort(-ref, axis=1)[:, :2]
    ban = sorted(set(top2.reshape(-1).tolist()))
    assert len(ban) <= 64
    dban = torch.tensor(ban, dtype=torch.int32, device="cuda")
    am = torch.empty(M, dtype=torch.int32, device="cuda")
    mx = torch.empty(M, dtype=torch.float32, device="cuda")
    lse = torch.empty(M, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.lm_head_verify(c["x"], c["w"], M, K, V, am, mx, None, dban, len(ban), T, lse)
    ctx.sync()
    got = host(lse).astype(np.float64)
    want = _lse64(ref, T, ban)
    own = _lse64(host(c["logits"]), T, ban)
    print("lse", got.tolist(), "err", np.abs(got - want).max(), flush=True)
    assert np.abs(got - want).max() < LSE_TOL
    assert np.abs(got - own).max() < LSE_TOL
    unbanned = _lse64(ref, T)
    assert np.abs(unbanned - want).min() > 10 * LSE_TOL  # the banned ids matter
    keep = np.ones(V, bool)
    keep[ban] = False
    ids = np.where(keep)[0]
    sub = ref[:, keep]
    assert (host(am) == ids[sub.argmax(1)]).all()
    assert (host(mx) == host(c["logits"])[:, keep].max(1)).all()


def test_lm_head_logsumexp_needs_temperature(ctx):
    import torch

    from momij_amd.ops import MomijError

    w = torch.zeros((256, 256), dtype=torch.float16, device="cuda")
    x = torch.zeros((1, 256), dtype=torch.float16, device="cuda")
    am = torch.empty(1, dtype=torch.int32, device="cuda")
    lse = torch.empty(1, dtype=torch.float32, device="cuda")
    with pytest.raises(MomijError):
        ctx.lm_head_verify(x, w, 1, 256, 256, am, temperature=0.0, out_lse=lse)
    ctx.lm_head_verify(x, w, 1, 256, 256, am, temperature=2.0, out_lse=lse)
    ctx.sync()
    # all logits 0: ln 256
    assert abs(float(host(lse)[0]) - np.log(256.0)) < 1e-5


def test_lm_head_banned_and_ties(ctx):
    import torch

    Vs, Ks, Ms = 4096, 256, 3
    w = torch.zeros((Vs, Ks), dtype=torch.float16, device="cuda")
    x = torch.ones((Ms, Ks), dtype=torch.float16, device="cuda")
    w[[17, 900, 901, 4000], 0] = 1.0  # four tied maxima
    am = torch.empty(Ms, dtype=torch.int32, device="cuda")
    banned = torch.tensor([17, 901], dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    ctx.lm_head_verify(x, w, Ms, Ks, Vs, am)
    ctx.sync()
    assert host(am).tolist() == [17, 17, 17]
    ctx.lm_head_verify(x, w, Ms, Ks, Vs, am, banned=banned, n_banned=2)
    ctx.sync()
    assert host(am).tolist() == [900, 900, 900]


@pytest.mark.parametrize("Ms", [17, 36, 64])
def test_lm_head_many_rows(ctx, orc, Ms):
    """17 verify rows (a 16-node tree + root) use the two-tile path; 36 and 64 rows (prefill
    chunks) go through in groups of 32."""
    import torch

    rng = np.random.default_rng(9 + Ms)
    Vs = 20000
    w = (rng.standard_normal((Vs, K)) * 0.02).astype(np.float16)
    x = rng.standard_normal((Ms, K)).astype(np.float16)
    am = torch.empty(Ms, dtype=torch.int32, device="cuda")
    lg = torch.empty((Ms, Vs), dtype=torch.float32, device="cuda")
    lse = torch.empty(Ms, dtype=torch.float32, device="cuda")
    dw, dx = dev(w), dev(x)
    torch.cuda.synchronize()
    ctx.lm_head_verify(dx, dw, Ms, K, Vs, am, None, lg, temperature=1.3, out_lse=lse)
    ctx.sync()
    ref = orc.lm_head_logits(x, w)
    idx, _, _ = orc.argmax_rows(ref)
    assert (host(am) == idx).all()
    want = _lse64(ref, 1.3)
    assert np.abs(host(lse) - want).max() < LSE_TOL
    assert_close(host(lg), ref, rel_tol=1e-5, abs_tol=1e-4, what=f"{Ms} rows")


def test_accept_greedy_config3(ctx, head_case, orc):
    import torch

    am = head_case["am"]
    rng = np.random.default_rng(11)
    draft = am[:M - 1].copy()
    for i in range(5, M - 1):
        while draft[i] == am[i]:
            draft[i] = rng.integers(0, V)
    tokens = np.concatenate([[123], draft]).astype(np.int32)
    out = torch.empty(2 + 2 * M, dtype=torch.int32, device="cuda")
    dt, da = dev(tokens), dev(am.astype(np.int32))
    torch.cuda.synchronize()
    ctx.accept_greedy(dt, None, da, M, out)
    ctx.sync()
    o = host(out)
    acc, path, emit = orc.accept_greedy(tokens, None, am)
    assert acc == 5 and o[0] == acc and o[1] == am[acc]
    assert list(o[2:3 + acc]) == list(path) and list(o[2 + M:3 + M + acc]) == list(emit)


def test_accept_greedy_trees(ctx, orc):
    import torch

    rng = np.random.default_rng(12)
    for trial in range(30):
        n = int(rng.integers(1, 20))
        parents = [-1] + [int(rng.integers(0, r)) for r in range(1, n)]
        argmax = rng.integers(0, 5, n).astype(np.int32)
        tokens = rng.integers(0, 5, n).astype(np.int32)
        out = torch.empty(2 + 2 * n, dtype=torch.int32, device="cuda")
        dt, da = dev(tokens), dev(argmax)
        torch.cuda.synchronize()
        ctx.accept_greedy(dt, parents, da, n, out)
        ctx.sync()
        o = host(out)
        acc, path, emit = orc.accept_greedy(tokens, parents, argmax)
        assert o[0] == acc and list(o[2:3 + acc]) == list(path), trial
        assert list(o[2 + n:3 + n + acc]) == list(emit), trial


@pytest.mark.parametrize("q_mode,temp", [(1, 0.7), (0, 0.7), (0, 0.1)])
def test_accept_sampled_bit_exact(ctx, head_case, orc, q_mode, temp):
    """Device rejection sampling == the oracle's canonical rule on the same logits and Philox
    uniforms: accepted count and emitted token, for many counters.  Uniform q at T = 0.7 is the
    config-3 case; a point-mass q (the reference default) accepts only where p is large, so it
    also runs at T = 0.1."""
    import torch

    am = head_case["am"]
    logits = head_case["logits"]
    lh = host(logits)
    rng = np.random.default_rng(13 + q_mode)
    out = torch.empty(2, dtype=torch.int32, device="cuda")
    seen = {}
    for trial in range(24):
        draft = am[:M - 1].copy()
        for i in range(5, M - 1):
            draft[i] = rng.integers(0, V)
        if trial % 3 == 0:
            draft[int(rng.integers(0, 5))] = rng.integers(0, V)  # early reject
        dd = dev(draft.astype(np.int32))
        torch.cuda.synchronize()
        ctx.accept_sampled(logits, M, V, dd, temp, q_mode, 2024, trial, out)
        ctx.sync()
        got = tuple(int(v) for v in host(out))
        u = orc.verify_uniforms(2024, trial, M)
        ref = orc.accept_sampled(lh, draft, temp, q_mode, u)
        assert got == ref, (trial, got, ref)
        seen[ref[0]] = seen.get(ref[0], 0) + 1
    print("accepted-count histogram", seen, flush=True)
    if temp < 0.5 or q_mode == 1:
        assert len(seen) >= 2  # both early rejects and long accepts were exercised


@pytest.mark.parametrize("opts", [
    dict(top_p=0.9),
    dict(top_p=0.5, rep=1.3, pres=0.4, freq=0.25),
    dict(rep=1.5, pres=0.8, freq=0.6),
    dict(top_p=0.02, rep=0.8),
])
def test_accept_sampled_ex_bit_exact(ctx, head_case, orc, opts):
    """LogitsProcessor options over the full 151936-token head: penalties on every row (the
    history plus the drafts accepted before it) and samplePrepared's nucleus for the bonus and
    for a residual without mass (the cut found by a radix selection over the row), bit for bit
    against the oracle's canonical rule on the same logits and uniforms; the caller's logits
    stay as they were."""
    import torch

    am = head_case["am"]
    logits = head_case["logits"]
    lh = host(logits)
    rng = np.random.default_rng(31)
    out = torch.empty(2, dtype=torch.int32, device="cuda")
    seen = {}
    for trial in range(8):
        draft = am[:M - 1].copy()
        for i in range(6, M - 1):
            draft[i] = rng.integers(0, V)
        if trial % 4 == 0:
            draft[int(rng.integers(0, 6))] = rng.integers(0, V)  # early reject
        hist = {int(t): int(c) for t, c in zip(rng.integers(0, V, 200), rng.integers(0, 4, 200))}
        for t in draft[:3]:
            hist[int(t)] = hist.get(int(t), 0) + 1  # drafts already in the history
        q_mode = trial % 2
        dd = dev(draft.astype(np.int32))
        torch.cuda.synchronize()
        ctx.accept_sampled_ex(logits, M, V, dd, q_mode, 77, trial, out, 0.7, hist=hist, **opts)
        ctx.sync()
        got = tuple(int(v) for v in host(out))
        u = orc.verify_uniforms(77, trial, M)
        ht = np.array(list(hist.keys()), np.int32)
        hc = np.array([hist[t] for t in ht.tolist()], np.int32)
        ref = orc.accept_sampled_ex(lh, draft, 0.7, q_mode, u, hist_tok=ht, hist_cnt=hc, **opts)
        assert got == ref, (trial, opts, got, ref)
        seen[ref[0]] = seen.get(ref[0], 0) + 1
    assert (host(logits).view(np.uint32) == lh.view(np.uint32)).all()
    print("accepted-count histogram", opts, seen, flush=True)


@pytest.mark.parametrize("opts", [None, dict(top_p=0.6, rep=1.3, pres=0.4, freq=0.25)])
def test_accept_sampled_point_q_bit_exact(ctx, head_case, orc, opts):
    """Fractional draft densities (qAlong-like count ratios, 1e-6, q = 0, q near p) passed as a
    device array q_point to mj_accept_sampled(_ex): accept count and emitted token bit for bit
    against the oracle on the same logits, q and uniforms, over the full 151936-token head."""
    import torch

    am = head_case["am"]
    logits = head_case["logits"]
    lh = host(logits)
    rng = np.random.default_rng(57 if opts is None else 58)
    out = torch.empty(2, dtype=torch.int32, device="cuda")
    seen = {}
    for trial in range(16):
        draft = am[:M - 1].copy()
        for i in range(6, M - 1):
            draft[i] = rng.integers(0, V)
        qp = draft_q_values(rng, lh, draft, 0.7)
        dd, dq = dev(draft.astype(np.int32)), dev(qp)
        u = orc.verify_uniforms(4049, trial, M)
        torch.cuda.synchronize()
        if opts is None:
            ctx.accept_sampled(logits, M, V, dd, 0.7, 0, 4049, trial, out, q_point=dq)
            ref = orc.accept_sampled(lh, draft, 0.7, 0, u, q_point=qp)
        else:
            hist = {int(t): int(c) for t, c in zip(rng.integers(0, V, 100), rng.integers(0, 4, 100))}
            ctx.accept_sampled_ex(logits, M, V, dd, 0, 4049, trial, out, 0.7, hist=hist,
                                  q_point=dq, **opts)
            ht = np.array(list(hist.keys()), np.int32)
            hc = np.array([hist[t] for t in ht.tolist()], np.int32)
            ref = orc.accept_sampled_ex(lh, draft, 0.7, 0, u, q_point=qp, hist_tok=ht,
                                        hist_cnt=hc, **opts)
        ctx.sync()
        got = tuple(int(v) for v in host(out))
        assert got == ref, (trial, qp.tolist(), got, ref)
        seen[ref[0]] = seen.get(ref[0], 0) + 1
    print("accepted-count histogram (point q)", opts, seen, flush=True)
    assert len(seen) >= 2


@pytest.mark.parametrize("levels,top_p", [(3, 0.5), (7, 0.9), (2, 0.02), (40, 0.6), (1, 0.37)])
def test_nucleus_ties_bit_exact(ctx, orc, levels, top_p):
    """Rows whose logits take only a few distinct values, so the nucleus cut falls inside a tie
    group spread over the whole vocabulary: the cut key from the four digit rounds, then the
    j-th tie in id order found across the selection's blocks.  Drafts of q = 1e-12 (below every
    p here) and, with one level, a uniform q equal to every p are accepted with certainty, so
    the bonus row goes through the nucleus.  Bit for bit against the oracle."""
    import torch

    rng = np.random.default_rng(levels)
    Vs, rows = 151936, 3
    lv = rng.integers(0, levels, (rows, Vs)).astype(np.float32) * 0.25
    logits = dev(lv)
    out = torch.empty(2, dtype=torch.int32, device="cuda")
    draft = rng.integers(0, Vs, rows - 1).astype(np.int32)
    dd = dev(draft)
    qp = np.full(rows - 1, 1e-12, np.float32)
    dq = dev(qp)
    q_mode = 1 if levels == 1 else 0
    for trial in range(4):
        torch.cuda.synchronize()
        ctx.accept_sampled_ex(logits, rows, Vs, dd, q_mode, 91, trial, out, 1.0,
                              q_point=dq if q_mode == 0 else None, top_p=top_p)
        ctx.sync()
        got = tuple(int(v) for v in host(out))
        u = orc.verify_uniforms(91, trial, rows)
        ref = orc.accept_sampled_ex(lv, draft, 1.0, q_mode, u,
                                    q_point=qp if q_mode == 0 else None, top_p=top_p)
        assert got == ref, (levels, top_p, trial, got, ref)
        assert ref[0] == rows - 1, ref  # the bonus, through the nucleus


@pytest.mark.parametrize("Vs,off,opts", [
    (151923, 0, None),                 # rows not 16-byte aligned, last chunk and block partial
    (1001, 0, None),                   # one block of 63 chunks, the last partial
    (V, 1, None),                      # aligned width, base pointer one float off
    (151923, 0, dict(top_p=0.5, rep=1.3, pres=0.4, freq=0.25)),
])
def test_accept_sampled_unaligned_rows_bit_exact(ctx, head_case, orc, Vs, off, opts):
    """Rows the kernels cannot read as float4 (width not a multiple of 4, or a base address off
    16 bytes) take the one-float-a-request path; partial chunks and blocks end the row.  Bit for
    bit against the oracle on the same logits and uniforms."""
    import torch

    logits = head_case["logits"]
    buf = torch.empty(M * Vs + off, dtype=torch.float32, device="cuda")
    lv = buf[off:].view(M, Vs)
    lv.copy_(logits[:, :Vs])
    torch.cuda.synchronize()
    lh = host(lv)
    am = lh.argmax(1).astype(np.int32)
    rng = np.random.default_rng(Vs + off)
    out = torch.empty(2, dtype=torch.int32, device="cuda")
    seen = {}
    for trial in range(10):
        draft = am[:M - 1].copy()
        for i in range(5, M - 1):
            draft[i] = rng.integers(0, Vs)
        if trial % 3 == 0:
            draft[int(rng.integers(0, 5))] = rng.integers(0, Vs)  # early reject
        q_mode = trial % 2
        dd = dev(draft.astype(np.int32))
        torch.cuda.synchronize()
        u = orc.verify_uniforms(2025, trial, M)
        if opts is None:
            ctx.accept_sampled(lv, M, Vs, dd, 0.7, q_mode, 2025, trial, out)
            ref = orc.accept_sampled(lh, draft, 0.7, q_mode, u)
        else:
            hist = {int(t): int(c) for t, c in zip(rng.integers(0, Vs, 50), rng.integers(0, 4, 50))}
            ctx.accept_sampled_ex(lv, M, Vs, dd, q_mode, 2025, trial, out, 0.7, hist=hist, **opts)
            ht = np.array(list(hist.keys()), np.int32)
            hc = np.array([hist[t] for t in ht.tolist()], np.int32)
            ref = orc.accept_sampled_ex(lh, draft, 0.7, q_mode, u, hist_tok=ht, hist_cnt=hc,
                                        **opts)
        ctx.sync()
        got = tuple(int(v) for v in host(out))
        assert got == ref, (Vs, off, trial, got, ref)
        seen[ref[0]] = seen.get(ref[0], 0) + 1
    print("accepted-count histogram", Vs, off, seen, flush=True)
