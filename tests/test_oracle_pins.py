"""Pins of the CPU oracle: known-answer vectors, closed forms and invariants.

Each test checks an oracle function against something it was not derived from: numpy's IEEE
float16, float64 closed forms, brute force, published RNG vectors, or the reference's own
known-answer tests (cited by file:line under swift/Tests/MomijCoreTests/).
"""
import math

import numpy as np
import pytest

from momij_amd import synth


# ----------------------------------------------------------------------------- fp16
def test_f16_decode_all_patterns(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = orc.h2f(h)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_f16_encode_matches_numpy_rne(orc):
    rng = np.random.default_rng(0)
    xs = [rng.standard_normal(200000).astype(np.float32) * s for s in (1e-7, 1e-5, 1e-3, 1, 1e3, 7e4)]
    # exact halfway cases between adjacent halves (ties to even)
    h = np.arange(0, 0x7bff, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    xs.append(((lo + hi) / 2).astype(np.float32))
    xs.append(np.array([65504, 65519.99, 65520, 1e9, -1e9, 0.0, -0.0, np.inf, -np.inf],
                       np.float32))
    x = np.concatenate(xs)
    ref = x.astype(np.float16).view(np.uint16)
    got = orc.f2h(x)
    assert (got == ref).all()


# ----------------------------------------------------------------------------- qmm2
def _qmm2_f64(x, w, s, b, inds, M, ktop, K, N, gs, lhs):
    dense = synth.dequant(w, s, b, gs)  # [E, N, K]
    y = np.zeros((M * ktop, N))
    for mk in range(M * ktop):
        xr = x[mk if lhs else mk // ktop].astype(np.float64)
        y[mk] = dense[inds[mk]] @ xr
    return y


@pytest.mark.parametrize("gs", [64, 128])
@pytest.mark.parametrize("lhs", [False, True])
def test_qmm2_closed_form(orc, gs, lhs):
    rng = np.random.default_rng(1 + gs + int(lhs))
    E, M, ktop, K, N = 5, 2, 3, 1024, 48
    w, s, b = synth.qweight(rng, (E,), N, K, gs)
    x = synth.normal_f16(rng, (M * ktop if lhs else M, K))
    inds = rng.integers(0, E, M * ktop).astype(np.int32)
    got = orc.qmm2(x, w, s, b, inds, M, ktop, K, N, gs, lhs).astype(np.float64)
    ref = _qmm2_f64(x, w, s, b, inds, M, ktop, K, N, gs, lhs)
    # fp16 output rounding (2^-11 rel) plus the reference's half 4-sums of x in the bias term
    err = np.abs(got - ref)
    assert err.max() <= 2e-3 * np.abs(ref).max() + 1e-3
    assert np.linalg.norm(got - ref) <= 2e-3 * np.linalg.norm(ref)


def test_qmm2_code_bit_order_and_affine(orc):
    """One-hot x at k with s=1, b=0 returns code k of the row (LSB-first layout)."""
    rng = np.random.default_rng(7)
    K, N, gs = 512, 16, 64
    codes = rng.integers(0, 4, (N, K))
    w = synth.pack_codes(codes)[None]
    s = np.ones((1, N, K // gs), np.float16)
    b = np.zeros((1, N, K // gs), np.float16)
    for k in (0, 1, 5, 15, 16, 17, 300, 511):
        x = np.zeros((1, K), np.float16)
        x[0, k] = 1.0
        y = orc.qmm2(x, w, s, b, np.zeros(1, np.int32), 1, 1, K, N, gs)
        assert (y[0].astype(np.int64) == codes[:, k]).all(), k
    # all-zero codes: y = sum_g b_g * sum_{k in g} x_k
    w0 = np.zeros((1, N, K // 16), np.uint32)
    bb = rng.uniform(-0.03, 0.03, (1, N, K // gs)).astype(np.float16)
    x = synth.normal_f16(rng, (1, K))
    y = orc.qmm2(x, w0, s, bb, np.zeros(1, np.int32), 1, 1, K, N, gs).astype(np.float64)
    gsum = x.astype(np.float64).reshape(K // gs, gs).sum(1)
    ref = bb[0].astype(np.float64) @ gsum
    assert np.allclose(y[0], ref, rtol=3e-3, atol=2e-3)


def test_qmm2_mrow_equals_sequential(orc):
    """MomijCoreTests.swift:251-314: the batched M-row gather equals M=1 calls row by row."""
    rng = np.random.default_rng(3)
    E, M, ktop, K, N, gs = 8, 2, 2, 512, 128, 128
    w, s, b = synth.qweight(rng, (E,), N, K, gs)
    x = synth.normal_f16(rng, (M, K))
    inds = np.array([1, 3, 2, 5], np.int32)
    yM = orc.qmm2(x, w, s, b, inds, M, ktop, K, N, gs)
    for m in range(M):
        y1 = orc.qmm2(x[m:m + 1], w, s, b, inds[m * ktop:(m + 1) * ktop], 1, ktop, K, N, gs)
        assert (y1.view(np.uint16) == yM[m * ktop:(m + 1) * ktop].view(np.uint16)).all()


# ----------------------------------------------------------------------------- epilogues
def test_swiglu_closed_form(orc):
    rng = np.random.default_rng(4)
    rows, I = 6, 256
    ug = (rng.standard_normal((rows, 2 * I)) * 5).astype(np.float16)  # exercises the +-7 clamps
    got = orc.clamped_swiglu(ug, rows, I).astype(np.float64)
    up = np.clip(ug[:, :I].astype(np.float64), -7, 7)
    gate = np.minimum(ug[:, I:].astype(np.float64), 7)
    ref = gate / (1 + np.exp(-gate)) * up
    assert np.allclose(got, ref, rtol=2e-3, atol=1e-3)
    assert (np.abs(ug[:, I:]) > 7).any() and (np.abs(ug[:, :I]) > 7).any()


def test_score_reduce_closed_form(orc):
    rng = np.random.default_rng(5)
    M, k, H = 3, 8, 64
    down = synth.normal_f16(rng, (M * k, H))
    sc = rng.dirichlet(np.ones(k), M).astype(np.float32)
    got = orc.score_reduce(down, sc, M, k, H).astype(np.float64)
    ref = np.einsum("mkh,mk->mh", down.astype(np.float64).reshape(M, k, H), sc.astype(np.float64))
    assert np.allclose(got, ref, rtol=2e-3, atol=1e-3)
    # ktop = 1 with score 1 is the identity combine
    one = orc.score_reduce(down[:M], np.ones((M, 1), np.float32), M, 1, H)
    assert (one.view(np.uint16) == down[:M].view(np.uint16)).all()


def test_rms_norm_closed_form(orc):
    rng = np.random.default_rng(6)
    x = synth.normal_f16(rng, (4, 2048), 3.0)
    w = (1 + 0.1 * rng.standard_normal(2048)).astype(np.float16)
    got = orc.rms_norm(x, w, 1e-6).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * w.astype(np.float64)
    assert np.allclose(got, ref, rtol=2e-3, atol=2e-3)


# ----------------------------------------------------------------------------- router
def test_router_topk_bruteforce(orc):
    rng = np.random.default_rng(8)
    M, E, H, k = 16, 64, 2048, 8
    W = synth.normal_f16(rng, (E, H), 0.02)
    x = synth.normal_f16(rng, (M, H))
    lg = orc.router_logits(W, x)
    ref_lg = x.astype(np.float64) @ W.astype(np.float64).T
    assert np.allclose(lg, ref_lg, rtol=1e-5, atol=1e-5)
    inds, scores = orc.route_topk(lg, k)
    for m in range(M):
        l = ref_lg[m]
        order = sorted(range(E), key=lambda e: (-l[e], e))[:k]
        assert list(inds[m]) == order
        g = np.exp(l - l.max())
        g /= g.sum()
        ref_sc = g[order] / g[order].sum()
        assert np.allclose(scores[m], ref_sc, rtol=1e-5)


def test_route_ties_pick_lowest_index(orc):
    lg = np.zeros((1, 16), np.float32)
    lg[0, [3, 9, 12]] = 2.0
    lg[0, [1, 14]] = 1.0
    inds, scores = orc.route_topk(lg, 5)
    assert list(inds[0]) == [3, 9, 12, 1, 14]
    assert abs(scores[0].sum() - 1) < 1e-6


# ----------------------------------------------------------------------------- attention
def test_qk_norm_rope_closed_form(orc):
    rng = np.random.default_rng(9)
    M, nQ, nKV, D, rope, eps, base = 3, 4, 2, 128, 64, 1e-6, 1e6
    qkv = synth.normal_f16(rng, (M, (nQ + 2 * nKV) * D))
    qn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float16)
    kn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float16)
    inv = orc.rope_inv_freq(rope, base)
    assert np.allclose(inv, base ** (-np.arange(rope // 2) / (rope // 2)), rtol=1e-6)
    pos = np.array([0, 4097, 123456], np.int64)
    qo, ko = orc.qk_norm_rope(qkv, qn, kn, inv, pos, nQ, nKV, D, rope, eps)
    for m in range(M):
        for hh in range(nQ + nKV):
            xh = qkv[m, hh * D:(hh + 1) * D].astype(np.float64)
            w = (qn if hh < nQ else kn).astype(np.float64)
            v = xh / np.sqrt((xh ** 2).mean() + eps) * w
            half = rope // 2
            th = pos[m] * inv.astype(np.float64)
            a, bb = v[:half].copy(), v[half:rope].copy()
            out = v.copy()
            out[:half] = a * np.cos(th) - bb * np.sin(th)
            out[half:rope] = bb * np.cos(th) + a * np.sin(th)
            got = (qo[m, hh] if hh < nQ else ko[m, hh - nQ]).astype(np.float64)
            assert np.allclose(got, out, rtol=4e-3, atol=4e-3), (m, hh)


def _attn_f64(q, kc, vc, C, L, parents, window):
    M, nQ, D = q.shape
    nKV = kc.shape[0]
    depth = np.zeros(M, int)
    anc = np.eye(M, dtype=bool)
    for r in range(M):
        p = parents[r]
        depth[r] = 0 if p < 0 else depth[p] + 1
        if p >= 0:
            anc[r] |= anc[p]          # transitive closure row by row
    out = np.zeros((M, nQ * D))
    for r in range(M):
        P = L + depth[r]
        lo = max(0, P - window + 1) if window > 0 else 0
        slots = [p % C for p in range(lo, L)] + [(L + a) % C for a in range(M)
                                                 if anc[r, a] and L + depth[a] >= lo]
        for h in range(nQ):
            g = h // (nQ // nKV)
            K = kc[g, slots].astype(np.float64)
            V = vc[g, slots].astype(np.float64)
            s = K @ q[r, h].astype(np.float64) / math.sqrt(D)
            p_ = np.exp(s - s.max())
            out[r, h * D:(h + 1) * D] = p_ @ V / p_.sum()
    return out


@pytest.mark.parametrize("shape", ["chain", "tree"])
def test_attention_textbook(orc, shape):
    rng = np.random.default_rng(10)
    nQ, nKV, D, W, C, L = 8, 2, 128, 64, 100, 150  # ring wraps; window narrower than prefix
    parents = ([-1] + list(range(7)) if shape == "chain"
               else [-1, 0, 0, 0, 1, 1, 2, 4, 4, 7, 9])
    M = len(parents)
    q = synth.normal_f16(rng, (M, nQ, D))
    kc = synth.normal_f16(rng, (nKV, C, D))
    vc = synth.normal_f16(rng, (nKV, C, D))
    got = orc.attention(q, kc, vc, C, L, np.array(parents, np.int32), W).astype(np.float64)
    ref = _attn_f64(q, kc, vc, C, L, parents, W)
    assert np.allclose(got, ref, rtol=3e-3, atol=3e-3)


def test_attention_tree_of_chain_equals_chain(orc):
    rng = np.random.default_rng(11)
    nQ, nKV, D, C, L, M = 4, 1, 128, 64, 40, 6
    q = synth.normal_f16(rng, (M, nQ, D))
    kc = synth.normal_f16(rng, (nKV, C, D))
    vc = synth.normal_f16(rng, (nKV, C, D))
    a = orc.attention(q, kc, vc, C, L, None, 16)
    b = orc.attention(q, kc, vc, C, L, np.array([-1, 0, 1, 2, 3, 4], np.int32), 16)
    assert (a.view(np.uint16) == b.view(np.uint16)).all()


def test_sliding_window_mask_kat(orc):
    """MomijCoreTests.swift:130-145: N=4, window=2, offset 0 -> row i attends [i-1, i].
    One-hot values read the attention weights back: out[r, d] = weight of key d."""
    D, M = 128, 4
    q = np.zeros((M, 1, D), np.float16)
    kc = np.zeros((1, 8, D), np.float16)
    vc = np.zeros((1, 8, D), np.float16)
    for s in range(8):
        vc[0, s, s] = 1.0
    out = orc.attention(q, kc, vc, 8, 0, None, 2).astype(np.float32)
    allowed = out[:, :4] > 0
    assert allowed.tolist() == [[True, False, False, False], [True, True, False, False],
                                [False, True, True, False], [False, False, True, True]]


# ----------------------------------------------------------------------------- lm_head
def test_lm_head_argmax(orc):
    rng = np.random.default_rng(12)
    M, K, V = 3, 256, 5000
    x = synth.normal_f16(rng, (M, K))
    w = synth.normal_f16(rng, (V, K), 0.02)
    lg = orc.lm_head_logits(x, w)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.allclose(lg, ref, rtol=1e-6, atol=1e-6)
    idx, best, second = orc.argmax_rows(lg)
    assert (idx == ref.argmax(1)).all()
    # ties -> lowest id; banned ids are skipped
    t = np.zeros((1, 10), np.float32)
    t[0, [4, 7]] = 3.0
    assert orc.argmax_rows(t)[0][0] == 4
    assert orc.argmax_rows(t, banned=np.array([4]))[0][0] == 7


def test_lm_head_q4_closed_form(orc):
    """The Maple 4-bit head against a float64 dequantised GEMV, plus the code order (nibble j
    of pack wk is k = 8 wk + j) and the group of a pack (wk >> 3) pinned with one-hot inputs."""
    rng = np.random.default_rng(13)
    M, K, V = 3, 512, 3000
    x = synth.normal_f16(rng, (M, K))
    w, s, b = synth.qweight4(rng, V, K)
    lg = orc.lm_head_q4_logits(x, w, s, b)
    ref = x.astype(np.float64) @ synth.dequant4(w, s, b).T
    assert np.allclose(lg, ref, rtol=1e-6, atol=1e-6)
    assert (orc.argmax_rows(lg)[0] == ref.argmax(1)).all()
    # one code set: pack 9 (group 1), nibble 5 = 11 -> weight at k = 77 is 11 s1 + b1
    w1 = np.zeros((1, K // 8), np.uint32)
    w1[0, 9] = np.uint32(11 << 20)
    s1 = np.full((1, K // 64), 0.5, np.float16)
    s1[0, 1] = 0.25
    b1 = np.zeros((1, K // 64), np.float16)
    b1[0, 1] = 1.0
    xo = np.zeros((1, K), np.float16)
    xo[0, 77] = 2.0
    assert orc.lm_head_q4_logits(xo, w1, s1, b1)[0, 0] == np.float32(2.0 * (11 * 0.25 + 1.0))
    xo[0, 77] = 0.0
    xo[0, 64] = 1.0  # another k of group 1: code 0 -> the bias alone
    assert orc.lm_head_q4_logits(xo, w1, s1, b1)[0, 0] == np.float32(1.0)


# ----------------------------------------------------------------------------- greedy accept
def test_accept_greedy_chain_kats(orc):
    """SpeculativeSamplingTests.swift:94-137 (walkDraft at temperature 0) as chain verifies."""
    # rows' argmax: 20, 21, 30 ; draft [20, 21] -> accept 2, next 30
    acc, path, emit = orc.accept_greedy([5, 20, 21], None, [20, 21, 30])
    assert acc == 2 and list(emit) == [20, 21, 30] and list(path) == [0, 1, 2]
    acc, _, emit = orc.accept_greedy([5, 99, 21], None, [20, 21, 10])
    assert acc == 0 and list(emit) == [20]
    acc, _, emit = orc.accept_greedy([5, 20, 99], None, [20, 21, 10])
    assert acc == 1 and list(emit) == [20, 21]


def test_accept_greedy_tree(orc):
    # row: 0(y) 1 2 3 4 5 6 ; parents; tokens at rows ; argmax per row
    parents = [-1, 0, 0, 0, 2, 2, 5]
    tokens = [9, 11, 12, 13, 21, 22, 31]
    argmax = [12, 0, 22, 0, 0, 31, 40]
    acc, path, emit = orc.accept_greedy(tokens, parents, argmax)
    assert acc == 3 and list(path) == [0, 2, 5, 6] and list(emit) == [12, 22, 31, 40]
    # duplicate sibling tokens: the lowest row index wins
    acc, path, _ = orc.accept_greedy([9, 12, 12], [-1, 0, 0], [12, 5, 6])
    assert acc == 1 and list(path) == [0, 1]
    # a chain written as a tree is the chain rule
    a1 = orc.accept_greedy([5, 20, 21, 22], None, [20, 21, 7, 1])
    a2 = orc.accept_greedy([5, 20, 21, 22], [-1, 0, 1, 2], [20, 21, 7, 1])
    assert a1[0] == a2[0] == 2 and list(a1[2]) == list(a2[2])


# ----------------------------------------------------------------------------- RNG
def test_philox_random123_kats(orc):
    kats = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for ctr, key, want in kats:
        assert [int(v) for v in orc.philox4x32_10(ctr, key)] == want


def test_splitmix64_vectors(orc):
    assert orc.splitmix64(1234567, 3) == [6457827717110365317, 3203168211198807973,
                                          9817491932198370423]


def test_canon_exp_vs_libm(orc):
    xs = np.concatenate([np.linspace(-87, 0, 20001, dtype=np.float32),
                         -np.logspace(-8, 1.9, 2000).astype(np.float32), [0.0, -0.0]])
    got = orc.canon_expf_array(xs).astype(np.float64)
    ref = np.exp(xs.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - ref) <= 2 * ulp).all()
    assert orc.canon_expf(-88.0) == 0.0 and orc.canon_expf(0.0) == 1.0


def test_canon_sum_and_walk_exact_cases(orc):
    rng = np.random.default_rng(13)
    for n in (1, 15, 16, 17, 1023, 1024, 1025, 5000, 151936):
        v = rng.integers(0, 8, n).astype(np.float32)  # integers: all sums exact in fp32
        assert orc.canon_sum(v) == float(v.sum())
        cs = np.cumsum(v.astype(np.int64))
        for t in rng.uniform(0, cs[-1], 20):
            want = int(np.searchsorted(cs, t, side="left"))
            assert orc.canon_walk(v, float(np.float32(t))) == min(want, n - 1), (n, t)
    v = rng.random(9).astype(np.float32)  # one chunk: plain sequential order
    acc = np.float32(0)
    for e in v:
        acc = np.float32(acc + e)
    assert orc.canon_sum(v) == float(acc)
    assert orc.canon_walk(np.zeros(10, np.float32), 1.0) == 9  # fallback: last id


# ----------------------------------------------------------------------------- sampling
def test_try_accept_kats(orc):
    """SpeculativeSamplingTests.swift:5-45."""
    ok, tok, _ = orc.try_accept(7, [7], [0.0], 1.0, 1.0, 1)
    assert ok and tok == 7
    ok, tok, _ = orc.try_accept(99, [1, 2, 3], [0, 5, 0], 0.0, 1.0, 99)
    assert not ok and tok == 2
    ok, tok, _ = orc.try_accept(1, [1, 2, 3], [0, 9, 0], 0.0, 1.0, 1)
    assert not ok and tok == 2
    ok, tok, _ = orc.try_accept(2, [1, 2, 3], [0, 5, 0], 0.0, 0.4, 1)
    assert ok and tok == 2


def test_walk_draft_kats(orc):
    """SpeculativeSamplingTests.swift:94-137."""
    ids = [[10, 20, 30], [10, 21, 30], [11, 22, 30]]
    assert orc.walk_draft([20, 21], ids, [[0, 5, 1], [0, 9, 1], [0, 1, 8]], 0.0, 1) == (2, 30)
    lg = [[0, 5, 1], [0, 9, 1], [8, 1, 0]]
    assert orc.walk_draft([99, 21], ids, lg, 0.0, 1) == (0, 20)
    assert orc.walk_draft([20, 99], ids, lg, 0.0, 1) == (1, 21)


def _sampled_f64(logits, draft, T, q_mode, u):
    rows, V = logits.shape
    for i in range(rows - 1):
        l = logits[i].astype(np.float64) / T
        p = np.exp(l - l.max())
        p /= p.sum()
        q = 1.0 / V if q_mode == 1 else 1.0
        if p[draft[i]] > 0 and u[i, 0] <= min(1.0, p[draft[i]] / q):
            continue
        r = np.maximum(p - q, 0) if q_mode == 1 else p.copy()
        if q_mode == 0:
            r[draft[i]] = max(0.0, r[draft[i]] - q)
        cs = np.cumsum(r)
        t = u[i, 1] * cs[-1]
        return i, min(int(np.searchsorted(cs, t)), V - 1), (p[draft[i]] / q, cs, t)
    l = logits[-1].astype(np.float64) / T
    e = np.exp(l - l.max())
    cs = np.cumsum(e)
    return rows - 1, min(int(np.searchsorted(cs, u[-1, 0] * cs[-1])), V - 1), None


@pytest.mark.parametrize("q_mode", [0, 1])
def test_accept_sampled_vs_float64(orc, q_mode):
    """Canonical fp32 rule vs a float64 textbook restatement on the same uniforms; cases whose
    decision lies within float rounding of a boundary are excluded (and counted)."""
    rng = np.random.default_rng(14 + q_mode)
    V, rows, T = 3000, 5, 0.7
    ambiguous = 0
    for trial in range(60):
        logits = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
        draft = rng.integers(0, V, rows - 1).astype(np.int32)
        draft[:2] = logits[:2].argmax(1)
        u = orc.verify_uniforms(1000 + trial, 7, rows)
        acc, tok = orc.accept_sampled(logits, draft, T, q_mode, u)
        racc, rtok, info = _sampled_f64(logits, draft, T, q_mode, u)
        if (acc, tok) != (racc, rtok):
            ambiguous += 1
            assert info is not None
            ratio, cs, t = info
            near = min(abs(u[racc, 0] - min(1, ratio)), np.abs(cs - t).min() / max(cs[-1], 1e-30))
            assert near < 1e-5, (trial, acc, tok, racc, rtok)
    assert ambiguous <= 2


def test_rejection_sampling_preserves_target(orc):
    """Leviathan et al.: with a uniform draft q, accept-or-resample emits tokens distributed as p."""
    V, T, n = 6, 1.0, 30000
    logits = np.array([[1.5, 0.2, -0.7, 0.9, 0.0, -2.0], [0, 0, 0, 0, 0, 0]], np.float32)
    p = np.exp(logits[0] / T)
    p /= p.sum()
    rng = np.random.default_rng(15)
    counts = np.zeros(V)
    for t in range(n):
        d = int(rng.integers(0, V))  # draft sampled from uniform q
        u = orc.verify_uniforms(77, t, 2)
        acc, tok = orc.accept_sampled(logits, np.array([d], np.int32), T, 1, u)
        counts[d if acc == 1 else tok] += 1
    chi2 = (((counts - n * p) ** 2) / (n * p)).sum()
    assert chi2 < 25.0, (counts / n, p)  # 5 dof, p ~ 1e-4
