"""Pins of the oracle's sampling rules beyond the plain temperature softmax: LogitsProcessor's
penalties and nucleus (LogitsProcessor.swift:57-164) and walkDraft's history growth
(SpeculativeSampling.swift:65-99), as restated in or_penalize_row / or_nucleus_sample /
or_accept_sampled_ex.

  * the reference's own known answers (LogitsProcessorTests.swift:12-53): presence, frequency
    and repetition penalties to the exact float, and the top-p tail drop;
  * a float64 textbook statement (numpy; stable sort by probability, then id) of penalties,
    softmax, nucleus and the acceptance walk agrees with the oracle's canonical fp32 rule on the
    same uniforms, except cases whose decision lies within float rounding of a boundary (counted
    and bounded);
  * planted mistakes in that statement -- a nucleus one token short, penalties that ignore the
    accepted drafts, presence applied before repetition -- disagree with the oracle on many of
    the same cases, so the comparison can tell each of them from the oracle;
  * with every option neutral the extended rule is or_accept_sampled bit for bit.
"""
import numpy as np
import pytest

from tests.gpu_util import draft_q_values as _q_values


# ---------------------------------------------------------------- float64 statement ------
def _penalize64(l, hist, extra, rep, pres, freq, order="rpf"):
    """hist: {token: count}; extra: accepted drafts (seen, counted once each)."""
    l = np.array(l, np.float64)
    counts = dict(hist)
    for t in extra:
        counts[t] = counts.get(t, 0) + 1
    for t, c in counts.items():
        x = l[t]
        for op in order:
            if op == "r" and abs(rep - 1) > 1e-6 and rep > 0:
                x = x / rep if x > 0 else x * rep
            elif op == "p" and pres != 0:
                x = x - pres
            elif op == "f" and freq != 0 and c > 0:
                x = x - freq * c
        l[t] = x
    return l


def _walk64(mass, t):
    """First index whose cumulative mass reaches t (last index otherwise) and the distance of t
    to the nearest cumulative boundary, relative to the total."""
    cs = np.cumsum(mass)
    i = min(int(np.searchsorted(cs, t)), len(mass) - 1)
    near = np.abs(cs - t).min() / max(cs[-1], 1e-300)
    return i, near


def _nucleus64(e, top_p, u, short=False):
    """samplePrepared's nucleus in float64: kept = shortest prefix (stable order by e desc, then
    id) whose sum reaches top_p * sum; sample at u * sum(kept) in id order."""
    order = sorted(range(len(e)), key=lambda i: (-e[i], i))
    cs = np.cumsum(np.asarray(e, np.float64)[order])
    cut = max(0.0, min(1.0, top_p)) * e.sum()
    k = min(int(np.searchsorted(cs, cut)), len(e) - 1)
    near_cut = np.abs(cs - cut).min() / max(cs[-1], 1e-300)
    if short:
        k = max(k - 1, 0)
    kept = np.zeros_like(e)
    kept[order[: k + 1]] = e[order[: k + 1]]
    if kept.sum() <= 0:
        return order[0], near_cut
    tok, near = _walk64(kept, u * kept.sum())
    return tok, min(near, near_cut)


def _accept64(logits, draft, T, q_mode, u, top_p, rep, pres, freq, hist, plant=None,
              q_point=None):
    """tryAccept / walkDraft in float64.  q_point (point mode): the draft density q_i on draft i
    (qAlong), max(0, q_i); None = 1 on every draft.  Plants: "q_row" reads q from the previous
    row, "q_one" ignores q_point, "q_resid" leaves the draft's mass in the residual."""
    rows, V = logits.shape
    D = rows - 1
    nuc = top_p < 1 - 1e-6
    near = 1.0

    def q_of(i):
        if q_mode == 1:
            return 1.0 / V
        if q_point is None or plant == "q_one":
            return 1.0
        j = (i - 1) % D if plant == "q_row" else i
        return max(0.0, float(np.float32(q_point[j])))

    for i in range(rows):
        extra = [] if plant == "no_drafts" else list(draft[:i])
        order = "prf" if plant == "order" else "rpf"
        l = _penalize64(logits[i], hist, extra, rep, pres, freq, order) / T
        e = np.exp(l - l.max())
        Z = e.sum()
        if i == D:
            if nuc:
                tok, n2 = _nucleus64(e, top_p, u[D, 0], short=plant == "short")
            else:
                tok, n2 = _walk64(e, u[D, 0] * Z)
            return D, tok, min(near, n2)
        p = e / Z
        d = draft[i]
        q = q_of(i)
        if q > 0 and p[d] > 0:
            edge = abs(u[i, 0] - min(1.0, p[d] / q))
            near = min(near, edge)
            if u[i, 0] <= min(1.0, p[d] / q):
                continue
        r = np.maximum(p - q, 0) if q_mode == 1 else p.copy()
        if q_mode == 0 and q > 0 and plant != "q_resid":
            r[d] = max(0.0, r[d] - q)
        if r.sum() > 0:
            tok, n2 = _walk64(r, u[i, 1] * r.sum())
        elif nuc:
            tok, n2 = _nucleus64(e, top_p, u[i, 1], short=plant == "short")
        else:
            tok, n2 = _walk64(e, u[i, 1] * Z)
        return i, tok, min(near, n2)


# ---------------------------------------------------------------- known answers ----------
def test_presence_penalty_kat(orc):
    # LogitsProcessorTests.swift:12-20: ids [1, 2, 3], logits 3, seen {2}, penalty 2
    l = orc.penalize_row(np.array([0, 3, 3, 3], np.float32), [2], [0], pres=2.0)
    assert l.tolist() == [0.0, 3.0, 1.0, 3.0]


def test_frequency_penalty_kat(orc):
    # LogitsProcessorTests.swift:22-28: ids [7, 8, 9], logits 0, counts {8: 3}, penalty 0.5
    l = orc.penalize_row(np.zeros(10, np.float32), [8], [3], freq=0.5)
    assert l[8] == -1.5 and (np.delete(l, 8) == 0).all()


def test_repetition_penalty_kat(orc):
    # LogitsProcessorTests.swift:30-36: [4, -2] at seen ids 1, 2, penalty 2 -> [2, -4]
    l = orc.penalize_row(np.array([0, 4, -2], np.float32), [1, 2], [1, 1], rep=2.0)
    assert l.tolist() == [0.0, 2.0, -4.0]
    # off at |r - 1| <= 1e-6 and at r <= 0 (LogitsProcessor.swift:81)
    for r in (1.0 + 5e-7, 0.0, -1.0):
        assert orc.penalize_row(np.array([0, 4, -2], np.float32), [1, 2], [1, 1],
                                rep=r).tolist() == [0.0, 4.0, -2.0]


def test_penalties_count_accepted_drafts(orc):
    """Drafts accepted along the walk join the seen set and add to the counts; a draft repeated
    or already in the history is penalised once with the summed count."""
    base = np.full(12, 1.0, np.float32)
    l = orc.penalize_row(base, [5], [1], extra=[5, 7, 7], rep=2.0, pres=0.5, freq=1.0)
    want = base.copy()
    want[5] = 1.0 / 2.0 - 0.5 - 2.0 * 1.0  # count 1 + 1
    want[7] = 1.0 / 2.0 - 0.5 - 2.0 * 1.0  # count 2
    assert l.tolist() == want.astype(np.float32).tolist()


def test_top_p_drops_tail_kat(orc):
    # LogitsProcessorTests.swift:39-53: temperature 1, top_p 0.5, logits [10, 0, -10]: of 200
    # samples more than 180 are id 0 (ids [1, 2, 3] there) and none is the last
    rng = np.random.default_rng(42)
    logits = np.array([[10.0, 0.0, -10.0]], np.float32)
    hits = np.zeros(3, int)
    for _ in range(200):
        u = rng.random((1, 2)).astype(np.float32)
        _, tok = orc.accept_sampled_ex(logits, np.zeros(0, np.int32), 1.0, 0, u, top_p=0.5)
        hits[tok] += 1
    assert hits[0] > 180 and hits[2] == 0


def test_neutral_options_equal_base_rule(orc):
    rng = np.random.default_rng(3)
    for trial in range(20):
        logits = (rng.standard_normal((4, 700)) * 2).astype(np.float32)
        draft = logits[:3].argmax(1).astype(np.int32)
        u = orc.verify_uniforms(50 + trial, 1, 4)
        for q_mode in (0, 1):
            assert orc.accept_sampled_ex(logits, draft, 0.7, q_mode, u) == \
                orc.accept_sampled(logits, draft, 0.7, q_mode, u)


# ---------------------------------------------------------------- float64 pins -----------
def _cases(seed, n, V=1500, rows=5):
    rng = np.random.default_rng(seed)
    for trial in range(n):
        logits = (rng.standard_normal((rows, V)) * 2.5).astype(np.float32)
        draft = rng.integers(0, V, rows - 1).astype(np.int32)
        # mostly high-probability drafts so that several rows are accepted
        hot = rng.random(rows - 1) < 0.8
        draft[hot] = logits[:-1][hot].argmax(1)
        ht = np.unique(np.concatenate([rng.integers(0, V, 40), draft[:2]])).astype(np.int32)
        hc = rng.integers(0, 4, ht.size).astype(np.int32)
        opts = dict(top_p=[1.0, 0.9, 0.6, 0.3][trial % 4], rep=[1.0, 1.3][trial % 2],
                    pres=[0.0, 0.4][(trial // 2) % 2], freq=[0.0, 0.25][(trial // 3) % 2])
        yield trial, logits, draft, ht, hc, opts


def _sharp_cases(seed, n, V=600, rows=5):
    """Rows sharing a few dominant tokens (the drafts), so that the penalties on the history
    and on the accepted drafts, and the nucleus cut, decide the outcome."""
    rng = np.random.default_rng(seed)
    for trial in range(n):
        base = (rng.standard_normal(V) * 1.0).astype(np.float32)
        top = rng.choice(V, 6, replace=False)
        base[top] += rng.uniform(4.0, 6.0, 6).astype(np.float32)
        logits = (base[None, :] + 0.4 * rng.standard_normal((rows, V))).astype(np.float32)
        draft = logits[:-1].argmax(1).astype(np.int32)
        ht = np.unique(rng.choice(top, 3, replace=False)).astype(np.int32)
        hc = rng.integers(1, 3, ht.size).astype(np.int32)
        opts = dict(top_p=[0.5, 0.3, 0.8][trial % 3], rep=1.6, pres=0.8, freq=0.6)
        yield trial, logits, draft, ht, hc, opts


@pytest.mark.parametrize("q_mode", [0, 1])
@pytest.mark.parametrize("gen", ["random", "sharp"])
def test_accept_sampled_ex_vs_float64(orc, q_mode, gen):
    T = 0.8
    ambiguous = agree = 0
    planted_miss = {"short": 0, "no_drafts": 0, "order": 0}
    cases = _cases(60 + q_mode, 80) if gen == "random" else _sharp_cases(70 + q_mode, 80)
    for trial, logits, draft, ht, hc, opts in cases:
        u = orc.verify_uniforms(900 + trial, 3, logits.shape[0])
        acc, tok = orc.accept_sampled_ex(logits, draft, T, q_mode, u, hist_tok=ht, hist_cnt=hc,
                                         **opts)
        hist = dict(zip(ht.tolist(), hc.tolist()))
        racc, rtok, near = _accept64(logits, draft, T, q_mode, u, opts["top_p"], opts["rep"],
                                     opts["pres"], opts["freq"], hist)
        if (acc, tok) != (racc, rtok):
            ambiguous += 1
            assert near < 1e-5, (trial, opts, acc, tok, racc, rtok, near)
            continue
        agree += 1
        for plant in planted_miss:
            pacc, ptok, _ = _accept64(logits, draft, T, q_mode, u, opts["top_p"], opts["rep"],
                                      opts["pres"], opts["freq"], hist, plant=plant)
            planted_miss[plant] += (pacc, ptok) != (acc, tok)
    assert ambiguous <= 3 and agree >= 70
    if gen == "sharp":
        # each planted mistake is caught on several cases where the true statement agrees (the
        # nucleus is reached through the bonus, i.e. when drafts are accepted: with a uniform q)
        need = ["no_drafts", "order"] + (["short"] if q_mode == 1 else [])
        assert all(planted_miss[k] >= 3 for k in need), planted_miss


def test_nucleus_vs_float64(orc):
    rng = np.random.default_rng(8)
    ambiguous = short_miss = 0
    for trial in range(200):
        V = int(rng.integers(2, 400))
        l = (rng.standard_normal(V) * rng.choice([0.5, 2.0, 6.0])).astype(np.float32)
        if trial % 5 == 0:  # ties in e
            l = np.round(l).astype(np.float32)
        e = np.array([orc.canon_expf(float(x)) for x in (l - l.max())], np.float32)
        Z = orc.canon_sum(e)
        top_p, u = float(rng.uniform(0.05, 0.99)), float(rng.random())
        tok = orc.nucleus_sample(e, Z, top_p, u)
        rtok, near = _nucleus64(e.astype(np.float64), top_p, u)
        if tok != rtok:
            ambiguous += 1
            assert near < 1e-5, (trial, V, top_p, u, tok, rtok, near)
            continue
        stok, _ = _nucleus64(e.astype(np.float64), top_p, u, short=True)
        short_miss += stok != tok
    assert ambiguous <= 3 and short_miss >= 10


# ---------------------------------------------------------------- fractional draft q ----
@pytest.mark.parametrize("ex", [False, True])
@pytest.mark.parametrize("gen", ["random", "sharp"])
def test_accept_sampled_point_q_vs_float64(orc, gen, ex):
    """tryAccept with the draft density of a draft source (draftQ from qAlong,
    SeedlessDecodeEngine.swift:1530-1559; SpeculativeSampling.swift:27-59): accept iff q > 0,
    p > 0 and u <= min(1, p / q), else the residual p with the draft's mass reduced by q.  The
    oracle agrees with the float64 statement on the same uniforms; planted mistakes -- q taken
    from the previous row, q ignored (1 everywhere), the draft's mass left in the residual --
    disagree on several of the same cases."""
    T = 0.8
    ambiguous = agree = 0
    planted_miss = {"q_row": 0, "q_one": 0, "q_resid": 0}
    cases = _cases(80 + ex, 80) if gen == "random" else _sharp_cases(90 + ex, 80)
    for trial, logits, draft, ht, hc, opts in cases:
        rng = np.random.default_rng(1000 + trial)
        qp = _q_values(rng, logits, draft, T)
        u = orc.verify_uniforms(700 + trial, 5, logits.shape[0])
        if ex:
            acc, tok = orc.accept_sampled_ex(logits, draft, T, 0, u, q_point=qp, hist_tok=ht,
                                             hist_cnt=hc, **opts)
            hist = dict(zip(ht.tolist(), hc.tolist()))
            o = (opts["top_p"], opts["rep"], opts["pres"], opts["freq"], hist)
        else:
            acc, tok = orc.accept_sampled(logits, draft, T, 0, u, q_point=qp)
            o = (1.0, 1.0, 0.0, 0.0, {})
        racc, rtok, near = _accept64(logits, draft, T, 0, u, *o, q_point=qp)
        if (acc, tok) != (racc, rtok):
            ambiguous += 1
            assert near < 1e-5, (trial, acc, tok, racc, rtok, near)
            continue
        agree += 1
        for plant in planted_miss:
            pacc, ptok, _ = _accept64(logits, draft, T, 0, u, *o, plant=plant, q_point=qp)
            planted_miss[plant] += (pacc, ptok) != (acc, tok)
    assert ambiguous <= 3 and agree >= 70
    print(gen, ex, "agree", agree, "ambiguous", ambiguous, "planted", planted_miss)
    assert all(v >= 3 for v in planted_miss.values()), planted_miss


def test_point_q_extremes(orc):
    """q = 0 rejects every draft (no uniform can accept it) and samples the target itself;
    q below p accepts with certainty; q = 1 is the reference default (q_point NULL)."""
    rng = np.random.default_rng(12)
    V, rows = 300, 4
    for trial in range(30):
        logits = (rng.standard_normal((rows, V)) * 3).astype(np.float32)
        draft = logits[:-1].argmax(1).astype(np.int32)
        u = orc.verify_uniforms(11, trial, rows)
        acc0, _ = orc.accept_sampled(logits, draft, 1.0, 0, u, q_point=np.zeros(rows - 1, np.float32))
        assert acc0 == 0
        acc_lo, _ = orc.accept_sampled(logits, draft, 1.0, 0, u,
                                       q_point=np.full(rows - 1, 1e-6, np.float32))
        assert acc_lo == rows - 1
        assert orc.accept_sampled(logits, draft, 1.0, 0, u, q_point=np.ones(rows - 1, np.float32)) \
            == orc.accept_sampled(logits, draft, 1.0, 0, u)


def test_nucleus_equal_values_cut_by_id(orc):
    """V equal e (= 1): the ranked order is the id order and each token carries mass 1, so the
    kept set is exactly the first ceil(t) ids, t = top_p * Z in fp32 (the fewest whose mass
    reaches the target, at least one), and the sample is the kept id at u * |kept|.  A cut one
    token short or long, or ties broken by the higher id, would miss."""
    for V in (1, 7, 100, 4096):
        e = np.ones(V, np.float32)
        Z = orc.canon_sum(e)
        assert Z == V
        for top_p in (0.0, 0.3, 0.5, 0.999, 1.0):
            t = float(np.float32(top_p) * np.float32(Z))
            n_kept = min(V, max(1, int(np.ceil(t))))
            for u in (0.0, 0.25, 0.5, 0.9999):
                tok = orc.nucleus_sample(e, Z, top_p, u)
                want = max(0, int(np.ceil(float(np.float32(u) * np.float32(n_kept)))) - 1)
                assert tok == want, (V, top_p, u, tok, want, n_kept)

