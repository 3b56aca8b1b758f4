"""GPU parity: the Maple 4-bit lm_head verify (maple_lm_head_argmax) against the oracle.

Head uint32 [151936 x 256] (4-bit codes uniform, group 64, scale ~ U(0.001, 0.004), bias
-7.5 scale), hidden fp16 [8 x 2048] ~ N(0, 1).  Argmax ids are compared bit for bit, with the
oracle's top-1/top-2 margin checked against the fp32 accumulation error bound so the match is
not luck; logits within 1e-5 relative to the norm and 1e-4 absolute.
"""
import numpy as np
import pytest

from momij_amd import synth
from tests.gpu_util import assert_close, dev, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from momij_amd.ops import Context

    c = Context(0)
    yield c
    c.close()


def _run(ctx, x, w, s, b, M, K, V, banned=None, logits=True, T=None):
    """Runs the head; with T it also returns the per-row log-sum-exp of logits / T."""
    import torch

    am = torch.empty(M, dtype=torch.int32, device="cuda")
    mx = torch.empty(M, dtype=torch.float32, device="cuda")
    lg = torch.empty((M, V), dtype=torch.float32, device="cuda") if logits else None
    lse = torch.empty(M, dtype=torch.float32, device="cuda") if T else None
    db = dev(np.asarray(banned, np.int32)) if banned is not None else None
    torch.cuda.synchronize()
    ctx.lm_head_verify_q4(dev(x), dev(w), dev(s), dev(b), M, K, V, am, mx, lg, db,
                          0 if banned is None else len(banned), temperature=T or 1.0,
                          out_lse=lse)
    ctx.sync()
    out = (host(am), host(mx), (host(lg) if logits else None))
    return out + (host(lse).astype(np.float64),) if T else out


# log-sum-exp bar: the fp32 running sums see at most a few hundred roundings (per-lane strip
# sums, then lane, wave and block merges), 2e-5 relative in the worst case, i.e. 2e-5 absolute
# in the logarithm; plus the logits' own rounding (1e-6 relative, |logit / T| < 10)
LSE_TOL = 3e-5


def _lse64(logits, T, banned=()):
    z = logits.astype(np.float64) / T
    if len(banned):
        z[:, list(banned)] = -np.inf
    mx = z.max(1, keepdims=True)
    return mx[:, 0] + np.log(np.exp(z - mx).sum(1))


def _bound(x, w, s, b, rows):
    """fp32 rounding bound of one logit: 8 sqrt(K) eps times the sum of |term| over the dot
    product, with the 16 s x term of the code offset counted too."""
    K = x.shape[1]
    out = []
    for m, vs in enumerate(rows):
        tot = 0.0
        for v in vs:
            q = ((w[v][:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15).reshape(-1)
            sg = np.repeat(np.abs(s[v].astype(np.float64)), 64)
            bg = np.repeat(np.abs(b[v].astype(np.float64)), 64)
            ax = np.abs(x[m].astype(np.float64))
            tot = max(tot, ((sg * (q + 16) + bg) * ax).sum())
        out.append(8 * np.sqrt(K) * 2.0 ** -24 * tot)
    return np.array(out)


def test_lm_head_q4_full_vocab(ctx, orc):
    V, K, M = 151936, 2048, 8
    print(f"case: lm_head q4 V={V} K={K} M={M}", flush=True)
    rng = np.random.default_rng(31)
    w, s, b = synth.qweight4(rng, V, K)
    x = synth.normal_f16(rng, (M, K))
    am, mx, lg = _run(ctx, x, w, s, b, M, K, V)
    ref = orc.lm_head_q4_logits(x, w, s, b)
    idx, best, second = orc.argmax_rows(ref)
    top2 = np.argsort(-ref, axis=1)[:, :2]
    bound = _bound(x, w, s, b, top2)
    print("margins", (best - second).tolist(), "bound", bound.tolist(), flush=True)
    assert ((best - second) > bound).all()
    assert (am == idx).all(), (am, idx)
    assert_close(lg, ref, rel_tol=1e-5, abs_tol=1e-4, what="q4 full vocab logits")
    assert (mx == lg.max(1)).all()
    # log-sum-exp of logits / 0.7 with each row's top two ids banned (moves it by ~1e-3)
    ban = sorted(set(top2.reshape(-1).tolist()))
    am2, _, _, lse = _run(ctx, x, w, s, b, M, K, V, banned=ban, logits=False, T=0.7)
    want = _lse64(ref, 0.7, ban)
    print("lse err", np.abs(lse - want).max(), flush=True)
    assert np.abs(lse - want).max() < LSE_TOL
    assert np.abs(_lse64(ref, 0.7) - want).min() > 10 * LSE_TOL
    keep = np.ones(V, bool)
    keep[ban] = False
    assert (am2 == np.where(keep)[0][ref[:, keep].argmax(1)]).all()


@pytest.mark.parametrize("M,K,V", [(17, 2048, 20000), (36, 1024, 5003), (9, 4096, 3000),
                                   (1, 512, 777)])
def test_lm_head_q4_shapes(ctx, orc, M, K, V):
    """17 rows (two 16-row tiles), 36 rows (groups of 32), K = 4096 (eight pieces a strip),
    K = 512 (one piece) and vocab sizes that leave a partial last strip."""
    print(f"case: lm_head q4 M={M} K={K} V={V}", flush=True)
    rng = np.random.default_rng(M * 7 + K + V)
    w, s, b = synth.qweight4(rng, V, K)
    x = synth.normal_f16(rng, (M, K))
    am, mx, lg, lse = _run(ctx, x, w, s, b, M, K, V, T=1.3)
    ref = orc.lm_head_q4_logits(x, w, s, b)
    want = _lse64(ref, 1.3)
    assert np.abs(lse - want).max() < LSE_TOL
    idx, best, second = orc.argmax_rows(ref)
    bound = _bound(x, w, s, b, np.argsort(-ref, axis=1)[:, :2])
    clear = (best - second) > bound
    assert clear.sum() >= M // 2
    assert (am[clear] == idx[clear]).all(), (am, idx)
    # a row whose top two lie within the rounding bound may pick either, never a worse id
    assert (ref[np.arange(M), am] >= best - bound).all()
    assert_close(lg, ref, rel_tol=1e-5, abs_tol=1e-4, what=f"q4 M={M} K={K} V={V}")


def test_lm_head_q4_banned_and_ties(ctx):
    """Codes 0 and scale 0 everywhere; bias 1 on group 0 of four rows gives them the same
    logit (the group sum of the hidden row): the lowest id wins, banned ids are skipped."""
    V, K, M = 4096, 512, 3
    w = np.zeros((V, K // 8), np.uint32)
    s = np.zeros((V, K // 64), np.float16)
    b = np.zeros((V, K // 64), np.float16)
    b[[17, 900, 901, 4000], 0] = 1.0
    x = np.ones((M, K), np.float16)
    am, mx, _ = _run(ctx, x, w, s, b, M, K, V, logits=False)
    assert am.tolist() == [17, 17, 17] and (mx == 64.0).all()
    am, _, _ = _run(ctx, x, w, s, b, M, K, V, banned=[17, 901], logits=False)
    assert am.tolist() == [900, 900, 900]


def test_lm_head_q4_code_order(ctx):
    """One set code per row (row v: code 15 at k = (37 v) % K, scale 1, bias 0) against a
    hidden row x[k] = k / 64: logit v is exactly ((37 v) % K) * 15 / 64, which fixes the
    nibble order within a word, the word order and the group of each scale."""
    V, K, M = 512, 1024, 2
    w = np.zeros((V, K // 8), np.uint32)
    ks = (37 * np.arange(V)) % K
    w[np.arange(V), ks // 8] = (np.uint32(15) << (4 * (ks % 8)).astype(np.uint32))
    s = np.zeros((V, K // 64), np.float16)
    s[np.arange(V), ks // 64] = 1.0
    b = np.zeros((V, K // 64), np.float16)
    x = np.tile((np.arange(K) / 64.0).astype(np.float16), (M, 1))
    am, mx, lg = _run(ctx, x, w, s, b, M, K, V)
    want = (ks * 15 / 64.0).astype(np.float32)
    assert (lg == want[None, :]).all()
    assert am.tolist() == [int(np.argmax(want))] * M


def test_lm_head_q4_shape_guards(ctx):
    import torch

    from momij_amd._lib import MomijError

    t = torch.zeros(4096, dtype=torch.int32, device="cuda")
    for K, gs, M in [(2304, 64, 1), (1024, 32, 1), (4096, 64, 17), (8192, 64, 1)]:
        with pytest.raises(MomijError) as e:
            ctx.lm_head_verify_q4(t, t, t, t, M, K, 64, t, group_size=gs)
        assert e.value.status == 3, (K, gs, M)
