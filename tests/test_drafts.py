"""CPU draft sources (drafts.cpp through the C ABI): the reference's own known-answer tests
(MomijCoreTests.swift:6-65, 147-174; SpeculativeSamplingTests.swift:47-56), and the suffix
index against brute-force substring counting over random sequences (a node's count is the
number of occurrences of its path, within the depth limit)."""
import numpy as np
import pytest

from momij_amd import drafts as D


# ---- SuffixSpec.suffixDraft (prompt lookup) ------------------------------------------------
def test_finds_repeated_suffix_draft():
    assert D.suffix_draft([7, 1, 2, 3, 9, 8, 1, 2, 3], 2) == [9, 8]


def test_finds_distant_prompt_lookup_draft():
    assert D.suffix_draft([10, 11, 12, 13, 14, 99, 98, 10, 11], 3) == [12, 13, 14]


def test_prefers_prompt_region_match():
    assert D.suffix_draft([1, 2, 3, 4, 5, 1, 2, 90, 91, 1, 2], 3, prompt_len=5) == [3, 4, 5]


def test_bigram_fallback_is_contiguous():
    assert D.suffix_draft([5, 7, 8, 9, 1, 2, 5], 3) == [7, 8, 9]


def test_adaptive_draft_length_tracks_match():
    assert D.suffix_draft([1, 2, 3, 4, 5, 6, 0, 1, 2, 3, 4], 8) == [5, 6, 0, 1, 2, 3, 4]
    assert D.adaptive_draft_k(0.0, 8) == 2
    assert D.adaptive_draft_k(0.9, 8) == 4
    assert D.adaptive_draft_k(1.6, 8) == 6
    assert D.adaptive_draft_k(3.0, 8) == 8


def test_prompt_lookup_edges():
    assert D.suffix_draft([], 4) == [] and D.suffix_draft([3], 4) == []
    assert D.suffix_draft([1, 2, 3], 0) == []
    assert D.suffix_draft([1, 2, 3, 4], 3) == []  # no repeated token


# ---- SuffixDraftIndex --------------------------------------------------------------------
def test_suffix_tree_draft_follows_frequency():
    idx = D.SuffixDraftIndex(max_depth=16)
    idx.insert([0, 1, 2, 3, 4, 4])
    idx.insert([7, 1, 2, 3, 4, 5])
    idx.insert([8, 1, 2, 3, 9])
    m, toks = idx.draft([1, 2, 3], 4, 1.0)
    assert m == 3 and toks[0] == 4
    assert D.max_spec(m, 4, 1.0) == 3
    assert idx.token_count == 17


def test_max_spec_scales_with_match_len():
    assert D.max_spec(4, 16, 1.0) == 4
    assert D.max_spec(4, 16, 2.0) == 8
    assert D.max_spec(4, 3, 2.0) == 3
    assert D.max_spec(0, 8, 1.0) == 0
    assert D.max_spec(1, 8, 0.3) == 1  # at least one with a match


def test_global_index_beats_empty_local():
    g = D.SuffixDraftIndex(max_depth=32)
    g.insert([1, 2, 3, 4, 5, 6])
    assert D.SuffixDraftIndex.best_draft(None, g, [1, 2, 3], 4, 1.0) == (3, [4, 5, 6])
    local = D.SuffixDraftIndex(max_depth=32)
    local.insert([2, 3, 7])  # shorter match: the global index still wins
    assert D.SuffixDraftIndex.best_draft(local, g, [1, 2, 3], 4, 1.0) == (3, [4, 5, 6])


def test_tree_draft_falls_back_to_pld():
    assert D.tree_draft([7, 1, 2, 3, 9, 8, 1, 2, 3], 2) == [9, 8]


def test_q_along_follows_child_frequency():
    idx = D.SuffixDraftIndex(max_depth=16)
    idx.insert([1, 2, 3, 4])
    idx.insert([1, 2, 3, 4])
    idx.insert([1, 2, 3, 9])
    q = idx.q_along([1, 2, 3], [4])
    assert len(q) == 1 and abs(q[0] - 2 / 3) < 1e-5
    assert idx.q_along([1, 2, 3], [7, 4]) == [1.0, 1.0]  # leaves the tree at once
    assert idx.q_along([1, 2, 3], []) == []


def _occurrences(seqs, pat, depth):
    if len(pat) > depth:
        return 0
    L = len(pat)
    return sum(1 for s in seqs for i in range(len(s) - L + 1) if s[i:i + L] == pat)


@pytest.mark.parametrize("seed", range(6))
def test_suffix_index_against_brute_force(seed):
    rng = np.random.default_rng(seed)
    depth = int(rng.integers(4, 9))
    seqs = [rng.integers(0, 5, int(rng.integers(3, 30))).tolist() for _ in range(5)]
    idx = D.SuffixDraftIndex(max_depth=depth)
    for s in seqs:
        idx.insert(s)
    for _ in range(20):
        hist = rng.integers(0, 5, int(rng.integers(1, 12))).tolist()
        k = int(rng.integers(1, 7))
        alpha = float(rng.choice([0.5, 1.0, 2.0]))
        m, toks = idx.draft(hist, k, alpha)
        # longest suffix (<= depth) that occurs and continues somewhere
        want_p = 0
        for p in range(min(depth, len(hist)), 0, -1):
            pat = hist[len(hist) - p:]
            if any(_occurrences(seqs, pat + [t], depth) for t in range(5)):
                want_p = p
                break
        assert m == want_p
        if want_p == 0:
            assert toks == []
            continue
        path = hist[len(hist) - want_p:]
        want = []
        for _ in range(D.max_spec(want_p, k, alpha)):
            counts = [_occurrences(seqs, path + [t], depth) for t in range(5)]
            if max(counts) == 0:
                break
            t = int(np.argmax(counts))  # lowest id among equal counts
            want.append(t)
            path = path + [t]
        assert toks == want, (hist, k, alpha, toks, want)


# ---- TokenRecycleIndex -------------------------------------------------------------------
def test_token_recycle_draft_chain():
    r = D.TokenRecycleIndex(top_k=4)
    r.observe(10, [20, 21, 22])
    r.observe(20, [30, 31])
    r.observe(30, [40])
    assert r.draft(10, 3) == [20, 30, 40]
    r.observe(10, [99, 20])  # the latest observation comes first
    assert r.draft(10, 1)[0] == 99


def test_token_recycle_merge_cycle_and_limits():
    r = D.TokenRecycleIndex(top_k=2)
    r.observe(1, [1, -5, 2, 3, 4])  # self and negative ids dropped, top_k kept
    r.observe(2, [1])
    assert r.draft(1, 5) == [2]      # 2 -> 1 would repeat: stop
    assert r.entry_count == 2
    r.observe(1, [7])
    assert r.draft(1, 1) == [7]      # merged [7, 2]
    r.observe(3, [])                 # nothing observed
    assert r.entry_count == 2
    assert r.draft(-1, 4) == [] and r.draft(5, 0) == []
    r.clear()
    assert r.entry_count == 0 and r.draft(1, 3) == []
