"""CPU draft sources for the verify step, through the C ABI (drafts.cpp): the online suffix
index (SuffixDraftIndex.swift), prompt-lookup drafting and the adaptive draft length
(SuffixSpec.swift:8-55), and token recycling (TokenRecycleIndex.swift).  Names and argument
meanings follow the reference's.
"""
from __future__ import annotations

import ctypes as C

from . import _lib

_ST = {}


def _check(st: int):
    if st != 0:
        raise _lib.MomijError(st, _lib.load().mj_status_str(st).decode())


def _arr(xs):
    xs = [int(x) for x in xs]
    return (C.c_int32 * max(len(xs), 1))(*xs), len(xs)


def max_spec(match_len: int, max_k: int, alpha: float) -> int:
    return int(_lib.load().mj_suffix_max_spec(match_len, max_k, alpha))


def adaptive_draft_k(mean_accept: float, draft_k: int) -> int:
    return int(_lib.load().mj_adaptive_draft_k(mean_accept, draft_k))


def suffix_draft(history, k: int, max_ngram: int = 16, prompt_len: int | None = None) -> list:
    """SuffixSpec.suffixDraft: prompt-lookup continuation of the history's longest suffix."""
    h, n = _arr(history)
    out = (C.c_int32 * max(k, 1))()
    m = C.c_int()
    _check(_lib.load().mj_suffix_draft_pld(h, n, k, max_ngram, prompt_len or 0, out,
                                           C.byref(m)))
    return list(out[: m.value])


class SuffixDraftIndex:
    def __init__(self, max_depth: int = 64):
        self._lib = _lib.load()
        h = C.c_void_p()
        _check(self._lib.mj_suffix_index_create(max_depth, C.byref(h)))
        self.h = h
        self.max_depth = max(4, max_depth)

    def __del__(self):
        if getattr(self, "h", None):
            self._lib.mj_suffix_index_destroy(self.h)
            self.h = None

    def clear(self):
        _check(self._lib.mj_suffix_index_clear(self.h))

    @property
    def token_count(self) -> int:
        return int(self._lib.mj_suffix_index_tokens(self.h))

    def insert(self, tokens):
        a, n = _arr(tokens)
        _check(self._lib.mj_suffix_index_insert(self.h, a, n))

    def draft(self, history, max_k: int, alpha: float = 1.0) -> tuple[int, list]:
        """(matchLen, tokens)."""
        a, n = _arr(history)
        out = (C.c_int32 * max(max_k, 1))()
        m, p = C.c_int(), C.c_int()
        _check(self._lib.mj_suffix_index_draft(self.h, a, n, max_k, alpha, out, C.byref(m),
                                               C.byref(p)))
        return p.value, list(out[: m.value])

    def q_along(self, history, draft) -> list:
        a, n = _arr(history)
        d, nd = _arr(draft)
        q = (C.c_float * max(nd, 1))()
        _check(self._lib.mj_suffix_index_q_along(self.h, a, n, d, nd, q))
        return list(q[:nd])

    @staticmethod
    def best_draft(local, global_, history, max_k: int, alpha: float) -> tuple[int, list]:
        a, n = _arr(history)
        out = (C.c_int32 * max(max_k, 1))()
        m, p = C.c_int(), C.c_int()
        _check(_lib.load().mj_suffix_best_draft(local.h if local else None,
                                                global_.h if global_ else None, a, n, max_k,
                                                alpha, out, C.byref(m), C.byref(p)))
        return p.value, list(out[: m.value])


def tree_draft(history, k: int, local=None, global_=None, alpha: float = 1.0,
               prompt_len: int | None = None) -> list:
    """SuffixSpec.treeDraft: the best tree draft, else the prompt lookup."""
    a, n = _arr(history)
    out = (C.c_int32 * max(k, 1))()
    m = C.c_int()
    _check(_lib.load().mj_tree_draft(a, n, k, local.h if local else None,
                                     global_.h if global_ else None, alpha, prompt_len or 0,
                                     out, C.byref(m)))
    return list(out[: m.value])


class TokenRecycleIndex:
    def __init__(self, top_k: int = 8):
        self._lib = _lib.load()
        h = C.c_void_p()
        _check(self._lib.mj_recycle_index_create(top_k, C.byref(h)))
        self.h = h
        self.top_k = max(2, top_k)

    def __del__(self):
        if getattr(self, "h", None):
            self._lib.mj_recycle_index_destroy(self.h)
            self.h = None

    def clear(self):
        _check(self._lib.mj_recycle_index_clear(self.h))

    def observe(self, from_token: int, candidates):
        a, n = _arr(candidates)
        _check(self._lib.mj_recycle_index_observe(self.h, from_token, a, n))

    def draft(self, last: int, max_k: int) -> list:
        out = (C.c_int32 * max(max_k, 1))()
        m = C.c_int()
        _check(self._lib.mj_recycle_index_draft(self.h, last, max_k, out, C.byref(m)))
        return list(out[: m.value])

    @property
    def entry_count(self) -> int:
        return int(self._lib.mj_recycle_index_entries(self.h))
