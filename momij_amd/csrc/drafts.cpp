// drafts.cpp -- the CPU draft sources that feed the verify step: the online suffix-tree index
// (SuffixDraftIndex.swift), prompt-lookup drafting and the adaptive draft length
// (SuffixSpec.swift:8-55), and token recycling (TokenRecycleIndex.swift).  Host code only.
//
// The index keeps its trie in one node array; a node's children are a small vector kept sorted
// by token, so lookups are binary searches and the walk order is deterministic.  The reference
// picks the most frequent child by iterating a Swift dictionary, whose order is unspecified: on
// equal counts this code takes the lowest token id.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <map>
#include <new>
#include <unordered_set>
#include <vector>

#include "momij_hip.h"

namespace {

struct SuffixNode {
    int64_t count = 0;                          // occurrences of the path ending here
    std::vector<std::pair<int32_t, int32_t>> kids;  // (token, node index), sorted by token
};

}  // namespace

struct mj_suffix_index {
    int max_depth = 64;
    int64_t token_count = 0;
    std::vector<SuffixNode> nodes{SuffixNode{}};  // node 0 = root

    int child(int node, int32_t t) const {
        const auto& k = nodes[node].kids;
        auto it = std::lower_bound(k.begin(), k.end(), std::make_pair(t, INT32_MIN));
        return (it != k.end() && it->first == t) ? it->second : -1;
    }
    int child_or_add(int node, int32_t t) {
        auto& k = nodes[node].kids;
        auto it = std::lower_bound(k.begin(), k.end(), std::make_pair(t, INT32_MIN));
        if (it != k.end() && it->first == t) return it->second;
        const int idx = (int)nodes.size();
        k.insert(it, {t, idx});  // may reallocate `k`'s storage only, not `nodes`
        nodes.emplace_back();
        return idx;
    }
    // deepest node matching the last p tokens of history, p = min(max_depth, n) .. 1, taking the
    // first match (with children when `need_kids`); returns (node, p) or (-1, 0)
    std::pair<int, int> match(const int32_t* h, int n, bool need_kids) const {
        for (int p = std::min(max_depth, n); p >= 1; --p) {
            int node = 0;
            bool ok = true;
            for (int j = n - p; j < n && ok; ++j) {
                node = child(node, h[j]);
                ok = node >= 0;
            }
            if (ok && (!need_kids || !nodes[node].kids.empty())) return {node, p};
        }
        return {-1, 0};
    }
};

struct mj_recycle_index {
    int top_k = 8;
    int64_t observe_count = 0;
    std::map<int32_t, std::vector<int32_t>> adj;
};

extern "C" {

int mj_suffix_max_spec(int match_len, int max_k, double alpha) {
    if (match_len <= 0 || max_k <= 0) return 0;
    const int raw = (int)std::trunc(alpha * (double)match_len);
    return std::max(1, std::min(max_k, raw));
}

int mj_adaptive_draft_k(double mean_accept, int draft_k) {
    const int k = std::max(1, draft_k);
    if (mean_accept >= 2.5) return k;
    if (mean_accept >= 1.5) return std::min(k, 6);
    if (mean_accept >= 0.8) return std::min(k, 4);
    if (mean_accept >= 0.4) return std::min(k, 3);
    return std::min(k, 2);
}

mj_status mj_suffix_index_create(int max_depth, mj_suffix_index** out) {
    if (!out) return MJ_INVALID_ARG;
    *out = new (std::nothrow) mj_suffix_index();
    if (!*out) return MJ_OUT_OF_MEMORY;
    (*out)->max_depth = std::max(4, max_depth);
    return MJ_OK;
}

mj_status mj_suffix_index_destroy(mj_suffix_index* idx) {
    delete idx;
    return MJ_OK;
}

mj_status mj_suffix_index_clear(mj_suffix_index* idx) {
    if (!idx) return MJ_INVALID_ARG;
    idx->nodes.assign(1, SuffixNode{});
    idx->token_count = 0;
    return MJ_OK;
}

int64_t mj_suffix_index_tokens(const mj_suffix_index* idx) { return idx ? idx->token_count : 0; }

mj_status mj_suffix_index_insert(mj_suffix_index* idx, const int32_t* tokens, int n) {
    if (!idx || n < 0 || (n > 0 && !tokens)) return MJ_INVALID_ARG;
    if (n == 0) return MJ_OK;
    try {
        idx->token_count += n;
        for (int i = 0; i < n; ++i) {
            int node = 0;
            const int end = std::min(n, i + idx->max_depth);
            for (int j = i; j < end; ++j) {
                node = idx->child_or_add(node, tokens[j]);
                idx->nodes[node].count += 1;
            }
        }
    } catch (const std::bad_alloc&) {
        return MJ_OUT_OF_MEMORY;
    }
    return MJ_OK;
}

mj_status mj_suffix_index_draft(const mj_suffix_index* idx, const int32_t* history, int n,
                                int max_k, double alpha, int32_t* out_tokens, int* out_n,
                                int* out_match_len) {
    if (!idx || !out_n || !out_match_len || n < 0 || (n > 0 && !history) ||
        (max_k > 0 && !out_tokens))
        return MJ_INVALID_ARG;
    *out_n = 0;
    *out_match_len = 0;
    if (n == 0 || max_k <= 0) return MJ_OK;
    const auto [start, p] = idx->match(history, n, true);
    if (start < 0) return MJ_OK;
    *out_match_len = p;
    const int spec = mj_suffix_max_spec(p, max_k, alpha);
    int node = start;
    for (int s = 0; s < spec; ++s) {
        const auto& kids = idx->nodes[node].kids;
        if (kids.empty()) break;
        int best = -1;
        int64_t best_c = -1;
        for (const auto& [t, c] : kids)  // ascending token: the first of equal counts wins
            if (idx->nodes[c].count > best_c) {
                best_c = idx->nodes[c].count;
                best = c;
                out_tokens[*out_n] = t;
            }
        if (best < 0) break;
        *out_n += 1;
        node = best;
    }
    return MJ_OK;
}

mj_status mj_suffix_best_draft(const mj_suffix_index* local, const mj_suffix_index* global,
                               const int32_t* history, int n, int max_k, double alpha,
                               int32_t* out_tokens, int* out_n, int* out_match_len) {
    if (!out_n || !out_match_len || (max_k > 0 && !out_tokens)) return MJ_INVALID_ARG;
    *out_n = 0;
    *out_match_len = 0;
    std::vector<int32_t> tmp(std::max(max_k, 1));
    for (const mj_suffix_index* idx : {local, global}) {
        if (!idx) continue;
        int dn = 0, dm = 0;
        const mj_status s = mj_suffix_index_draft(idx, history, n, max_k, alpha, tmp.data(), &dn,
                                                  &dm);
        if (s != MJ_OK) return s;
        if (dm > *out_match_len || (dm == *out_match_len && dn > *out_n)) {
            *out_match_len = dm;
            *out_n = dn;
            std::copy(tmp.begin(), tmp.begin() + dn, out_tokens);
        }
    }
    return MJ_OK;
}

mj_status mj_suffix_index_q_along(const mj_suffix_index* idx, const int32_t* history, int n,
                                  const int32_t* draft, int n_draft, float* out_q) {
    if (!idx || n < 0 || n_draft < 0 || (n > 0 && !history) ||
        (n_draft > 0 && (!draft || !out_q)))
        return MJ_INVALID_ARG;
    for (int i = 0; i < n_draft; ++i) out_q[i] = 1.0f;
    if (n_draft == 0 || n == 0) return MJ_OK;
    int node = idx->match(history, n, false).first;
    if (node < 0) return MJ_OK;
    for (int i = 0; i < n_draft; ++i) {
        int64_t total = 0;
        for (const auto& kc : idx->nodes[node].kids) total += idx->nodes[kc.second].count;
        const int c = idx->child(node, draft[i]);
        if (total <= 0 || c < 0) break;
        out_q[i] = std::max(1e-6f, (float)idx->nodes[c].count / (float)total);
        node = c;
    }
    return MJ_OK;
}

mj_status mj_suffix_draft_pld(const int32_t* history, int n, int k, int max_ngram,
                              int prompt_len, int32_t* out_tokens, int* out_n) {
    if (!out_n || n < 0 || (n > 0 && !history) || (k > 0 && !out_tokens)) return MJ_INVALID_ARG;
    *out_n = 0;
    if (n < 2 || k <= 0) return MJ_OK;
    const int max_pattern = std::min(max_ngram, n - 1);
    auto search = [&](bool prefer_prompt) -> bool {
        for (int plen = max_pattern; plen >= 1; --plen) {
            const int ps = n - plen;
            for (int st = ps - 1; st >= 0; --st) {
                if (prefer_prompt && prompt_len > 0 && st >= prompt_len) continue;
                bool ok = true;
                for (int j = 0; j < plen && ok; ++j) ok = history[st + j] == history[ps + j];
                if (!ok) continue;
                const int cont = st + plen, avail = n - cont;
                if (avail <= 0) continue;
                const int take = std::min(k, avail);
                std::copy(history + cont, history + cont + take, out_tokens);
                *out_n = take;
                return true;
            }
        }
        return false;
    };
    if (prompt_len > 0 && search(true)) return MJ_OK;
    search(false);
    return MJ_OK;
}

mj_status mj_tree_draft(const int32_t* history, int n, int k, const mj_suffix_index* local,
                        const mj_suffix_index* global, double alpha, int prompt_len,
                        int32_t* out_tokens, int* out_n) {
    int m = 0;
    mj_status s = mj_suffix_best_draft(local, global, history, n, k, alpha, out_tokens, out_n, &m);
    if (s != MJ_OK || *out_n > 0) return s;
    return mj_suffix_draft_pld(history, n, k, 16, prompt_len, out_tokens, out_n);
}

mj_status mj_recycle_index_create(int top_k, mj_recycle_index** out) {
    if (!out) return MJ_INVALID_ARG;
    *out = new (std::nothrow) mj_recycle_index();
    if (!*out) return MJ_OUT_OF_MEMORY;
    (*out)->top_k = std::max(2, top_k);
    return MJ_OK;
}

mj_status mj_recycle_index_destroy(mj_recycle_index* r) {
    delete r;
    return MJ_OK;
}

mj_status mj_recycle_index_clear(mj_recycle_index* r) {
    if (!r) return MJ_INVALID_ARG;
    r->adj.clear();
    r->observe_count = 0;
    return MJ_OK;
}

mj_status mj_recycle_index_observe(mj_recycle_index* r, int32_t from_token,
                                   const int32_t* candidates, int n) {
    if (!r || n < 0 || (n > 0 && !candidates)) return MJ_INVALID_ARG;
    if (from_token < 0 || n == 0) return MJ_OK;
    r->observe_count += 1;
    std::vector<int32_t> merged;
    std::unordered_set<int32_t> seen;
    auto add = [&](int32_t t) {
        if ((int)merged.size() >= r->top_k || t < 0 || t == from_token) return;
        if (seen.insert(t).second) merged.push_back(t);
    };
    for (int i = 0; i < n; ++i) add(candidates[i]);
    auto it = r->adj.find(from_token);
    if (it != r->adj.end())
        for (int32_t t : it->second) add(t);
    if (!merged.empty()) r->adj[from_token] = merged;
    return MJ_OK;
}

mj_status mj_recycle_index_draft(const mj_recycle_index* r, int32_t last, int max_k,
                                 int32_t* out_tokens, int* out_n) {
    if (!r || !out_n || (max_k > 0 && !out_tokens)) return MJ_INVALID_ARG;
    *out_n = 0;
    if (max_k <= 0 || last < 0) return MJ_OK;
    std::unordered_set<int32_t> seen{last};
    int32_t cur = last;
    for (int i = 0; i < max_k; ++i) {
        auto it = r->adj.find(cur);
        if (it == r->adj.end() || it->second.empty()) break;
        const int32_t nx = it->second.front();
        if (!seen.insert(nx).second) break;
        out_tokens[(*out_n)++] = nx;
        cur = nx;
    }
    return MJ_OK;
}

int mj_recycle_index_entries(const mj_recycle_index* r) { return r ? (int)r->adj.size() : 0; }

}  // extern "C"
