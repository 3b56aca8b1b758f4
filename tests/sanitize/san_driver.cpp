// Sanitizer driver (test infrastructure): runs the CPU oracle and the host-side draft sources
// under AddressSanitizer + UndefinedBehaviorSanitizer on small seeded inputs, including the
// edge cases their callers hit (empty drafts, single rows, ring wrap, banned ids, ties, empty
// histories, repeated tokens).  Built and run by tests/test_sanitizers.py; exits non-zero (the
// sanitizers abort) on the first invalid access or undefined operation.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "momij_hip.h"
#include "momij_oracle.h"

namespace {

std::mt19937_64 rng(12345);

std::vector<uint16_t> normal_f16(size_t n, float sd) {
    std::normal_distribution<float> d(0.0f, sd);
    std::vector<uint16_t> v(n);
    for (auto& x : v) x = or_f2h(d(rng));
    return v;
}

std::vector<uint32_t> codes(size_t n) {
    std::vector<uint32_t> v(n);
    for (auto& x : v) x = (uint32_t)rng();
    return v;
}

std::vector<uint16_t> scales(size_t n) {
    std::uniform_real_distribution<float> d(0.005f, 0.02f);
    std::vector<uint16_t> v(n);
    for (auto& x : v) x = or_f2h(d(rng));
    return v;
}

std::vector<uint16_t> neg15(const std::vector<uint16_t>& s) {
    std::vector<uint16_t> b(s.size());
    for (size_t i = 0; i < s.size(); ++i) b[i] = or_f2h(-1.5f * or_h2f(s[i]));
    return b;
}

void check(bool ok, const char* what) {
    if (!ok) {
        std::fprintf(stderr, "check failed: %s\n", what);
        std::exit(2);
    }
}

void run_qmm2() {
    const int E = 3, N = 64, K = 512, gs = 64, ktop = 2, M = 3;
    auto w = codes((size_t)E * N * K / 16);
    auto s = scales((size_t)E * N * K / gs);
    auto b = neg15(s);
    auto x = normal_f16((size_t)M * ktop * K, 1.0f);
    std::vector<int32_t> inds = {0, 2, 1, 1, 2, 0};
    std::vector<uint16_t> y((size_t)M * ktop * N);
    or_qmm2(x.data(), w.data(), s.data(), b.data(), inds.data(), y.data(), M, ktop, K, N, gs, 0);
    or_qmm2(x.data(), w.data(), s.data(), b.data(), inds.data(), y.data(), M, ktop, K, N, gs, 1);
}

struct Moe {
    int E, k, H, I, gs;
    std::vector<uint16_t> norm, router, ugs, ugb, ds, db;
    std::vector<uint32_t> ugw, dw;
    or_moe_w w;
    Moe(int E_, int k_, int H_, int I_, int gs_) : E(E_), k(k_), H(H_), I(I_), gs(gs_) {
        norm = normal_f16(H, 0.1f);
        for (auto& v : norm) v = or_f2h(1.0f + or_h2f(v));
        router = normal_f16((size_t)E * H, 0.02f);
        ugw = codes((size_t)E * 2 * I * H / 16);
        ugs = scales((size_t)E * 2 * I * H / gs);
        ugb = neg15(ugs);
        dw = codes((size_t)E * H * I / 16);
        ds = scales((size_t)E * H * I / gs);
        db = neg15(ds);
        w = {norm.data(), router.data(), ugw.data(), ugs.data(), ugb.data(),
             dw.data(), ds.data(), db.data(), E, k, H, I, gs, 1e-6f};
    }
};

void run_moe() {
    Moe m(8, 4, 512, 512, 64);
    for (int M : {1, 5}) {
        auto x = normal_f16((size_t)M * m.H, 1.0f);
        std::vector<uint16_t> y(x.size());
        std::vector<int32_t> inds((size_t)M * m.k);
        std::vector<float> sc((size_t)M * m.k);
        or_moe_block(&m.w, x.data(), y.data(), M, OR_MOE_PRENORM | OR_MOE_RESIDUAL, inds.data(),
                     sc.data());
        for (int v : inds) check(v >= 0 && v < m.E, "moe expert id");
        or_moe_block(&m.w, x.data(), y.data(), M, 0, inds.data(), sc.data());
    }
    // all-tied router: lowest ids win
    std::vector<float> logits(2 * 8, 0.0f);
    std::vector<int32_t> inds(2 * 4);
    std::vector<float> sc(2 * 4);
    or_route_topk(logits.data(), inds.data(), sc.data(), 2, 8, 4);
    check(inds[0] == 0 && inds[3] == 3, "tied route order");
}

struct Attn {
    or_cfg cfg;
    std::vector<uint16_t> norm, qkvs, qkvb, qn, kn, os, ob;
    std::vector<uint32_t> qkvw, ow;
    or_attn_w w;
    std::vector<float> inv_freq;
    Attn(int window, int rope_dim, int64_t C) {
        const int H = 512, nQ = 4, nKV = 2, D = 128, gs = 64;
        cfg = {H, nQ, nKV, D, rope_dim, window, gs, 1e6f, 1e-6f, C};
        norm = normal_f16(H, 0.1f);
        const int nqkv = (nQ + 2 * nKV) * D;
        qkvw = codes((size_t)nqkv * H / 16);
        qkvs = scales((size_t)nqkv * H / gs);
        qkvb = neg15(qkvs);
        qn = normal_f16(D, 0.1f);
        kn = normal_f16(D, 0.1f);
        ow = codes((size_t)H * nQ * D / 16);
        os = scales((size_t)H * nQ * D / gs);
        ob = neg15(os);
        w = {norm.data(), qkvw.data(), qkvs.data(), qkvb.data(), qn.data(), kn.data(),
             ow.data(), os.data(), ob.data()};
        inv_freq.resize(rope_dim > 0 ? rope_dim / 2 : 1);
        if (rope_dim > 0) or_rope_inv_freq(inv_freq.data(), rope_dim, 1e6f);
    }
};

void run_attention() {
    for (int window : {0, 16}) {
        for (int rope_dim : {0, 64, 128}) {
            const int64_t C = 40;
            Attn a(window, rope_dim, C);
            auto kc = normal_f16((size_t)a.cfg.nKV * C * a.cfg.D, 1.0f);
            auto vc = normal_f16(kc.size(), 1.0f);
            // chain, tree and one row; L past the ring size (wrap)
            std::vector<std::vector<int32_t>> trees = {{-1}, {-1, 0, 1, 2}, {-1, 0, 0, 1, 1, 2}};
            for (auto& par : trees) {
                const int M = (int)par.size();
                auto h = normal_f16((size_t)M * a.cfg.H, 1.0f);
                or_attn_block(&a.cfg, &a.w, a.inv_freq.data(), h.data(), kc.data(), vc.data(),
                              53, par.data(), M);
            }
            std::vector<int32_t> path = {0, 2, 5};
            or_kv_commit(kc.data(), vc.data(), a.cfg.nKV, C, a.cfg.D, 53, path.data(), 3);
        }
    }
}

void run_layer() {
    Attn a(16, 64, 48);
    Moe m(8, 4, 512, 512, 64);
    or_layer_w lw = {a.w, m.w};
    auto kc = normal_f16((size_t)a.cfg.nKV * 48 * a.cfg.D, 1.0f);
    auto vc = normal_f16(kc.size(), 1.0f);
    std::vector<int32_t> par = {-1, 0, 1};
    auto h = normal_f16((size_t)3 * 512, 1.0f);
    std::vector<int32_t> inds(3 * 4);
    std::vector<float> sc(3 * 4);
    or_layer_forward(&a.cfg, &lw, a.inv_freq.data(), h.data(), kc.data(), vc.data(), 20,
                     par.data(), 3, inds.data(), sc.data());
}

void run_head_and_accept() {
    const int M = 4, K = 256, V = 300;
    auto x = normal_f16((size_t)M * K, 1.0f);
    auto w = normal_f16((size_t)V * K, 0.02f);
    std::vector<float> logits((size_t)M * V);
    or_lm_head_logits(x.data(), w.data(), logits.data(), M, K, V);
    std::vector<int32_t> am(M);
    std::vector<float> best(M), second(M);
    std::vector<int32_t> banned = {7, 299};
    or_argmax_rows(logits.data(), M, V, banned.data(), 2, am.data(), best.data(), second.data());
    or_argmax_rows(logits.data(), M, V, nullptr, 0, am.data(), best.data(), second.data());
    // greedy: chain, tree, a single row
    std::vector<int32_t> tokens = {5, am[0], 9, am[2]}, parents = {-1, 0, 1, 2};
    std::vector<int32_t> path(M + 1), emit(M + 1);
    int acc = or_accept_greedy(tokens.data(), parents.data(), am.data(), M, path.data(), emit.data());
    check(acc >= 0 && acc < M, "greedy accepted");
    acc = or_accept_greedy(tokens.data(), parents.data(), am.data(), 1, path.data(), emit.data());
    check(acc == 0, "one row accepts nothing");
    // sampled, both q modes, with and without penalties / top-p; an empty draft
    std::vector<float> u((size_t)M * 2);
    or_verify_uniforms(7, 3, M, u.data());
    std::vector<int32_t> draft = {am[0], 17, am[2]};
    int32_t tok = -1;
    for (int qm : {0, 1}) {
        acc = or_accept_sampled(logits.data(), M, V, draft.data(), 0.7f, qm, nullptr, u.data(), &tok);
        check(acc >= 0 && acc < M && tok >= 0 && tok < V, "sampled");
        acc = or_accept_sampled(logits.data(), 1, V, draft.data(), 0.7f, qm, nullptr, u.data(), &tok);
        check(acc == 0 && tok >= 0 && tok < V, "sampled one row");
    }
    std::vector<int32_t> ht = {3, 17, 250}, hc = {1, 4, 2};
    for (float top_p : {1.0f, 0.9f, 1e-6f}) {
        acc = or_accept_sampled_ex(logits.data(), M, V, draft.data(), 0.7f, top_p, 1.1f, 0.1f, 0.1f,
                                   ht.data(), hc.data(), 3, 1, nullptr, u.data(), &tok);
        check(acc >= 0 && tok >= 0 && tok < V, "sampled ex");
        acc = or_accept_sampled_ex(logits.data(), M, V, draft.data(), 0.7f, top_p, 1.0f, 0.0f, 0.0f,
                                   nullptr, nullptr, 0, 0, nullptr, u.data(), &tok);
        check(acc >= 0 && tok >= 0 && tok < V, "sampled ex no history");
    }
    std::vector<float> e(V);
    for (int i = 0; i < V; ++i) e[i] = (float)((i * 37) % 11) / 11.0f;
    const float Z = or_canon_sum(e.data(), V);
    check(or_canon_walk(e.data(), V, Z * 0.5f) < V, "canonical walk");
    check(or_nucleus_sample(e.data(), V, Z, 0.5f, 0.3f) < V, "nucleus");
    uint64_t st = 42;
    std::vector<int32_t> ids = {4, 9, 11};
    std::vector<float> cl = {1.0f, 2.0f, 0.5f};
    (void)or_try_accept(9, ids.data(), cl.data(), 3, 0.7f, 1.0f, &st, &tok);
}

void run_drafts() {
    mj_suffix_index *loc = nullptr, *glob = nullptr;
    check(mj_suffix_index_create(8, &loc) == MJ_OK && mj_suffix_index_create(8, &glob) == MJ_OK,
          "suffix create");
    std::vector<int32_t> seq;
    for (int i = 0; i < 400; ++i) seq.push_back((int32_t)((i * i + 3 * i) % 23));
    check(mj_suffix_index_insert(glob, seq.data(), (int)seq.size()) == MJ_OK, "insert");
    check(mj_suffix_index_insert(loc, seq.data(), 50) == MJ_OK, "insert local");
    check(mj_suffix_index_insert(loc, seq.data(), 0) == MJ_OK, "insert empty");
    int32_t out[16];
    int n = 0, match = 0;
    for (int hn : {0, 1, 5, 40}) {
        mj_suffix_index_draft(glob, seq.data() + 100, hn, 8, 1.0, out, &n, &match);
        mj_suffix_best_draft(loc, glob, seq.data() + 100, hn, 8, 1.0, out, &n, &match);
        mj_suffix_best_draft(nullptr, glob, seq.data() + 100, hn, 8, 1.0, out, &n, &match);
        mj_suffix_draft_pld(seq.data(), 200 + hn, 8, 16, 50, out, &n);
        mj_tree_draft(seq.data(), 200 + hn, 8, loc, glob, 1.0, 50, out, &n);
        float q[8];
        if (n > 0) mj_suffix_index_q_along(glob, seq.data() + 100, hn, out, n, q);
    }
    mj_suffix_draft_pld(seq.data(), 1, 8, 16, 0, out, &n);
    (void)mj_adaptive_draft_k(0.0, 8);
    (void)mj_adaptive_draft_k(7.5, 8);
    (void)mj_suffix_max_spec(0, 8, 1.0);
    check(mj_suffix_index_clear(loc) == MJ_OK, "clear");
    mj_suffix_index_destroy(loc);
    mj_suffix_index_destroy(glob);
    mj_recycle_index* r = nullptr;
    check(mj_recycle_index_create(4, &r) == MJ_OK, "recycle create");
    for (int i = 0; i < 200; ++i) {
        int32_t cands[5] = {(int32_t)((i + 1) % 31), (int32_t)((i + 7) % 31), 3, 3, (int32_t)(i % 5)};
        mj_recycle_index_observe(r, (int32_t)(i % 31), cands, 1 + i % 5);
    }
    mj_recycle_index_observe(r, 1, nullptr, 0);
    mj_recycle_index_draft(r, 3, 8, out, &n);
    mj_recycle_index_draft(r, 1000, 8, out, &n);
    (void)mj_recycle_index_entries(r);
    mj_recycle_index_clear(r);
    mj_recycle_index_destroy(r);
    // small limits are raised to the minimum (depth 4, top_k 2); a missing out pointer refused
    check(mj_suffix_index_create(1, &loc) == MJ_OK, "depth raised");
    mj_suffix_index_insert(loc, seq.data(), 30);
    mj_suffix_index_draft(loc, seq.data(), 30, 8, 1.0, out, &n, &match);
    mj_suffix_index_destroy(loc);
    check(mj_recycle_index_create(1, &r) == MJ_OK, "top_k raised");
    mj_recycle_index_destroy(r);
    check(mj_suffix_index_create(8, nullptr) == MJ_INVALID_ARG, "null out");
    check(mj_recycle_index_create(4, nullptr) == MJ_INVALID_ARG, "null out");
}

}  // namespace

int main() {
    or_set_threads(2);
    run_qmm2();
    run_moe();
    run_attention();
    run_layer();
    run_head_and_accept();
    run_drafts();
    std::printf("sanitizer driver: all cases ran\n");
    return 0;
}
