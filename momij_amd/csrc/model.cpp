// model.cpp -- the resident verify stack behind the C ABI.
//
// mj_model mirrors SeedlessLayerStack / SeedlessDecodeEngine (SeedlessAttn.swift:369-593,
// SeedlessDecodeEngine.swift:194-327, 516-545, 1541-1603): caller-owned weights, a KV ring per
// layer ([2][n_kv][C][128] fp16, committed position p at slot p % C), scratch sized for
// MJ_MAX_ROWS rows, an absolute offset (committed tokens).  A verify pass is one stream of
// kernels (embed -> layers -> final norm -> lm_head (+ greedy acceptance in its final launch)
// -> sampled acceptance -> KV commit for a tree -> result copy) with a single host wait.  Per-pass parameters live in a device StepDesc so the pass can be
// captured once per (kind, rows) into a HIP graph and replayed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstring>
#include <map>
#include <vector>

#include "mj_abi_internal.h"
#include "mj_internal.h"

// PASS_SAMPLED_NUC: a sampled pass whose bonus (or zero-mass residual) takes a nucleus.
// PASS_PEN marks a sampled pass with penalties: the logits are rewritten, so the row maxima are
// recomputed; without it the lm_head's maxima are used and those launches are left out.
// PASS_TREE marks a greedy pass over a draft tree that is not a chain: only then can the
// accepted path leave the rows' KV out of place (path[i] != i), so only then is it compacted.
enum PassKind {
    PASS_PREFILL = 0,
    PASS_CHAIN = 1,
    PASS_GREEDY = 2,
    PASS_SAMPLED = 3,
    PASS_SAMPLED_NUC = 4,
    PASS_PEN = 8,
    PASS_TREE = 16
};

static bool sampled_pass(int kind) {
    return (kind & ~PASS_PEN) == PASS_SAMPLED || (kind & ~PASS_PEN) == PASS_SAMPLED_NUC;
}

struct mj_model {
    mj_ctx* ctx = nullptr;
    mj_model_config cfg{};
    std::vector<mj_layer_weights> layers;
    std::vector<int> lwin, lrope;  // per-layer sliding window (0 = full) and rope dims
    const uint16_t* embed = nullptr;
    const uint16_t* final_norm = nullptr;
    const uint16_t* lm_head = nullptr;
    uint16_t* kv = nullptr;
    int64_t layer_stride = 0;  // halves per layer
    float* inv_freq = nullptr;
    int max_chunks = 0;
    // pass scratch
    void* arena = nullptr;
    uint16_t *h, *xperm, *qkv, *aperm, *xf;
    float2* rope_cs;
    float2 *xsum, *asum, *mlpart;
    float *opart, *pval, *rowmax, *logits, *bsum, *maxv;
    int* pidx;
    int32_t* argmax;
    int32_t *hist_tok, *hist_cnt;  // sampled passes: the seen tokens (ascending) and counts
    int32_t* hist_host = nullptr;   // pinned [2][MJ_MAX_HIST]: the history now on the device
    int hist_n = -1;                // its length (-1: none uploaded)
    NucleusBuf nuc{};
    int32_t *inds_all;
    float* scores_all;
    MoeScratch ms{};
    StepDesc* sd_dev = nullptr;
    StepDesc* sd_host = nullptr;
    StepResult* res_dev = nullptr;
    StepResult* res_host = nullptr;
    int64_t offset = 0;
    bool graphs = true;
    std::map<int, hipGraphExec_t> graph_cache;
    mj_capture cap{};  // debug capture (device pointers; all null: off)
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    float last_ms = -1.0f;
    bool profiling = false;
    Prof prof;
    double prof_ms[PROF_CLASSES] = {};
    long prof_n[PROF_CLASSES] = {};
};

static mj_status model_fail(mj_model* m, mj_status s, const char* what) {
    return mj_fail(m->ctx, s, "%s", what);
}

// Depth and ancestor masks of a pass; parents == nullptr means a chain.
static mj_status fill_tree(mj_ctx* ctx, StepDesc* sd, const int32_t* parents, int M) {
    sd->chain = 1;
    for (int r = 0; r < M; ++r) {
        const int p = parents ? parents[r] : r - 1;
        if (r == 0 ? p != -1 : (p < 0 || p >= r))
            return mj_fail(ctx, MJ_INVALID_ARG, "bad tree: parents[%d] = %d (need parents[0] = -1,"
                           " 0 <= parents[r] < r)", r, p);
        sd->parents[r] = p;
        if (p != r - 1) sd->chain = 0;
        sd->depth[r] = r == 0 ? 0 : sd->depth[p] + 1;
        sd->anc[r] = (r == 0 ? 0ull : sd->anc[p]) | (1ull << r);
    }
    return MJ_OK;
}

hipError_t set_kernel_attributes();

// Layer l of a pass.  Its input norm (attention RMSNorm into xperm / xsum) was written by
// whatever produced h: the embedding for layer 0, the previous layer's expert combine
// otherwise; its own expert combine writes the next one (or the final norm into xf).
static mj_status enqueue_layer(mj_model* m, int l, int M, int kind, hipStream_t st) {
    mj_ctx* ctx = m->ctx;
    const mj_model_config& c = m->cfg;
    const mj_layer_weights& w = m->layers[l];
    const int H = c.H, nQ = c.n_heads, nKV = c.n_kv_heads, D = c.head_dim;
    const int qkvN = (nQ + 2 * nKV) * D;
    const int* ab = ctx->abort_dev;
    mj_status s;
    GatherArgs q{};
    q.xperm = m->xperm;
    q.xsum = m->xsum;
    q.w = w.attn.qkv_w;
    q.s = (const uint16_t*)w.attn.qkv_s;
    q.b = (const uint16_t*)w.attn.qkv_b;
    q.bk = nullptr;
    q.dense_rows = M;
    q.y = m->qkv;
    q.K = H;
    q.N = qkvN;
    q.gs = c.gs;
    q.x_div = 1;
    q.abort = ab;
    Prof* pf = m->profiling ? &m->prof : nullptr;
    // raw q / k / v rows; the attention kernel finishes q and k and appends k and v
    if (pf) pf->begin(PROF_DENSE, st);
    s = mj_hip(ctx, launch_gather(q, EPI_STORE, M, 1, st), "qkv");
    if (pf) pf->end(st);
    if (s != MJ_OK) return s;
    AttnArgs a{};
    a.qkv = m->qkv;
    a.q_norm_w = (const uint16_t*)w.attn.q_norm_w;
    a.k_norm_w = (const uint16_t*)w.attn.k_norm_w;
    a.rope_cs = m->rope_cs;
    a.sd = m->sd_dev;
    a.kc = m->kv + (int64_t)l * m->layer_stride;
    a.vc = a.kc + (int64_t)nKV * c.kv_capacity * 128;
    a.opart = m->opart;
    a.mlpart = m->mlpart;
    a.out_perm = m->aperm;
    a.out_sum = m->asum;
    a.M = M;
    a.nQ = nQ;
    a.nKV = nKV;
    a.rope_dim = m->lrope[l];
    a.window = m->lwin[l];
    a.max_chunks = m->max_chunks;
    a.C = c.kv_capacity;
    a.eps = c.eps;
    a.scale = (float)std::pow((double)D, -0.5);
    a.abort = ab;
    if (pf) pf->begin(PROF_ATTN, st);
    s = mj_hip(ctx, launch_attn(a, st), "attention");
    if (pf) pf->end(st);
    if (s != MJ_OK) return s;
    GatherArgs o{};
    o.xperm = m->aperm;
    o.xsum = m->asum;
    o.w = w.attn.o_w;
    o.s = (const uint16_t*)w.attn.o_s;
    o.b = (const uint16_t*)w.attn.o_b;
    o.bk = nullptr;
    o.dense_rows = M;
    o.y = m->h;
    o.K = nQ * D;
    o.N = H;
    o.gs = c.gs;
    o.x_div = 1;
    o.abort = ab;
    if (pf) pf->begin(PROF_DENSE, st);
    s = mj_hip(ctx, launch_gather(o, EPI_ADD, M, 1, st), "o proj");
    if (pf) pf->end(st);
    if (s != MJ_OK) return s;
    const size_t rowsH = (size_t)MJ_MAX_ROWS * H;
    if (m->cap.attn_out) {
        s = mj_hip(ctx, hipMemcpyAsync((uint16_t*)m->cap.attn_out + l * rowsH, m->h, (size_t)M * H * 2,
                                       hipMemcpyDeviceToDevice, st), "capture");
        if (s != MJ_OK) return s;
    }
    int32_t* inds = m->inds_all + (size_t)l * MJ_MAX_ROWS * c.top_k;
    float* scores = m->scores_all + (size_t)l * MJ_MAX_ROWS * c.top_k;
    NormOut next{};
    const bool last = l + 1 == c.n_layers;
    if (!last)
        next = NormOut{(const uint16_t*)m->layers[l + 1].attn.norm_w, c.eps, nullptr, m->xperm,
                       m->xsum};
    else
        next = NormOut{m->final_norm, c.eps, m->xf, nullptr, nullptr};
    s = run_moe(ctx, &w.moe, m->h, m->h, M, MJ_MOE_PRENORM | MJ_MOE_RESIDUAL, m->ms, inds,
                scores, st, pf, (last && kind == PASS_PREFILL) ? nullptr : &next);
    if (s != MJ_OK) return s;
    // the route wrote the normed rows plain into ms.xn (want_plain) and the logits into ms.logits
    if (m->cap.moe_in) {
        s = mj_hip(ctx, hipMemcpyAsync((uint16_t*)m->cap.moe_in + l * rowsH, m->ms.xn,
                                       (size_t)M * H * 2, hipMemcpyDeviceToDevice, st), "capture");
        if (s != MJ_OK) return s;
    }
    if (m->cap.router_logits) {
        s = mj_hip(ctx, hipMemcpyAsync(m->cap.router_logits + (size_t)l * MJ_MAX_ROWS * c.E,
                                       m->ms.logits, (size_t)M * c.E * 4, hipMemcpyDeviceToDevice,
                                       st), "capture");
        if (s != MJ_OK) return s;
    }
    return MJ_OK;
}

static mj_status enqueue_pass(mj_model* m, int kind, int M, hipStream_t st) {
    mj_ctx* ctx = m->ctx;
    const mj_model_config& c = m->cfg;
    const int H = c.H;
    const int* ab = ctx->abort_dev;
    mj_status s;
    const NormOut first{(const uint16_t*)m->layers[0].attn.norm_w, c.eps, nullptr, m->xperm,
                        m->xsum};
    const RopeTab rt{m->inv_freq, m->rope_cs, c.rope_dim / 2};
    if (H == 2048) {
        s = mj_hip(ctx, launch_embed_norm(m->embed, m->sd_dev, M, H, m->h, first, rt, ab, st),
                   "embed + norm");
    } else {
        s = mj_hip(ctx, launch_embed(m->embed, m->sd_dev, M, H, m->h, rt, ab, st), "embed");
        if (s == MJ_OK)
            s = mj_hip(ctx, launch_rmsnorm_qx(m->h, first.w, c.eps, nullptr, m->xperm, m->xsum, M,
                                              H, ab, st), "attn norm");
    }
    if (s != MJ_OK) return s;
    if (m->cap.h) {
        s = mj_hip(ctx, hipMemcpyAsync(m->cap.h, m->h, (size_t)M * H * 2, hipMemcpyDeviceToDevice,
                                       st), "capture");
        if (s != MJ_OK) return s;
    }
    for (int l = 0; l < c.n_layers; ++l) {
        s = enqueue_layer(m, l, M, kind, st);
        if (s != MJ_OK) return s;
        if (m->cap.h) {
            s = mj_hip(ctx, hipMemcpyAsync((uint16_t*)m->cap.h + (size_t)(l + 1) * MJ_MAX_ROWS * H,
                                           m->h, (size_t)M * H * 2, hipMemcpyDeviceToDevice, st),
                       "capture");
            if (s != MJ_OK) return s;
        }
        if (m->cap.inds) {
            s = mj_hip(ctx, hipMemcpyAsync(m->cap.inds + (size_t)l * MJ_MAX_ROWS * c.top_k,
                                           m->inds_all + (size_t)l * MJ_MAX_ROWS * c.top_k,
                                           (size_t)M * c.top_k * 4, hipMemcpyDeviceToDevice, st),
                       "capture");
            if (s != MJ_OK) return s;
        }
    }
    if (m->cap.kv_rows) {
        s = mj_hip(ctx, launch_kv_rows(m->kv, m->layer_stride, c.n_layers, c.kv_capacity,
                                       c.n_kv_heads, m->sd_dev, (uint16_t*)m->cap.kv_rows, st),
                   "capture");
        if (s != MJ_OK) return s;
    }
    if (kind != PASS_PREFILL) {
        // the last layer's expert combine wrote the final norm into xf
        if (m->cap.head_in) {
            s = mj_hip(ctx, hipMemcpyAsync(m->cap.head_in, m->xf, (size_t)M * H * 2,
                                           hipMemcpyDeviceToDevice, st), "capture");
            if (s != MJ_OK) return s;
        }
        float* logits =
            (sampled_pass(kind) || m->cap.logits) ? m->logits : nullptr;
        // a greedy pass's acceptance runs in the head's final launch
        const int32_t* toks = (const int32_t*)((char*)m->sd_dev + offsetof(StepDesc, tokens));
        const int32_t* pars = (const int32_t*)((char*)m->sd_dev + offsetof(StepDesc, parents));
        const GreedyAccept ga{toks, pars, m->res_dev};
        const GreedyAccept* gap = sampled_pass(kind) ? nullptr : &ga;
        if (m->profiling) m->prof.begin(PROF_HEAD, st);
        if (c.head_bits == 4)
            s = mj_hip(ctx,
                       launch_lm_head_q4(m->xf, (const uint32_t*)m->lm_head,
                                         (const uint16_t*)c.lm_head_scales,
                                         (const uint16_t*)c.lm_head_biases, M, H, c.vocab, nullptr,
                                         0, logits, m->pval, m->pidx, m->argmax, m->maxv,
                                         HeadLse{}, ab, st, gap),
                       "lm_head q4");
        else
            s = mj_hip(ctx, launch_lm_head(m->xf, m->lm_head, M, H, c.vocab, nullptr, 0, logits,
                                           m->pval, m->pidx, m->argmax, m->maxv, HeadLse{}, ab,
                                           st, gap),
                       "lm_head");
        if (m->profiling) m->prof.end(st);
        if (s != MJ_OK) return s;
        if (m->cap.logits) {
            s = mj_hip(ctx, hipMemcpyAsync(m->cap.logits, m->logits, (size_t)M * c.vocab * 4,
                                           hipMemcpyDeviceToDevice, st), "capture");
            if (s != MJ_OK) return s;
        }
        if (sampled_pass(kind)) {
            SampleOpts o{};
            o.hist_tok = m->hist_tok;
            o.hist_cnt = m->hist_cnt;
            const bool nuc = (kind & ~PASS_PEN) == PASS_SAMPLED_NUC;
            s = mj_hip(ctx, launch_accept_sampled(m->logits, M, c.vocab, nullptr, 1.0f, 0, nullptr,
                                                  0, 0, o, nuc ? &m->nuc : nullptr, m->rowmax,
                                                  m->bsum, nullptr, m->res_dev, m->sd_dev, ab, st,
                                                  (kind & PASS_PEN) ? nullptr : m->maxv),
                       "sampled accept");
        }
        if (s != MJ_OK) return s;
        if (kind & PASS_TREE) {
            s = mj_hip(ctx, launch_kv_commit(m->kv, m->layer_stride, c.n_layers, c.kv_capacity,
                                             c.n_kv_heads, m->sd_dev, m->res_dev, ab, st),
                       "kv commit");
            if (s != MJ_OK) return s;
        }
        s = mj_hip(ctx, hipMemcpyAsync(m->res_host, m->res_dev, sizeof(StepResult),
                                       hipMemcpyDeviceToHost, st), "result copy");
    }
    return s;
}

// Upload the descriptor, run the pass (graph or eager), wait once.
static mj_status run_pass(mj_model* m, int kind, int M) {
    mj_ctx* ctx = m->ctx;
    hipStream_t st = ctx->stream;
    unsigned gen = 0;
    mj_status s = mj_abort_begin(ctx, &gen);  // set: nothing is queued
    if (s != MJ_OK) return s;
    hipSetDevice(ctx->device);
    s = mj_hip(ctx, hipMemcpyAsync(m->sd_dev, m->sd_host, sizeof(StepDesc),
                                   hipMemcpyHostToDevice, st), "descriptor upload");
    if (s != MJ_OK) return s;
    const mj_capture& cp = m->cap;
    const bool capturing = cp.h || cp.inds || cp.logits || cp.attn_out || cp.moe_in ||
                           cp.router_logits || cp.head_in || cp.kv_rows;
    const bool capture_ok = m->graphs && !capturing && !m->profiling;
    m->prof.used = 0;
    // A profiled pass is queued behind a hold, so every kernel starts as soon as its
    // predecessor ends: its event pair then brackets the kernel, not the host's launch gap.
    if (m->profiling && !capture_ok) {
        s = mj_hip(ctx, launch_hold(15000, st), "hold");
        if (s != MJ_OK) return s;
        // timer calibration: the same event bracket around holds of known length
        for (int j = 0; j < 8; ++j) {
            m->prof.begin(PROF_TIMER, st);
            s = mj_hip(ctx, launch_hold(PROF_TIMER_US, st), "hold");
            m->prof.end(st);
            if (s != MJ_OK) return s;
        }
    }
    hipEventRecord(m->ev0, st);
    if (capture_ok) {
        const int key = kind * 1000 + M;
        auto it = m->graph_cache.find(key);
        if (it == m->graph_cache.end()) {
            hipGraph_t g = nullptr;
            s = mj_hip(ctx, hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "capture");
            if (s != MJ_OK) return s;
            mj_status es = enqueue_pass(m, kind, M, st);
            hipError_t ee = hipStreamEndCapture(st, &g);
            if (es != MJ_OK) return es;
            s = mj_hip(ctx, ee, "end capture");
            if (s != MJ_OK) return s;
            hipGraphExec_t ex = nullptr;
            s = mj_hip(ctx, hipGraphInstantiate(&ex, g, nullptr, nullptr, 0), "instantiate");
            hipGraphDestroy(g);
            if (s != MJ_OK) return s;
            it = m->graph_cache.emplace(key, ex).first;
        }
        s = mj_hip(ctx, hipGraphLaunch(it->second, st), "graph launch");
    } else {
        s = enqueue_pass(m, kind, M, st);
    }
    if (s != MJ_OK) return s;
    hipEventRecord(m->ev1, st);
    s = mj_hip(ctx, hipStreamSynchronize(st), "pass sync");
    if (s != MJ_OK) return s;
    hipEventElapsedTime(&m->last_ms, m->ev0, m->ev1);
    if (m->profiling) {
        for (int i = 0; i + 1 < m->prof.used; i += 2) {
            float ms = 0.0f;
            if (m->prof.valid[i / 2] &&
                hipEventElapsedTime(&ms, m->prof.pool[i], m->prof.pool[i + 1]) == hipSuccess) {
                m->prof_ms[m->prof.cls[i / 2]] += ms;
                m->prof_n[m->prof.cls[i / 2]] += 1;
            }
        }
    }
    return mj_abort_end(ctx, gen);
}

static mj_status check_rows(mj_model* m, int M) {
    const mj_model_config& c = m->cfg;
    if (M < 1 || M > MJ_MAX_ROWS)
        return mj_fail(m->ctx, MJ_INVALID_ARG, "rows %d outside 1..%d", M, MJ_MAX_ROWS);
    bool any_full = false;
    for (int w : m->lwin) any_full = any_full || w <= 0;
    if (any_full && m->offset + M > c.kv_capacity)
        return mj_fail(m->ctx, MJ_CAPACITY, "kv capacity %lld exceeded at offset %lld + %d",
                       (long long)c.kv_capacity, (long long)m->offset, M);
    return MJ_OK;
}

extern "C" {

mj_status mj_model_create(mj_ctx* ctx, const mj_model_config* cfg, const mj_layer_weights* layers,
                          const void* embed, const void* final_norm_w, const void* lm_head,
                          mj_model** out) {
    if (!ctx || !cfg || !layers || !embed || !final_norm_w || !lm_head || !out)
        return mj_fail(ctx, MJ_INVALID_ARG, "model_create: null argument");
    *out = nullptr;
    const mj_model_config& c = *cfg;
    if (c.head_dim != 128 || c.n_heads % 4 != 0 || c.n_kv_heads < 1 ||
        c.n_heads % c.n_kv_heads != 0 || c.H % 2048 != 0 || c.H > 4096 ||
        (c.rope_dim != 0 && c.rope_dim != 32 && c.rope_dim != 64 && c.rope_dim != 128) ||
        c.top_k < 1 || c.top_k > 8 || c.E < c.top_k || c.E > MJ_MAX_EXPERTS ||
        c.I % 512 != 0 || c.I > 4096 || (c.gs != 64 && c.gs != 128) || c.vocab < 16 ||
        c.vocab > 196608 || c.n_layers < 1 || c.n_heads * 128 % 512 != 0)
        return mj_fail(ctx, MJ_UNSUPPORTED_SHAPE, "model_create: unsupported configuration");
    std::vector<int> lwin(c.n_layers, c.window), lrope(c.n_layers, c.rope_dim);
    for (int l = 0; l < c.n_layers; ++l) {
        if (c.layer_window) lwin[l] = c.layer_window[l];
        if (c.layer_rope_dim) lrope[l] = c.layer_rope_dim[l];
        if (lrope[l] != 0 && lrope[l] != c.rope_dim)
            return mj_fail(ctx, MJ_UNSUPPORTED_SHAPE,
                           "model_create: layer %d rope_dim %d (0 or rope_dim %d)", l, lrope[l],
                           c.rope_dim);
        if (lwin[l] > 0 && c.kv_capacity < (int64_t)lwin[l] + MJ_MAX_ROWS)
            return mj_fail(ctx, MJ_CAPACITY, "kv_capacity must be >= window + %d", MJ_MAX_ROWS);
        if (lwin[l] <= 0 && c.kv_capacity < MJ_MAX_ROWS)
            return mj_fail(ctx, MJ_CAPACITY, "kv_capacity too small");
    }
    if (c.head_bits != 0 && c.head_bits != 16 &&
        (c.head_bits != 4 || !c.lm_head_scales || !c.lm_head_biases || c.H > 2048 ||
         c.gs <= 0))
        return mj_fail(ctx, MJ_UNSUPPORTED_SHAPE,
                       "model_create: head_bits %d (16, or 4 with scales and biases, H <= 2048)",
                       c.head_bits);
    for (int l = 0; l < c.n_layers; ++l) {
        const mj_moe_weights& mw = layers[l].moe;
        if (!mw.router_w || !mw.up_gate_w || !mw.up_gate_s || !mw.up_gate_b || !mw.down_w ||
            !mw.down_s || !mw.down_b || !mw.norm_w ||
            ((uintptr_t)mw.up_gate_alpha | (uintptr_t)mw.down_alpha) % 16 != 0)
            return mj_fail(ctx, MJ_INVALID_ARG,
                           "model_create: layer %d expert weights: null pointer or row-alpha "
                           "array not 16-byte aligned", l);
        // the pass scratch is sized from the model configuration: every layer's expert shape
        // must be that one
        if (mw.E != c.E || mw.top_k != c.top_k || mw.H != c.H || mw.I != c.I || mw.gs != c.gs)
            return mj_fail(ctx, MJ_INVALID_ARG,
                           "model_create: layer %d experts E=%d top_k=%d H=%d I=%d gs=%d differ "
                           "from the model's E=%d top_k=%d H=%d I=%d gs=%d", l, mw.E, mw.top_k,
                           mw.H, mw.I, mw.gs, c.E, c.top_k, c.H, c.I, c.gs);
        const mj_attn_weights& aw = layers[l].attn;
        if (!aw.norm_w || !aw.qkv_w || !aw.qkv_s || !aw.qkv_b || !aw.q_norm_w || !aw.k_norm_w ||
            !aw.o_w || !aw.o_s || !aw.o_b)
            return mj_fail(ctx, MJ_INVALID_ARG, "model_create: layer %d attention weights: null "
                           "pointer", l);
    }
    hipSetDevice(ctx->device);
    mj_status s = mj_hip(ctx, set_kernel_attributes(), "kernel attributes");
    if (s != MJ_OK) return s;
    mj_model* m = new mj_model();
    m->ctx = ctx;
    m->cfg = c;
    m->layers.assign(layers, layers + c.n_layers);
    m->lwin = lwin;
    m->lrope = lrope;
    // the layer arrays are the caller's: the copy keeps no pointer to them
    m->cfg.layer_window = nullptr;
    m->cfg.layer_rope_dim = nullptr;
    m->embed = (const uint16_t*)embed;
    m->final_norm = (const uint16_t*)final_norm_w;
    m->lm_head = (const uint16_t*)lm_head;
    const int H = c.H, nQ = c.n_heads, nKV = c.n_kv_heads, R = MJ_MAX_ROWS;
    const int qkvN = (nQ + 2 * nKV) * 128;
    m->layer_stride = 2LL * nKV * c.kv_capacity * 128;
    m->max_chunks = 0;
    for (int w : lwin) m->max_chunks = std::max(m->max_chunks, attn_max_chunks(w, c.kv_capacity, R));
    const int gqa = nQ / nKV;
    const int nqt16 = ((R * gqa + 15) / 16) * 16;
    auto layout = [&](Arena& a) {
        m->h = (uint16_t*)a.take((size_t)R * H * 2);
        m->xperm = (uint16_t*)a.take((size_t)R * H * 2);
        m->xsum = (float2*)a.take((size_t)R * (H / 64) * 8);
        m->qkv = (uint16_t*)a.take((size_t)R * qkvN * 2);
        m->rope_cs = (float2*)a.take((size_t)R * MJ_ROPE_F * sizeof(float2));
        m->opart = (float*)a.take((size_t)nKV * m->max_chunks * nqt16 * 128 * 4);
        m->mlpart = (float2*)a.take((size_t)nKV * m->max_chunks * nqt16 * 8);
        m->aperm = (uint16_t*)a.take((size_t)R * nQ * 128 * 2);
        m->asum = (float2*)a.take((size_t)R * nQ * 2 * 8);
        m->xf = (uint16_t*)a.take((size_t)R * H * 2);
        m->pval = (float*)a.take((size_t)head_blocks() * 32 * 4);
        m->pidx = (int*)a.take((size_t)head_blocks() * 32 * 4);
        m->argmax = (int32_t*)a.take((size_t)R * 4);
        m->maxv = (float*)a.take((size_t)R * 4);
        m->rowmax = (float*)a.take((size_t)R * 4);
        m->logits = (float*)a.take((size_t)R * c.vocab * 4);
        m->bsum = (float*)a.take(sample_scratch_floats(R, c.vocab) * 4);
        m->hist_tok = (int32_t*)a.take((size_t)MJ_MAX_HIST * 4);
        m->hist_cnt = (int32_t*)a.take((size_t)MJ_MAX_HIST * 4);
        nucleus_layout(a.take(nucleus_bytes(c.vocab)), c.vocab, m->nuc);
        m->inds_all = (int32_t*)a.take((size_t)c.n_layers * R * c.top_k * 4);
        m->scores_all = (float*)a.take((size_t)c.n_layers * R * c.top_k * 4);
        m->sd_dev = (StepDesc*)a.take(sizeof(StepDesc));
        m->res_dev = (StepResult*)a.take(sizeof(StepResult));
        MoeScratch& ms = m->ms;
        ms.xn = (uint16_t*)a.take((size_t)R * H * 2);
        ms.xperm = (uint16_t*)a.take((size_t)R * H * 2);
        ms.xsum = (float2*)a.take((size_t)R * (H / 64) * 8);
        ms.logits = (float*)a.take((size_t)R * c.E * 4);
        ms.inds = (int32_t*)a.take((size_t)R * c.top_k * 4);
        ms.scores = (float*)a.take((size_t)R * c.top_k * 4);
        ms.bk = (Buckets*)a.take(sizeof(Buckets));
        ms.act = (uint16_t*)a.take((size_t)R * c.top_k * c.I * 2);
        ms.act_sum = (float2*)a.take((size_t)R * c.top_k * (c.I / 64) * 8);
        ms.down = (uint16_t*)a.take((size_t)R * c.top_k * H * 2);
        ms.ecnt = (int*)a.take((size_t)c.E * 4);
        ms.eplist = (int*)a.take((size_t)c.E * MJ_MAX_ROWS * 4);
        ms.srec = (int*)a.take((size_t)64 * 64 * 4);
    };
    Arena count;
    layout(count);
    std::vector<float> inv(c.rope_dim > 0 ? c.rope_dim / 2 : 1, 1.0f);
    for (int i = 0; c.rope_dim > 0 && i < c.rope_dim / 2; ++i)
        inv[i] = powf(c.rope_base, -(float)i / (float)(c.rope_dim / 2));
    if (hipMalloc(&m->arena, count.off) != hipSuccess ||
        hipMalloc(&m->kv, (size_t)c.n_layers * m->layer_stride * 2) != hipSuccess ||
        hipMalloc(&m->inv_freq, inv.size() * 4) != hipSuccess ||
        hipHostMalloc(&m->sd_host, sizeof(StepDesc), hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc(&m->res_host, sizeof(StepResult), hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc(&m->hist_host, (size_t)2 * MJ_MAX_HIST * 4, hipHostMallocDefault) !=
            hipSuccess ||
        hipEventCreate(&m->ev0) != hipSuccess || hipEventCreate(&m->ev1) != hipSuccess) {
        mj_model_destroy(m);
        return mj_fail(ctx, MJ_HIP_ERROR, "model_create: allocation failed");
    }
    Arena real{m->arena, 0};
    layout(real);
    std::memset(m->sd_host, 0, sizeof(StepDesc));
    std::memset(m->res_host, 0, sizeof(StepResult));
    s = mj_hip(ctx, hipMemcpy(m->inv_freq, inv.data(), inv.size() * 4, hipMemcpyHostToDevice),
               "inv_freq upload");
    if (s == MJ_OK)
        s = mj_hip(ctx, hipMemset(m->kv, 0, (size_t)c.n_layers * m->layer_stride * 2), "kv clear");
    // pass scratch starts zeroed: an aborted pass leaves empty expert buckets behind
    if (s == MJ_OK) s = mj_hip(ctx, hipMemset(m->arena, 0, count.off), "scratch clear");
    if (s == MJ_OK) s = mj_hip(ctx, hipDeviceSynchronize(), "create sync");
    if (s != MJ_OK) {
        mj_model_destroy(m);
        return s;
    }
    *out = m;
    return MJ_OK;
}

mj_status mj_model_destroy(mj_model* m) {
    if (!m) return MJ_INVALID_ARG;
    hipSetDevice(m->ctx->device);
    hipStreamSynchronize(m->ctx->stream);
    for (auto& kv : m->graph_cache) hipGraphExecDestroy(kv.second);
    for (int i = 0; i < m->prof.cap; ++i) hipEventDestroy(m->prof.pool[i]);
    delete[] m->prof.pool;
    if (m->arena) hipFree(m->arena);
    if (m->kv) hipFree(m->kv);
    if (m->inv_freq) hipFree(m->inv_freq);
    if (m->sd_host) hipHostFree(m->sd_host);
    if (m->res_host) hipHostFree(m->res_host);
    if (m->hist_host) hipHostFree(m->hist_host);
    if (m->ev0) hipEventDestroy(m->ev0);
    if (m->ev1) hipEventDestroy(m->ev1);
    delete m;
    return MJ_OK;
}

int64_t mj_model_offset(const mj_model* m) { return m ? m->offset : -1; }

mj_status mj_model_rewind(mj_model* m, int64_t offset) {
    if (!m) return MJ_INVALID_ARG;
    if (offset < 0 || offset > m->offset)
        return mj_fail(m->ctx, MJ_INVALID_ARG, "rewind to %lld outside 0..%lld", (long long)offset,
                       (long long)m->offset);
    m->offset = offset;
    return MJ_OK;
}

mj_status mj_model_kv(mj_model* m, int layer, void** k, void** v) {
    if (!m || !k || !v || layer < 0 || layer >= m->cfg.n_layers) return MJ_INVALID_ARG;
    *k = m->kv + (int64_t)layer * m->layer_stride;
    *v = (uint16_t*)*k + (int64_t)m->cfg.n_kv_heads * m->cfg.kv_capacity * 128;
    return MJ_OK;
}

mj_status mj_model_set_capture(mj_model* m, void* h, int32_t* inds, float* logits) {
    if (!m) return MJ_INVALID_ARG;
    m->cap = mj_capture{};
    m->cap.h = h;
    m->cap.inds = inds;
    m->cap.logits = logits;
    m->ms.want_plain = false;
    return MJ_OK;
}

mj_status mj_model_set_capture_ex(mj_model* m, const mj_capture* cap) {
    if (!m) return MJ_INVALID_ARG;
    m->cap = cap ? *cap : mj_capture{};
    m->ms.want_plain = m->cap.moe_in != nullptr;
    return MJ_OK;
}

mj_status mj_model_set_graphs(mj_model* m, int enable) {
    if (!m) return MJ_INVALID_ARG;
    m->graphs = enable != 0;
    return MJ_OK;
}

float mj_model_last_pass_ms(const mj_model* m) { return m ? m->last_ms : -1.0f; }

mj_status mj_model_profile(mj_model* m, int enable) {
    if (!m) return MJ_INVALID_ARG;
    if (enable && !m->prof.pool) {
        m->prof.cap = 2048;
        m->prof.pool = new hipEvent_t[m->prof.cap];
        // timing-only events: no system-scope cache write-back / invalidate at each record,
        // which would otherwise sit inside every bracketed kernel's measured time
        for (int i = 0; i < m->prof.cap; ++i)
            if (hipEventCreateWithFlags(&m->prof.pool[i], hipEventDisableSystemFence) !=
                hipSuccess)
                return mj_fail(m->ctx, MJ_HIP_ERROR, "profile events");
    }
    m->profiling = enable != 0;
    for (int c = 0; c < PROF_CLASSES; ++c) {
        m->prof_ms[c] = 0.0;
        m->prof_n[c] = 0;
    }
    return MJ_OK;
}

float mj_model_kernel_ms(const mj_model* m, int kernel_class, int64_t* launches) {
    if (!m || kernel_class < 0 || kernel_class >= PROF_CLASSES) return -1.0f;
    if (launches) *launches = m->prof_n[kernel_class];
    return (float)m->prof_ms[kernel_class];
}

static mj_status feed_rows(mj_model* m, const int32_t* tokens, const int32_t* parents, int M,
                           int kind) {
    mj_status s = check_rows(m, M);
    if (s != MJ_OK) return s;
    StepDesc* sd = m->sd_host;
    sd->L = m->offset;
    sd->M = M;
    for (int r = 0; r < M; ++r) {
        if (tokens[r] < 0 || tokens[r] >= m->cfg.vocab)
            return mj_fail(m->ctx, MJ_INVALID_ARG, "token %d outside the vocabulary", tokens[r]);
        sd->tokens[r] = tokens[r];
    }
    s = fill_tree(m->ctx, sd, parents, M);
    if (s != MJ_OK) return s;
    if (kind == PASS_GREEDY && !sd->chain) kind |= PASS_TREE;
    return run_pass(m, kind, M);
}

mj_status mj_prefill(mj_model* m, const int32_t* tokens, int n, int chunk, int32_t* out_next) {
    if (!m || !tokens || n < 1) return MJ_INVALID_ARG;
    if (chunk < 1 || chunk > MJ_MAX_ROWS) chunk = MJ_MAX_ROWS;
    for (int i = 0; i < n; i += chunk) {
        const int M = n - i < chunk ? n - i : chunk;
        const bool last = i + M >= n;
        mj_status s = feed_rows(m, tokens + i, nullptr, M, last ? PASS_CHAIN : PASS_PREFILL);
        if (s != MJ_OK) return s;
        m->offset += M;
        if (last && out_next) *out_next = m->res_host->argmax[M - 1];
    }
    return MJ_OK;
}

mj_status mj_step_chain_feeds(mj_model* m, const int32_t* feeds, int M, int32_t* out_evals) {
    if (!m || !feeds) return MJ_INVALID_ARG;
    mj_status s = feed_rows(m, feeds, nullptr, M, PASS_CHAIN);
    if (s != MJ_OK) return s;
    m->offset += M;
    if (out_evals)
        for (int r = 0; r < M; ++r) out_evals[r] = m->res_host->argmax[r];
    return MJ_OK;
}

mj_status mj_verify_greedy(mj_model* m, int32_t y, const int32_t* draft, int n_draft,
                           const int32_t* parents, int32_t* out_accepted, int32_t* out_tokens) {
    if (!m || (n_draft > 0 && !draft) || n_draft < 0) return MJ_INVALID_ARG;
    const int M = n_draft + 1;
    if (M > MJ_MAX_ROWS)
        return mj_fail(m->ctx, MJ_INVALID_ARG, "draft of %d nodes exceeds %d", n_draft,
                       MJ_MAX_ROWS - 1);
    int32_t rows[MJ_MAX_ROWS];
    rows[0] = y;
    for (int i = 0; i < n_draft; ++i) rows[i + 1] = draft[i];
    mj_status s = feed_rows(m, rows, parents, M, PASS_GREEDY);
    if (s != MJ_OK) return s;
    const StepResult* r = m->res_host;
    m->offset += r->accepted + 1;
    if (out_accepted) *out_accepted = r->accepted;
    if (out_tokens)
        for (int i = 0; i <= r->accepted; ++i) out_tokens[i] = r->emit[i];
    return MJ_OK;
}

// The LogitsProcessor options of a sampled call, checked, with the history ranked by token
// (the penalty kernel looks drafts up in it); NULL = temperature only.
static mj_status sampling_prep(mj_ctx* ctx, const mj_sampling* sp, SampleOpts& o,
                               std::vector<int32_t>& tok, std::vector<int32_t>& cnt) {
    o = SampleOpts{};
    tok.clear();
    cnt.clear();
    if (!sp) return MJ_OK;
    if (!std::isfinite(sp->top_p) || !std::isfinite(sp->repetition_penalty) ||
        !std::isfinite(sp->presence_penalty) || !std::isfinite(sp->frequency_penalty) ||
        sp->n_hist < 0 || sp->n_hist > MJ_MAX_HIST ||
        (sp->n_hist > 0 && (!sp->hist_tokens || !sp->hist_counts)))
        return mj_fail(ctx, MJ_INVALID_ARG, "sampling options: bad argument");
    o.top_p = sp->top_p;
    o.rep = sp->repetition_penalty;
    o.pres = sp->presence_penalty;
    o.freq = sp->frequency_penalty;
    std::vector<std::pair<int32_t, int32_t>> h(sp->n_hist);
    bool sorted = true;
    for (int i = 0; i < sp->n_hist; ++i) {
        if (sp->hist_counts[i] < 0)
            return mj_fail(ctx, MJ_INVALID_ARG, "sampling options: negative count");
        h[i] = {sp->hist_tokens[i], sp->hist_counts[i]};
        sorted = sorted && (i == 0 || h[i - 1].first <= h[i].first);
    }
    if (!sorted) std::sort(h.begin(), h.end());
    for (size_t i = 1; i < h.size(); ++i)
        if (h[i].first == h[i - 1].first)
            return mj_fail(ctx, MJ_INVALID_ARG, "sampling options: token %d listed twice",
                           h[i].first);
    for (auto& e : h) {
        tok.push_back(e.first);
        cnt.push_back(e.second);
    }
    o.n_hist = (int)h.size();
    return MJ_OK;
}

mj_status mj_verify_sampled_ex(mj_model* m, int32_t y, const int32_t* draft, int n_draft,
                               const mj_sampling* sp, int q_mode, const float* q_point,
                               uint64_t seed, uint64_t counter, int32_t* out_accepted,
                               int32_t* out_token) {
    if (!m || !sp || (n_draft > 0 && !draft) || n_draft < 0) return MJ_INVALID_ARG;
    if (!(sp->temperature > 1e-5f))
        return mj_fail(m->ctx, MJ_INVALID_ARG, "sampled verify needs temperature > 1e-5");
    if (q_mode != MJ_Q_POINT && q_mode != MJ_Q_UNIFORM)
        return mj_fail(m->ctx, MJ_INVALID_ARG, "unknown q_mode %d", q_mode);
    const int M = n_draft + 1;
    if (M > MJ_MAX_ROWS) return mj_fail(m->ctx, MJ_INVALID_ARG, "draft too long");
    SampleOpts o;
    std::vector<int32_t> ht, hc;
    mj_status s = sampling_prep(m->ctx, sp, o, ht, hc);
    if (s != MJ_OK) return s;
    StepDesc* sd = m->sd_host;
    sd->seed = seed;
    sd->counter = counter;
    sd->temperature = sp->temperature;
    sd->q_mode = q_mode;
    sd->q_uniform = 1.0f / (float)m->cfg.vocab;
    sd->has_qpoint = q_point ? 1 : 0;
    for (int i = 0; i < n_draft; ++i) sd->q_point[i] = q_point ? q_point[i] : 1.0f;
    sd->top_p = o.top_p;
    sd->rep = o.rep;
    sd->pres = o.pres;
    sd->freq = o.freq;
    sd->n_hist = o.n_hist;
    // the history goes up only when it differs from the one already on the device (the previous
    // call waited for its pass, so the pinned copy is free to rewrite)
    const size_t hn = ht.size();
    if (o.n_hist > 0 &&
        (m->hist_n != (int)hn || std::memcmp(m->hist_host, ht.data(), hn * 4) != 0 ||
         std::memcmp(m->hist_host + MJ_MAX_HIST, hc.data(), hn * 4) != 0)) {
        std::memcpy(m->hist_host, ht.data(), hn * 4);
        std::memcpy(m->hist_host + MJ_MAX_HIST, hc.data(), hn * 4);
        hipSetDevice(m->ctx->device);
        s = mj_hip(m->ctx, hipMemcpyAsync(m->hist_tok, m->hist_host, hn * 4,
                                          hipMemcpyHostToDevice, m->ctx->stream), "history");
        if (s == MJ_OK)
            s = mj_hip(m->ctx, hipMemcpyAsync(m->hist_cnt, m->hist_host + MJ_MAX_HIST, hn * 4,
                                              hipMemcpyHostToDevice, m->ctx->stream), "history");
        m->hist_n = s == MJ_OK ? (int)hn : -1;
        if (s != MJ_OK) return s;
    }
    int32_t rows[MJ_MAX_ROWS];
    rows[0] = y;
    for (int i = 0; i < n_draft; ++i) rows[i + 1] = draft[i];
    const bool pen = (std::fabs(o.rep - 1.0f) > 1e-6f && o.rep > 0.0f) || o.pres != 0.0f ||
                     o.freq != 0.0f;
    s = feed_rows(m, rows, nullptr, M,
                  (o.top_p < 1.0f - 1e-6f ? PASS_SAMPLED_NUC : PASS_SAMPLED) | (pen ? PASS_PEN : 0));
    if (s != MJ_OK) return s;
    const StepResult* r = m->res_host;
    m->offset += r->accepted + 1;
    if (out_accepted) *out_accepted = r->accepted;
    if (out_token) *out_token = r->token;
    return MJ_OK;
}

mj_status mj_verify_sampled(mj_model* m, int32_t y, const int32_t* draft, int n_draft,
                            float temperature, int q_mode, const float* q_point, uint64_t seed,
                            uint64_t counter, int32_t* out_accepted, int32_t* out_token) {
    mj_sampling sp{};
    sp.temperature = temperature;
    sp.top_p = 1.0f;
    sp.repetition_penalty = 1.0f;
    return mj_verify_sampled_ex(m, y, draft, n_draft, &sp, q_mode, q_point, seed, counter,
                                out_accepted, out_token);
}

// ------------------------------------------------------------------ op-level entries
mj_status mj_attn_block(mj_ctx* ctx, const mj_attn_config* cfg, const mj_attn_weights* w,
                        void* h, void* kcache, void* vcache, int64_t L,
                        const int32_t* parents_host, int M) {
    if (!ctx) return MJ_INVALID_ARG;
    if (!cfg || !w || !h || !kcache || !vcache || M < 1 || M > MJ_MAX_ROWS || L < 0)
        return mj_fail(ctx, MJ_INVALID_ARG, "attn_block: bad argument");
    const mj_attn_config& c = *cfg;
    if (c.head_dim != 128 || c.n_heads % 4 != 0 || c.n_heads % c.n_kv_heads != 0 ||
        c.H % 2048 != 0 || (c.rope_dim != 0 && c.rope_dim != 32 && c.rope_dim != 64 &&
                            c.rope_dim != 128) || (c.gs != 64 && c.gs != 128))
        return mj_fail(ctx, MJ_UNSUPPORTED_SHAPE, "attn_block: unsupported configuration");
    if (c.window > 0 ? c.kv_capacity < (int64_t)c.window + M : c.kv_capacity < L + M)
        return mj_fail(ctx, MJ_CAPACITY, "attn_block: kv capacity %lld too small",
                       (long long)c.kv_capacity);
    hipSetDevice(ctx->device);
    mj_status s = mj_hip(ctx, set_kernel_attributes(), "kernel attributes");
    if (s != MJ_OK) return s;
    StepDesc sd{};
    sd.L = L;
    sd.M = M;
    s = fill_tree(ctx, &sd, parents_host, M);
    if (s != MJ_OK) return s;
    const int H = c.H, nQ = c.n_heads, nKV = c.n_kv_heads;
    const int qkvN = (nQ + 2 * nKV) * 128;
    const int maxc = attn_max_chunks(c.window, L, M);
    const int nqt16 = ((M * (nQ / nKV) + 15) / 16) * 16;
    std::vector<float> inv(c.rope_dim > 0 ? c.rope_dim / 2 : 1, 1.0f);
    for (int i = 0; c.rope_dim > 0 && i < c.rope_dim / 2; ++i)
        inv[i] = powf(c.rope_base, -(float)i / (float)(c.rope_dim / 2));
    auto layout = [&](Arena& a, void** p) {
        p[0] = a.take((size_t)M * H * 2);                 // xperm
        p[1] = a.take((size_t)M * (H / 64) * 8);          // xsum
        p[2] = a.take((size_t)M * qkvN * 2);              // qkv
        p[3] = a.take((size_t)M * MJ_ROPE_F * sizeof(float2));  // RoPE table
        p[4] = a.take((size_t)nKV * maxc * nqt16 * 128 * 4);
        p[5] = a.take((size_t)nKV * maxc * nqt16 * 8);
        p[6] = a.take((size_t)M * nQ * 128 * 2);          // aperm
        p[7] = a.take((size_t)M * nQ * 2 * 8);            // asum
        p[8] = a.take(sizeof(StepDesc));
        p[9] = a.take(inv.size() * 4);
    };
    void* p[10];
    Arena count;
    layout(count, p);
    s = mj_scratch_reserve(ctx, count.off);
    if (s != MJ_OK) return s;
    Arena real{ctx->scratch, 0};
    layout(real, p);
    hipStream_t st = ctx->stream;
    s = mj_hip(ctx, hipMemcpyAsync(p[8], &sd, sizeof sd, hipMemcpyHostToDevice, st), "sd upload");
    if (s == MJ_OK)
        s = mj_hip(ctx, hipMemcpyAsync(p[9], inv.data(), inv.size() * 4, hipMemcpyHostToDevice, st),
                   "inv_freq upload");
    if (s == MJ_OK) s = mj_hip(ctx, hipStreamSynchronize(st), "upload sync");
    if (s != MJ_OK) return s;
    const int* ab = ctx->abort_dev;
    s = mj_hip(ctx, launch_rmsnorm_qx((const uint16_t*)h, (const uint16_t*)w->norm_w, c.eps,
                                      nullptr, (uint16_t*)p[0], (float2*)p[1], M, H, ab, st),
               "attn norm");
    if (s != MJ_OK) return s;
    GatherArgs q{};
    q.xperm = (uint16_t*)p[0];
    q.xsum = (float2*)p[1];
    q.w = w->qkv_w;
    q.s = (const uint16_t*)w->qkv_s;
    q.b = (const uint16_t*)w->qkv_b;
    q.dense_rows = M;
    q.y = (uint16_t*)p[2];
    q.K = H;
    q.N = qkvN;
    q.gs = c.gs;
    q.x_div = 1;
    q.abort = ab;
    const RopeTab rt{(const float*)p[9], (float2*)p[3], c.rope_dim / 2};
    s = mj_hip(ctx, launch_rope_table((const StepDesc*)p[8], M, rt, st), "rope table");
    if (s != MJ_OK) return s;
    s = mj_hip(ctx, launch_gather(q, EPI_STORE, M, 1, st), "qkv");
    if (s != MJ_OK) return s;
    AttnArgs a{};
    a.qkv = (uint16_t*)p[2];
    a.q_norm_w = (const uint16_t*)w->q_norm_w;
    a.k_norm_w = (const uint16_t*)w->k_norm_w;
    a.rope_cs = (const float2*)p[3];
    a.sd = (StepDesc*)p[8];
    a.kc = (uint16_t*)kcache;
    a.vc = (uint16_t*)vcache;
    a.opart = (float*)p[4];
    a.mlpart = (float2*)p[5];
    a.out_perm = (uint16_t*)p[6];
    a.out_sum = (float2*)p[7];
    a.M = M;
    a.nQ = nQ;
    a.nKV = nKV;
    a.rope_dim = c.rope_dim;
    a.window = c.window;
    a.max_chunks = maxc;
    a.C = c.kv_capacity;
    a.eps = c.eps;
    a.scale = (float)std::pow(128.0, -0.5);
    a.abort = ab;
    s = mj_hip(ctx, launch_attn(a, st), "attention");
    if (s != MJ_OK) return s;
    GatherArgs o{};
    o.xperm = (uint16_t*)p[6];
    o.xsum = (float2*)p[7];
    o.w = w->o_w;
    o.s = (const uint16_t*)w->o_s;
    o.b = (const uint16_t*)w->o_b;
    o.dense_rows = M;
    o.y = (uint16_t*)h;
    o.K = nQ * 128;
    o.N = H;
    o.gs = c.gs;
    o.x_div = 1;
    o.abort = ab;
    return mj_hip(ctx, launch_gather(o, EPI_ADD, M, 1, st), "o proj");
}

// Scratch for the head's block partials: value/index and, with a log-sum-exp output, the
// (max, sum) pairs.  Returns the pointers in p[0..3] (p[2], p[3] null without lse).
static mj_status head_scratch(mj_ctx* ctx, bool lse, void* p[4]) {
    const size_t part = (size_t)head_blocks() * 32 * 4;
    Arena count;
    for (int i = 0; i < (lse ? 4 : 2); ++i) count.take(part);
    mj_status s = mj_scratch_reserve(ctx, count.off);
    if (s != MJ_OK) return s;
    Arena real{ctx->scratch, 0};
    for (int i = 0; i < 4; ++i) p[i] = i < (lse ? 4 : 2) ? real.take(part) : nullptr;
    return MJ_OK;
}

// Temperature check shared by both heads: the log-sum-exp is of logits / T, T > 1e-5 (the
// sampled regime of LogitsProcessor.probabilities, LogitsProcessor.swift:168-189).
static bool head_lse_arg_ok(float temperature, const float* out_lse) {
    return !out_lse || (temperature > 1e-5f && std::isfinite(temperature));
}

mj_status mj_lm_head_verify(mj_ctx* ctx, const void* x, const void* w, int M, int K, int V,
                            const int32_t* banned, int n_banned, float temperature,
                            int32_t* out_argmax, float* out_row_max, float* out_row_logsumexp,
                            float* out_logits) {
    if (!ctx) return MJ_INVALID_ARG;
    if (!x || !w || !out_argmax || M < 1 || M > MJ_MAX_ROWS || V < 1 || n_banned < 0 ||
        (n_banned > 0 && !banned))
        return mj_fail(ctx, MJ_INVALID_ARG, "lm_head_verify: bad argument (M must be 1..%d)",
                       MJ_MAX_ROWS);
    if (n_banned > MJ_HEAD_MAX_BANNED)
        return mj_fail(ctx, MJ_INVALID_ARG, "lm_head_verify: n_banned=%d (at most %d)", n_banned,
                       MJ_HEAD_MAX_BANNED);
    if (!head_lse_arg_ok(temperature, out_row_logsumexp))
        return mj_fail(ctx, MJ_INVALID_ARG,
                       "lm_head_verify: temperature %g (the log-sum-exp needs T > 1e-5)",
                       (double)temperature);
    if (K % 256 != 0 || K > 4096)
        return mj_fail(ctx, MJ_UNSUPPORTED_SHAPE, "lm_head_verify: K=%d (need K%%256==0, <=4096)",
                       K);
    hipSetDevice(ctx->device);
    mj_status s = mj_hip(ctx, set_kernel_attributes(), "kernel attributes");
    if (s != MJ_OK) return s;
    void* p[4];
    s = head_scratch(ctx, out_row_logsumexp != nullptr, p);
    if (s != MJ_OK) return s;
    const HeadLse lse{1.4426950408889634f / temperature, (float*)p[2], (float*)p[3],
                      out_row_logsumexp};
    return mj_hip(ctx, launch_lm_head((const uint16_t*)x, (const uint16_t*)w, M, K, V, banned,
                                      n_banned, out_logits, (float*)p[0], (int*)p[1], out_argmax,
                                      out_row_max, lse, ctx->abort_dev, ctx->stream),
                  "lm_head");
}

mj_status mj_lm_head_verify_q4(mj_ctx* ctx, const void* x, const void* w, const void* scales,
                               const void* biases, int M, int K, int V, int group_size,
                               const int32_t* banned, int n_banned, float temperature,
                               int32_t* out_argmax, float* out_row_max,
                               float* out_row_logsumexp, float* out_logits) {
    if (!ctx) return MJ_INVALID_ARG;
    if (!x || !w || !scales || !biases || !out_argmax || M < 1 || M > MJ_MAX_ROWS || V < 1 ||
        n_banned < 0 || (n_banned > 0 && !banned))
        return mj_fail(ctx, MJ_INVALID_ARG, "lm_head_verify_q4: bad argument (M must be 1..%d)",
                       MJ_MAX_ROWS);
    if (n_banned > MJ_HEAD_MAX_BANNED)
        return mj_fail(ctx, MJ_INVALID_ARG, "lm_head_verify_q4: n_banned=%d (at most %d)",
                       n_banned, MJ_HEAD_MAX_BANNED);
    if (!head_lse_arg_ok(temperature, out_row_logsumexp))
        return mj_fail(ctx, MJ_INVALID_ARG,
                       "lm_head_verify_q4: temperature %g (the log-sum-exp needs T > 1e-5)",
                       (double)temperature);
    if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)scales | (uintptr_t)biases) & 15)
        return mj_fail(ctx, MJ_INVALID_ARG, "lm_head_verify_q4: operands need 16-byte alignment");
    const int kmax = M > 16 ? 2048 : 4096;  // staged hidden rows fit 140 KB of LDS
    if (group_size != 64 || K % 512 != 0 || K > kmax)
        return mj_fail(ctx, MJ_UNSUPPORTED_SHAPE,
                       "lm_head_verify_q4: K=%d gs=%d (need gs 64, K%%512==0, K<=%d)", K,
                       group_size, kmax);
    hipSetDevice(ctx->device);
    mj_status s = mj_hip(ctx, set_kernel_attributes(), "kernel attributes");
    if (s != MJ_OK) return s;
    void* p[4];
    s = head_scratch(ctx, out_row_logsumexp != nullptr, p);
    if (s != MJ_OK) return s;
    const HeadLse lse{1.4426950408889634f / temperature, (float*)p[2], (float*)p[3],
                      out_row_logsumexp};
    return mj_hip(ctx,
                  launch_lm_head_q4((const uint16_t*)x, (const uint32_t*)w,
                                    (const uint16_t*)scales, (const uint16_t*)biases, M, K, V,
                                    banned, n_banned, out_logits, (float*)p[0], (int*)p[1],
                                    out_argmax, out_row_max, lse, ctx->abort_dev, ctx->stream),
                  "lm_head q4");
}

mj_status mj_accept_greedy(mj_ctx* ctx, const int32_t* tokens, const int32_t* parents_host,
                           const int32_t* argmax, int n_rows, int32_t* out) {
    if (!ctx) return MJ_INVALID_ARG;
    if (!tokens || !argmax || !out || n_rows < 1 || n_rows > MJ_MAX_ROWS)
        return mj_fail(ctx, MJ_INVALID_ARG, "accept_greedy: bad argument");
    StepDesc sd{};
    mj_status s = fill_tree(ctx, &sd, parents_host, n_rows);
    if (s != MJ_OK) return s;
    s = mj_scratch_reserve(ctx, MJ_MAX_ROWS * 4 + 256);
    if (s != MJ_OK) return s;
    hipSetDevice(ctx->device);
    int32_t* pdev = (int32_t*)ctx->scratch;
    s = mj_hip(ctx, hipMemcpyAsync(pdev, sd.parents, n_rows * 4, hipMemcpyHostToDevice,
                                   ctx->stream), "parents upload");
    if (s == MJ_OK) s = mj_hip(ctx, hipStreamSynchronize(ctx->stream), "upload sync");
    if (s != MJ_OK) return s;
    return mj_hip(ctx, launch_accept_greedy(tokens, pdev, argmax, n_rows, nullptr, out,
                                            ctx->abort_dev, ctx->stream), "accept greedy");
}

mj_status mj_accept_sampled_ex(mj_ctx* ctx, const float* logits, int rows, int V,
                               const int32_t* draft, const mj_sampling* sp, int q_mode,
                               const float* q_point, uint64_t seed, uint64_t counter,
                               int32_t* out) {
    if (!ctx) return MJ_INVALID_ARG;
    if (!logits || !out || !sp || rows < 1 || rows > MJ_MAX_ROWS || V < 1 || V > 196608 ||
        (rows > 1 && !draft) || !(sp->temperature > 1e-5f) ||
        (q_mode != MJ_Q_POINT && q_mode != MJ_Q_UNIFORM))
        return mj_fail(ctx, MJ_INVALID_ARG, "accept_sampled: bad argument");
    SampleOpts o;
    std::vector<int32_t> ht, hc;
    mj_status s = sampling_prep(ctx, sp, o, ht, hc);
    if (s != MJ_OK) return s;
    const bool pen = (std::fabs(o.rep - 1.0f) > 1e-6f && o.rep > 0.0f) || o.pres != 0.0f ||
                     o.freq != 0.0f;
    const bool nucleus = o.top_p < 1.0f - 1e-6f;
    hipSetDevice(ctx->device);
    auto layout = [&](Arena& a, float** rowmax, float** bsum, float** lcopy, int32_t** dt,
                      int32_t** dc, void** nbase) {
        *rowmax = (float*)a.take((size_t)rows * 4);
        *bsum = (float*)a.take(sample_scratch_floats(rows, V) * 4);
        *lcopy = pen ? (float*)a.take((size_t)rows * V * 4) : nullptr;
        *dt = (int32_t*)a.take((size_t)ht.size() * 4 + 4);
        *dc = (int32_t*)a.take((size_t)hc.size() * 4 + 4);
        *nbase = nucleus ? a.take(nucleus_bytes(V)) : nullptr;
    };
    float *rowmax, *bsum, *lcopy;
    int32_t *dt, *dc;
    void* nbase;
    Arena count;
    layout(count, &rowmax, &bsum, &lcopy, &dt, &dc, &nbase);
    s = mj_scratch_reserve(ctx, count.off);
    if (s != MJ_OK) return s;
    Arena real{ctx->scratch, 0};
    layout(real, &rowmax, &bsum, &lcopy, &dt, &dc, &nbase);
    hipStream_t st = ctx->stream;
    // the penalties rewrite the logits: on a copy, the caller's buffer is read-only here
    float* lg = const_cast<float*>(logits);
    if (pen) {
        s = mj_hip(ctx, hipMemcpyAsync(lcopy, logits, (size_t)rows * V * 4,
                                       hipMemcpyDeviceToDevice, st), "logits copy");
        if (s != MJ_OK) return s;
        lg = lcopy;
    }
    if (!ht.empty()) {
        s = mj_hip(ctx, hipMemcpyAsync(dt, ht.data(), ht.size() * 4, hipMemcpyHostToDevice, st),
                   "history");
        if (s == MJ_OK)
            s = mj_hip(ctx, hipMemcpyAsync(dc, hc.data(), hc.size() * 4, hipMemcpyHostToDevice,
                                           st), "history");
        if (s == MJ_OK) s = mj_hip(ctx, hipStreamSynchronize(st), "history upload");
        if (s != MJ_OK) return s;
    }
    o.hist_tok = dt;
    o.hist_cnt = dc;
    NucleusBuf nb{};
    if (nucleus) nucleus_layout(nbase, V, nb);
    return mj_hip(ctx, launch_accept_sampled(lg, rows, V, draft, sp->temperature, q_mode, q_point,
                                             seed, counter, o, nucleus ? &nb : nullptr, rowmax,
                                             bsum, out, nullptr, nullptr, ctx->abort_dev, st),
                  "accept sampled");
}

mj_status mj_accept_sampled(mj_ctx* ctx, const float* logits, int rows, int V,
                            const int32_t* draft, float temperature, int q_mode,
                            const float* q_point, uint64_t seed, uint64_t counter, int32_t* out) {
    mj_sampling sp{};
    sp.temperature = temperature;
    sp.top_p = 1.0f;
    sp.repetition_penalty = 1.0f;
    return mj_accept_sampled_ex(ctx, logits, rows, V, draft, &sp, q_mode, q_point, seed, counter,
                                out);
}

}  // extern "C"
