/*
 * momij_hip.h -- C ABI of the MI355X (gfx950) speculative-decode verify step.
 *
 * Plain C: device pointers are `void*` / typed scalars, sizes are ints.  No HIP or torch types
 * cross this boundary.  Every call is asynchronous on the context's stream unless it says it
 * synchronises; a context is not re-entrant (the reference engine is single-request too,
 * README.md:32, Server.swift:677-700); distinct contexts may be driven from distinct threads.
 * The caller owns every tensor it allocates (weights, activations, outputs); the library owns
 * only its scratch and, for a model, the KV cache.
 *
 * Reference paths below are relative to penta2himajin/momij, swift/Sources/MomijCore/.
 * Tensor layouts follow MLX (WeightStore.swift:48-92): 2-bit affine weights as uint32 words
 * packing 16 codes LSB-first, [rows][K/16]; fp16 scales and biases [rows][K/gs]; up||gate
 * packed with the up rows first.
 */
#ifndef MOMIJ_HIP_H
#define MOMIJ_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MJ_ABI_VERSION 1
#define MJ_MAX_ROWS 64 /* verify rows per pass (draft tree nodes + 1), prefill chunk */

/* Errors -- SeedlessError {noMetal, notReady, unsupportedShape(N,K,gs)}
 * (SeedlessMetal.swift:3718-3728) plus argument, abort, capacity and runtime failures.
 * mj_last_error() gives the message (shape errors carry N, K and gs). */
typedef enum mj_status {
    MJ_OK = 0,
    MJ_NO_DEVICE = 1,          /* no gfx950 device (noMetal) */
    MJ_NOT_READY = 2,          /* library / model not initialised (notReady) */
    MJ_UNSUPPORTED_SHAPE = 3,  /* unsupportedShape(N:K:gs:) */
    MJ_INVALID_ARG = 4,        /* null pointer, bad index, bad tree */
    MJ_ABORTED = 5,            /* abort word set (stopBuf, SeedlessMetal.swift:60, 69-70) */
    MJ_HIP_ERROR = 6,          /* HIP runtime failure */
    MJ_CAPACITY = 7,           /* KV capacity / prompt too long (SeedlessAttn.swift:279-286) */
    MJ_OUT_OF_MEMORY = 8       /* host allocation failed (draft indexes) */
} mj_status;

typedef struct mj_ctx mj_ctx;
typedef struct mj_model mj_model;

/* ---------------------------------------------------------------- context ---- */
/* SeedlessMetal.ensureCompiled (SeedlessMetal.swift:63-104): device, queue, stop buffer. */
mj_status mj_init(int device, mj_ctx** out);
mj_status mj_destroy(mj_ctx* ctx);
const char* mj_last_error(const mj_ctx* ctx);
const char* mj_status_str(mj_status s);
int mj_abi_version(void);
/* Use an external hipStream_t (e.g. the caller's current stream); NULL restores the own one. */
mj_status mj_set_stream(mj_ctx* ctx, void* hip_stream);
void* mj_get_stream(const mj_ctx* ctx);
/* Abort word (stopBuf, SeedlessMetal.swift:60, 69-70): non-zero makes every kernel of this
 * context that starts after the call return early.  Safe from any thread at any time, also
 * while the owning thread's pass is queued, running or being captured into a graph: the word is
 * written by a copy on a stream of the context's own that no pass uses, and mj_set_abort waits
 * for that copy only.  A synchronising call (mj_sync, mj_prefill's chunks, the verify and step
 * calls) reports MJ_ABORTED when the word is set at its entry (then nothing is queued) or at its
 * end, or was set at any time in between -- whenever some of its kernels may have skipped their
 * work -- and its results are then void (a model's offset does not advance).  Cleared with
 * flag = 0; the next call runs normally. */
mj_status mj_set_abort(mj_ctx* ctx, int flag);
/* Bound of the fused MoE launch's waits (no counterpart in the reference: it has no fused
 * launch).  Passes of at most 32 rows run the up||gate and down products as one launch whose
 * blocks all stay resident; a down item computes once the act rows it stages hold no value the
 * up product has yet to write, staging them again at most `polls` times (default 131072, each
 * after a short sleep: well under a second).  A wait that runs out its bound -- the launch's
 * blocks were not all resident, e.g. kernels of another stream held CUs -- sets the context's
 * fault word, and the next synchronising call reports MJ_HIP_ERROR (the results since the
 * previous one are invalid) and clears it.  polls = 0 forces that report whenever a down item's
 * rows are not complete at its first check.  A pass replayed from a graph keeps the bound it
 * was captured with. */
mj_status mj_set_wait_limit(mj_ctx* ctx, int polls);
/* One wait for everything queued (cb.commit + waitUntilCompleted,
 * SeedlessDecodeEngine.swift:324-325).  Reports MJ_ABORTED if the abort word is set or was set
 * since the previous synchronising call. */
mj_status mj_sync(mj_ctx* ctx);

/* ---------------------------------------------------------------- memory ----- */
mj_status mj_alloc(mj_ctx* ctx, size_t bytes, void** out);
mj_status mj_free(mj_ctx* ctx, void* p);
mj_status mj_h2d(mj_ctx* ctx, void* dst, const void* src, size_t bytes);  /* synchronous */
mj_status mj_d2h(mj_ctx* ctx, void* dst, const void* src, size_t bytes);  /* synchronous */

/* ------------------------------------------------------------------ ops ------ */
/* 2-bit affine gather-qmv / verify GEMM -- SeedlessMetal.gqmm2 (SeedlessMetal.swift:312-438),
 * kernel gqmm2_rows (2168-2221):
 *   y[mk, n] = half( sum_k (s[e,n,k/gs]*q[e,n,k] + b[e,n,k/gs]) * x[row(mk), k] ),
 *   e = inds[mk], row(mk) = lhs_per_expert ? mk : mk / ktop, mk < M*ktop.
 * x fp16 [M or M*ktop][K], w uint32 [E][N][K/16], scales/biases fp16 [E][N][K/gs],
 * inds int32 [M*ktop] (device), y fp16 [M*ktop][N].
 * Shapes: K % 512 == 0 (as the reference, SeedlessMetal.swift:336-338), N % 16 == 0,
 * gs in {64, 128}, M*ktop <= MJ_MAX_ROWS*8.
 * epilogue MJ_EPI_STORE writes y; MJ_EPI_ADD writes y = half(y + half(acc)) (o-proj residual,
 * gqmm2_rows_fold_add 3488-3543; requires ktop == 1). */
#define MJ_EPI_STORE 0
#define MJ_EPI_ADD 1
mj_status mj_gather_qmm2(mj_ctx* ctx, const void* x, const uint32_t* w, const void* scales,
                         const void* biases, const int32_t* inds, void* y, int M, int ktop,
                         int K, int N, int gs, int lhs_per_expert, int epilogue);

/* MoE expert weights of one layer (MapleMoE.swift:6-33 / SeedlessAttn.swift:93-99). */
typedef struct mj_moe_weights {
    const void* norm_w;        /* fp16 [H] post_attention_layernorm (MJ_MOE_PRENORM) */
    const void* router_w;      /* fp16 [E][H] mlp.gate */
    const uint32_t* up_gate_w; /* [E][2I][H/16], rows 0..I-1 up, I..2I-1 gate */
    const void* up_gate_s;     /* fp16 [E][2I][H/gs] */
    const void* up_gate_b;
    const uint32_t* down_w;    /* [E][H][I/16] */
    const void* down_s;        /* fp16 [E][H][I/gs] */
    const void* down_b;
    int E, top_k, H, I, gs;  /* H 2048 or 4096; I a multiple of 512, <= 4096; gs 64 or 128 */
    float eps;
    /* optional row-alpha form (WeightStore.swift:47-63: scales = alpha in every group of a
     * row, biases = -alpha): fp16 [E][2I] and [E][H], 16-byte aligned, or NULL.  When set,
     * up_gate_s/_b and down_s/_b must still hold that expansion: the batched expert kernels
     * read one alpha per row, the one-row and general kernels read the arrays, and the two are
     * not compared (an alpha that is not the arrays' expansion makes decode and verify
     * disagree). */
    const void* up_gate_alpha;
    const void* down_alpha;
} mj_moe_weights;

/* MoE block -- encodeMoEBlock (SeedlessMetal.swift:576-609), MapleMoE.callAsFunction
 * (MapleMoE.swift:58-80): [rms(x)] -> router logits -> softmax top-k (lowest index on ties,
 * renormalised) -> up||gate gather -> clamped SwiGLU -> down gather -> score-weighted combine.
 * flags: MJ_MOE_PRENORM applies norm_w first; MJ_MOE_RESIDUAL writes y = x + moe.
 * x, y fp16 [M][H] (may alias); out_inds int32 [M][top_k], out_scores fp32 [M][top_k]
 * (device, nullable).  Rows are bucketed by expert so each routed expert's weights stream
 * once per call. */
#define MJ_MOE_PRENORM 1
#define MJ_MOE_RESIDUAL 2
mj_status mj_moe_block(mj_ctx* ctx, const mj_moe_weights* w, const void* x, void* y, int M,
                       int flags, int32_t* out_inds, float* out_scores);

/* mj_moe_block without any device allocation.  No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same kernels, arguments and results as mj_moe_block, with the
 * scratch in one statically allocated device array of MJ_MOE_NOALLOC_BYTES per GPU (held until
 * the process ends) instead of the context's growable scratch.  A call whose scratch would
 * exceed it (M rows x top_k x (I + H) halves dominate: H <= 2048 fits any I <= 4096 at
 * M = 64) is refused with MJ_CAPACITY before any work is queued.  Every call on one GPU shares
 * that GPU's array, which keeps the last call's contents: calls that overlap on one GPU (from
 * several contexts, or one context whose stream mj_set_stream changed between calls) race, so
 * the caller must order them -- issue them on one stream, or make each stream wait for the
 * previous call's completion event.  No synchronisation is added here: a wait on an event
 * recorded outside a graph capture would break the capture this entry point exists for. */
#define MJ_MOE_NOALLOC_BYTES (8u << 20)
mj_status mj_moe_block_noalloc(mj_ctx* ctx, const mj_moe_weights* w, const void* x, void* y,
                               int M, int flags, int32_t* out_inds, float* out_scores);

/* Attention weights of one layer (SeedlessAttn.swift:74-92). */
typedef struct mj_attn_weights {
    const void* norm_w;      /* fp16 [H] input_layernorm */
    const uint32_t* qkv_w;   /* [(nQ+2nKV)*D][H/16], q rows then k then v (WeightStore 66-79) */
    const void* qkv_s;
    const void* qkv_b;
    const void* q_norm_w;    /* fp16 [D] */
    const void* k_norm_w;    /* fp16 [D] */
    const uint32_t* o_w;     /* [H][nQ*D/16] */
    const void* o_s;
    const void* o_b;
} mj_attn_weights;

typedef struct mj_attn_config {
    int H, n_heads, n_kv_heads, head_dim; /* head_dim must be 128 */
    int rope_dim;                         /* rotated leading dims (0 = NoPE) */
    float rope_base, eps;
    int window;                           /* sliding window (0 = full attention) */
    int64_t kv_capacity;                  /* slots C of the cache; >= window + M */
    int gs;
} mj_attn_config;

/* Attention block with residual -- encodeAttnBlock (SeedlessMetal.swift:926-1005) with the
 * input RMSNorm of encodeLayerBlock (1008-1048): h += o_proj(attn(rms(h))).
 * Verify row r sits at position L + depth(r); parents_host[r] < r gives the draft tree
 * (NULL = linear chain, parents[0] = -1).  Row r attends the committed positions inside its
 * window plus its ancestors and itself.  New K/V rows are written at slot (L + r) % C of the
 * caches kcache/vcache fp16 [n_kv][C][128]; committed position p lives at slot p % C. */
mj_status mj_attn_block(mj_ctx* ctx, const mj_attn_config* cfg, const mj_attn_weights* w,
                        void* h, void* kcache, void* vcache, int64_t L,
                        const int32_t* parents_host, int M);

/* lm_head verify -- encodeMetalHead -> maple_lm_head_argmax/reduce
 * (SeedlessDecodeEngine.swift:481-498, SeedlessMetal.swift:3005-3111) for an fp16 head:
 * logits[m][v] = sum_k w[v][k] * x[m][k] (fp32), argmax per row with the lowest id winning
 * ties and banned ids skipped.  x fp16 [M][K], w fp16 [V][K]; out_argmax int32 [M];
 * out_row_max fp32 [M] (nullable): the row's largest logit; out_row_logsumexp fp32 [M]
 * (nullable): ln sum_v exp(logits[m][v] / temperature) over the ids not banned, so that
 * ln p = logits / T - logsumexp is LogitsProcessor.probabilities' softmax
 * (LogitsProcessor.swift:168-189; needs temperature > 1e-5, otherwise ignored);
 * out_logits fp32 [M][V] (nullable; written when sampling).  banned int32 [n_banned] device
 * (nullable), n_banned <= 64 (the reference stages at most 16, SeedlessDecodeEngine.swift:470). */
mj_status mj_lm_head_verify(mj_ctx* ctx, const void* x, const void* w, int M, int K, int V,
                            const int32_t* banned, int n_banned, float temperature,
                            int32_t* out_argmax, float* out_row_max, float* out_row_logsumexp,
                            float* out_logits);

/* lm_head verify over the Maple checkpoint's 4-bit head -- maple_lm_head_argmax/reduce
 * (SeedlessMetal.swift:3005-3111, bound by SeedlessDecodeEngine.swift:481-498 when head_bits
 * is 4, SeedlessDecodeEngine.swift:144): logits[m][v] = sum_k (q[v][k] s[v][k/64] +
 * b[v][k/64]) x[m][k] (fp32), argmax per row with the lowest id winning ties and banned ids
 * skipped.  w uint32 [V][K/8] (8 codes a word, LSB first), scales/biases fp16 [V][K/64],
 * x fp16 [M][K]; group_size must be 64 and K a multiple of 512 (K <= 4096, <= 2048 for
 * M > 16); all four operands 16-byte aligned; n_banned <= 64 (the reference stages at most
 * 16, SeedlessDecodeEngine.swift:470).  Outputs as mj_lm_head_verify. */
mj_status mj_lm_head_verify_q4(mj_ctx* ctx, const void* x, const void* w, const void* scales,
                               const void* biases, int M, int K, int V, int group_size,
                               const int32_t* banned, int n_banned, float temperature,
                               int32_t* out_argmax, float* out_row_max,
                               float* out_row_logsumexp, float* out_logits);

/* Greedy acceptance -- verifyDraftChain (SeedlessDecodeEngine.swift:1574-1603) generalised to
 * a tree: from row 0 step to the lowest-index child whose token equals the current row's
 * argmax; stop when none does.  tokens/argmax int32 [n_rows] device, parents_host as above.
 * out int32 device [2 + 2*n_rows]: out[0] = accepted, out[1] = bonus token,
 * out[2 .. 2+acc] = accepted row path (row 0 first), out[2+n_rows .. 2+n_rows+acc] = emitted
 * tokens (accepted drafts then the bonus). */
mj_status mj_accept_greedy(mj_ctx* ctx, const int32_t* tokens, const int32_t* parents_host,
                           const int32_t* argmax, int n_rows, int32_t* out);

/* Sampled acceptance over the full vocabulary -- SpeculativeSampling.tryAccept / walkDraft
 * (SpeculativeSampling.swift:27-99) with LogitsProcessor.probabilities / samplePrepared
 * (LogitsProcessor.swift:116-189), no penalties.  logits fp32 [rows][V] device (row i = target
 * after feed i), draft int32 [rows-1] device.  q_mode MJ_Q_POINT: q = q_point[i] at the draft
 * token (q_point: a DEVICE float array [rows-1], read by the kernels; NULL = 1 on every draft, the
 * reference default); MJ_Q_UNIFORM: q = 1/V.  q < 0 counts as 0 (max(0, draftQ)): such a
 * draft is rejected without a uniform and the residual is the target itself.
 * Uniforms: Philox4x32-10, key = seed, counter = (row, counter lo, counter hi, 0x6d6a6a76),
 * u0 = accept test, u1 = residual walk (row rows-1: u0 = bonus).  Sums and walks use a fixed
 * blocked order (16-element chunks, 64-chunk blocks) so results are reproducible bit for bit.
 * out int32 device [2]: accepted count, emitted token.  temperature must be > 1e-5. */
#define MJ_Q_POINT 0
#define MJ_Q_UNIFORM 1
mj_status mj_accept_sampled(mj_ctx* ctx, const float* logits, int rows, int V,
                            const int32_t* draft, float temperature, int q_mode,
                            const float* q_point, uint64_t seed, uint64_t counter, int32_t* out);

/* LogitsProcessor options (LogitsProcessor.swift:17-49): temperature > 1e-5; top_p (nucleus,
 * 1 = off, clamped to [0, 1]); repetition (1 = off, > 0), presence and frequency (0 = off)
 * penalties.  hist_tokens / hist_counts (host, n_hist <= MJ_MAX_HIST, tokens distinct): the
 * seen set and the counts the penalties read (prepare, 91-104); drafts accepted in the walk
 * join both before the next row (walkDraft, SpeculativeSampling.swift:86-87). */
#define MJ_MAX_HIST 65536
typedef struct mj_sampling {
    float temperature;
    float top_p;
    float repetition_penalty;
    float presence_penalty;
    float frequency_penalty;
    const int32_t* hist_tokens;
    const int32_t* hist_counts;
    int n_hist;
} mj_sampling;

/* mj_accept_sampled with the options: every row's logits penalised (row i with the history
 * plus drafts 0 .. i-1; the caller's logits are not modified), the bonus and a residual of zero
 * mass sampled through samplePrepared's nucleus (LogitsProcessor.swift:137-164): tokens ranked
 * by e descending, the lower id first among equal e, kept up to the first ranked prefix whose
 * blocked prefix sum reaches top_p * Z, sampled in id order at u * (kept mass). */
mj_status mj_accept_sampled_ex(mj_ctx* ctx, const float* logits, int rows, int V,
                               const int32_t* draft, const mj_sampling* s, int q_mode,
                               const float* q_point, uint64_t seed, uint64_t counter,
                               int32_t* out);

/* ---------------------------------------------------------------- model ------ */
typedef struct mj_model_config {
    int n_layers;
    int H, n_heads, n_kv_heads, head_dim, rope_dim;
    float rope_base, eps;
    int window;            /* sliding window of every layer (0 = full) */
    int64_t kv_capacity;   /* ring slots per layer (>= window + MJ_MAX_ROWS when windowed) */
    int E, top_k, I, gs;
    int vocab;
    /* Maple's layer mix (MapleConfig.isSliding, MapleConfig.swift:145-148; SeedlessAttn.swift
     * 81-83): host arrays [n_layers] overriding window and rope_dim per layer -- sliding layers
     * window w with partial RoPE, full-attention layers 0 / 0 (NoPE).  NULL: every layer takes
     * window / rope_dim.  The non-zero rope dims must all equal rope_dim. */
    const int32_t* layer_window;
    const int32_t* layer_rope_dim;
    /* 4: lm_head is the 4-bit gs64 head of the checkpoint (headBits, MapleConfig.swift:141),
     * uint32 [V][H/8] with lm_head_scales / lm_head_biases fp16 [V][H/64], decoded by
     * mj_lm_head_verify_q4's kernel (H <= 2048).  0 or 16: fp16 [V][H]. */
    int head_bits;
    const void* lm_head_scales;
    const void* lm_head_biases;
} mj_model_config;

typedef struct mj_layer_weights {
    mj_attn_weights attn;
    mj_moe_weights moe;    /* moe.norm_w = post_attention_layernorm */
} mj_layer_weights;

/* A resident stack (SeedlessLayerStack, SeedlessAttn.swift:369-456): caller-owned weights,
 * library-owned KV caches and scratch sized for MJ_MAX_ROWS rows.  layers [n_layers] is copied;
 * the device buffers it points to must outlive the model.  embed fp16 [V][H], final_norm_w
 * fp16 [H], lm_head fp16 [V][H]. */
mj_status mj_model_create(mj_ctx* ctx, const mj_model_config* cfg, const mj_layer_weights* layers,
                          const void* embed, const void* final_norm_w, const void* lm_head,
                          mj_model** out);
mj_status mj_model_destroy(mj_model* model);
/* Committed tokens (SeedlessLayerBlock.offset) and rewind (rewindOffset, SeedlessAttn.swift
 * 319-322; the reject rollback of snapshotForChain 540-586 when writes are append-only). */
int64_t mj_model_offset(const mj_model* model);
mj_status mj_model_rewind(mj_model* model, int64_t offset);
/* Device pointers of layer `layer`'s caches, fp16 [n_kv][kv_capacity][head_dim]. */
mj_status mj_model_kv(mj_model* model, int layer, void** kcache, void** vcache);

/* prefillPrompt (SeedlessDecodeEngine.swift:516-545): feed tokens in chunks of <= chunk rows
 * (<= MJ_MAX_ROWS), commit them, return the argmax after the last token.  Synchronises. */
mj_status mj_prefill(mj_model* model, const int32_t* tokens, int n, int chunk,
                     int32_t* out_next);

/* stepChainFeeds (SeedlessDecodeEngine.swift:194-228): one pass over the chain `feeds`
 * (M rows), commit all M, return the greedy argmax after each row.  Synchronises. */
mj_status mj_step_chain_feeds(mj_model* model, const int32_t* feeds, int M, int32_t* out_evals);

/* verifyDraftChain (SeedlessDecodeEngine.swift:1574-1603), tree-capable: one pass over rows
 * [y] + draft (parents NULL = chain; else parents[0] = -1 and parents[r] < r over the rows),
 * greedy acceptance on the device, accepted rows compacted into the cache, offset advanced by
 * accepted + 1.  out_tokens [n_draft + 1]: accepted drafts then the bonus token.
 * One device wait per call. */
mj_status mj_verify_greedy(mj_model* model, int32_t y, const int32_t* draft, int n_draft,
                           const int32_t* parents, int32_t* out_accepted, int32_t* out_tokens);

/* verifyDraftSampled (SeedlessDecodeEngine.swift:1541-1571) over the exact fp16 head and the
 * full vocabulary (chain drafts): one pass, device-side sampled acceptance (mj_accept_sampled
 * rules), commit accepted + 1 rows.  out_token = resampled token or bonus.  Unlike
 * mj_accept_sampled, draft and q_point are HOST arrays here: q_point float [n_draft] holds
 * draftQ (qAlong's q on draft i, mergedDraftQ at SeedlessDecodeEngine.swift:1530-1538) and is
 * copied into the pass's descriptor; NULL = 1 on every draft. */
mj_status mj_verify_sampled(mj_model* model, int32_t y, const int32_t* draft, int n_draft,
                            float temperature, int q_mode, const float* q_point, uint64_t seed,
                            uint64_t counter, int32_t* out_accepted, int32_t* out_token);
/* mj_verify_sampled with LogitsProcessor options (mj_accept_sampled_ex's rules) --
 * verifyDraftSampled (SeedlessDecodeEngine.swift:1541-1571) with the processor's penalties
 * and nucleus. */
mj_status mj_verify_sampled_ex(mj_model* model, int32_t y, const int32_t* draft, int n_draft,
                               const mj_sampling* s, int q_mode, const float* q_point,
                               uint64_t seed, uint64_t counter, int32_t* out_accepted,
                               int32_t* out_token);

/* Debug capture for layer-by-layer checks: when set, each pass copies h after the embedding
 * and after every layer into h_capture fp16 [n_layers+1][MJ_MAX_ROWS][H], the routing into
 * inds_capture int32 [n_layers][MJ_MAX_ROWS][top_k] and the head logits into logits_capture
 * fp32 [MJ_MAX_ROWS][V] (device pointers, any may be NULL; all NULL disables). */
mj_status mj_model_set_capture(mj_model* model, void* h_capture, int32_t* inds_capture,
                               float* logits_capture);

/* The same capture with every block boundary, so each block can be re-run from the exact
 * inputs the device used (no counterpart in the reference; its layer-by-layer checks read
 * MTLBuffers directly).  Device pointers, any may be NULL (all NULL disables); while any is
 * set, passes run without graphs.  R = MJ_MAX_ROWS, rows beyond the pass's M are untouched. */
typedef struct mj_capture {
    void* h;               /* fp16 [n_layers+1][R][H]: after the embedding and after each layer */
    int32_t* inds;         /* int32 [n_layers][R][top_k]: each layer's routing */
    float* logits;         /* fp32 [R][V]: lm_head logits */
    void* attn_out;        /* fp16 [n_layers][R][H]: h after each layer's attention block */
    void* moe_in;          /* fp16 [n_layers][R][H]: the normed MoE input (router and up gather) */
    float* router_logits;  /* fp32 [n_layers][R][E]: router logits */
    void* head_in;         /* fp16 [R][H]: the final-normed rows fed to the lm_head */
    void* kv_rows;         /* fp16 [n_layers][2][n_kv_heads][R][head_dim]: the K and V rows the
                              pass appended (row r at slot (L + r) % C), before any commit */
} mj_capture;
mj_status mj_model_set_capture_ex(mj_model* model, const mj_capture* cap);

/* Use HIP graphs for verify passes (one graph per row count and mode, replayed with a device
 * step descriptor).  On by default. */
mj_status mj_model_set_graphs(mj_model* model, int enable);

/* Per-pass device timing of the last verify call (ms), from HIP events on the model stream. */
float mj_model_last_pass_ms(const mj_model* model);

/* Per-kernel timing for measurement: when enabled, verify passes run without graphs and record
 * HIP events around each launch of the classes below on the model stream (counters reset on
 * every call).  A profiled pass waits behind a 15 ms hold kernel, so its launches are queued
 * before the GPU reaches them, and starts with 8 brackets around a kernel that waits 20 us of
 * wall-clock time: each bracketed time is the kernel's duration plus the timer's own cost, and
 * MJ_KERNEL_TIMER minus 20 us per launch is that cost.  mj_model_kernel_ms returns the summed
 * milliseconds and the launch count. */
#define MJ_KERNEL_EXPERT_UP 0   /* bucketed up||gate gather + SwiGLU */
#define MJ_KERNEL_EXPERT_DOWN 1 /* bucketed down gather */
#define MJ_KERNEL_LM_HEAD 2     /* fp16 lm_head + argmax partials */
#define MJ_KERNEL_ATTENTION 3   /* split-K attention + combine */
#define MJ_KERNEL_DENSE 4       /* qkv and o projections */
#define MJ_KERNEL_TIMER 5       /* the same bracket around a 20 us wall-clock hold */
#define MJ_KERNEL_EXPERT_MOE 6  /* up||gate + SwiGLU then down, one launch (passes of at most
                                   32 rows over at most 64 experts, H 2048, intermediate 1024) */
mj_status mj_model_profile(mj_model* model, int enable);
float mj_model_kernel_ms(const mj_model* model, int kernel_class, int64_t* launches);

/* Hardware self-check of the MFMA operand layout the kernels rely on (16x16x32 f16):
 * D = A[16x32] * B[32x16] with A, B fp16 row-major device, D fp32 [16][16] device. */
mj_status mj_selftest_mfma(mj_ctx* ctx, const void* A, const void* B, float* D);

/* ---------------------------------------------------------- draft sources ---- */
/* Host-only drafters that propose the rows a verify pass checks (no device work).
 *
 * Online suffix-tree index -- SuffixDraftIndex (SuffixDraftIndex.swift:12-156): every suffix of
 * the inserted sequences, truncated to max_depth (>= 4), with occurrence counts.  A draft takes
 * the longest suffix of `history` (at most max_depth) that ends at a node with children, then
 * follows the most frequent child mj_suffix_max_spec(match, max_k, alpha) times; equal counts
 * take the lowest token id (the reference's order there is its dictionary's).  out_tokens
 * holds max_k ids; *out_n drafted, *out_match_len the suffix length (0: no match). */
typedef struct mj_suffix_index mj_suffix_index;
mj_status mj_suffix_index_create(int max_depth, mj_suffix_index** out);
mj_status mj_suffix_index_destroy(mj_suffix_index* idx);
mj_status mj_suffix_index_clear(mj_suffix_index* idx);
int64_t mj_suffix_index_tokens(const mj_suffix_index* idx);
mj_status mj_suffix_index_insert(mj_suffix_index* idx, const int32_t* tokens, int n);
mj_status mj_suffix_index_draft(const mj_suffix_index* idx, const int32_t* history, int n,
                                int max_k, double alpha, int32_t* out_tokens, int* out_n,
                                int* out_match_len);
/* MAX_SPEC = alpha * match, at least 1 with a match, at most max_k -- maxSpec (48-53). */
int mj_suffix_max_spec(int match_len, int max_k, double alpha);
/* bestDraft (103-121): the local then the global index (either NULL), longer match first, then
 * the longer draft. */
mj_status mj_suffix_best_draft(const mj_suffix_index* local, const mj_suffix_index* global,
                               const int32_t* history, int n, int max_k, double alpha,
                               int32_t* out_tokens, int* out_n, int* out_match_len);
/* qAlong (123-156): the draft model's q along `draft`, child count over sibling mass from the
 * longest matching suffix; positions past the tree stay 1.  out_q float [n_draft]. */
mj_status mj_suffix_index_q_along(const mj_suffix_index* idx, const int32_t* history, int n,
                                  const int32_t* draft, int n_draft, float* out_q);
/* Prompt-lookup draft -- SuffixSpec.suffixDraft (SuffixSpec.swift:17-55): the longest pattern
 * (<= max_ngram, reference default 16) ending the history, its latest earlier occurrence (one
 * inside the first prompt_len tokens first, when prompt_len > 0), and up to k tokens after it. */
mj_status mj_suffix_draft_pld(const int32_t* history, int n, int k, int max_ngram,
                              int prompt_len, int32_t* out_tokens, int* out_n);
/* treeDraft (SuffixDraftIndex.swift:160-178): best tree draft, else the prompt lookup. */
mj_status mj_tree_draft(const int32_t* history, int n, int k, const mj_suffix_index* local,
                        const mj_suffix_index* global, double alpha, int prompt_len,
                        int32_t* out_tokens, int* out_n);
/* adaptiveDraftK (SuffixSpec.swift:8-15): draft length from the mean accepted length. */
int mj_adaptive_draft_k(double mean_accept, int draft_k);

/* Token recycling -- TokenRecycleIndex (TokenRecycleIndex.swift:9-57): per token the top_k
 * (>= 2) latest candidate successors, newest first; a draft follows first successors until one
 * repeats or is missing. */
typedef struct mj_recycle_index mj_recycle_index;
mj_status mj_recycle_index_create(int top_k, mj_recycle_index** out);
mj_status mj_recycle_index_destroy(mj_recycle_index* r);
mj_status mj_recycle_index_clear(mj_recycle_index* r);
mj_status mj_recycle_index_observe(mj_recycle_index* r, int32_t from_token,
                                   const int32_t* candidates, int n);
mj_status mj_recycle_index_draft(const mj_recycle_index* r, int32_t last, int max_k,
                                 int32_t* out_tokens, int* out_n);
int mj_recycle_index_entries(const mj_recycle_index* r);

#ifdef __cplusplus
}
#endif
#endif
