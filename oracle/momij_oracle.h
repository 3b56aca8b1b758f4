/*
 * momij_oracle.h -- CPU restatement of momij's speculative-decode verify step.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the parity reference / the timed CPU
 * baseline.  The product library (libmomij_hip.so) never links or calls it.
 *
 * Every function cites the reference file:line whose semantics it restates
 * (paths relative to the penta2himajin/momij checkout, under swift/Sources/MomijCore/).
 * fp16 values travel as uint16_t bit patterns; all arithmetic is fp32 unless noted.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   or_h2f/or_f2h          all 65536 patterns + random floats vs numpy float16 (IEEE RNE)
 *   or_qmm2                float64 numpy closed form; one-hot / all-zero-code special cases;
 *                          M-row == sequential (MomijCoreTests.swift:251-314)
 *   or_rms_norm etc.       float64 closed forms
 *   or_route_topk          float64 softmax + full sort brute force, lowest-index ties
 *   or_attention           textbook masked softmax in float64; sliding mask KAT
 *                          (MomijCoreTests.swift:130-145); tree-of-a-chain == causal chain
 *   or_philox4x32_10       Random123 known-answer vectors
 *   or_splitmix64          published SplitMix64 vectors (seed 1234567)
 *   or_try_accept/walk     SpeculativeSamplingTests.swift:5-45, 94-137 KATs
 *   or_canon_expf          libm expf within 2 ulp on a dense grid
 *   or_moe_block, or_attn_block, or_layer_forward, or_score_resid
 *                          float64 numpy restatement at the reference's fp16 rounding points
 *                          (tests/restate64.py), with planted-mistake negative controls; the
 *                          double rounding of the residual by an exact special case
 *   or_kv_commit           a tree verify + commit leaves the cache a chain verify of the
 *                          accepted path leaves, bit for bit; a chain path is the identity
 */
#ifndef MOMIJ_ORACLE_H
#define MOMIJ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 ---------------------------------------------------------------- */
float or_h2f(uint16_t h);
uint16_t or_f2h(float f);
void or_h2f_array(const uint16_t* in, float* out, size_t n);
void or_f2h_array(const float* in, uint16_t* out, size_t n);

/* ---- a2: 2-bit affine gather-qmv (gqmm2_rows) ----------------------------- */
void or_qmm2(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
             const uint16_t* biases, const int32_t* inds, uint16_t* y,
             int M, int ktop, int K, int N, int gs, int lhs_per_expert);

/* ---- a3: expert epilogues ------------------------------------------------- */
void or_clamped_swiglu(const uint16_t* ug, uint16_t* act, int rows, int I);
void or_score_reduce(const uint16_t* down, const float* scores, uint16_t* y,
                     int M, int ktop, int H);
void or_score_resid(const uint16_t* down, const float* scores, uint16_t* h,
                    int M, int ktop, int H);

/* ---- a4: norm / router ---------------------------------------------------- */
void or_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* out, int M, int H, float eps);
void or_router_logits(const uint16_t* W, const uint16_t* x, float* logits, int M, int E, int H);
void or_route_topk(const float* logits, int32_t* inds, float* scores, int M, int E, int k);

/* MoE block.  flags: bit0 = pre-norm with norm_w, bit1 = residual (y = x + moe).
 * out_inds int32 [M][top_k] and out_scores fp32 [M][top_k] are required (the gathers read them). */
#define OR_MOE_PRENORM 1
#define OR_MOE_RESIDUAL 2
typedef struct or_moe_w {
    const uint16_t* norm_w;      /* [H] (used with OR_MOE_PRENORM) */
    const uint16_t* router_w;    /* [E][H] */
    const uint32_t* up_gate_w;   /* [E][2I][H/16] rows 0..I-1 up, I..2I-1 gate */
    const uint16_t* up_gate_s;   /* [E][2I][H/gs] */
    const uint16_t* up_gate_b;
    const uint32_t* down_w;      /* [E][H][I/16] */
    const uint16_t* down_s;      /* [E][H][I/gs] */
    const uint16_t* down_b;
    int E, top_k, H, I, gs;
    float eps;
} or_moe_w;
void or_moe_block(const or_moe_w* w, const uint16_t* x, uint16_t* y, int M, int flags,
                  int32_t* out_inds, float* out_scores);

/* ---- a5/a6: attention ----------------------------------------------------- */
void or_rope_inv_freq(float* inv_freq, int rope_dim, float base);
void or_qk_norm_rope(const uint16_t* qkv, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                     const float* inv_freq, const int64_t* pos, uint16_t* q_out, uint16_t* k_out,
                     int M, int nQ, int nKV, int D, int rope_dim, float eps);
/* Tree/chain sliding-window attention over a cache [nKV][C][D] (slot = position % C for the
 * committed prefix, (L + r) % C for verify row r).  parents[r] < r (row 0: -1).  window == 0
 * means full attention.  q [M][nQ][D] fp16, out [M][nQ*D] fp16. */
void or_attention(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache,
                  int64_t C, int64_t L, const int32_t* parents, int M, int nQ, int nKV, int D,
                  int window, uint16_t* out);

typedef struct or_attn_w {
    const uint16_t* norm_w;      /* [H] input_layernorm */
    const uint32_t* qkv_w;       /* [(nQ+2nKV)D][H/16] */
    const uint16_t* qkv_s;
    const uint16_t* qkv_b;
    const uint16_t* q_norm_w;    /* [D] */
    const uint16_t* k_norm_w;    /* [D] */
    const uint32_t* o_w;         /* [H][nQ*D/16] */
    const uint16_t* o_s;
    const uint16_t* o_b;
} or_attn_w;

typedef struct or_cfg {
    int H, nQ, nKV, D, rope_dim, window, gs;
    float rope_base, eps;
    int64_t C;                    /* KV slots per layer */
} or_cfg;

/* One attention block with residual: h += o_proj(attn(norm(h))).  Writes the M new K/V rows. */
void or_attn_block(const or_cfg* cfg, const or_attn_w* w, const float* inv_freq, uint16_t* h,
                   uint16_t* kcache, uint16_t* vcache, int64_t L, const int32_t* parents, int M);

/* ---- a7: lm_head ---------------------------------------------------------- */
void or_lm_head_logits(const uint16_t* x, const uint16_t* w, float* logits, int M, int K, int V);
void or_argmax_rows(const float* logits, int M, int V, const int32_t* banned, int n_banned,
                    int32_t* out_idx, float* out_best, float* out_second);

/* ---- a8: greedy acceptance ------------------------------------------------ */
/* rows 0..n (row 0 = fed token y, rows 1..n = draft nodes), parents[r] row index (< r),
 * tokens[r] = token fed at row r, argmax[r] = target argmax after row r.
 * Returns accepted count; out_path[0..acc] = accepted row indices (row 0 first);
 * out_emit[0..acc] = emitted tokens (accepted drafts then the bonus). */
int or_accept_greedy(const int32_t* tokens, const int32_t* parents, const int32_t* argmax,
                     int n_rows, int32_t* out_path, int32_t* out_emit);

/* ---- a9: sampled acceptance ----------------------------------------------- */
void or_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
float or_u01_from_u32(uint32_t x);
void or_verify_uniforms(uint64_t seed, uint64_t counter, int rows, float* u /* [rows][2] */);
uint64_t or_splitmix64_next(uint64_t* state);
float or_canon_expf(float x);

/* Canonical-order sum and walk (chunks of 16 summed sequentially, blocks of 64 chunks). */
float or_canon_sum(const float* v, int n);
int or_canon_walk(const float* v, int n, float t);

/* Full-vocab verify: logits [rows][V] fp32 (row i is the target distribution after feed i),
 * draft[0..rows-2].  q_mode 0: point mass q at the draft token (q_point[i], NULL = 1);
 * q_mode 1: uniform q = 1/V.  uniforms [rows][2].  Returns accepted count; *out_token = the
 * resampled token on reject or the bonus sample on full accept. */
int or_accept_sampled(const float* logits, int rows, int V, const int32_t* draft,
                      float temperature, int q_mode, const float* q_point,
                      const float* uniforms, int32_t* out_token);

/* LogitsProcessor.prepare over a full row in place: history tokens (unique) with counts plus
 * the first n_extra drafts (seen, counted once each). */
void or_penalize_row(float* l, int V, const int32_t* hist_tok, const int32_t* hist_cnt,
                     int n_hist, const int32_t* extra, int n_extra, float rep, float pres,
                     float freq);
/* Nucleus + multinomial in the canonical order (ranked by e descending, lower id first). */
int or_nucleus_sample(const float* e, int V, float Z, float top_p, float u);
/* the fixed-point mass of one e in the nucleus cut: trunc(e * 2^40) */
uint64_t or_nucleus_fixed(float e);
/* or_accept_sampled with penalties (history + accepted drafts) and top-p. */
int or_accept_sampled_ex(const float* logits, int rows, int V, const int32_t* draft,
                         float temperature, float top_p, float rep, float pres, float freq,
                         const int32_t* hist_tok, const int32_t* hist_cnt, int n_hist,
                         int q_mode, const float* q_point, const float* uniforms,
                         int32_t* out_token);

/* Restatement of SpeculativeSampling.tryAccept / LogitsProcessor over a candidate list
 * (used for the reference's own KATs).  rng: SplitMix64 state. */
int or_try_accept(int draft_token, const int32_t* ids, const float* logits, int n,
                  float temperature, float draft_q, uint64_t* rng, int32_t* out_token);
int or_walk_draft(const int32_t* draft, int n_draft, const int32_t* row_ids,
                  const float* row_logits, int n_cand, float temperature, uint64_t* rng,
                  int32_t* out_next);
int or_walk_draft_greedy(const int32_t* draft, int n_draft, const int32_t* row_ids,
                         const float* row_logits, int n_cand, int32_t* out_next);

/* ---- full model (small configs; composition of the above) ---------------- */
typedef struct or_layer_w {
    or_attn_w attn;
    or_moe_w moe;
} or_layer_w;

/* One decoder layer: attention block then MoE block (pre-norm + residual), in place on h. */
void or_layer_forward(const or_cfg* cfg, const or_layer_w* w, const float* inv_freq, uint16_t* h,
                      uint16_t* kcache, uint16_t* vcache, int64_t L, const int32_t* parents, int M,
                      int32_t* out_inds, float* out_scores);
/* accepted tree path compacted into consecutive positions (SeedlessAttn.swift:219-225,
 * 540-586): rows at slot (L + path[i]) % C move to (L + i) % C; caches [nKV][C][D] */
void or_kv_commit(uint16_t* kcache, uint16_t* vcache, int nKV, int64_t C, int D, int64_t L,
                  const int32_t* path, int n_path);

/* OpenMP threads of the parallel loops (the timed CPU baseline runs at 1 and at all cores). */
void or_set_threads(int n);
int or_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
