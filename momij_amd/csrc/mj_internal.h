// mj_internal.h -- launchers shared between the kernel files and the C ABI layer.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

// Kernel-duration timing for measurement: when armed, the next launch made through
// launch_timed() passes `start` / `stop` to hipExtLaunchKernel, which stamps the kernel's own
// start and end (the interval a kernel trace reports, without the dispatch gap an event pair
// recorded around the launch would add); the launch disarms it.
struct TimedLaunch {
    hipEvent_t start = nullptr, stop = nullptr;
    bool armed = false;
};
TimedLaunch& timed_launch();  // per host thread

template <typename K, typename... Args>
inline void launch_timed(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st,
                         Args... args) {
    TimedLaunch& t = timed_launch();
    if (t.armed) {
        t.armed = false;
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, st, t.start, t.stop, 0u, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
    }
}

#define MJ_MAX_EXPERTS 256
#define MJ_MAX_PAIRS 512  // rows * top_k per pass

// Rows of one pass grouped by expert (filled on the device by the router, or implied for a
// dense projection).  pair[start[u] .. start[u+1]) lists the (row * top_k + slot) indices
// routed to expert[u], in increasing order; experts are listed in increasing id.
struct Buckets {
    int count;
    int expert[MJ_MAX_EXPERTS];
    int start[MJ_MAX_EXPERTS + 1];
    int pair[MJ_MAX_PAIRS];
};

enum { EPI_STORE = 0, EPI_ADD = 1, EPI_SWIGLU = 2 };

// Outputs of a fused RMSNorm over 2048-element rows: out = half(x * rsqrt(mean x^2 + eps) * w)
// written plain and / or in qx order with its per-64 block sums.
struct NormOut {
    const uint16_t* w;   // [2048]
    float eps;
    uint16_t* plain;     // [rows][2048] (nullable)
    uint16_t* xperm;     // [rows][2048] qx (nullable)
    float2* xsum;        // [rows][32]
};

#define MJ_ROWS 64  // == MJ_MAX_ROWS of the C ABI

// Per-pass parameters read by the kernels from device memory, so one captured graph serves
// every step with the same row count.  Row r of a pass sits at position L + depth[r]; anc[r]
// has bit a set iff row a is row r or one of its ancestors; tokens[r] is the token fed there.
struct StepDesc {
    int64_t L;
    int32_t M;
    int32_t chain;           // 1: parents[r] = r - 1 for every row (depth[r] = r)
    int32_t tokens[MJ_ROWS];
    int32_t parents[MJ_ROWS];
    int32_t depth[MJ_ROWS];
    uint64_t anc[MJ_ROWS];
    uint64_t seed, counter;  // sampled acceptance
    float temperature;
    float q_uniform;         // 1/V (q_mode uniform)
    int32_t q_mode;
    int32_t has_qpoint;
    float q_point[MJ_ROWS];
    // LogitsProcessor options of a sampled pass (the history itself is in a device buffer)
    float top_p, rep, pres, freq;
    int32_t n_hist;
};

// Result of a verify pass (device, copied back once per step).
struct StepResult {
    int32_t accepted;
    int32_t token;           // bonus (greedy) / resampled or bonus (sampled)
    int32_t path[MJ_ROWS];   // accepted rows, row 0 first
    int32_t emit[MJ_ROWS];   // accepted drafts then the final token
    int32_t argmax[MJ_ROWS];
};


// Row sets of a gather launch (grid = groups x column blocks):
//   ecnt != nullptr (tile kernel): group u = expert u with ecnt[u] pairs listed, in no
//   particular order, at eplist[u * MJ_ROWS ..] (pair = row * top_k + slot);
//   bk != nullptr: group u = bucket u of the table;  neither: dense, one group of dense_rows.
struct GatherArgs {
    const uint16_t* xperm;  // qx activations [rows_x][K]
    const float2* xsum;     // [rows_x][K/64] {sum x, sum base*x}
    const uint32_t* w;      // [E][N][K/16]
    const uint16_t* s;      // [E][N][K/gs]
    const uint16_t* b;
    const Buckets* bk;      // fallback kernel: rows grouped by expert (nullptr: dense)
    const int* ecnt;        // tile kernel: pairs per expert [E]
    const int* eplist;      // tile kernel: pair lists [E][MJ_ROWS]
    const int* srec;        // tile kernel, persistent: one record per routed-expert slot
                            // [64][64]: lane j = pair j (low 16 bits); lane 0 also holds the
                            // expert id, lane 1 the pair count (high 16 bits); count 0 past the
                            // last routed expert
    int dense_rows;         // dense: rows 0 .. dense_rows-1 of expert 0
    const uint16_t* alpha;  // row-alpha weights [E][N] fp16 (scale alpha, bias -alpha in
                            // every group): the tile expert kernels read it instead of s / b
    uint16_t* y;            // STORE/ADD: [pairs][N] ; SWIGLU: act qx [pairs][I]
    float2* ysum;           // SWIGLU: act sums [pairs][I/64]
    int K, N, gs;
    int x_div;              // x row of pair p = p / x_div
    const int* abort;
    // persistent expert mode with fused routing (rlogits set, at most MJ_G5_FUSED_ROWS rows,
    // E <= 64): every block ranks the router logits [rM][rE] itself and builds the slot records
    // in LDS; block 0 writes inds / scores [rM][rk] and the records (rsrec) for the next product
    const float* rlogits;
    int rM, rE, rk;
    int32_t* rinds;
    float* rscores;
    int* rsrec;
    // fused MoE launch (up || gate then down in one kernel): the up product's column blocks,
    // and the bound of a down item's wait for act rows still holding the router launch's
    // marker, in re-stagings of its rows
    int fup_ncb;
    int fpolls;
    int* ffault;  // set (system scope) by a wait that ran out its bound (nullable)
};
#define MJ_G5_FUSED_ROWS 16  // rows the standalone up || gate gather ranks itself
#define MJ_MOE_FUSED_ROWS 32  // rows the fused MoE launch ranks itself

struct QmvArgs {
    const uint16_t* x;      // plain fp16 [rows_x][K]
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
    const int32_t* inds;    // [pairs]
    uint16_t* y;            // STORE: [pairs][N]; SWIGLU: act plain [pairs][I]
    int K, N, gs, pairs, lhs_per, rows_per_wave, waves_per_pair;
    const int* abort;
};

// qmm2.hip
hipError_t launch_qx_prep(const uint16_t* x, uint16_t* xperm, float2* xsum, int rows, int K,
                          const int* abort, hipStream_t st);
hipError_t launch_qx_sums(const uint16_t* xperm, float2* xsum, int rows, int K, const int* abort,
                          hipStream_t st);
hipError_t launch_qmv2(const QmvArgs& a, int epi, hipStream_t st);
hipError_t launch_gather(const GatherArgs& a, int epi, int max_rows_per_bucket, int n_buckets_max,
                         hipStream_t st);
hipError_t launch_selftest_mfma(const uint16_t* A, const uint16_t* B, float* D, hipStream_t st);

// gather.hip: the tile gather (one 16-row weight tile over the whole K per wave)
bool gather3_supported(int epi, int K, int N, int gs);
// the fused MoE launch: up || gate with its routing, then down, in one persistent kernel
// (the shapes, and two blocks of the launch resident a CU: its waits assume every block runs)
bool moe_fused_supported(int H, int I, int E, int gs, int M, bool rowa);
hipError_t launch_moe_fused(const GatherArgs& up, const GatherArgs& dn, int rows, hipStream_t st);
hipError_t launch_gather3(const GatherArgs& a, int epi, int max_rows_per_bucket, int n_buckets,
                          hipStream_t st);

// RoPE angles of a pass: rope_cs[r * MJ_ROPE_F + f] = {cos, sin} of (L + depth[r]) *
// inv_freq[f] for row r and frequency f < rope_dim / 2, written by the pass's embedding kernel
// (or k_rope_table) so that no layer evaluates a sine.
#define MJ_ROPE_F 64
struct RopeTab {
    const float* inv_freq;  // [half]
    float2* cs;             // [MJ_ROWS][MJ_ROPE_F]
    int half;               // rope_dim / 2 (0: no RoPE layer in the model)
};

struct AttnArgs {
    const uint16_t* qkv;     // [M][(nQ+2nKV)*128] projection output (plain, raw q / k / v)
    const uint16_t* q_norm_w;
    const uint16_t* k_norm_w;
    const float2* rope_cs;   // RopeTab::cs of the pass
    const StepDesc* sd;
    uint16_t* kc;            // [nKV][C][128]
    uint16_t* vc;
    float* opart;            // [nKV][max_chunks][nqt*16][128] partial outputs
    float2* mlpart;          // [nKV][max_chunks][nqt*16] {max, sum}
    uint16_t* out_perm;      // attention output, qx [M][nQ*128]
    float2* out_sum;         // [M][nQ*2]
    int M, nQ, nKV, rope_dim, window, max_chunks;
    int64_t C;
    float eps, scale;
    const int* abort;
};

// attn.hip
hipError_t launch_attn(const AttnArgs& a, hipStream_t st);
int attn_max_chunks(int window, int64_t L_max, int M);

// head.hip
// Optional per-row log-sum-exp of logits / T: k = log2(e) / T, block partials pm / ps
// [blocks][32] (log2-unit max and scaled sum), out [M] natural-log result.  out == nullptr: off.
struct HeadLse {
    float k;
    float* pm;
    float* ps;
    float* out;
};
// Greedy acceptance of a verify pass over the head's argmax ids (tokens / parents: the step
// descriptor's rows), folded into the head's final launch.
struct GreedyAccept {
    const int32_t* tokens;
    const int32_t* parents;
    StepResult* res;
};
hipError_t launch_lm_head(const uint16_t* x, const uint16_t* w, int M, int K, int V,
                          const int32_t* banned, int n_banned, float* logits, float* pval,
                          int* pidx, int32_t* out_idx, float* out_max, HeadLse lse,
                          const int* abort, hipStream_t st, const GreedyAccept* ga = nullptr);
// Banned ids the 4-bit head stages in LDS (the reference passes at most 16,
// SeedlessDecodeEngine.swift:470, 496).
#define MJ_HEAD_MAX_BANNED 64
hipError_t launch_lm_head_q4(const uint16_t* x, const uint32_t* w, const uint16_t* s,
                             const uint16_t* b, int M, int K, int V, const int32_t* banned,
                             int n_banned, float* logits, float* pval, int* pidx,
                             int32_t* out_idx, float* out_max, HeadLse lse, const int* abort,
                             hipStream_t st, const GreedyAccept* ga = nullptr);
int head_blocks();
hipError_t launch_accept_greedy(const int32_t* tokens, const int32_t* parents,
                                const int32_t* argmax, int n, StepResult* res, int32_t* out_flat,
                                const int* abort, hipStream_t st);
hipError_t launch_kv_commit(uint16_t* kv, int64_t layer_stride, int n_layers, int64_t C, int nKV,
                            const StepDesc* sd, const StepResult* res, const int* abort,
                            hipStream_t st);
hipError_t launch_kv_rows(const uint16_t* kv, int64_t layer_stride, int n_layers, int64_t C,
                          int nKV, const StepDesc* sd, uint16_t* dst, hipStream_t st);
// The embedding kernels also write the pass's RoPE table (rt.half == 0: none).
hipError_t launch_embed(const uint16_t* table, const StepDesc* sd, int M, int H, uint16_t* h,
                        const RopeTab& rt, const int* abort, hipStream_t st);
hipError_t launch_embed_norm(const uint16_t* table, const StepDesc* sd, int M, int H, uint16_t* h,
                             const NormOut& no, const RopeTab& rt, const int* abort,
                             hipStream_t st);  // H = 2048
hipError_t launch_rope_table(const StepDesc* sd, int M, const RopeTab& rt, hipStream_t st);
// One wave that waits `us` microseconds of wall-clock time (bounded), so that the host can
// queue the launches that follow it before the GPU reaches them.
hipError_t launch_hold(unsigned us, hipStream_t st);

// sample.hip
// LogitsProcessor options (LogitsProcessor.swift:17-104): the penalties change the logits in
// place (the buffer must be writable), the nucleus needs a NucleusBuf.
struct SampleOpts {
    float top_p = 1.0f, rep = 1.0f, pres = 0.0f, freq = 0.0f;
    const int32_t* hist_tok = nullptr;  // device, ascending, distinct (the seen set)
    const int32_t* hist_cnt = nullptr;  // device, their counts
    int n_hist = 0;
};
struct NucState {
    int need, row, acc;
    float u, Z;
};
// Scratch of a nucleus sample over one row of V: the row's keys (e bits), the selection's four
// rounds of digit histograms (counts [4][256], exact masses [4][256]), the last round's counts
// per block [blocks][256], and the deferred decision.
struct NucleusBuf {
    uint32_t* keys;
    uint32_t* hcnt;
    uint64_t* hmass;
    uint32_t* hblk;
    NucState* st;
};
size_t nucleus_bytes(int V);
void nucleus_layout(void* base, int V, NucleusBuf& nb);
// Full-vocabulary sampled acceptance.  With sd the temperature, q, uniforms' seed / counter,
// the drafts and the options' scalars come from the step descriptor (hist arrays from o).
// head_max: the exact maxima of the rows as given (the lm_head's), for a call without
// penalties only (the caller knows): the penalty and row-maximum launches are then left out.
hipError_t launch_accept_sampled(float* logits, int rows, int V, const int32_t* draft,
                                 float temperature, int q_mode, const float* q_point,
                                 uint64_t seed, uint64_t counter, const SampleOpts& o,
                                 const NucleusBuf* nb, float* rowmax, float* bsum, int32_t* out,
                                 StepResult* res, const StepDesc* sd, const int* abort,
                                 hipStream_t st, const float* head_max = nullptr);
int sample_nblocks(int V);
size_t sample_scratch_floats(int rows, int V);  // the bsum buffer of launch_accept_sampled

// large-LDS kernels need their limit raised once per process
hipError_t set_kernel_attributes();

// moe.hip
hipError_t launch_rmsnorm_qx(const uint16_t* x, const uint16_t* w, float eps, uint16_t* out_plain,
                             uint16_t* xperm, float2* xsum, int rows, int H, const int* abort,
                             hipStream_t st);
hipError_t launch_router(const uint16_t* W, const uint16_t* x, float* logits, int M, int E, int H,
                         const int* abort, hipStream_t st);
hipError_t launch_topk_bucket(const float* logits, int M, int E, int k, int32_t* inds,
                              float* scores, Buckets* bk, const int* abort, hipStream_t st);
hipError_t launch_bucket_inds(const int32_t* inds, int P, Buckets* bk, const int* abort,
                              hipStream_t st);
struct RouteArgs {
    const uint16_t* x;       // [M][H] rows
    const uint16_t* norm_w;  // [H] RMSNorm weight, nullptr: rows are already normed
    const uint16_t* W;       // router [E][H]
    uint16_t* xn;            // normed rows, plain [M][H] (optional)
    uint16_t* xperm;         // normed rows, qx [M][H] (optional)
    float2* xsum;            // [M][H/64]
    int32_t* inds;           // [M][k]
    float* scores;           // [M][k]
    float* logits;           // [M][E] router logits
    int* ecnt;               // pairs per expert [E] (route lists)
    int* eplist;             // pair lists [E][MJ_ROWS] (route lists)
    int* srec;               // slot records of the persistent gathers [64][64] (E <= 64;
                             // nullable: then ecnt / eplist, when set, are written instead)
    int M, E, k;
    float eps;
    const int* abort;
    uint16_t* act_mark;      // act rows of the fused MoE launch that follows (nullable): every
    int act_n16;             // 16-byte chunk of them set to the marker 0xFFFF here, before it
};
bool route_supported(int H, int E, int k);
hipError_t launch_route_logits(const RouteArgs& a, int H, hipStream_t st);
// inds and scores of every row from the logits, and (when a.ecnt is set, M <= MJ_ROWS) the
// per-expert pair lists ecnt / eplist
hipError_t launch_route_topk(const RouteArgs& a, hipStream_t st);
// y = [x_resid +] combine of the k expert rows (as launch_score_combine), then the norm of y
// into `no`; H must be 2048.
hipError_t launch_combine_norm(const uint16_t* down, const float* scores, const uint16_t* x_resid,
                               uint16_t* y, int M, int k, int H, const NormOut& no,
                               const int* abort, hipStream_t st);
hipError_t launch_score_combine(const uint16_t* down, const float* scores, const uint16_t* x_resid,
                                uint16_t* y, int M, int k, int H, const int* abort,
                                hipStream_t st);
