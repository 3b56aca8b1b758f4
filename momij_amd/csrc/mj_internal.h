// mj_internal.h -- launchers shared between the kernel files and the C ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

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

struct GatherArgs {
    const uint16_t* xperm;  // qx activations [rows_x][K]
    const float2* xsum;     // [rows_x][K/64] {sum x, sum base*x}
    const uint32_t* w;      // [E][N][K/16]
    const uint16_t* s;      // [E][N][K/gs]
    const uint16_t* b;
    const Buckets* bk;      // nullptr: dense, one bucket (expert 0) with pairs 0..dense_rows-1
    int dense_rows;
    uint16_t* y;            // STORE/ADD: [pairs][N] ; SWIGLU: act qx [pairs][I]
    float2* ysum;           // SWIGLU: act sums [pairs][I/64]
    int K, N, gs;
    int x_div;              // x row of pair p = p / x_div
    const int* abort;
};

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
hipError_t launch_qmv2(const QmvArgs& a, int epi, hipStream_t st);
hipError_t launch_gather(const GatherArgs& a, int epi, int max_rows_per_bucket, int n_buckets_max,
                         hipStream_t st);
hipError_t launch_selftest_mfma(const uint16_t* A, const uint16_t* B, float* D, hipStream_t st);

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
hipError_t launch_score_combine(const uint16_t* down, const float* scores, const uint16_t* x_resid,
                                uint16_t* y, int M, int k, int H, const int* abort,
                                hipStream_t st);
