// moe.hip -- RMSNorm into the qx activation format, router logits, top-k routing with
// expert bucketing, and the score-weighted expert combine.
//
// RMSNorm    maple_rms_norm (SeedlessMetal.swift:2496-2526): out = half(x * rsqrt(mean x^2 +
//            eps) * w), fp32.  Written plain (router input) and in qx order (2-bit product
//            input) with per-64-block {sum x, sum base*x}.
// Router     maple_batched_gemv (2574-2595): logits[m][e] = sum_k W[e][k] x[m][k], fp32.
// Route      maple_route_top8 (2720-2791): softmax with exp, top-k by logit (lowest index
//            on ties), scores = gate / sum of the k gates.  Then the (row, slot) pairs are
//            grouped by expert so every routed expert is streamed once for all its rows.
// Combine    maple_score_reduce / maple_score_resid (2452-2493):
//            y = [x +] half(sum_j half(down_j) * score_j), j in slot order.
#include "mj_device.h"
#include "mj_internal.h"

// One 256-thread block per row; H % 2048 == 0, H <= 8192.
__global__ __launch_bounds__(256) void k_rmsnorm_qx(const uint16_t* __restrict__ x,
                                                    const uint16_t* __restrict__ w, float eps,
                                                    uint16_t* out_plain, uint16_t* xperm,
                                                    float2* xsum, int H, const int* abort) {
    if (aborted(abort)) return;
    const int row = blockIdx.x, t = threadIdx.x, lane = t & 63;
    const uint16_t* xr = x + (size_t)row * H;
    const int nch = H / 2048;
    u4v xv[4];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        if (c >= nch) break;
        xv[c] = *(const u4v*)(xr + 2048 * c + 8 * t);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float a = h2f(xv[c][j] & 0xFFFFu), b = h2f(xv[c][j] >> 16);
            ss += a * a;
            ss += b * b;
        }
    }
    ss = wave_sum(ss);
    __shared__ float red[4];
    if (lane == 0) red[t >> 6] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(tot / (float)H + eps);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        if (c >= nch) break;
        const int k0 = 2048 * c + 8 * t;
        const u4v wv = *(const u4v*)(w + k0);
        u4v o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float a = h2f(xv[c][j] & 0xFFFFu) * inv * h2f(wv[j] & 0xFFFFu);
            const float b = h2f(xv[c][j] >> 16) * inv * h2f(wv[j] >> 16);
            o[j] = (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16);
        }
        if (out_plain) *(u4v*)(out_plain + (size_t)row * H + k0) = o;
        if (xperm) emit_qx(o, lane, xperm + (size_t)row * H, xsum + (size_t)row * (H / 64), k0);
    }
}

hipError_t launch_rmsnorm_qx(const uint16_t* x, const uint16_t* w, float eps, uint16_t* out_plain,
                             uint16_t* xperm, float2* xsum, int rows, int H, const int* abort,
                             hipStream_t st) {
    hipLaunchKernelGGL(k_rmsnorm_qx, dim3(rows), dim3(256), 0, st, x, w, eps, out_plain, xperm,
                       xsum, H, abort);
    return hipGetLastError();
}

// One wave per expert: the expert's router row stays in registers, every token row is dotted
// against it.  H % 512 == 0, H <= 4096.
__global__ __launch_bounds__(256) void k_router(const uint16_t* __restrict__ W,
                                                const uint16_t* __restrict__ x, float* logits,
                                                int M, int E, int H, const int* abort) {
    if (aborted(abort)) return;
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (e >= E) return;
    const int nch = H / 512;
    u4v wr[8];
#pragma unroll
    for (int c = 0; c < 8; ++c)
        if (c < nch) wr[c] = *(const u4v*)(W + (size_t)e * H + 512 * c + 8 * lane);
    for (int m = 0; m < M; ++m) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            if (c >= nch) break;
            const u4v xv = *(const u4v*)(x + (size_t)m * H + 512 * c + 8 * lane);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = dot2(wr[c][j], xv[j], acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) logits[(size_t)m * E + e] = acc;
    }
}

hipError_t launch_router(const uint16_t* W, const uint16_t* x, float* logits, int M, int E, int H,
                         const int* abort, hipStream_t st) {
    hipLaunchKernelGGL(k_router, dim3((E + 3) / 4), dim3(256), 0, st, W, x, logits, M, E, H,
                       abort);
    return hipGetLastError();
}

// Group pair indices 0..P-1 by expert id (ids in s_ids, LDS): experts in increasing id, pairs
// in increasing index inside each expert.  Ids outside [0, E) are left out.  Whole block.
__device__ void bucket_pairs(const int* s_ids, int P, int E, Buckets* bk, int* s_cnt,
                             int* s_slot) {
    const int t = threadIdx.x;
    for (int e = t; e < E; e += blockDim.x) s_cnt[e] = 0;
    __syncthreads();
    for (int p = t; p < P; p += blockDim.x) {
        const int e = s_ids[p];
        if (e >= 0 && e < E) atomicAdd(&s_cnt[e], 1);
    }
    __syncthreads();
    if (t == 0) {
        int u = 0, pos = 0;
        for (int e = 0; e < E; ++e) {
            if (s_cnt[e] > 0) {
                bk->expert[u] = e;
                bk->start[u] = pos;
                s_slot[e] = pos;
                pos += s_cnt[e];
                ++u;
            }
        }
        bk->start[u] = pos;
        bk->count = u;
        for (int p = 0; p < P; ++p) {
            const int e = s_ids[p];
            if (e >= 0 && e < E) bk->pair[s_slot[e]++] = p;
        }
    }
}

__global__ __launch_bounds__(256) void k_bucket_inds(const int32_t* __restrict__ inds, int P,
                                                     Buckets* bk, const int* abort) {
    if (aborted(abort)) return;
    __shared__ int s_ids[MJ_MAX_PAIRS];
    __shared__ int s_cnt[MJ_MAX_EXPERTS];
    __shared__ int s_slot[MJ_MAX_EXPERTS];
    for (int p = threadIdx.x; p < P; p += blockDim.x) s_ids[p] = inds[p];
    __syncthreads();
    bucket_pairs(s_ids, P, MJ_MAX_EXPERTS, bk, s_cnt, s_slot);
}

hipError_t launch_bucket_inds(const int32_t* inds, int P, Buckets* bk, const int* abort,
                              hipStream_t st) {
    hipLaunchKernelGGL(k_bucket_inds, dim3(1), dim3(256), 0, st, inds, P, bk, abort);
    return hipGetLastError();
}

// Single block: softmax + top-k per row (one wave per row), then expert bucketing.
__global__ __launch_bounds__(256) void k_topk_bucket(const float* __restrict__ logits, int M,
                                                     int E, int k, int32_t* inds, float* scores,
                                                     Buckets* bk, const int* abort) {
    if (aborted(abort)) return;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    __shared__ int s_inds[MJ_MAX_PAIRS];
    __shared__ int s_cnt[MJ_MAX_EXPERTS];
    __shared__ int s_slot[MJ_MAX_EXPERTS];
    for (int m = wv; m < M; m += 4) {
        const float* lg = logits + (size_t)m * E;
        float lv[4], work[4];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = lane + 64 * i;
            lv[i] = e < E ? lg[e] : -INFINITY;
            mx = fmaxf(mx, lv[i]);
        }
        mx = wave_max(mx);
        float z = 0.0f, g[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = lane + 64 * i;
            g[i] = e < E ? expf(lv[i] - mx) : 0.0f;
            z += g[i];
            work[i] = lv[i];
        }
        z = wave_sum(z);
        float sel[8];
        int seli[8];
        for (int j = 0; j < k; ++j) {
            float bv = work[0];
            int bi = lane;
#pragma unroll
            for (int i = 1; i < 4; ++i)
                if (work[i] > bv) {
                    bv = work[i];
                    bi = lane + 64 * i;
                }
            wave_argmax(bv, bi);
            // owner lane marks it taken and publishes the gate
            float gsel = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (lane + 64 * i == bi) {
                    work[i] = -INFINITY;
                    gsel = g[i] / z;
                }
            gsel = __shfl(gsel, bi & 63, MJ_WAVE);
            sel[j] = gsel;
            seli[j] = bi;
        }
        if (lane == 0) {
            float ssum = 0.0f;
            for (int j = 0; j < k; ++j) ssum += sel[j];
            for (int j = 0; j < k; ++j) {
                inds[m * k + j] = seli[j];
                scores[m * k + j] = sel[j] / ssum;
                s_inds[m * k + j] = seli[j];
            }
        }
    }
    if (bk == nullptr) return;
    __syncthreads();
    bucket_pairs(s_inds, M * k, E, bk, s_cnt, s_slot);
}

hipError_t launch_topk_bucket(const float* logits, int M, int E, int k, int32_t* inds,
                              float* scores, Buckets* bk, const int* abort, hipStream_t st) {
    hipLaunchKernelGGL(k_topk_bucket, dim3(1), dim3(256), 0, st, logits, M, E, k, inds, scores,
                       bk, abort);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_score_combine(const uint16_t* __restrict__ down,
                                                       const float* __restrict__ scores,
                                                       const uint16_t* x_resid, uint16_t* y,
                                                       int M, int k, int H, const int* abort) {
    if (aborted(abort)) return;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= M * H) return;
    const int m = i / H, c = i % H;
    float acc = 0.0f;
    for (int j = 0; j < k; ++j) acc += h2f(down[((size_t)m * k + j) * H + c]) * scores[m * k + j];
    if (x_resid)
        y[i] = f2h(h2f(x_resid[i]) + hround(acc));
    else
        y[i] = f2h(acc);
}

hipError_t launch_score_combine(const uint16_t* down, const float* scores, const uint16_t* x_resid,
                                uint16_t* y, int M, int k, int H, const int* abort,
                                hipStream_t st) {
    hipLaunchKernelGGL(k_score_combine, dim3((M * H + 255) / 256), dim3(256), 0, st, down, scores,
                       x_resid, y, M, k, H, abort);
    return hipGetLastError();
}

#define RT_H 2048

// ---------------------------------------------------------------------------------------
// MoE front, one 512-thread block per pass row: RMSNorm of the row (written plain and in qx
// order with its block sums), its E router logits and its top-k, with no dependency between
// blocks.  Every block reads the whole router (E x 2048 fp16, L2-resident after the first
// rows) -- the price of needing no grid-wide synchronisation.
// Arithmetic as maple_rms_norm / maple_batched_gemv / maple_route_top8: fp32 sums (the logit
// sums in v_dot2 lane partials and a fixed shuffle tree), softmax with max subtraction, top-k
// by logit with the lowest index winning ties, weights renormalised over the k in rank order.
// The top-k ranks every expert against all E logits (broadcast LDS reads), so the selection
// comes out sorted without a chain of cross-lane reductions.
// ---------------------------------------------------------------------------------------
#define RR_EPW 8  // router rows per wave per round (8 waves -> 64 experts a round)

__global__ __launch_bounds__(512) void k_route_row(RouteArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = blockIdx.x, E = a.E, k = a.k;
    // the other count buffer is cleared for the next launch even when this one is aborted (the
    // launch that used it has completed: stream order)
    if (blockIdx.x == 0 && a.ecnt_clear)
        for (int e = tid; e < E; e += 512) a.ecnt_clear[e] = 0;
    __shared__ __align__(16) uint16_t xn[RT_H];
    __shared__ float s_ss[4];
    __shared__ __align__(16) float s_lg[MJ_MAX_EXPERTS];
    __shared__ float s_gate[8];
    if (aborted(a.abort)) return;  // whole grid: the abort word is fixed during a launch

    // row r: threads 0..255 hold 8 consecutive elements each
    u4v xv = {0u, 0u, 0u, 0u}, nw = {0u, 0u, 0u, 0u};
    if (tid < 256) {
        xv = *(const u4v*)(a.x + (size_t)r * RT_H + 8 * tid);
        if (a.norm_w) nw = *(const u4v*)(a.norm_w + 8 * tid);
    }
    // the first round of router rows: expert wv + 8 j, k = 512 c + 8 lane .. +7
    u4v wr[RR_EPW][4];
    auto load_round = [&](int e0) {
#pragma unroll
        for (int j = 0; j < RR_EPW; ++j) {
            const int e = min(e0 + wv + 8 * j, E - 1);
#pragma unroll
            for (int c = 0; c < 4; ++c)
                wr[j][c] = *(const u4v*)(a.W + (size_t)e * RT_H + 512 * c + 8 * lane);
        }
    };
    load_round(0);

    // RMSNorm
    if (a.norm_w) {
        float ss = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float x0 = h2f(xv[q] & 0xFFFFu), x1 = h2f(xv[q] >> 16);
            ss += x0 * x0;
            ss += x1 * x1;
        }
        ss = wave_sum(ss);
        if (lane == 0 && wv < 4) s_ss[wv] = ss;
        __syncthreads();
        const float tot = (s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3]);
        const float inv = 1.0f / sqrtf(tot / (float)RT_H + a.eps);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float x0 = h2f(xv[q] & 0xFFFFu) * inv * h2f(nw[q] & 0xFFFFu);
            const float x1 = h2f(xv[q] >> 16) * inv * h2f(nw[q] >> 16);
            xv[q] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
        }
    }
    if (tid < 256) {
        *(u4v*)(xn + 8 * tid) = xv;
        if (a.xn) *(u4v*)(a.xn + (size_t)r * RT_H + 8 * tid) = xv;
        if (a.xperm)
            emit_qx(xv, lane, a.xperm + (size_t)r * RT_H, a.xsum + (size_t)r * (RT_H / 64), 8 * tid);
    }
    __syncthreads();

    // logits: all partial dot products of a round, then their reductions together
    u4v xa[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) xa[c] = *(const u4v*)(xn + 512 * c + 8 * lane);
    for (int e0 = 0; e0 < E; e0 += 8 * RR_EPW) {
        if (e0 > 0) load_round(e0);
        float acc[RR_EPW];
#pragma unroll
        for (int j = 0; j < RR_EPW; ++j) {
            acc[j] = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[j] = dot2(wr[j][c][q], xa[c][q], acc[j]);
        }
#pragma unroll
        for (int m = 32; m > 0; m >>= 1)
#pragma unroll
            for (int j = 0; j < RR_EPW; ++j) acc[j] += __shfl_xor(acc[j], m, MJ_WAVE);
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < RR_EPW; ++j) {
                const int e = e0 + wv + 8 * j;
                if (e < E) s_lg[e] = acc[j];
            }
        }
    }
    __syncthreads();
    if (wv != 0) return;

    // top-k of the row (wave 0): lane holds experts lane + 64 i
    float lv[4];
    int rank[4];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = lane + 64 * i;
        lv[i] = e < E ? s_lg[e] : -INFINITY;
        mx = fmaxf(mx, lv[i]);
        rank[i] = 0;
    }
    for (int e2 = 0; e2 < E; e2 += 4) {
        const f4 o = *(const f4*)(s_lg + e2);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int e = lane + 64 * i;
                rank[i] += (int)(o[c] > lv[i]) + (int)(o[c] == lv[i]) * (int)(e2 + c < e);
            }
    }
    mx = wave_max(mx);
    float z = 0.0f, g[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = lane + 64 * i;
        g[i] = e < E ? expf(lv[i] - mx) : 0.0f;
        z += g[i];
    }
    z = wave_sum(z);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = lane + 64 * i;
        if (e < E && rank[i] < k) {
            s_gate[rank[i]] = g[i] / z;
            a.inds[r * k + rank[i]] = e;
        }
    }
    __builtin_amdgcn_wave_barrier();
    if (lane < k) {
        float ssum = 0.0f;
        for (int j = 0; j < k; ++j) ssum += s_gate[j];  // in rank order
        a.scores[r * k + lane] = s_gate[lane] / ssum;
    }
    // append (row, slot) pairs to the experts' lists (order inside a list is immaterial: every
    // pair's output is computed the same way wherever it sits)
    for (int i = 0; i < 4; ++i) {
        const int e = lane + 64 * i;
        if (e < E && rank[i] < k) {
            const int pos = atomicAdd(&a.ecnt[e], 1);
            a.eplist[e * MJ_ROWS + pos] = r * k + rank[i];
        }
    }
}

__global__ void k_zero_i32(int* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

hipError_t launch_zero_i32(int* p, int n, hipStream_t st) {
    hipLaunchKernelGGL(k_zero_i32, dim3((n + 255) / 256), dim3(256), 0, st, p, n);
    return hipGetLastError();
}

bool route_supported(int H, int E, int k) {
    return H == RT_H && E >= 8 && E <= MJ_MAX_EXPERTS && E % 4 == 0 && k >= 1 && k <= 8 && k <= E;
}

hipError_t launch_route(const RouteArgs& a, int H, hipStream_t st) {
    if (!route_supported(H, a.E, a.k) || a.M < 1 || a.M > MJ_ROWS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_route_row, dim3(a.M), dim3(512), 0, st, a);
    return hipGetLastError();
}

hipError_t set_moe_attributes() { return hipSuccess; }
