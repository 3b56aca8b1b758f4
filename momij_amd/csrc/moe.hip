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

// Writes 8 consecutive plain values (4 fp16 pairs in v, elements k0..k0+7 of a row, k0 a
// multiple of 8) in qx order, and the block sums from lanes with (lane & 7) == 0.  Lanes must
// come in aligned groups of 8 covering one 64-block.
__device__ __forceinline__ void emit_qx(const u4v v, int lane, uint16_t* xperm_row,
                                        float2* xsum_row, int k0) {
    u4v o;
    o.x = __shfl_xor(v.x, 1, MJ_WAVE);
    o.y = __shfl_xor(v.y, 1, MJ_WAVE);
    o.z = __shfl_xor(v.z, 1, MJ_WAVE);
    o.w = __shfl_xor(v.w, 1, MJ_WAVE);
    const bool odd = lane & 1;
    const uint32_t u[8] = {odd ? o.x : v.x, odd ? o.y : v.y, odd ? o.z : v.z, odd ? o.w : v.w,
                           odd ? v.x : o.x, odd ? v.y : o.y, odd ? v.z : o.z, odd ? v.w : o.w};
    uint32_t p[8];
    perm16(u, p);
    u4v out;
    out.x = odd ? p[4] : p[0];
    out.y = odd ? p[5] : p[1];
    out.z = odd ? p[6] : p[2];
    out.w = odd ? p[7] : p[3];
    *(u4v*)(xperm_row + k0) = out;
    float X = 0.0f, Bx = 0.0f;
    X = dot2(v.x, 0x3C003C00u, X);
    X = dot2(v.y, 0x3C003C00u, X);
    X = dot2(v.z, 0x3C003C00u, X);
    X = dot2(v.w, 0x3C003C00u, X);
    Bx = dot2(v.x, 0x44004C00u, Bx);
    Bx = dot2(v.y, 0x44004C00u, Bx);
    Bx = dot2(v.z, 0x44004C00u, Bx);
    Bx = dot2(v.w, 0x44004C00u, Bx);
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
        X += __shfl_xor(X, m, MJ_WAVE);
        Bx += __shfl_xor(Bx, m, MJ_WAVE);
    }
    if ((lane & 7) == 0) xsum_row[k0 >> 6] = make_float2(X, Bx);
}

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
