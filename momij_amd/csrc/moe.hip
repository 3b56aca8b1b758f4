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
#include "moe_topk.h"

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

// The same combine, 8 elements a thread (H % 8 == 0, k <= 8) with every load issued before
// the first wait: one memory round trip instead of one per expert.
__global__ __launch_bounds__(256) void k_score_combine8(const uint16_t* __restrict__ down,
                                                        const float* __restrict__ scores,
                                                        const uint16_t* x_resid, uint16_t* y,
                                                        int M, int k, int H, const int* abort) {
    const int i = 8 * (blockIdx.x * 256 + threadIdx.x);
    if (i >= M * H) return;
    const int m = i / H, c = i % H;
    u4v d[8];
    float sc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int jj = min(j, k - 1);
        d[j] = *(const u4v*)(down + ((size_t)m * k + jj) * H + c);
        sc[j] = scores[m * k + jj];
    }
    const u4v xr = *(const u4v*)((x_resid ? x_resid : down) + (size_t)i);
    if (aborted(abort)) return;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if (j < k) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[2 * q] += h2f(d[j][q] & 0xFFFFu) * sc[j];
                acc[2 * q + 1] += h2f(d[j][q] >> 16) * sc[j];
            }
        }
    }
    u4v o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (x_resid)
            o[q] = (uint32_t)f2h(h2f(xr[q] & 0xFFFFu) + hround(acc[2 * q])) |
                   ((uint32_t)f2h(h2f(xr[q] >> 16) + hround(acc[2 * q + 1])) << 16);
        else
            o[q] = (uint32_t)f2h(acc[2 * q]) | ((uint32_t)f2h(acc[2 * q + 1]) << 16);
    }
    *(u4v*)(y + (size_t)i) = o;
}

hipError_t launch_score_combine(const uint16_t* down, const float* scores, const uint16_t* x_resid,
                                uint16_t* y, int M, int k, int H, const int* abort,
                                hipStream_t st) {
    if (H % 8 == 0 && k >= 1 && k <= 8) {
        hipLaunchKernelGGL(k_score_combine8, dim3((M * H / 8 + 255) / 256), dim3(256), 0, st, down,
                           scores, x_resid, y, M, k, H, abort);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_score_combine, dim3((M * H + 255) / 256), dim3(256), 0, st, down, scores,
                       x_resid, y, M, k, H, abort);
    return hipGetLastError();
}

// The expert combine of one row followed by the next RMSNorm (of the next layer's attention,
// or the final norm), H = 2048: one 256-thread block per row, thread t owns elements
// 8t .. 8t+7.  The combine is k_score_combine's arithmetic, the norm k_rmsnorm_qx's.  Every
// load is issued before the first wait (the k <= 8 expert rows at clamped indices, their
// weights, the residual, the norm weights and the abort word): one memory round trip, not one
// per expert.
__global__ __launch_bounds__(256) void k_combine_norm(const uint16_t* __restrict__ down,
                                                      const float* __restrict__ scores,
                                                      const uint16_t* x_resid, uint16_t* y, int k,
                                                      NormOut no, const int* abort) {
    const int r = blockIdx.x, t = threadIdx.x;
    constexpr int H = 2048;
    u4v d[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        d[j] = *(const u4v*)(down + ((size_t)r * k + min(j, k - 1)) * H + 8 * t);
    // the weights as one vector load (lane j holds weight j), not eight scalar ones
    const float scv = scores[r * k + min(t & 7, k - 1)];
    const u4v xr = *(const u4v*)((x_resid ? x_resid : down) + (size_t)r * H + 8 * t);
    const u4v wn = *(const u4v*)(no.w + 8 * t);
    if (aborted(abort)) return;
    float sc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) sc[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(scv), j));
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if (j < k) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[2 * q] += h2f(d[j][q] & 0xFFFFu) * sc[j];
                acc[2 * q + 1] += h2f(d[j][q] >> 16) * sc[j];
            }
        }
    }
    u4v hv;
    if (x_resid) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            hv[q] = (uint32_t)f2h(h2f(xr[q] & 0xFFFFu) + hround(acc[2 * q])) |
                    ((uint32_t)f2h(h2f(xr[q] >> 16) + hround(acc[2 * q + 1])) << 16);
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            hv[q] = (uint32_t)f2h(acc[2 * q]) | ((uint32_t)f2h(acc[2 * q + 1]) << 16);
    }
    *(u4v*)(y + (size_t)r * H + 8 * t) = hv;
    norm_row_2048_w(hv, wn, no, r);
}

hipError_t launch_combine_norm(const uint16_t* down, const float* scores, const uint16_t* x_resid,
                               uint16_t* y, int M, int k, int H, const NormOut& no,
                               const int* abort, hipStream_t st) {
    if (H != 2048 || k < 1 || k > 8) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_combine_norm, dim3(M), dim3(256), 0, st, down, scores, x_resid, y, k, no,
                       abort);
    return hipGetLastError();
}

#define RT_H 2048

// ---------------------------------------------------------------------------------------
// MoE front, two launches:
//   k_route_logits  one 256-thread block per (row, group of RS_EPB experts), M * E / RS_EPB
//                   blocks: RMSNorm of the row (the group-0 block writes it out, plain and in
//                   qx order with its block sums) and the logits of the group's experts.  The
//                   router matrix is read in 32 KB pieces by many CUs (a single CU streams only
//                   a few tens of GB/s).
//   k_route_topk    one wave per row: top-k of the row's logits, renormalised scores, and the
//                   row's (row, slot) pairs appended to the experts' lists.
// The kernel boundary orders the two: a grid-wide handoff inside one kernel needs a device-
// scope release (an L2 write-back on this chip), which costs more than the launch.
// Arithmetic as maple_rms_norm / maple_batched_gemv / maple_route_top8: fp32 sums (the logit
// sums in v_dot2 lane partials and a fixed shuffle tree), softmax with max subtraction, top-k
// by logit with the lowest index winning ties, weights renormalised over the k in rank order.
// The top-k ranks every expert against all E logits (broadcast LDS reads), so the selection
// comes out sorted without a chain of cross-lane reductions.
// ---------------------------------------------------------------------------------------
#define RS_EPB 8  // router rows (experts) per block: two per wave

__global__ __launch_bounds__(256) void k_route_logits(RouteArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int E = a.E, S = E / RS_EPB;
    const int r = blockIdx.x / S, grp = blockIdx.x - r * S;
    __shared__ __align__(16) uint16_t xn[RT_H];
    __shared__ float s_ss[4];
    if (aborted(a.abort)) return;

    // router rows of this wave first (k = 512 c + 8 lane .. +7), then the row
    const int e0 = grp * RS_EPB + 2 * wv;
    u4v wr[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c)
            wr[j][c] = *(const u4v*)(a.W + (size_t)(e0 + j) * RT_H + 512 * c + 8 * lane);
    u4v xv = *(const u4v*)(a.x + (size_t)r * RT_H + 8 * tid);
    u4v nw = {0u, 0u, 0u, 0u};
    if (a.norm_w) nw = *(const u4v*)(a.norm_w + 8 * tid);

    if (a.norm_w) {
        float ss = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float x0 = h2f(xv[q] & 0xFFFFu), x1 = h2f(xv[q] >> 16);
            ss += x0 * x0;
            ss += x1 * x1;
        }
        ss = wave_sum(ss);
        if (lane == 0) s_ss[wv] = ss;
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
    *(u4v*)(xn + 8 * tid) = xv;
    // the fused MoE launch's act rows: the "not yet written" marker, before that launch starts
    for (int i = blockIdx.x * 256 + tid; i < a.act_n16; i += gridDim.x * 256)
        ((u4v*)a.act_mark)[i] = (u4v){~0u, ~0u, ~0u, ~0u};
    if (grp == 0) {
        if (a.xn) *(u4v*)(a.xn + (size_t)r * RT_H + 8 * tid) = xv;
        if (a.xperm)
            emit_qx(xv, lane, a.xperm + (size_t)r * RT_H, a.xsum + (size_t)r * (RT_H / 64), 8 * tid);
    }
    __syncthreads();

    u4v xa[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) xa[c] = *(const u4v*)(xn + 512 * c + 8 * lane);
    float acc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        acc[j] = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[j] = dot2(wr[j][c][q], xa[c][q], acc[j]);
    }
#pragma unroll
    for (int m = 32; m > 0; m >>= 1)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[j] += __shfl_xor(acc[j], m, MJ_WAVE);
    if (lane == 0) *(float2*)(a.logits + (size_t)r * E + e0) = make_float2(acc[0], acc[1]);
}

// inds and scores of every row, and the pair lists of the tile gathers: one 1024-thread block,
// wave w ranks rows w, w + 16, ... (M <= 64: at most four each, all their logits requested
// before the first is ranked).  Pairs are grouped by expert with LDS atomics.  With slot records
// (E <= 64) the routed experts are numbered in increasing id and slot s's record gets expert,
// count and pairs (count 0 for every slot past the last); otherwise each expert's count and list
// go to ecnt / eplist.  Every entry a reader uses is rewritten each launch, so nothing needs
// clearing.  Order inside a list is immaterial: every pair's output is computed the same way
// wherever it sits.
#define RT_WAVES 16
template <int NI>
__global__ __launch_bounds__(64 * RT_WAVES) void k_route_topk(RouteArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, E = a.E, k = a.k, M = a.M;
    constexpr bool SLOTS_OK = NI == 1;  // slot records: at most 64 experts
    __shared__ __align__(16) float s_row[RT_WAVES][64 * NI];
    __shared__ __align__(16) float s_gate[RT_WAVES][8];
    __shared__ int s_ind[RT_WAVES][8];
    __shared__ int s_cnt[MJ_MAX_EXPERTS];
    __shared__ int s_pairs[SLOTS_OK ? 64 : 1][SLOTS_OK ? MJ_ROWS : 1];
    __shared__ int s_wsum[RT_WAVES];
    if (aborted(a.abort)) return;
    const bool slots = SLOTS_OK && a.srec != nullptr;
    if (tid < E) s_cnt[tid] = 0;
    // all of the wave's rows (at most four) requested up front, every load unconditional
    // (clamped row and expert) so no branch waits on one
    float v[4][NI];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < NI; ++i)
            v[s][i] = a.logits[min(wv + RT_WAVES * s, M - 1) * E + min(lane + 64 * i, E - 1)];
    __syncthreads();  // s_cnt cleared
#pragma unroll 1
    for (int s = 0, r = wv; r < M; ++s, r += RT_WAVES) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const float t = s == 0 ? v[0][i] : s == 1 ? v[1][i] : s == 2 ? v[2][i] : v[3][i];
            s_row[wv][lane + 64 * i] = lane + 64 * i < E ? t + 0.0f : -INFINITY;
        }
        __builtin_amdgcn_wave_barrier();
        int e = 0;
        float gate = 0.0f;
        row_topk<NI>(s_row[wv], E, k, s_ind[wv], s_gate[wv], e, gate);
        if (lane < k) {
            a.inds[r * k + lane] = e;
            a.scores[r * k + lane] = gate;
            if (slots) {
                const int pos = atomicAdd(&s_cnt[e], 1);
                if constexpr (SLOTS_OK) s_pairs[e][pos] = r * k + lane;
            } else if (a.ecnt) {
                const int pos = atomicAdd(&s_cnt[e], 1);
                a.eplist[e * MJ_ROWS + pos] = r * k + lane;
            }
        }
    }
    if (!slots && !a.ecnt) return;
    __syncthreads();
    if (!slots) {
        if (tid < E) a.ecnt[tid] = s_cnt[tid];
        return;
    }
    // routed experts numbered in increasing id: slot = routed experts below this one
    const bool on = tid < E && s_cnt[tid] > 0;
    const uint64_t bal = __ballot(on);
    if (lane == 0) s_wsum[wv] = __popcll(bal);
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < RT_WAVES; ++w) {
        before += w < wv ? s_wsum[w] : 0;
        total += s_wsum[w];
    }
    if constexpr (SLOTS_OK) {
        if (on) {
            const int cnt = s_cnt[tid];
            int* rec = a.srec + (before + __popcll(bal & ((1ull << lane) - 1))) * MJ_ROWS;
            for (int j = 0; j < cnt; ++j)
                rec[j] = s_pairs[tid][j] | (j == 0 ? tid << 16 : j == 1 ? cnt << 16 : 0);
            if (cnt == 1) rec[1] = 1 << 16;
        }
        if (tid >= total && tid < 64) {
            a.srec[tid * MJ_ROWS] = 0;
            a.srec[tid * MJ_ROWS + 1] = 0;
        }
    }
}

bool route_supported(int H, int E, int k) {
    return H == RT_H && E >= RS_EPB && E <= MJ_MAX_EXPERTS && E % RS_EPB == 0 && k >= 1 &&
           k <= 8 && k <= E;
}

hipError_t launch_route_logits(const RouteArgs& a, int H, hipStream_t st) {
    if (!route_supported(H, a.E, a.k) || a.M < 1 || a.M > MJ_ROWS) return hipErrorInvalidValue;
    if (!a.logits) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_route_logits, dim3(a.M * (a.E / RS_EPB)), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_route_topk(const RouteArgs& a, hipStream_t st) {
    // one block: 16 waves with at most four rows each
    if (a.E < 1 || a.E > MJ_MAX_EXPERTS || a.k < 1 || a.k > 8 || a.k > a.E || a.M < 1 ||
        a.M > 4 * RT_WAVES || a.M > MJ_ROWS || (a.srec && a.E > 64))
        return hipErrorInvalidValue;
    if (a.E <= 64)
        hipLaunchKernelGGL(k_route_topk<1>, dim3(1), dim3(64 * RT_WAVES), 0, st, a);
    else
        hipLaunchKernelGGL(k_route_topk<MJ_MAX_EXPERTS / 64>, dim3(1), dim3(64 * RT_WAVES), 0, st, a);
    return hipGetLastError();
}
