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

// ---------------------------------------------------------------------------------------
// Fused MoE front: RMSNorm of the pass rows, router logits on MFMA, softmax / top-k per row
// and the expert buckets, in one 512-thread block (the whole step is a few hundred KB, so
// one launch with every load issued up front beats four dependent launches).
// Arithmetic as above except the order of the logit sum (MFMA over 32-element k slices,
// then the two K-halves in order).  H = 2048: rows go in chunks of 16 (wave w normalises
// rows w and w + 8 of the chunk); for the router the 8 waves are 4 expert tiles x 2 K-halves
// of 1024 and each keeps its slice of the router rows of one 64-expert chunk in registers.
// ---------------------------------------------------------------------------------------
#define RT_H 2048
#define RT_XS (RT_H + 8)  // LDS row stride (halves)
#define RT_NS 32          // MFMA k-steps per wave (1024 / 32)

static constexpr size_t route_lds_bytes() {
    return (size_t)16 * RT_XS * 2 + 2 * 16 * 64 * 4 + 16 * MJ_MAX_EXPERTS * 4 +
           MJ_MAX_EXPERTS * 8 + MJ_MAX_PAIRS * 4 + MJ_MAX_EXPERTS * 4 + 16;
}

__global__ __launch_bounds__(512) void k_route(RouteArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int M = a.M, E = a.E, k = a.k;
    extern __shared__ __align__(16) char rt_lds[];
    uint16_t* xs = (uint16_t*)rt_lds;                                  // [16][RT_XS]
    float* red = (float*)(xs + 16 * RT_XS);                            // [2][16][64]
    float* lg = red + 2 * 16 * 64;                                     // [16][E]
    unsigned long long* s_mask = (unsigned long long*)(lg + 16 * MJ_MAX_EXPERTS);  // [E]
    int* s_inds = (int*)(s_mask + MJ_MAX_EXPERTS);                     // [M*k]
    int* s_start = s_inds + MJ_MAX_PAIRS;                              // [E]
    int* s_abort = s_start + MJ_MAX_EXPERTS;

    const int et = wv & 3, kh = wv >> 2;
    const int ecol = et * 16 + (lane & 15);
    const int kl = kh * 1024 + 8 * (lane >> 4);
    u4v wr[RT_NS];
#pragma unroll
    for (int s = 0; s < RT_NS; ++s)
        wr[s] = *(const u4v*)(a.W + (size_t)ecol * RT_H + kl + 32 * s);
    for (int e = tid; e < MJ_MAX_EXPERTS; e += 512) s_mask[e] = 0ull;

    for (int c0 = 0; c0 < M; c0 += 16) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int rl = wv + 8 * half, r = c0 + rl;
            u4v o[4];
            if (r < M) {
                const uint16_t* xr = a.x + (size_t)r * RT_H;
                u4v nw[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    o[c] = *(const u4v*)(xr + 512 * c + 8 * lane);
                    nw[c] = a.norm_w ? *(const u4v*)(a.norm_w + 512 * c + 8 * lane)
                                     : (u4v){0u, 0u, 0u, 0u};
                }
                if (a.norm_w) {
                    float ss = 0.0f;
#pragma unroll
                    for (int c = 0; c < 4; ++c)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const float x0 = h2f(o[c][j] & 0xFFFFu), x1 = h2f(o[c][j] >> 16);
                            ss += x0 * x0;
                            ss += x1 * x1;
                        }
                    ss = wave_sum(ss);
                    const float inv = 1.0f / sqrtf(ss / (float)RT_H + a.eps);
#pragma unroll
                    for (int c = 0; c < 4; ++c)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const float x0 = h2f(o[c][j] & 0xFFFFu) * inv * h2f(nw[c][j] & 0xFFFFu);
                            const float x1 = h2f(o[c][j] >> 16) * inv * h2f(nw[c][j] >> 16);
                            o[c][j] = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
                        }
                }
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) o[c] = (u4v){0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) *(u4v*)(xs + rl * RT_XS + 512 * c + 8 * lane) = o[c];
        }
        if (c0 == 0 && tid == 0) *s_abort = a.abort ? *a.abort : 0;
        __syncthreads();
        if (*s_abort) {
            if (tid == 0 && a.bk) a.bk->count = 0;
            return;  // block-uniform
        }
        // normed rows out (plain and / or qx)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int rl = wv + 8 * half, r = c0 + rl;
            if (r < M && (a.xn || a.xperm)) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int k0 = 512 * c + 8 * lane;
                    const u4v o = *(const u4v*)(xs + rl * RT_XS + k0);
                    if (a.xn) *(u4v*)(a.xn + (size_t)r * RT_H + k0) = o;
                    if (a.xperm)
                        emit_qx(o, lane, a.xperm + (size_t)r * RT_H,
                                a.xsum + (size_t)r * (RT_H / 64), k0);
                }
            }
        }
        for (int e0 = 0; e0 < E; e0 += 64) {
            if (e0 > 0 || c0 > 0) {
#pragma unroll
                for (int s = 0; s < RT_NS; ++s)
                    wr[s] = *(const u4v*)(a.W + (size_t)(e0 + ecol) * RT_H + kl + 32 * s);
            }
            f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < RT_NS; ++s) {
                const u4v av = *(const u4v*)(xs + (lane & 15) * RT_XS + kl + 32 * s);
                d = mfma16x16x32(as_h8(av), as_h8(wr[s]), d);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) red[(kh * 16 + 4 * (lane >> 4) + q) * 64 + ecol] = d[q];
            __syncthreads();
#pragma unroll
            for (int rep = 0; rep < 2; ++rep) {
                const int idx = tid + 512 * rep, row = idx >> 6, col = idx & 63;
                lg[row * E + e0 + col] =
                    red[(0 * 16 + row) * 64 + col] + red[(1 * 16 + row) * 64 + col];
            }
            __syncthreads();
        }
        // softmax + top-k, wave wv <-> rows wv and wv + 8 of the chunk
        for (int half = 0; half < 2; ++half) {
            const int rl = wv + 8 * half, r = c0 + rl;
            if (r >= M) continue;
            const float* lr = lg + rl * E;
            float lv[4], work[4], g[4];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = lane + 64 * i;
                lv[i] = e < E ? lr[e] : -INFINITY;
                mx = fmaxf(mx, lv[i]);
            }
            mx = wave_max(mx);
            float z = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = lane + 64 * i;
                g[i] = e < E ? expf(lv[i] - mx) : 0.0f;
                z += g[i];
                work[i] = lv[i];
            }
            z = wave_sum(z);
            // lane j keeps the j-th pick
            float mysel = 0.0f, ssum = 0.0f;
            int myidx = 0;
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
                float gsel = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (lane + 64 * i == bi) {
                        work[i] = -INFINITY;
                        gsel = g[i] / z;
                    }
                gsel = __shfl(gsel, bi & 63, MJ_WAVE);
                ssum += gsel;
                if (lane == j) {
                    mysel = gsel;
                    myidx = bi;
                }
            }
            if (lane < k) {
                a.inds[r * k + lane] = myidx;
                a.scores[r * k + lane] = mysel / ssum;
                s_inds[r * k + lane] = myidx;
                atomicOr(&s_mask[myidx], 1ull << r);
            }
        }
        __syncthreads();  // xs / lg reuse, masks complete
    }
    if (a.bk == nullptr) return;
    Buckets* bk = a.bk;
    // experts in increasing id; each bucket lists its pairs in increasing (row, slot) order
    if (wv == 0) {
        int cnt[4], tot = 0, nz = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            cnt[i] = e < E ? __popcll(s_mask[e]) : 0;
            tot += cnt[i];
            nz += cnt[i] > 0;
        }
        int ptot = tot, pnz = nz;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t1 = __shfl_up(ptot, o, MJ_WAVE), t2 = __shfl_up(pnz, o, MJ_WAVE);
            if (lane >= o) {
                ptot += t1;
                pnz += t2;
            }
        }
        int pos = ptot - tot, u = pnz - nz;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            if (e < E) s_start[e] = pos;
            if (cnt[i] > 0) {
                bk->expert[u] = e;
                bk->start[u] = pos;
                ++u;
            }
            pos += cnt[i];
        }
        if (lane == 63) {
            bk->count = pnz;
            bk->start[pnz] = ptot;
        }
    }
    __syncthreads();
    for (int p = tid; p < M * k; p += 512) {
        const int e = s_inds[p], r = p / k;
        const int rank = __popcll(s_mask[e] & ((1ull << r) - 1ull));
        bk->pair[s_start[e] + rank] = p;
    }
}

bool route_supported(int H, int E, int k) {
    return H == RT_H && E % 64 == 0 && E <= MJ_MAX_EXPERTS && k >= 1 && k <= 8;
}

hipError_t launch_route(const RouteArgs& a, int H, hipStream_t st) {
    if (!route_supported(H, a.E, a.k) || a.M < 1 || a.M > MJ_ROWS || a.M * a.k > MJ_MAX_PAIRS)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_route, dim3(1), dim3(512), route_lds_bytes(), st, a);
    return hipGetLastError();
}

hipError_t set_moe_attributes() {
    return hipFuncSetAttribute((const void*)k_route, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)route_lds_bytes());
}
