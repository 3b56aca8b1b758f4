// qmm2.hip -- 2-bit affine products in the MLX layout on gfx950.
//
// Semantics: gqmm2_rows (SeedlessMetal.swift:2168-2221):
//   y[mk, n] = half( sum_k (s[e,n,k/gs] * q[e,n,k] + b[e,n,k/gs]) * x[row(mk), k] ), fp32 sums,
// computed here per 64-input block as s * (sum q*x) + b * (sum x), which is the same sum.
//
// k_qmv2    one activation row: VALU GEMV, v_dot2_f32_f16 on expanded code pairs, each row
//           split over LPR = K/64 lanes (one 64-block each), shuffle reduction.
// k_gather  verify rows: rows grouped by expert, each expert's weights streamed once for all
//           its rows through v_mfma_f32_16x16x32_f16.  B operand = 16 output rows x 32 k of
//           expanded codes; A operand = up to 4 activation rows placed on the A rows of the
//           k quarter they belong to (row 4q+m of A carries x_m only in quarter q), so one
//           MFMA yields separate per-quarter sums D[4q+m][n] and every 64-block keeps its own
//           scale and bias.  Lane (n = l%16, q = l/16) loads the 16 bytes of codes of its row
//           and 64-block, and applies that block's scale/bias to its own D values.
#include "mj_device.h"
#include "mj_internal.h"

// ---------------------------------------------------------------------------------------
// qx prep: plain fp16 rows -> permuted rows + per-64-block {sum x, sum base*x}.
// One wave per 512 elements of a row; lane t owns plain elements 8t..8t+7.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_qx_prep(const uint16_t* __restrict__ x,
                                                 uint16_t* __restrict__ xperm,
                                                 float2* __restrict__ xsum, int rows, int K,
                                                 const int* abort) {
    if (aborted(abort)) return;
    const int lane = threadIdx.x & 63;
    const int chunks = K / 512;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gw >= rows * chunks) return;
    const int row = gw / chunks, c = gw % chunks;
    const size_t base = (size_t)row * K + 512 * c + 8 * lane;
    const u4v v = *(const u4v*)(x + base);
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
    *(u4v*)(xperm + base) = out;
    float X = 0.0f, Bx = 0.0f;
    X = dot2(v.x, 0x3C003C00u, X);
    X = dot2(v.y, 0x3C003C00u, X);
    X = dot2(v.z, 0x3C003C00u, X);
    X = dot2(v.w, 0x3C003C00u, X);
    // plain pairs (x_2j, x_2j+1): bases (256, 64) and (16, 4)
    Bx = dot2(v.x, plain_base2(0), Bx);
    Bx = dot2(v.y, plain_base2(1), Bx);
    Bx = dot2(v.z, plain_base2(2), Bx);
    Bx = dot2(v.w, plain_base2(3), Bx);
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
        X += __shfl_xor(X, m, MJ_WAVE);
        Bx += __shfl_xor(Bx, m, MJ_WAVE);
    }
    if ((lane & 7) == 0) xsum[(size_t)row * (K / 64) + 8 * c + (lane >> 3)] = make_float2(X, Bx);
}

// Block sums {sum x, sum base*x} of rows already in qx order (one thread per 64-block).
__global__ __launch_bounds__(256) void k_qx_sums(const uint16_t* __restrict__ xperm,
                                                 float2* __restrict__ xsum, int rows, int K,
                                                 const int* abort) {
    if (aborted(abort)) return;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * (K / 64)) return;
    const uint16_t* xr = xperm + (size_t)i * 64;
    float X = 0.0f, Bx = 0.0f;
    for (int c = 0; c < 8; ++c) {
        const u4v v = *(const u4v*)(xr + 8 * c);
        for (int j = 0; j < 4; ++j) {
            const float base = code_base(4 * c + j);  // pair (x_i, x_{i+8}), i = (4c+j)%8
            const float lo = h2f((uint16_t)v[j]), hi = h2f((uint16_t)(v[j] >> 16));
            X += lo + hi;
            Bx += base * (lo + hi);
        }
    }
    xsum[i] = make_float2(X, Bx);
}

hipError_t launch_qx_sums(const uint16_t* xperm, float2* xsum, int rows, int K, const int* abort,
                          hipStream_t st) {
    const int n = rows * (K / 64);
    hipLaunchKernelGGL(k_qx_sums, dim3((n + 255) / 256), dim3(256), 0, st, xperm, xsum, rows, K,
                       abort);
    return hipGetLastError();
}

hipError_t launch_qx_prep(const uint16_t* x, uint16_t* xperm, float2* xsum, int rows, int K,
                          const int* abort, hipStream_t st) {
    const int waves = rows * (K / 512);
    hipLaunchKernelGGL(k_qx_prep, dim3((waves + 3) / 4), dim3(256), 0, st, x, xperm, xsum, rows, K,
                       abort);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// VALU GEMV for one activation row per pair (M = 1 decode, MoE at M = 1).
// Wave = (pair p, run of rows_per_wave outputs).  LPR lanes share one weight row, lane li
// owns 64-block li; SUB = 64/LPR rows in flight, U rows per lane per iteration.
// EPI_SWIGLU: up row j and gate row I+j sit on lanes li and li+LPR; output = act (plain).
// ---------------------------------------------------------------------------------------
template <int LPR, int U, int EPI>
__global__ __launch_bounds__(256) void k_qmv2(QmvArgs a) {
    constexpr int SUB = 64 / LPR;
    constexpr int OUT_PER_IT = (EPI == EPI_SWIGLU ? SUB / 2 : SUB) * U;
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int p = gw / a.waves_per_pair;
    if (p >= a.pairs) return;
    const int nout = EPI == EPI_SWIGLU ? a.N / 2 : a.N;
    const int wb = (gw % a.waves_per_pair) * a.rows_per_wave;
    const int wend = min(wb + a.rows_per_wave, nout);
    const int sub = lane / LPR, li = lane % LPR;
    const int kw = a.K >> 4, kg = a.K / a.gs;
    const int gidx = (64 * li) / a.gs;
    // The weight stream is the long latency: the expert id, the abort word and the activation
    // block are fetched together first, the first iteration's codes, scales and biases
    // requested as soon as the id is in, and the activation block formed while they arrive.
    // The abort word is tested before anything is written (an aborted call writes nothing).
    const int e = a.inds[p];
    // (a relaxed atomic load, with no branch around it: a vector load, waited for where it is
    // tested; a scalar load, or one inside a branch, is waited for before the next loads)
    const int ab = __hip_atomic_load(a.abort != nullptr ? a.abort : &a.inds[p], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) &
                   (a.abort != nullptr ? ~0 : 0);
    const uint16_t* xr = a.x + (size_t)(a.lhs_per ? p : 0) * a.K + 64 * li;
    u4v xraw[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) xraw[c] = *(const u4v*)(xr + 8 * c);
    int oi[U];
    bool ok[U];
    u4v cw[U];
    uint16_t sh[U], bh[U];
    auto request = [&](int o0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int row;
            if constexpr (EPI == EPI_SWIGLU) {
                oi[u] = o0 + (sub >> 1) + (SUB / 2) * u;
                row = (sub & 1) ? nout + oi[u] : oi[u];
            } else {
                oi[u] = o0 + sub + SUB * u;
                row = oi[u];
            }
            ok[u] = oi[u] < wend;
            const size_t rr = (size_t)e * a.N + (ok[u] ? row : 0);
            cw[u] = *(const u4v*)(a.w + rr * kw + 4 * li);
            sh[u] = a.s[rr * kg + gidx];
            bh[u] = a.b[rr * kg + gidx];
        }
    };
    if (wb < wend) request(wb);

    // activation block li in qx order, with its sums
    uint32_t xp[32];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const u4v lo = xraw[2 * c], hi = xraw[2 * c + 1];
        const uint32_t u[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        perm16(u, xp + 8 * c);
    }
    float X = 0.0f, Bx = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        X = dot2(xp[i], 0x3C003C00u, X);
        Bx = dot2(xp[i], code_base2(i), Bx);
    }

    if (ab != 0) return;
    for (int o0 = wb; o0 < wend; o0 += OUT_PER_IT) {
        if (o0 != wb) request(o0);
        float part[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int wd = 0; wd < 4; ++wd) {
                uint32_t v[8];
                unpack16(cw[u][wd], v);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[wd] = dot2(v[i], xp[8 * wd + i], acc[wd]);
            }
            const float t = (acc[0] + acc[1]) + (acc[2] + acc[3]);
            part[u] = h2f(sh[u]) * (t - Bx) + h2f(bh[u]) * X;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int m = LPR / 2; m > 0; m >>= 1) part[u] += __shfl_xor(part[u], m, MJ_WAVE);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if constexpr (EPI == EPI_SWIGLU) {
                const float gate_raw = __shfl_xor(part[u], LPR, MJ_WAVE);
                if (li == 0 && (sub & 1) == 0 && ok[u]) {
                    float up = hround(part[u]);
                    float g = hround(gate_raw);
                    g = fminf(g, 7.0f);
                    up = fminf(fmaxf(up, -7.0f), 7.0f);
                    const float act = g / (1.0f + expf(-g)) * up;
                    a.y[(size_t)p * nout + oi[u]] = f2h(act);
                }
            } else {
                if (li == 0 && ok[u]) a.y[(size_t)p * nout + oi[u]] = f2h(part[u]);
            }
        }
    }
}

template <int LPR, int EPI>
static hipError_t launch_qmv2_t(QmvArgs a, hipStream_t st) {
    constexpr int U = 2;
    constexpr int SUB = 64 / LPR;
    constexpr int OPI = (EPI == EPI_SWIGLU ? SUB / 2 : SUB) * U;
    const int nout = EPI == EPI_SWIGLU ? a.N / 2 : a.N;
    // enough waves to cover the chip (~2048), whole iterations per wave
    int rpw = (nout * a.pairs + 2047) / 2048;
    rpw = ((rpw + OPI - 1) / OPI) * OPI;
    if (rpw < OPI) rpw = OPI;
    a.rows_per_wave = rpw;
    a.waves_per_pair = (nout + rpw - 1) / rpw;
    const int waves = a.waves_per_pair * a.pairs;
    hipLaunchKernelGGL((k_qmv2<LPR, U, EPI>), dim3((waves + 3) / 4), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_qmv2(const QmvArgs& a, int epi, hipStream_t st) {
    const int lpr = a.K / 64;
    if (epi == EPI_SWIGLU) {
        if (lpr == 8) return launch_qmv2_t<8, EPI_SWIGLU>(a, st);
        if (lpr == 16) return launch_qmv2_t<16, EPI_SWIGLU>(a, st);
        if (lpr == 32) return launch_qmv2_t<32, EPI_SWIGLU>(a, st);
        return hipErrorInvalidValue;
    }
    if (lpr == 8) return launch_qmv2_t<8, EPI_STORE>(a, st);
    if (lpr == 16) return launch_qmv2_t<16, EPI_STORE>(a, st);
    if (lpr == 32) return launch_qmv2_t<32, EPI_STORE>(a, st);
    if (lpr == 64) return launch_qmv2_t<64, EPI_STORE>(a, st);
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------------
// MFMA gather GEMM over expert buckets.
// ---------------------------------------------------------------------------------------
template <int RG, int EPI, int TPW>
__global__ __launch_bounds__(EPI == EPI_SWIGLU ? 512 : 256) void k_gather(GatherArgs a) {
    if (aborted(a.abort)) return;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nq = lane >> 4, nn = lane & 15;
    const Buckets* bk = a.bk;
    const int nbk = bk ? bk->count : 1;
    const int I = a.N / 2;
    int u, tile0 = 0, kbo = 0;
    const int tiles = a.N / 16;
    if constexpr (EPI == EPI_SWIGLU) {
        const int kbo_n = I / 64;
        u = blockIdx.x / kbo_n;
        kbo = blockIdx.x % kbo_n;
        if (u >= nbk) return;  // whole block
    } else {
        const int groups = (tiles + TPW - 1) / TPW;
        const int gw = blockIdx.x * 4 + wv;
        u = gw / groups;
        if (u >= nbk) return;  // whole wave
        tile0 = (gw % groups) * TPW;
    }
    const int e = bk ? bk->expert[u] : 0;
    const int p0 = bk ? bk->start[u] : 0;
    const int np = bk ? bk->start[u + 1] - p0 : a.dense_rows;
    const int kb_n = a.K >> 6, kw = a.K >> 4, kg = a.K / a.gs;
    const int xm = lane & 3;
    const bool arow = ((lane & 15) >> 2) == nq;

    __shared__ float act_lds[EPI == EPI_SWIGLU ? 64 * 65 : 1];

    constexpr int NT = EPI == EPI_SWIGLU ? 1 : TPW;
    for (int ti = 0; ti < NT; ++ti) {
        int nrow, tile = 0, j0 = 0;
        if constexpr (EPI == EPI_SWIGLU) {
            j0 = kbo * 64 + wv * 8;
            nrow = nn < 8 ? j0 + nn : I + j0 + nn - 8;
        } else {
            tile = tile0 + ti;
            if (tile >= tiles) break;
            nrow = tile * 16 + nn;
        }
        const size_t rr = (size_t)e * a.N + nrow;
        const u4v* wp = (const u4v*)(a.w + rr * kw);
        const uint16_t* sp = a.s + rr * kg;
        const uint16_t* bp = a.b + rr * kg;

        for (int pb = 0; pb < np; pb += RG * 4) {
            float acc[RG][4];
            int xrow[RG];
            bool xok[RG];
            int srow[RG][4];
            bool sok[RG][4];
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
                const int i = pb + rg * 4 + xm;
                xok[rg] = arow && i < np;
                xrow[rg] = xok[rg] ? (bk ? bk->pair[p0 + i] : i) / a.x_div : 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int ir = pb + rg * 4 + r;
                    sok[rg][r] = ir < np;
                    srow[rg][r] = sok[rg][r] ? (bk ? bk->pair[p0 + ir] : ir) / a.x_div : 0;
                    acc[rg][r] = 0.0f;
                }
            }
            for (int t = 0; t < (a.K >> 8); ++t) {
                const int kb = 4 * t + nq;
                const u4v cw = wp[kb];
                const float sc = h2f(sp[(kb * 64) / a.gs]);
                const float bi = h2f(bp[(kb * 64) / a.gs]);
                uint32_t v[4][8];
#pragma unroll
                for (int wd = 0; wd < 4; ++wd) unpack16(cw[wd], v[wd]);
#pragma unroll
                for (int rg = 0; rg < RG; ++rg) {
                    if (pb + rg * 4 >= np) break;
                    f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
                    const u4v* xq = (const u4v*)(a.xperm + (size_t)xrow[rg] * a.K + 64 * kb);
#pragma unroll
                    for (int s = 0; s < 8; ++s) {
                        u4v av = {0u, 0u, 0u, 0u};
                        if (xok[rg]) av = xq[s];
                        u4v bv;
                        bv.x = v[s >> 1][4 * (s & 1) + 0];
                        bv.y = v[s >> 1][4 * (s & 1) + 1];
                        bv.z = v[s >> 1][4 * (s & 1) + 2];
                        bv.w = v[s >> 1][4 * (s & 1) + 3];
                        d = mfma16x16x32(as_h8(av), as_h8(bv), d);
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (sok[rg][r]) {
                            const float2 xs = a.xsum[(size_t)srow[rg][r] * kb_n + kb];
                            acc[rg][r] += sc * (d[r] - xs.y) + bi * xs.x;
                        }
                    }
                }
            }
#pragma unroll
            for (int rg = 0; rg < RG; ++rg)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    acc[rg][r] += __shfl_xor(acc[rg][r], 16, MJ_WAVE);
                    acc[rg][r] += __shfl_xor(acc[rg][r], 32, MJ_WAVE);
                }
            if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
                for (int rg = 0; rg < RG; ++rg)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float gate_raw = __shfl_xor(acc[rg][r], 8, MJ_WAVE);
                        const int i = pb + rg * 4 + r;
                        if (nq == 0 && nn < 8 && i < np) {
                            float up = hround(acc[rg][r]);
                            float g = hround(gate_raw);
                            g = fminf(g, 7.0f);
                            up = fminf(fmaxf(up, -7.0f), 7.0f);
                            const float act = hround(g / (1.0f + expf(-g)) * up);
                            const int pr = bk ? bk->pair[p0 + i] : i;
                            const int j = j0 + nn;
                            a.y[(size_t)pr * I + (j & ~15) + perm_pos(j & 15)] = f2h(act);
                            act_lds[i * 65 + wv * 8 + nn] = act;
                        }
                    }
            } else {
                if (nq == 0) {
#pragma unroll
                    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int i = pb + rg * 4 + r;
                            if (i < np) {
                                const int pr = bk ? bk->pair[p0 + i] : i;
                                uint16_t* yp = a.y + (size_t)pr * a.N + nrow;
                                if constexpr (EPI == EPI_ADD)
                                    *yp = f2h(h2f(*yp) + hround(acc[rg][r]));
                                else
                                    *yp = f2h(acc[rg][r]);
                            }
                        }
                }
            }
        }
    }
    if constexpr (EPI == EPI_SWIGLU) {
        __syncthreads();
        // per-row sums of this 64-block of act, fixed sequential order
        if ((int)threadIdx.x < np && np <= 64) {
            const int i = threadIdx.x;
            float X = 0.0f, Bx = 0.0f;
            for (int c = 0; c < 64; ++c) {
                const float v = act_lds[i * 65 + c];
                X += v;
                Bx += code_base(c % 8) * v;  // plain element c: the base of its qx pair
            }
            const int pr = bk ? bk->pair[p0 + i] : i;
            a.ysum[(size_t)pr * (I / 64) + kbo] = make_float2(X, Bx);
        }
    }
}

template <int RG, int EPI>
static hipError_t launch_gather_t(const GatherArgs& a, int n_buckets_max, hipStream_t st) {
    constexpr int TPW = 2;
    if constexpr (EPI == EPI_SWIGLU) {
        const int blocks = n_buckets_max * (a.N / 2 / 64);
        launch_timed(k_gather<RG, EPI, TPW>, dim3(blocks), dim3(512), 0, st, a);
    } else {
        const int groups = (a.N / 16 + TPW - 1) / TPW;
        const int waves = n_buckets_max * groups;
        launch_timed(k_gather<RG, EPI, TPW>, dim3((waves + 3) / 4), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

hipError_t launch_gather(const GatherArgs& a, int epi, int max_rows_per_bucket, int n_buckets_max,
                         hipStream_t st) {
    if (gather3_supported(epi, a.K, a.N, a.gs))
        return launch_gather3(a, epi, max_rows_per_bucket, n_buckets_max, st);
    if (a.ecnt != nullptr || a.srec != nullptr)  // expert modes are the tile kernel's
        return hipErrorInvalidValue;
    // generic fallback (any K % 256 == 0, N % 16 == 0): K inside each wave, RG row groups
    const int rows = max_rows_per_bucket;
    const int rg = rows <= 4 ? 1 : (rows <= 8 ? 2 : 4);
#define MJ_G(R, E)                                      \
    if (rg == R && epi == E) return launch_gather_t<R, E>(a, n_buckets_max, st);
    MJ_G(1, EPI_STORE) MJ_G(2, EPI_STORE) MJ_G(4, EPI_STORE)
    MJ_G(1, EPI_ADD) MJ_G(2, EPI_ADD) MJ_G(4, EPI_ADD)
    MJ_G(1, EPI_SWIGLU) MJ_G(2, EPI_SWIGLU) MJ_G(4, EPI_SWIGLU)
#undef MJ_G
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------------
// MFMA operand-layout self-check: D = A[16x32] * B[32x16] with the lane mapping the
// kernels assume (A: row l%16, k 8(l/16)+j; B: col l%16, k 8(l/16)+j; D: row 4(l/16)+r).
// ---------------------------------------------------------------------------------------
__global__ void k_selftest_mfma(const uint16_t* A, const uint16_t* B, float* D) {
    const int l = threadIdx.x & 63;
    u4v av, bv;
    uint32_t bw[4];
    av = *(const u4v*)(A + (l & 15) * 32 + 8 * (l >> 4));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t lo = B[(8 * (l >> 4) + 2 * j) * 16 + (l & 15)];
        const uint32_t hi = B[(8 * (l >> 4) + 2 * j + 1) * 16 + (l & 15)];
        bw[j] = lo | (hi << 16);
    }
    bv.x = bw[0];
    bv.y = bw[1];
    bv.z = bw[2];
    bv.w = bw[3];
    f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
    d = mfma16x16x32(as_h8(av), as_h8(bv), d);
#pragma unroll
    for (int r = 0; r < 4; ++r) D[(4 * (l >> 4) + r) * 16 + (l & 15)] = d[r];
}

hipError_t launch_selftest_mfma(const uint16_t* A, const uint16_t* B, float* D, hipStream_t st) {
    hipLaunchKernelGGL(k_selftest_mfma, dim3(1), dim3(64), 0, st, A, B, D);
    return hipGetLastError();
}
