// attn.hip -- sliding-window attention over the fp16 KV cache for a pass of M verify rows
// arranged as a chain or a draft tree.
//
// k_qknorm_rope_kv  maple_qk_norm_rope + maple_write_kv_pair (SeedlessMetal.swift:2794-2901):
//                   per head RMSNorm(eps) * w, non-traditional half-split RoPE on the first
//                   rope_dim dims at the row's position L + depth(r); K and V rows appended at
//                   slot (L + r) % C.  One wave per (row, head), two dims per lane.
// k_attn_chunk      maple_sdpa_d128 math (2919-2997): softmax(q k^T / sqrt(128)) v in fp32, GQA.
//                   Split-K over 64-key chunks ("flash decoding"); one 256-thread block per
//                   (kv head, chunk) stages Q (all rows x heads of the group), K and V^T in LDS
//                   and runs QK^T and PV on v_mfma_f32_16x16x32_f16.  Mask: committed
//                   positions inside the row's window [P-W+1, L-1] (AttentionMasks.swift:10-27)
//                   plus the row's ancestors and itself; a chain is the causal M-row pass.
// k_attn_combine    merges the chunk partials per (row, head) and writes the output in the qx
//                   format consumed by the o-projection.
#include "mj_device.h"
#include "mj_internal.h"

#define HD 128
#define AK 64     // keys per chunk
#define QSTR 136  // LDS row stride (halves) of Q and K tiles
#define VSTR 72   // LDS row stride (halves) of V^T and P tiles

int attn_max_chunks(int window, int64_t L_max, int M) {
    const int64_t keys = (window > 0 ? (int64_t)window - 1 : L_max) + M;
    return (int)((keys + AK - 1) / AK);
}

__global__ __launch_bounds__(256) void k_qknorm_rope_kv(AttnArgs a) {
    if (aborted(a.abort)) return;
    const int lane = threadIdx.x & 63;
    const int nh = a.nQ + a.nKV;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int r = gw / nh, hh = gw % nh;
    if (r >= a.M) return;
    const int qkvN = (a.nQ + 2 * a.nKV) * HD;
    const uint32_t xv = *(const uint32_t*)(a.qkv + (size_t)r * qkvN + hh * HD + 2 * lane);
    const float x0 = h2f(xv & 0xFFFFu), x1 = h2f(xv >> 16);
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float sc = 1.0f / sqrtf(ss / (float)HD + a.eps);
    const uint16_t* wn = hh < a.nQ ? a.q_norm_w : a.k_norm_w;
    const uint32_t wv = *(const uint32_t*)(wn + 2 * lane);
    float v0 = x0 * sc * h2f(wv & 0xFFFFu);
    float v1 = x1 * sc * h2f(wv >> 16);
    const int rd = a.rope_dim;
    if (rd > 0) {
        const int half = rd / 2;
        const float u0 = __shfl_xor(v0, half / 2, MJ_WAVE);
        const float u1 = __shfl_xor(v1, half / 2, MJ_WAVE);
        const float pos = (float)(a.sd->L + a.sd->depth[r]);
        const int j0 = 2 * lane;
        if (j0 < rd) {
            const int p0 = j0 < half ? j0 : j0 - half;
            const float t0 = pos * a.inv_freq[p0], t1 = pos * a.inv_freq[p0 + 1];
            const float c0 = cosf(t0), s0 = sinf(t0), c1 = cosf(t1), s1 = sinf(t1);
            if (j0 < half) {
                v0 = v0 * c0 - u0 * s0;
                v1 = v1 * c1 - u1 * s1;
            } else {
                v0 = v0 * c0 + u0 * s0;
                v1 = v1 * c1 + u1 * s1;
            }
        }
    }
    const uint32_t o = (uint32_t)f2h(v0) | ((uint32_t)f2h(v1) << 16);
    if (hh < a.nQ) {
        *(uint32_t*)(a.qbuf + ((size_t)r * a.nQ + hh) * HD + 2 * lane) = o;
    } else {
        const int g = hh - a.nQ;
        const int64_t slot = (a.sd->L + r) % a.C;
        const size_t dst = ((size_t)g * a.C + slot) * HD + 2 * lane;
        *(uint32_t*)(a.kc + dst) = o;
        *(uint32_t*)(a.vc + dst) =
            *(const uint32_t*)(a.qkv + (size_t)r * qkvN + (a.nQ + a.nKV) * HD + g * HD + 2 * lane);
    }
}

hipError_t launch_qknorm_rope_kv(const AttnArgs& a, hipStream_t st) {
    const int waves = a.M * (a.nQ + a.nKV);
    hipLaunchKernelGGL(k_qknorm_rope_kv, dim3((waves + 3) / 4), dim3(256), 0, st, a);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_attn_chunk(AttnArgs a) {
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int g = blockIdx.x / a.max_chunks, c = blockIdx.x % a.max_chunks;
    const StepDesc* sd = a.sd;
    const int64_t L = sd->L;
    const int gqa = a.nQ / a.nKV;
    const int nqv = a.M * gqa, nqt = (nqv + 15) / 16;
    const int64_t lo_min = a.window > 0 ? (L - a.window + 1 > 0 ? L - a.window + 1 : 0) : 0;
    const int64_t ncm = L - lo_min;
    const int64_t nk = ncm + a.M;
    if ((int64_t)c * AK >= nk) return;  // whole block

    extern __shared__ uint16_t lds[];
    uint16_t* Qs = lds;                          // [nqt*16][QSTR]
    uint16_t* Ks = Qs + nqt * 16 * QSTR;         // [AK][QSTR]
    uint16_t* Vt = Ks + AK * QSTR;               // [HD][VSTR]
    uint16_t* Ps = Vt + HD * VSTR;               // [4 waves][16][VSTR]
    int64_t* kpos = (int64_t*)(Ps + 4 * 16 * VSTR);
    int64_t* rlo = kpos + AK;                    // [MJ_ROWS] first key position of a row's window
    uint64_t* ranc = (uint64_t*)(rlo + MJ_ROWS);  // [MJ_ROWS] ancestor masks
    int* ktree = (int*)(ranc + MJ_ROWS);
    int* s_abort = ktree + AK;

    // Every load of the block is issued before the first wait: this thread's K/V quarter row
    // (key kk = t / 4, dims 32 (t % 4) ..), its share of the Q rows, and the key metadata.
    const int kk = t >> 2, dq = t & 3;
    const int64_t ki = (int64_t)c * AK + kk;
    const bool kvalid = ki < nk;
    int64_t kslot_v = 0;
    if (kvalid) kslot_v = (ki < ncm ? lo_min + ki : L + (ki - ncm)) % a.C;
    u4v kv[4], vv[4];
    {
        const size_t base = ((size_t)g * a.C + kslot_v) * HD + 32 * dq;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            kv[q] = (u4v){0u, 0u, 0u, 0u};
            vv[q] = (u4v){0u, 0u, 0u, 0u};
            if (kvalid) {
                kv[q] = *(const u4v*)(a.kc + base + 8 * q);
                vv[q] = *(const u4v*)(a.vc + base + 8 * q);
            }
        }
    }
    if (t < AK) {
        const int64_t i = (int64_t)c * AK + t;
        int64_t pos = INT64_MIN / 2;
        int tree = -2;  // -2 invalid, -1 committed, >=0 tree row
        if (i < nk) {
            if (i < ncm) {
                pos = lo_min + i;
                tree = -1;
            } else {
                const int ar = (int)(i - ncm);
                pos = L + sd->depth[ar];
                tree = ar;
            }
        }
        kpos[t] = pos;
        ktree[t] = tree;
    }
    // the rows' window starts and ancestor masks, fetched with everything else
    if (t < a.M) {
        rlo[t] = a.window > 0 ? L + sd->depth[t] - a.window + 1 : INT64_MIN;
        ranc[t] = sd->anc[t];
    }
    // Q rows of this kv group: qv = r * gqa + j  <-  head g*gqa + j of row r; four 16-byte
    // parts per thread per round
    for (int base = 0; base < nqt * 256; base += 1024) {
        u4v qv4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int idx = base + t + 256 * j;
            const int qv = idx >> 4, part = idx & 15;
            qv4[j] = (u4v){0u, 0u, 0u, 0u};
            if (idx < nqt * 256 && qv < nqv) {
                const int r = qv / gqa, jj = qv % gqa;
                qv4[j] = *(const u4v*)(a.qbuf + ((size_t)r * a.nQ + g * gqa + jj) * HD + 8 * part);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int idx = base + t + 256 * j;
            if (idx < nqt * 256) *(u4v*)(Qs + (idx >> 4) * QSTR + 8 * (idx & 15)) = qv4[j];
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        *(u4v*)(Ks + kk * QSTR + 32 * dq + 8 * q) = kv[q];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = 32 * dq + 8 * q + 2 * j;
            Vt[d * VSTR + kk] = (uint16_t)(vv[q][j] & 0xFFFFu);
            Vt[(d + 1) * VSTR + kk] = (uint16_t)(vv[q][j] >> 16);
        }
    }
    if (t == 0) *s_abort = a.abort ? *a.abort : 0;
    __syncthreads();
    if (*s_abort) return;  // block-uniform

    const int ln = lane & 15, lq = lane >> 4;
    uint16_t* Pw = Ps + wv * 16 * VSTR;
    const int iters = (nqt + 3) / 4;
    for (int it = 0; it < iters; ++it) {
        const int qt = wv + 4 * it;
        const bool active = qt < nqt;
        float m[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        float l[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        f4 S[4];
        if (active) {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                S[kt] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const u4v av = *(const u4v*)(Qs + (qt * 16 + ln) * QSTR + 32 * s + 8 * lq);
                    const u4v bv = *(const u4v*)(Ks + (16 * kt + ln) * QSTR + 32 * s + 8 * lq);
                    S[kt] = mfma16x16x32(as_h8(av), as_h8(bv), S[kt]);
                }
            }
            // mask + scale; lane holds rows qv = qt*16 + 4*lq + r, key 16*kt + ln
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qv = qt * 16 + 4 * lq + r;
                const int row = qv < nqv ? qv / gqa : 0;
                const int64_t lo_r = rlo[row];
                const uint64_t anc = ranc[row];
#pragma unroll
                for (int kt = 0; kt < 4; ++kt) {
                    const int kk = 16 * kt + ln;
                    const int tr = ktree[kk];
                    bool ok = qv < nqv && tr != -2 && kpos[kk] >= lo_r;
                    if (tr >= 0) ok = ok && ((anc >> tr) & 1ull);
                    const float s = ok ? S[kt][r] * a.scale : -INFINITY;
                    S[kt][r] = s;
                    m[r] = fmaxf(m[r], s);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) m[r] = fmaxf(m[r], __shfl_xor(m[r], o, MJ_WAVE));
        }
        if (active) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
#pragma unroll
                for (int kt = 0; kt < 4; ++kt) {
                    const float p = m[r] == -INFINITY ? 0.0f : expf(S[kt][r] - m[r]);
                    l[r] += p;
                    Pw[(4 * lq + r) * VSTR + 16 * kt + ln] = f2h(p);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) l[r] += __shfl_xor(l[r], o, MJ_WAVE);
        }
        __syncthreads();  // P tile visible to the whole wave
        if (active) {
            f4 O[8];
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) O[dt] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const u4v av = *(const u4v*)(Pw + ln * VSTR + 32 * ks + 8 * lq);
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) {
                    const u4v bv = *(const u4v*)(Vt + (16 * dt + ln) * VSTR + 32 * ks + 8 * lq);
                    O[dt] = mfma16x16x32(as_h8(av), as_h8(bv), O[dt]);
                }
            }
            const size_t pbase = ((size_t)g * a.max_chunks + c) * (size_t)(nqt * 16);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qv = qt * 16 + 4 * lq + r;
                float* op = a.opart + (pbase + qv) * HD;
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) op[16 * dt + ln] = O[dt][r];
                if (ln == 0) a.mlpart[pbase + qv] = make_float2(m[r], l[r]);
            }
        }
        __syncthreads();  // before the next tile overwrites P
    }
}

// One 256-thread block per (row, query head): wave w merges chunks w, w + 4, ... (lane = two
// dims), then the four wave sums are added in wave order and the row is written in qx order.
// Every chunk below the row's count holds a partial (a fully masked one has max -inf, sum 0).
__global__ __launch_bounds__(256) void k_attn_combine(AttnArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = blockIdx.x / a.nQ, hq = blockIdx.x % a.nQ;
    const int gqa = a.nQ / a.nKV;
    const int g = hq / gqa, qv = r * gqa + (hq % gqa);
    const size_t nq16 = (size_t)((a.M * gqa + 15) / 16) * 16;
    const int64_t L = a.sd->L;
    const int64_t lo_min = a.window > 0 ? (L - a.window + 1 > 0 ? L - a.window + 1 : 0) : 0;
    const int64_t nk = (L - lo_min) + a.M;
    const int nch = (int)((nk + AK - 1) / AK);
    const float2* ml = a.mlpart + (size_t)g * a.max_chunks * nq16 + qv;
    const float* op = a.opart + ((size_t)g * a.max_chunks * nq16 + qv) * HD + 2 * lane;
    float mx = -INFINITY;
    for (int c = lane; c < nch; c += 64) mx = fmaxf(mx, ml[(size_t)c * nq16].x);
    mx = wave_max(mx);
    float o0 = 0.0f, o1 = 0.0f, ls = 0.0f;
    for (int c0 = wv; c0 < nch; c0 += 16) {
        float2 m4[4], p4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = c0 + 4 * j;
            m4[j] = make_float2(-INFINITY, 0.0f);
            p4[j] = make_float2(0.0f, 0.0f);
            if (c < nch) {
                m4[j] = ml[(size_t)c * nq16];
                p4[j] = *(const float2*)(op + (size_t)c * nq16 * HD);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float w = m4[j].x == -INFINITY ? 0.0f : expf(m4[j].x - mx);
            ls += m4[j].y * w;
            o0 += w * p4[j].x;
            o1 += w * p4[j].y;
        }
    }
    __shared__ float s_o[4][HD];
    __shared__ float s_l[4];
    __shared__ int s_abort;
    s_o[wv][2 * lane] = o0;
    s_o[wv][2 * lane + 1] = o1;
    if (lane == 0) s_l[wv] = ls;
    if (tid == 0) s_abort = a.abort ? *a.abort : 0;
    __syncthreads();
    if (s_abort) return;
    if (tid < 16) {
        const float lsum = ((s_l[0] + s_l[1]) + s_l[2]) + s_l[3];
        const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
        u4v ov;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = 8 * tid + 2 * j;
            const float v0 = (((s_o[0][d] + s_o[1][d]) + s_o[2][d]) + s_o[3][d]) * inv;
            const float v1 =
                (((s_o[0][d + 1] + s_o[1][d + 1]) + s_o[2][d + 1]) + s_o[3][d + 1]) * inv;
            ov[j] = (uint32_t)f2h(v0) | ((uint32_t)f2h(v1) << 16);
        }
        const int K = a.nQ * HD;
        emit_qx(ov, tid, a.out_perm + (size_t)r * K, a.out_sum + (size_t)r * (K / 64),
                hq * HD + 8 * tid);
    }
}

hipError_t launch_attn(const AttnArgs& a, hipStream_t st) {
    if (a.M < 1 || a.M > MJ_ROWS) return hipErrorInvalidValue;  // row metadata is staged per row
    const int gqa = a.nQ / a.nKV;
    const int nqt = (a.M * gqa + 15) / 16;
    const size_t lds = (size_t)(nqt * 16 * QSTR + AK * QSTR + HD * VSTR + 4 * 16 * VSTR) * 2 +
                       AK * (8 + 4) + MJ_ROWS * 16 + 16;
    launch_timed(k_attn_chunk, dim3(a.nKV * a.max_chunks), dim3(256), lds, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_combine, dim3(a.M * a.nQ), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t set_attn_attributes() {
    return hipFuncSetAttribute((const void*)k_attn_chunk,
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
}
