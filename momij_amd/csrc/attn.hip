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
    if (aborted(a.abort)) return;
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
    int* ktree = (int*)(kpos + AK);
    int* kslot = ktree + AK;

    // keys of this chunk
    if (t < AK) {
        const int64_t i = (int64_t)c * AK + t;
        int64_t pos = INT64_MIN / 2, slot = 0;
        int tree = -2;  // -2 invalid, -1 committed, >=0 tree row
        if (i < nk) {
            if (i < ncm) {
                pos = lo_min + i;
                slot = pos % a.C;
                tree = -1;
            } else {
                const int ar = (int)(i - ncm);
                slot = (L + ar) % a.C;
                pos = L + sd->depth[ar];
                tree = ar;
            }
        }
        kpos[t] = pos;
        ktree[t] = tree;
        kslot[t] = (int)slot;
    }
    // Q rows of this kv group: qv = r * gqa + j  <-  head g*gqa + j of row r
    for (int idx = t; idx < nqt * 16 * 16; idx += 256) {
        const int qv = idx >> 4, part = idx & 15;
        u4v v = {0u, 0u, 0u, 0u};
        if (qv < nqv) {
            const int r = qv / gqa, j = qv % gqa;
            v = *(const u4v*)(a.qbuf + ((size_t)r * a.nQ + g * gqa + j) * HD + 8 * part);
        }
        *(u4v*)(Qs + qv * QSTR + 8 * part) = v;
    }
    __syncthreads();
    // K rows and V transposed
    {
        const int kk = t >> 2, dq = t & 3;
        const bool valid = ktree[kk] != -2;
        const size_t base = ((size_t)g * a.C + (valid ? kslot[kk] : 0)) * HD + 32 * dq;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            u4v kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
            if (valid) {
                kv = *(const u4v*)(a.kc + base + 8 * q);
                vv = *(const u4v*)(a.vc + base + 8 * q);
            }
            *(u4v*)(Ks + kk * QSTR + 32 * dq + 8 * q) = kv;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = 32 * dq + 8 * q + 2 * j;
                Vt[d * VSTR + kk] = (uint16_t)(vv[j] & 0xFFFFu);
                Vt[(d + 1) * VSTR + kk] = (uint16_t)(vv[j] >> 16);
            }
        }
    }
    __syncthreads();

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
                const int64_t lo_r = a.window > 0 ? L + sd->depth[row] - a.window + 1 : INT64_MIN;
                const uint64_t anc = sd->anc[row];
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

// One wave per (row, group of 4 query heads): lane = head (lane/16) x 8 dims (lane%16).
__global__ __launch_bounds__(256) void k_attn_combine(AttnArgs a) {
    if (aborted(a.abort)) return;
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int hgroups = a.nQ / 4;
    const int r = gw / hgroups, hg = gw % hgroups;
    if (r >= a.M) return;
    const int gqa = a.nQ / a.nKV;
    const int hq = hg * 4 + (lane >> 4), d0 = 8 * (lane & 15);
    const int g = hq / gqa, qv = r * gqa + (hq % gqa);
    const int nqt = (a.M * gqa + 15) / 16;
    const int64_t L = a.sd->L;
    const int64_t lo_min = a.window > 0 ? (L - a.window + 1 > 0 ? L - a.window + 1 : 0) : 0;
    const int64_t nk = (L - lo_min) + a.M;
    const int nch = (int)((nk + AK - 1) / AK);
    float mx = -INFINITY;
    for (int c = 0; c < nch; ++c) {
        const float2 ml = a.mlpart[((size_t)g * a.max_chunks + c) * (nqt * 16) + qv];
        mx = fmaxf(mx, ml.x);
    }
    float lsum = 0.0f, o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int c = 0; c < nch; ++c) {
        const size_t idx = ((size_t)g * a.max_chunks + c) * (nqt * 16) + qv;
        const float2 ml = a.mlpart[idx];
        if (ml.x == -INFINITY) continue;
        const float w = expf(ml.x - mx);
        lsum += ml.y * w;
        const float4* op = (const float4*)(a.opart + idx * HD + d0);
        const float4 p0 = op[0], p1 = op[1];
        o[0] += w * p0.x;
        o[1] += w * p0.y;
        o[2] += w * p0.z;
        o[3] += w * p0.w;
        o[4] += w * p1.x;
        o[5] += w * p1.y;
        o[6] += w * p1.z;
        o[7] += w * p1.w;
    }
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    u4v ov;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        ov[j] = (uint32_t)f2h(o[2 * j] * inv) | ((uint32_t)f2h(o[2 * j + 1] * inv) << 16);
    // qx emit: lanes in aligned groups of 8 hold one 64-block
    u4v ox;
    ox.x = __shfl_xor(ov.x, 1, MJ_WAVE);
    ox.y = __shfl_xor(ov.y, 1, MJ_WAVE);
    ox.z = __shfl_xor(ov.z, 1, MJ_WAVE);
    ox.w = __shfl_xor(ov.w, 1, MJ_WAVE);
    const bool odd = lane & 1;
    const uint32_t u[8] = {odd ? ox.x : ov.x, odd ? ox.y : ov.y, odd ? ox.z : ov.z, odd ? ox.w : ov.w,
                           odd ? ov.x : ox.x, odd ? ov.y : ox.y, odd ? ov.z : ox.z, odd ? ov.w : ox.w};
    uint32_t p[8];
    perm16(u, p);
    u4v pv;
    pv.x = odd ? p[4] : p[0];
    pv.y = odd ? p[5] : p[1];
    pv.z = odd ? p[6] : p[2];
    pv.w = odd ? p[7] : p[3];
    const int K = a.nQ * HD;
    const int k0 = hq * HD + d0;
    *(u4v*)(a.out_perm + (size_t)r * K + k0) = pv;
    float X = 0.0f, Bx = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        X = dot2(ov[j], 0x3C003C00u, X);
        Bx = dot2(ov[j], 0x44004C00u, Bx);
    }
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
        X += __shfl_xor(X, m, MJ_WAVE);
        Bx += __shfl_xor(Bx, m, MJ_WAVE);
    }
    if ((lane & 7) == 0) a.out_sum[(size_t)r * (K / 64) + (k0 >> 6)] = make_float2(X, Bx);
}

hipError_t launch_attn(const AttnArgs& a, hipStream_t st) {
    const int gqa = a.nQ / a.nKV;
    const int nqt = (a.M * gqa + 15) / 16;
    const size_t lds = (size_t)(nqt * 16 * QSTR + AK * QSTR + HD * VSTR + 4 * 16 * VSTR) * 2 +
                       AK * (8 + 4 + 4);
    hipLaunchKernelGGL(k_attn_chunk, dim3(a.nKV * a.max_chunks), dim3(256), lds, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int waves = a.M * (a.nQ / 4);
    hipLaunchKernelGGL(k_attn_combine, dim3((waves + 3) / 4), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t set_attn_attributes() {
    return hipFuncSetAttribute((const void*)k_attn_chunk,
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
}
