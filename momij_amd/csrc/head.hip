// head.hip -- exact fp16 lm_head verify, greedy acceptance, KV commit and token embedding.
//
// k_lm_head      maple_lm_head_argmax semantics (SeedlessMetal.swift:3005-3090) for an fp16
//                head: logits[m][v] = sum_k w[v][k] x[m][k] (fp32), banned ids skipped, lowest
//                id wins ties.  One 512-thread block per CU streams 16-row vocab strips through
//                v_mfma_f32_16x16x32_f16 (A = 16 vocab rows x 32 k straight from HBM, B = the
//                M <= 32 hidden rows staged once in LDS); per-lane running argmax, optional
//                fp32 logits, one partial per (block, row).
// k_head_final   maple_lm_head_reduce (3093-3111): folds the block partials per row.
// k_accept_greedy verifyDraftChain's longest-prefix rule (SeedlessDecodeEngine.swift:1574-1603)
//                walked over a draft tree: lowest-index child whose token equals the argmax.
// k_kv_commit    keeps the accepted rows: the KV written at slot L + path[i] moves to L + i
//                (SeedlessAttn.swift:219-270 rewinds the offset for append-only writes; a tree
//                also needs the accepted path compacted into consecutive positions).
#include "mj_device.h"
#include "mj_internal.h"

struct HeadArgs {
    const uint16_t* x;   // [M][K] fp16
    const uint16_t* w;   // [V][K] fp16
    int M, K, V;
    const int32_t* banned;
    int n_banned;
    float* logits;       // [M][V] or nullptr
    float* pval;         // [blocks][32]
    int* pidx;           // [blocks][32]
    const int* abort;
    HeadLse lse;
};

template <int NT, int PL>
__global__ __launch_bounds__(512) void k_lm_head(HeadArgs a) {
    if (aborted(a.abort)) return;
    extern __shared__ uint16_t xs[];  // [NT*16][K + 8]
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int K = a.K, XS = K + 8;
    for (int idx = t; idx < NT * 16 * (K / 8); idx += 512) {
        const int m = idx / (K / 8), part = idx % (K / 8);
        u4v v = {0u, 0u, 0u, 0u};
        if (m < a.M) v = *(const u4v*)(a.x + (size_t)m * K + 8 * part);
        *(u4v*)(xs + m * XS + 8 * part) = v;
    }
    __shared__ int s_ban[MJ_HEAD_MAX_BANNED];  // banned ids (read with LDS, not vector, loads)
    for (int idx = t; idx < a.n_banned; idx += 512) s_ban[idx] = a.banned[idx];
    __syncthreads();
    const int ln = lane & 15, lq = lane >> 4;
    const int nstrips = (a.V + 15) / 16;
    float bv[NT];
    int bi[NT];
    float lm[NT], ls[NT];  // running log-sum-exp of logits / T (log2 units) per lane and tile
#pragma unroll
    for (int tl = 0; tl < NT; ++tl) {
        bv[tl] = -INFINITY;
        bi[tl] = 0x7fffffff;
        lm[tl] = -INFINITY;
        ls[tl] = 0.0f;
    }
    // Work unit: one K half of a 16-row strip.  Wave (slot, h) of a block takes half h of
    // strips blockIdx.x * 4 + slot + round * gridDim.x * 4; the h = 1 partial meets the h = 0
    // one in LDS (two slot sets by round parity), so twice as many units as strips keep the
    // waves' loads even.  A wave's halves are one stream of pieces of PL 32-k chunks (16 rows x
    // 256 k, 8 KB, when K / 2 allows) through two register sets taken in turn: a set is
    // refilled with the piece two ahead as soon as it has been multiplied, so one piece is
    // always in flight behind the one in use and no set is copied.  Every load is issued --
    // past the stream's end at the clamped last row, a cached line -- which keeps the wait
    // before a set's use from covering the other set's requests.
    const int slot = wv & 3, h = wv >> 2;
    const int NH = K / 64 / PL;                // pieces per half strip
    const int SW = gridDim.x * 4;
    const int rounds = (nstrips - (int)blockIdx.x * 4 + SW - 1) / SW;  // of this block's slot 0
    const int strip0 = blockIdx.x * 4 + slot, TP = rounds * NH;
    struct Piece {
        u4v c[PL];
    };
    int ld_strip = strip0, ld_pc = 0;
    auto issue = [&](Piece& pz) {
        const int vr = min(ld_strip * 16 + ln, a.V - 1);
        const u4v* wr = (const u4v*)(a.w + (size_t)vr * K) + lq + 4 * PL * (h * NH + ld_pc);
#pragma unroll
        for (int u = 0; u < PL; ++u) pz.c[u] = wr[4 * u];
        if (++ld_pc == NH) {
            ld_pc = 0;
            ld_strip += SW;
        }
    };
    // h = 1 partials: two sets by round parity for one tile; one set for two tiles (their rows
    // take most of the LDS), reused after a barrier
    constexpr int NPB = NT == 1 ? 2 : 1;
    __shared__ f4 s_part[NPB][4][NT][64];
    f4 acc[NT];
#pragma unroll
    for (int tl = 0; tl < NT; ++tl) acc[tl] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
    int c_strip = strip0, c_pc = 0, c_rd = 0;
    auto step = [&](Piece& cur, int i) {
        const int s0 = PL * (h * NH + c_pc);
#pragma unroll
        for (int u = 0; u < PL; ++u) {
#pragma unroll
            for (int tl = 0; tl < NT; ++tl) {
                const u4v xb = *(const u4v*)(xs + (tl * 16 + ln) * XS + 32 * (s0 + u) + 8 * lq);
                acc[tl] = mfma16x16x32(as_h8(cur.c[u]), as_h8(xb), acc[tl]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        issue(cur);  // the piece two ahead
        __builtin_amdgcn_sched_barrier(0);
        if (++c_pc < NH) return;
        c_pc = 0;
        if (i < TP) {  // end of a round: the same for every wave of the block
            const bool live = c_strip < nstrips;
            const int v0 = c_strip * 16;
            if (h == 1) {
#pragma unroll
                for (int tl = 0; tl < NT; ++tl) s_part[c_rd % NPB][slot][tl][lane] = acc[tl];
            }
            __syncthreads();  // the h = 1 halves are in LDS
            if (live && h == 0) {
#pragma unroll
                for (int tl = 0; tl < NT; ++tl) {
                    const f4 o = s_part[c_rd % NPB][slot][tl][lane];
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[tl][r] += o[r];
                }
                // lane holds logits for vocab v0 + 4*lq + r, row tl*16 + ln
                bool keep[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int v = v0 + 4 * lq + r;
                    keep[r] = v < a.V;
                    for (int b = 0; b < a.n_banned; ++b)
                        if (s_ban[b] == v) keep[r] = false;
                }
#pragma unroll
                for (int tl = 0; tl < NT; ++tl) {
                    const int m = tl * 16 + ln;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int v = v0 + 4 * lq + r;
                        const float sc = acc[tl][r];
                        if (keep[r] && (sc > bv[tl] || (sc == bv[tl] && v < bi[tl]))) {
                            bv[tl] = sc;
                            bi[tl] = v;
                        }
                    }
                    if (a.lse.pm) {
                        float xk[4], mx = -INFINITY;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            xk[r] = keep[r] ? acc[tl][r] * a.lse.k : -INFINITY;
                            mx = fmaxf(mx, xk[r]);
                        }
                        if (mx != -INFINITY) {
                            const float mn = fmaxf(lm[tl], mx);
                            float sum = ls[tl] * __builtin_amdgcn_exp2f(lm[tl] - mn);
#pragma unroll
                            for (int r = 0; r < 4; ++r) sum += __builtin_amdgcn_exp2f(xk[r] - mn);
                            lm[tl] = mn;
                            ls[tl] = sum;
                        }
                    }
                    if (a.logits && m < a.M) {
                        float* lp = a.logits + (size_t)m * a.V + v0 + 4 * lq;
                        if (v0 + 4 * lq + 3 < a.V) {
                            *(float4*)lp =
                                make_float4(acc[tl][0], acc[tl][1], acc[tl][2], acc[tl][3]);
                        } else {
                            for (int r = 0; r < 4; ++r)
                                if (v0 + 4 * lq + r < a.V) lp[r] = acc[tl][r];
                        }
                    }
                }
            }
            if (NPB == 1) __syncthreads();  // the partials were read before the set is reused
        }
        c_strip += SW;
        ++c_rd;
#pragma unroll
        for (int tl = 0; tl < NT; ++tl) acc[tl] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
    };
    Piece pa, pb;
    issue(pa);
    __builtin_amdgcn_sched_barrier(0);  // all of pa's requests before pb's
    issue(pb);
    __builtin_amdgcn_sched_barrier(0);
    for (int i = 0; i < TP; i += 2) {
        step(pa, i);
        step(pb, i + 1);
    }
    // reduce across lanes of the same row (lane, lane^16, lane^32, lane^48)
#pragma unroll
    for (int tl = 0; tl < NT; ++tl) {
#pragma unroll
        for (int o = 16; o < 64; o <<= 1) {
            const float ov = __shfl_xor(bv[tl], o, MJ_WAVE);
            const int oi = __shfl_xor(bi[tl], o, MJ_WAVE);
            if (ov > bv[tl] || (ov == bv[tl] && oi < bi[tl])) {
                bv[tl] = ov;
                bi[tl] = oi;
            }
        }
    }
    __shared__ float sv[8][32];
    __shared__ int si[8][32];
    __shared__ float slm[4][32], sls[4][32];
    if (a.lse.pm) {  // the h = 0 waves hold the sums
#pragma unroll
        for (int tl = 0; tl < NT; ++tl)
#pragma unroll
            for (int o = 16; o < 64; o <<= 1)
                lse_merge(lm[tl], ls[tl], __shfl_xor(lm[tl], o, MJ_WAVE),
                          __shfl_xor(ls[tl], o, MJ_WAVE));
        if (lane < 16 && h == 0) {
#pragma unroll
            for (int tl = 0; tl < NT; ++tl) {
                slm[slot][tl * 16 + lane] = lm[tl];
                sls[slot][tl * 16 + lane] = ls[tl];
            }
        }
    }
    if (lane < 16) {
#pragma unroll
        for (int tl = 0; tl < NT; ++tl) {
            sv[wv][tl * 16 + lane] = bv[tl];
            si[wv][tl * 16 + lane] = bi[tl];
        }
    }
    __syncthreads();
    if (t < NT * 16 && t < a.M) {
        float b = sv[0][t];
        int i = si[0][t];
        for (int w = 1; w < 8; ++w)
            if (sv[w][t] > b || (sv[w][t] == b && si[w][t] < i)) {
                b = sv[w][t];
                i = si[w][t];
            }
        a.pval[(size_t)blockIdx.x * 32 + t] = b;
        a.pidx[(size_t)blockIdx.x * 32 + t] = i;
        if (a.lse.pm) {
            float m = slm[0][t], sm = sls[0][t];
            for (int w = 1; w < 4; ++w) lse_merge(m, sm, slm[w][t], sls[w][t]);
            a.lse.pm[(size_t)blockIdx.x * 32 + t] = m;
            a.lse.ps[(size_t)blockIdx.x * 32 + t] = sm;
        }
    }
}

// ---------------------------------------------------------------------------------------
// The Maple head: maple_lm_head_argmax (SeedlessMetal.swift:3005-3068) over its 4-bit affine
// weight -- w uint32 [V][K/8] (8 codes a word, LSB first), scale / bias fp16 [V][K/64];
// logits[m][v] = sum_k (q s + b) x[m][k].  Same partials as k_lm_head (lowest id on ties,
// banned ids skipped), folded by k_head_final.
//
// MFMA 16x16x32 f16 with A = 16 hidden rows (staged in LDS) and B = a 16-row vocab strip's
// codes, each widened to fp16 16 + q (code q in the top four mantissa bits under exponent 16:
// one shift and one mask-or per nibble pair (j, j + 4) of a word).  The products x (16 + q)
// are exact in fp32; per 64-group g the MFMA sum is scaled by s_g, and the remainder
// sum_g (b_g - 16 s_g) X_g (X_g = group sum of the hidden row, staged beside it) is a chain
// of fp32 MFMAs.
//
// Loads: lane (n, q) reads 16 B -- words 16 j + 4 q of a group pair j -- so a strip row's
// 64 B come in one request; one lane swap across the wave's halves (lanes 32..63 <-> 0..31)
// then leaves lane q holding words (0, 1) of both groups for q = 0, (4, 5) for q = 1, (2, 3)
// for q = 2 and (6, 7) for q = 3, so each MFMA takes one group.  The hidden rows are staged to
// match: 8-k chunk c of a group at chunk position c with bits 1 and 2 swapped, and within a
// chunk the order k 0 4 1 5 2 6 3 7 of the nibble pairs.
//
// Work unit: one K half of a strip, as k_lm_head: wave (slot, h) takes half h of strips
// blockIdx.x * 4 + slot + round * gridDim.x * 4, the h = 1 partial meets the h = 0 one in
// LDS.  A half streams as pieces of PL group pairs (16 rows x PL x 128 k codes plus their
// scales and biases), the next requested before the current one is multiplied.
struct HeadQ4Args {
    const uint16_t* x;   // [M][K] fp16
    const uint32_t* w;   // [V][K/8]
    const uint16_t* s;   // [V][K/64]
    const uint16_t* b;
    int M, K, V;
    const int32_t* banned;
    int n_banned;
    float* logits;       // [M][V] or nullptr
    float* pval;         // [blocks][32]
    int* pidx;
    const int* abort;
    HeadLse lse;
};

template <int PL>
struct Q4Piece {
    u4v c[PL];                          // codes: group pair j, words 16 j + 4 q .. + 3
    uint32_t sc[PL], bs[PL];            // scales / biases of groups 2 j, 2 j + 1 (lo, hi)
};

template <int NT, int PL>
__global__ __launch_bounds__(512) void k_lm_head_q4(HeadQ4Args a) {
    if (aborted(a.abort)) return;
    extern __shared__ __align__(16) char q4lds[];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int K = a.K, XS = K + 8, G = K / 64, GS1 = G + 1;
    uint16_t* xs = (uint16_t*)q4lds;                 // [NT*16][XS] hidden rows, code order
    float* xg = (float*)(xs + NT * 16 * XS);         // [NT*16][G + 1] group sums
    for (int idx = t; idx < NT * 16 * (K / 8); idx += 512) {
        const int m = idx / (K / 8), c = idx % (K / 8);
        u4v v = {0u, 0u, 0u, 0u};
        if (m < a.M) v = *(const u4v*)(a.x + (size_t)m * K + 8 * c);
        u4v o;
        o[0] = (v[0] & 0xFFFFu) | (v[2] << 16);
        o[1] = (v[0] >> 16) | (v[2] & 0xFFFF0000u);
        o[2] = (v[1] & 0xFFFFu) | (v[3] << 16);
        o[3] = (v[1] >> 16) | (v[3] & 0xFFFF0000u);
        const int cp = (c & ~6) | ((c & 2) << 1) | ((c & 4) >> 1);
        *(u4v*)(xs + m * XS + 8 * cp) = o;
    }
    __shared__ int s_ban[MJ_HEAD_MAX_BANNED];  // banned ids (read with LDS, not vector, loads)
    for (int idx = t; idx < a.n_banned; idx += 512) s_ban[idx] = a.banned[idx];
    for (int idx = t; idx < NT * 16 * G; idx += 512) {
        const int m = idx / G, g = idx % G;
        float sum = 0.0f;
        if (m < a.M)
            for (int c = 0; c < 8; ++c) {
                const u4v v = *(const u4v*)(a.x + (size_t)m * K + 64 * g + 8 * c);
#pragma unroll
                for (int j = 0; j < 4; ++j) sum += h2f(v[j] & 0xFFFFu) + h2f(v[j] >> 16);
            }
        xg[m * GS1 + g] = sum;
    }
    __syncthreads();

    const int n = lane & 15, q = lane >> 4;
    const int nstrips = (a.V + 15) / 16;
    const int slot = wv & 3, h = wv >> 2;
    const int NH = G / 2 / (2 * PL);   // pieces per half strip
    const int SW = gridDim.x * 4;
    const int rounds = (nstrips - (int)blockIdx.x * 4 + SW - 1) / SW;
    // the code offset 0x4C00 (fp16 16) kept in a VGPR so each nibble pair is one mask-or
    uint32_t c16 = 0x4C004C00u;
    asm("" : "+v"(c16));
    const uint32_t nmask = 0x03C003C0u;
    const int hsh = 16 * (q & 1);      // this lane's half of a scale word in the remainder chain
    float bv[NT][4];
    int bi[NT][4];
    float lm[NT][4], ls[NT][4];  // running log-sum-exp of logits / T (log2 units)
#pragma unroll
    for (int tl = 0; tl < NT; ++tl)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            bv[tl][r] = -INFINITY;
            bi[tl][r] = 0x7fffffff;
            lm[tl][r] = -INFINITY;
            ls[tl][r] = 0.0f;
        }
    auto load_piece = [&](int strip, int pc, Q4Piece<PL>& pz) {
        const int vr = min(strip * 16 + n, a.V - 1);
        const int g0 = 2 * PL * (h * NH + pc);   // first group of the piece
        const u4v* wr = (const u4v*)(a.w + (size_t)vr * (K / 8) + 8 * g0) + q;
#pragma unroll
        for (int j = 0; j < PL; ++j) pz.c[j] = wr[4 * j];
        const uint16_t* sr = a.s + (size_t)vr * G + g0;
        const uint16_t* br = a.b + (size_t)vr * G + g0;
        if constexpr (PL == 4) {
            const u4v sv4 = *(const u4v*)sr, bv4 = *(const u4v*)br;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                pz.sc[j] = sv4[j];
                pz.bs[j] = bv4[j];
            }
        } else {
            const uint2 sv2 = *(const uint2*)sr, bv2 = *(const uint2*)br;
            pz.sc[0] = sv2.x;
            pz.sc[1] = sv2.y;
            pz.bs[0] = bv2.x;
            pz.bs[1] = bv2.y;
        }
    };
    constexpr int NPB = NT == 1 ? 2 : 1;
    __shared__ f4 s_part[NPB][4][NT][64];
    // The wave's pieces form one stream (rounds x NH) through two register sets taken in
    // turn: a set is refilled with the piece two ahead as soon as it has been multiplied, so
    // one piece is always in flight behind the one in use and no set is copied.  Every load is
    // issued -- past the stream's end at the clamped last row, a cached line -- which keeps the
    // wait before a set's use from covering the other set's requests.
    const int strip0 = blockIdx.x * 4 + slot, TP = rounds * NH;
    int ld_strip = strip0, ld_pc = 0;
    auto issue = [&](Q4Piece<PL>& pz) {
        load_piece(ld_strip, ld_pc, pz);
        if (++ld_pc == NH) {
            ld_pc = 0;
            ld_strip += SW;
        }
    };
    f4 acc[NT];
#pragma unroll
    for (int tl = 0; tl < NT; ++tl) acc[tl] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
    int c_strip = strip0, c_pc = 0, c_rd = 0;
    auto step = [&](Q4Piece<PL>& cur, int i) {
        const int g0 = 2 * PL * (h * NH + c_pc);
        // remainder: lane q's group of chain step u is 4 u + q of the piece
#pragma unroll
        for (int u = 0; u < PL / 2; ++u) {
            const uint32_t sw = (q >> 1) ? cur.sc[2 * u + 1] : cur.sc[2 * u];
            const uint32_t bw = (q >> 1) ? cur.bs[2 * u + 1] : cur.bs[2 * u];
            const float cg = h2f((uint16_t)(bw >> hsh)) - 16.0f * h2f((uint16_t)(sw >> hsh));
#pragma unroll
            for (int tl = 0; tl < NT; ++tl)
                acc[tl] = mfma16x16x4f32(xg[(tl * 16 + n) * GS1 + g0 + 4 * u + q], cg, acc[tl]);
        }
#pragma unroll
        for (int j = 0; j < PL; ++j) {
            u4v cw = cur.c[j];
            {
                const auto r0 = __builtin_amdgcn_permlane32_swap(cw[0], cw[2], false, false);
                const auto r1 = __builtin_amdgcn_permlane32_swap(cw[1], cw[3], false, false);
                cw[0] = r0[0];
                cw[2] = r0[1];
                cw[1] = r1[0];
                cw[3] = r1[1];
            }
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                const int g = g0 + 2 * j + gi;
                u4v b0, b1;
                const uint32_t w0 = cw[2 * gi], w1 = cw[2 * gi + 1];
                b0[0] = ((w0 << 6) & nmask) | c16;
                b0[1] = ((w0 << 2) & nmask) | c16;
                b0[2] = ((w0 >> 2) & nmask) | c16;
                b0[3] = ((w0 >> 6) & nmask) | c16;
                b1[0] = ((w1 << 6) & nmask) | c16;
                b1[1] = ((w1 << 2) & nmask) | c16;
                b1[2] = ((w1 >> 2) & nmask) | c16;
                b1[3] = ((w1 >> 6) & nmask) | c16;
                const float sg = h2f((uint16_t)(cur.sc[j] >> (16 * gi)));
#pragma unroll
                for (int tl = 0; tl < NT; ++tl) {
                    const uint16_t* xr = xs + (tl * 16 + n) * XS + 64 * g + 16 * q;
                    f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
                    d = mfma16x16x32(as_h8(*(const u4v*)xr), as_h8(b0), d);
                    d = mfma16x16x32(as_h8(*(const u4v*)(xr + 8)), as_h8(b1), d);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[tl][r] += sg * d[r];
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        issue(cur);  // the piece two ahead
        __builtin_amdgcn_sched_barrier(0);
        if (++c_pc < NH) return;
        c_pc = 0;
        if (i < TP) {  // end of a round: the same for every wave of the block
            const bool live = c_strip < nstrips;
            if (h == 1) {
#pragma unroll
                for (int tl = 0; tl < NT; ++tl) s_part[c_rd % NPB][slot][tl][lane] = acc[tl];
            }
            __syncthreads();  // the h = 1 halves are in LDS
            if (live && h == 0) {
#pragma unroll
                for (int tl = 0; tl < NT; ++tl) {
                    const f4 o = s_part[c_rd % NPB][slot][tl][lane];
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[tl][r] += o[r];
                }
                // lane (n, q): vocab row v0 + n, hidden rows tl * 16 + 4 q + r
                const int v = c_strip * 16 + n;
                bool keep = v < a.V;
                for (int bb = 0; bb < a.n_banned; ++bb)
                    if (s_ban[bb] == v) keep = false;
#pragma unroll
                for (int tl = 0; tl < NT; ++tl)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int m = tl * 16 + 4 * q + r;
                        const float val = acc[tl][r];
                        if (keep && (val > bv[tl][r] || (val == bv[tl][r] && v < bi[tl][r]))) {
                            bv[tl][r] = val;
                            bi[tl][r] = v;
                        }
                        if (keep && a.lse.pm) {
                            const float xk = val * a.lse.k, mn = fmaxf(lm[tl][r], xk);
                            ls[tl][r] = ls[tl][r] * __builtin_amdgcn_exp2f(lm[tl][r] - mn) +
                                        __builtin_amdgcn_exp2f(xk - mn);
                            lm[tl][r] = mn;
                        }
                        if (a.logits && m < a.M && v < a.V) a.logits[(size_t)m * a.V + v] = val;
                    }
            }
            if (NPB == 1) __syncthreads();  // the partials were read before the set is reused
        }
        c_strip += SW;
        ++c_rd;
#pragma unroll
        for (int tl = 0; tl < NT; ++tl) acc[tl] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
    };
    Q4Piece<PL> pa, pb;
    issue(pa);
    __builtin_amdgcn_sched_barrier(0);  // all of pa's requests before pb's
    issue(pb);
    __builtin_amdgcn_sched_barrier(0);
    for (int i = 0; i < TP; i += 2) {
        step(pa, i);
        step(pb, i + 1);
    }
    // across the 16 vocab lanes of a row group, then across the h = 0 waves
#pragma unroll
    for (int tl = 0; tl < NT; ++tl)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const float ov = __shfl_xor(bv[tl][r], o, MJ_WAVE);
                const int oi = __shfl_xor(bi[tl][r], o, MJ_WAVE);
                if (ov > bv[tl][r] || (ov == bv[tl][r] && oi < bi[tl][r])) {
                    bv[tl][r] = ov;
                    bi[tl][r] = oi;
                }
            }
    __shared__ float sv[4][32];
    __shared__ int si[4][32];
    __shared__ float slm[4][32], sls[4][32];
    if (a.lse.pm) {
#pragma unroll
        for (int tl = 0; tl < NT; ++tl)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int o = 1; o < 16; o <<= 1)
                    lse_merge(lm[tl][r], ls[tl][r], __shfl_xor(lm[tl][r], o, MJ_WAVE),
                              __shfl_xor(ls[tl][r], o, MJ_WAVE));
    }
    if (h == 0 && n == 0) {
#pragma unroll
        for (int tl = 0; tl < NT; ++tl)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sv[slot][tl * 16 + 4 * q + r] = bv[tl][r];
                si[slot][tl * 16 + 4 * q + r] = bi[tl][r];
                slm[slot][tl * 16 + 4 * q + r] = lm[tl][r];
                sls[slot][tl * 16 + 4 * q + r] = ls[tl][r];
            }
    }
    __syncthreads();
    if (t < NT * 16 && t < a.M) {
        float bb = sv[0][t];
        int ii = si[0][t];
        for (int w2 = 1; w2 < 4; ++w2)
            if (sv[w2][t] > bb || (sv[w2][t] == bb && si[w2][t] < ii)) {
                bb = sv[w2][t];
                ii = si[w2][t];
            }
        a.pval[(size_t)blockIdx.x * 32 + t] = bb;
        a.pidx[(size_t)blockIdx.x * 32 + t] = ii;
        if (a.lse.pm) {
            float m = slm[0][t], sm = sls[0][t];
            for (int w2 = 1; w2 < 4; ++w2) lse_merge(m, sm, slm[w2][t], sls[w2][t]);
            a.lse.pm[(size_t)blockIdx.x * 32 + t] = m;
            a.lse.ps[(size_t)blockIdx.x * 32 + t] = sm;
        }
    }
}

// One wave per row: fold the block partials (value, lowest id on ties; log-sum-exp pairs).
// Row m's fold by one wave: its nblk partials, eight a lane requested together.  Every lane
// returns the row's argmax id; lane 0 writes out_idx / out_max / the log-sum-exp.
__device__ __forceinline__ int head_fold_row(const float* pval, const int* pidx, int nblk, int m,
                                             int lane, int32_t* out_idx, float* out_max,
                                             const HeadLse& lse) {
    float b = -INFINITY;
    int i = 0x7fffffff;
    float lm = -INFINITY, ls = 0.0f;
    for (int k0 = 0; k0 < nblk; k0 += 8 * 64) {
        float v[8];
        int j[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int k = k0 + 64 * u + lane;
            v[u] = k < nblk ? pval[(size_t)k * 32 + m] : -INFINITY;
            j[u] = k < nblk ? pidx[(size_t)k * 32 + m] : 0x7fffffff;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (v[u] > b || (v[u] == b && j[u] < i)) {
                b = v[u];
                i = j[u];
            }
        if (lse.out) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int k = k0 + 64 * u + lane;
                if (k < nblk) lse_merge(lm, ls, lse.pm[(size_t)k * 32 + m], lse.ps[(size_t)k * 32 + m]);
            }
        }
    }
    wave_argmax(b, i);
    if (lse.out) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
            lse_merge(lm, ls, __shfl_xor(lm, o, MJ_WAVE), __shfl_xor(ls, o, MJ_WAVE));
    }
    if (lane == 0) {
        out_idx[m] = i;
        if (out_max) out_max[m] = b;
        // ln sum_v exp(logit_v / T) = ln 2 * (m + log2 s); -inf when every id is banned
        if (lse.out) lse.out[m] = lm == -INFINITY ? -INFINITY : 0.69314718f * (lm + __log2f(ls));
    }
    return i;
}

__global__ __launch_bounds__(64) void k_head_final(const float* pval, const int* pidx, int nblk,
                                                   int M, int32_t* out_idx, float* out_max,
                                                   HeadLse lse, const int* abort) {
    if (aborted(abort)) return;
    const int m = blockIdx.x;
    if (m >= M) return;
    head_fold_row(pval, pidx, nblk, m, threadIdx.x, out_idx, out_max, lse);
}

// Greedy acceptance by one wave, lane c = row c < n (n <= 64): tok / par / am are row c's token,
// parent and argmax.  verifyDraftChain's longest-prefix rule walked over the draft tree: from
// row 0, the lowest-index child whose token equals the current row's argmax, while one exists
// (a ballot a level).  Writes res (path, emit, argmax) and / or out_flat ([acc, token,
// path[0..n), emit[0..n)]).
__device__ __forceinline__ void accept_greedy_wave(int tok, int par, int am, int n,
                                                   StepResult* res, int32_t* out_flat) {
    const int lane = threadIdx.x & 63;
    // (cur and next are wave-uniform: the row values are read with readlane, no LDS permute)
    int cur = 0, acc = 0, my_path = 0, my_emit = 0;
    for (;;) {
        const int amc = __builtin_amdgcn_readlane(am, cur);
        const uint64_t kids = __ballot(lane < n && par == cur && tok == amc);
        if (!kids) break;
        const int next = __ffsll((unsigned long long)kids) - 1;
        const int tn = __builtin_amdgcn_readlane(tok, next);
        if (lane == acc) my_emit = tn;
        ++acc;
        if (lane == acc) my_path = next;
        cur = next;
    }
    const int fin = __builtin_amdgcn_readlane(am, cur);
    if (lane == acc) my_emit = fin;
    if (res) {
        if (lane == 0) {
            res->accepted = acc;
            res->token = fin;
        }
        if (lane <= acc) {
            res->path[lane] = my_path;
            res->emit[lane] = my_emit;
        }
        if (lane < n) res->argmax[lane] = am;
    }
    if (out_flat) {
        if (lane == 0) {
            out_flat[0] = acc;
            out_flat[1] = fin;
        }
        if (lane <= acc) {
            out_flat[2 + lane] = my_path;
            out_flat[2 + n + lane] = my_emit;
        }
    }
}

// k_head_final over every row of one launch group (M <= 32; no log-sum-exp), then the greedy
// acceptance from the argmax ids it just formed: one launch where there were two.  512
// threads read the partials contiguously: float4 f = t + 512 i of the [nblk][32] arrays is
// rows 4 (t % 8) .. + 3 of partial block f / 8, so a thread keeps four rows over nblk / 64
// blocks (one round of requests for nblk <= 512); lanes of one row group meet by shuffles (xor 8, 16, 32), the eight waves in LDS.
// Highest value, lowest id among equal values: the same pick in any order.
__device__ __forceinline__ void argmax_merge(float& b, int& i, float v, int j) {
    if (v > b || (v == b && j < i)) {
        b = v;
        i = j;
    }
}

__global__ __launch_bounds__(512) void k_head_final_accept(const float* pval, const int* pidx,
                                                           int nblk, int M, int32_t* out_idx,
                                                           float* out_max, const int* abort,
                                                           GreedyAccept ga) {
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    // the abort word requested with the partials, tested before anything is written (a
    // relaxed atomic load, no branch around it: waited for only where it is tested)
    const int ab = __hip_atomic_load(abort != nullptr ? abort : ga.tokens, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) &
                   (abort != nullptr ? ~0 : 0);
    const int g = t & 7;                 // row group: rows 4g .. 4g + 3
    const int ng = (M + 3) >> 2;         // row groups in use
    __shared__ float s_v[8][32];
    __shared__ int s_i[8][32];
    // the accept's per-row inputs, requested with the partials
    const int tok = lane < M ? ga.tokens[lane] : -1;
    const int par = lane < M ? ga.parents[lane] : -2;
    float b[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    int bi[4] = {0x7fffffff, 0x7fffffff, 0x7fffffff, 0x7fffffff};
    if (g < ng) {
        const f4* pv4 = (const f4*)pval;
        const u4v* pi4 = (const u4v*)pidx;
        const int F = nblk * 8;  // float4s of each array
        for (int f0 = t; f0 < F; f0 += 512 * 8) {  // one round for nblk <= 512
            f4 v[8];
            u4v j[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int f = min(f0 + 512 * u, F - 8 + g);  // clamped: a repeat changes no pick
                v[u] = pv4[f];
                j[u] = pi4[f];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
#pragma unroll
                for (int c = 0; c < 4; ++c) argmax_merge(b[c], bi[c], v[u][c], (int)j[u][c]);
        }
    }
#pragma unroll
    for (int o = 8; o < 64; o <<= 1)
#pragma unroll
        for (int c = 0; c < 4; ++c)
            argmax_merge(b[c], bi[c], __shfl_xor(b[c], o, MJ_WAVE), __shfl_xor(bi[c], o, MJ_WAVE));
    if (lane < 8) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            s_v[wv][4 * lane + c] = b[c];
            s_i[wv][4 * lane + c] = bi[c];
        }
    }
    __syncthreads();
    if (wv != 0 || ab != 0) return;
    float bm = -INFINITY;
    int im = 0x7fffffff;
    if (lane < M)
#pragma unroll
        for (int w = 0; w < 8; ++w) argmax_merge(bm, im, s_v[w][lane], s_i[w][lane]);
    if (lane < M) {
        out_idx[lane] = im;
        if (out_max) out_max[lane] = bm;
    }
    accept_greedy_wave(tok, par, lane < M ? im : -1, M, ga.res, nullptr);
}

// The fold of rows m0 .. m0 + mg of M.  With ga the greedy acceptance follows: in the same
// launch when the rows are one group (M <= 32, no log-sum-exp), else after the last fold.
static hipError_t launch_head_final(const float* pval, const int* pidx, int nb, int M, int m0,
                                    int mg, int32_t* out_idx, float* out_max, const HeadLse& gl,
                                    const int* abort, hipStream_t st, const GreedyAccept* ga) {
    if (ga && M <= 32 && !gl.out) {
        hipLaunchKernelGGL(k_head_final_accept, dim3(1), dim3(512), 0, st, pval, pidx, nb, mg,
                           out_idx, out_max, abort, *ga);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_head_final, dim3(mg), dim3(64), 0, st, pval, pidx, nb, mg, out_idx + m0,
                       out_max ? out_max + m0 : nullptr, gl, abort);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !ga || m0 + mg < M) return e;
    return launch_accept_greedy(ga->tokens, ga->parents, out_idx, M, ga->res, nullptr, abort, st);
}

// two 512-thread blocks per CU (the staged rows take at most 66 KB of LDS each)
int head_blocks() {
    static int nb = 0;
    if (nb == 0) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        nb = 2 * cus;
    }
    return nb;
}

// Rows go through in groups of <= 32 (two 16-row MFMA tiles staged in LDS per group).
hipError_t launch_lm_head(const uint16_t* x, const uint16_t* w, int M, int K, int V,
                          const int32_t* banned, int n_banned, float* logits, float* pval,
                          int* pidx, int32_t* out_idx, float* out_max, HeadLse lse,
                          const int* abort, hipStream_t st, const GreedyAccept* ga) {
    if (K % 256 != 0 || M < 1 || n_banned > MJ_HEAD_MAX_BANNED)  // halves of 128-k multiples
        return hipErrorInvalidValue;
    for (int m0 = 0; m0 < M; m0 += 32) {
        const int mg = M - m0 < 32 ? M - m0 : 32;
        // two blocks per CU for one 16-row tile; a 32-row group's LDS allows one
        const int nb = mg <= 16 ? head_blocks() : head_blocks() / 2;
        HeadLse gl = lse;
        if (!gl.out) gl.pm = gl.ps = nullptr;
        else gl.out += m0;
        HeadArgs a{x + (size_t)m0 * K, w, mg, K, V, banned, n_banned,
                   logits ? logits + (size_t)m0 * V : nullptr, pval, pidx, abort, gl};
        const bool pl8 = (K / 64) % 8 == 0;  // 8-chunk pieces when the half strip allows
        if (mg <= 16) {
            const size_t lds = (size_t)16 * (K + 8) * 2;
            if (pl8)
                launch_timed(k_lm_head<1, 8>, dim3(nb), dim3(512), lds, st, a);
            else
                launch_timed(k_lm_head<1, 4>, dim3(nb), dim3(512), lds, st, a);
        } else {
            const size_t lds = (size_t)32 * (K + 8) * 2;
            if (lds > 140 * 1024) return hipErrorInvalidValue;  // K <= 2232 for 17..32 rows
            if (pl8)
                launch_timed(k_lm_head<2, 8>, dim3(nb), dim3(512), lds, st, a);
            else
                launch_timed(k_lm_head<2, 4>, dim3(nb), dim3(512), lds, st, a);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        e = launch_head_final(pval, pidx, nb, M, m0, mg, out_idx, out_max, gl, abort, st, ga);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// ---------------------------------------------------------------------------------------
// Greedy acceptance over rows 0..n-1 (row 0 = the fed token y).  tokens/parents from the
// step descriptor (or explicit arrays), argmax per row.  One wave: n <= 64.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_accept_greedy(const int32_t* tokens,
                                                      const int32_t* parents,
                                                      const int32_t* argmax, int n,
                                                      StepResult* res, int32_t* out_flat,
                                                      const int* abort) {
    if (aborted(abort)) return;
    const int lane = threadIdx.x;
    const int tok = lane < n ? tokens[lane] : -1;
    const int par = lane < n ? parents[lane] : -2;
    const int am = lane < n ? argmax[lane] : -1;
    accept_greedy_wave(tok, par, am, n, res, out_flat);
}

hipError_t launch_accept_greedy(const int32_t* tokens, const int32_t* parents,
                                const int32_t* argmax, int n, StepResult* res, int32_t* out_flat,
                                const int* abort, hipStream_t st) {
    hipLaunchKernelGGL(k_accept_greedy, dim3(1), dim3(64), 0, st, tokens, parents, argmax, n, res,
                       out_flat, abort);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// KV commit: block per (layer, kv head).  Reads every accepted row first, then writes.
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_kv_commit(uint16_t* kv, int64_t layer_stride,
                                                   int64_t C, int nKV, const StepDesc* sd,
                                                   const StepResult* res, const int* abort) {
    if (aborted(abort)) return;
    const int t = threadIdx.x;
    // the accepted count and path (one entry a thread) requested together
    const int acc = res->accepted;
    const int pv = res->path[t & (MJ_ROWS - 1)];
    const int layer = blockIdx.x / (2 * nKV), rest = blockIdx.x % (2 * nKV);
    uint16_t* base = kv + layer * layer_stride + (int64_t)rest * C * 128;  // K heads then V heads
    const int64_t L = sd->L;
    __shared__ u4v rows[MJ_ROWS][16];
    __shared__ int s_path[MJ_ROWS];
    if (t < MJ_ROWS) s_path[t] = pv;
    if (!__syncthreads_or(t >= 1 && t <= acc && t < MJ_ROWS && pv != t)) return;  // in place
    for (int idx = t; idx < (acc + 1) * 16; idx += 256) {
        const int i = idx >> 4, part = idx & 15;
        const int64_t src = (L + s_path[i]) % C;
        rows[i][part] = *(const u4v*)(base + src * 128 + 8 * part);
    }
    __syncthreads();
    for (int idx = t; idx < (acc + 1) * 16; idx += 256) {
        const int i = idx >> 4, part = idx & 15;
        const int64_t dst = (L + i) % C;
        *(u4v*)(base + dst * 128 + 8 * part) = rows[i][part];
    }
}

// Debug capture: the K and V rows a pass appended, dst [n_layers][2][nKV][R][128] (R =
// MJ_ROWS), block per (layer, K|V, kv head).
__global__ __launch_bounds__(256) void k_kv_rows(const uint16_t* kv, int64_t layer_stride, int64_t C,
                                                 int nKV, const StepDesc* sd, uint16_t* dst) {
    const int layer = blockIdx.x / (2 * nKV), rest = blockIdx.x % (2 * nKV);
    const uint16_t* base = kv + layer * layer_stride + (int64_t)rest * C * 128;
    uint16_t* out = dst + ((size_t)layer * 2 * nKV + rest) * MJ_ROWS * 128;
    const int64_t L = sd->L;
    for (int idx = threadIdx.x; idx < sd->M * 16; idx += 256) {
        const int r = idx >> 4, part = idx & 15;
        *(u4v*)(out + (size_t)r * 128 + 8 * part) =
            *(const u4v*)(base + ((L + r) % C) * 128 + 8 * part);
    }
}

hipError_t launch_kv_rows(const uint16_t* kv, int64_t layer_stride, int n_layers, int64_t C,
                          int nKV, const StepDesc* sd, uint16_t* dst, hipStream_t st) {
    hipLaunchKernelGGL(k_kv_rows, dim3(n_layers * 2 * nKV), dim3(256), 0, st, kv, layer_stride, C,
                       nKV, sd, dst);
    return hipGetLastError();
}

hipError_t launch_kv_commit(uint16_t* kv, int64_t layer_stride, int n_layers, int64_t C, int nKV,
                            const StepDesc* sd, const StepResult* res, const int* abort,
                            hipStream_t st) {
    hipLaunchKernelGGL(k_kv_commit, dim3(n_layers * 2 * nKV), dim3(256), 0, st, kv, layer_stride,
                       C, nKV, sd, res, abort);
    return hipGetLastError();
}

// RoPE angles of pass row r (its position L + depth[r]) for frequencies t < rt.half; called by
// the first rt.half threads of the row's block.  The same cosf / sinf of pos * inv_freq[f] as
// maple_qk_norm_rope's angle (SeedlessMetal.swift:2832-2846), evaluated once per pass.
__device__ __forceinline__ void rope_row(const StepDesc* sd, const RopeTab& rt, int r, int t) {
    if (t < rt.half) {
        const float pos = (float)(sd->L + sd->depth[r]);
        const float th = pos * rt.inv_freq[t];
        rt.cs[r * MJ_ROPE_F + t] = make_float2(cosf(th), sinf(th));
    }
}

// Token embedding: h[r] = table[tokens[r]] (maple_embed_token, SeedlessMetal.swift:3114-3126).
__global__ __launch_bounds__(256) void k_embed(const uint16_t* table, const StepDesc* sd, int M,
                                               int H, uint16_t* h, RopeTab rt, const int* abort) {
    if (aborted(abort)) return;
    const int r = blockIdx.x;
    if (r >= M) return;
    rope_row(sd, rt, r, threadIdx.x);
    const int tok = sd->tokens[r];
    for (int i = threadIdx.x; i < H / 8; i += 256)
        *(u4v*)(h + (size_t)r * H + 8 * i) = *(const u4v*)(table + (size_t)tok * H + 8 * i);
}

hipError_t launch_embed(const uint16_t* table, const StepDesc* sd, int M, int H, uint16_t* h,
                        const RopeTab& rt, const int* abort, hipStream_t st) {
    if (rt.half > MJ_ROPE_F || M > MJ_ROWS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_embed, dim3(M), dim3(256), 0, st, table, sd, M, H, h, rt, abort);
    return hipGetLastError();
}

// Token embedding of a 2048-wide row followed by the first layer's input RMSNorm.
__global__ __launch_bounds__(256) void k_embed_norm(const uint16_t* table, const StepDesc* sd,
                                                    uint16_t* h, NormOut no, RopeTab rt,
                                                    const int* abort) {
    if (aborted(abort)) return;
    const int r = blockIdx.x, t = threadIdx.x;
    rope_row(sd, rt, r, t);
    const int tok = sd->tokens[r];
    const u4v v = *(const u4v*)(table + (size_t)tok * 2048 + 8 * t);
    *(u4v*)(h + (size_t)r * 2048 + 8 * t) = v;
    norm_row_2048(v, no, r);
}

hipError_t launch_embed_norm(const uint16_t* table, const StepDesc* sd, int M, int H, uint16_t* h,
                             const NormOut& no, const RopeTab& rt, const int* abort,
                             hipStream_t st) {
    if (H != 2048 || rt.half > MJ_ROPE_F || M > MJ_ROWS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_embed_norm, dim3(M), dim3(256), 0, st, table, sd, h, no, rt, abort);
    return hipGetLastError();
}

__global__ __launch_bounds__(64) void k_rope_table(const StepDesc* sd, RopeTab rt) {
    rope_row(sd, rt, blockIdx.x, threadIdx.x);
}

hipError_t launch_rope_table(const StepDesc* sd, int M, const RopeTab& rt, hipStream_t st) {
    if (rt.half > MJ_ROPE_F || M > MJ_ROWS) return hipErrorInvalidValue;
    if (rt.half == 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope_table, dim3(M), dim3(64), 0, st, sd, rt);
    return hipGetLastError();
}

// The wall clock (s_memrealtime) ticks at 100 MHz; the loop also stops after a fixed number
// of sleeps, so it ends even if the clock were not to advance.
__global__ __launch_bounds__(64) void k_hold(unsigned ticks) {
    const unsigned long long t0 = wall_clock64();
    for (int i = 0; i < (1 << 22); ++i) {
        if (wall_clock64() - t0 >= ticks) break;
        __builtin_amdgcn_s_sleep(8);
    }
}

hipError_t launch_hold(unsigned us, hipStream_t st) {
    if (us > 100000) us = 100000;
    launch_timed(k_hold, dim3(1), dim3(64), 0, st, us * 100u);
    return hipGetLastError();
}

hipError_t set_attn_attributes();
hipError_t set_gather3_attributes();

// Rows in groups of <= 32 as launch_lm_head; K % 512 == 0 (a half strip is 4 groups or a
// multiple of 8), K <= 4096 (<= 2048 for 17..32 rows).
hipError_t launch_lm_head_q4(const uint16_t* x, const uint32_t* w, const uint16_t* s,
                             const uint16_t* b, int M, int K, int V, const int32_t* banned,
                             int n_banned, float* logits, float* pval, int* pidx,
                             int32_t* out_idx, float* out_max, HeadLse lse, const int* abort,
                             hipStream_t st, const GreedyAccept* ga) {
    if (K % 512 != 0 || K > 4096 || M < 1 || n_banned > MJ_HEAD_MAX_BANNED)
        return hipErrorInvalidValue;
    const bool pl4 = (K / 128) % 8 == 0;  // half strip of K / 128 groups: 8-group pieces
    for (int m0 = 0; m0 < M; m0 += 32) {
        const int mg = M - m0 < 32 ? M - m0 : 32;
        const int nt = mg <= 16 ? 1 : 2;
        const size_t lds = (size_t)nt * 16 * (K + 8) * 2 + (size_t)nt * 16 * (K / 64 + 1) * 4;
        if (lds > 140 * 1024) return hipErrorInvalidValue;
        const int nb = nt == 1 ? head_blocks() : head_blocks() / 2;
        HeadLse gl = lse;
        if (!gl.out) gl.pm = gl.ps = nullptr;
        else gl.out += m0;
        HeadQ4Args qa{x + (size_t)m0 * K, w, s, b, mg, K, V, banned, n_banned,
                      logits ? logits + (size_t)m0 * V : nullptr, pval, pidx, abort, gl};
        if (nt == 1 && pl4)
            launch_timed(k_lm_head_q4<1, 4>, dim3(nb), dim3(512), lds, st, qa);
        else if (nt == 1)
            launch_timed(k_lm_head_q4<1, 2>, dim3(nb), dim3(512), lds, st, qa);
        else if (pl4)
            launch_timed(k_lm_head_q4<2, 4>, dim3(nb), dim3(512), lds, st, qa);
        else
            launch_timed(k_lm_head_q4<2, 2>, dim3(nb), dim3(512), lds, st, qa);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        e = launch_head_final(pval, pidx, nb, M, m0, mg, out_idx, out_max, gl, abort, st, ga);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t set_kernel_attributes() {
    static bool done = false;
    if (done) return hipSuccess;
    const void* hk[8] = {(const void*)k_lm_head<1, 8>,    (const void*)k_lm_head<1, 4>,
                         (const void*)k_lm_head<2, 8>,    (const void*)k_lm_head<2, 4>,
                         (const void*)k_lm_head_q4<1, 4>, (const void*)k_lm_head_q4<1, 2>,
                         (const void*)k_lm_head_q4<2, 4>, (const void*)k_lm_head_q4<2, 2>};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 8 && e == hipSuccess; ++i)
        e = hipFuncSetAttribute(hk[i], hipFuncAttributeMaxDynamicSharedMemorySize, 140 * 1024);
    if (e == hipSuccess) e = set_attn_attributes();
    if (e == hipSuccess) e = set_gather3_attributes();
    if (e == hipSuccess) done = true;
    return e;
}
