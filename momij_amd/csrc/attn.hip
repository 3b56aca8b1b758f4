// attn.hip -- sliding-window attention over the fp16 KV cache for a pass of M verify rows
// arranged as a chain or a draft tree.
//
// k_attn_chunk      maple_sdpa_d128 math (SeedlessMetal.swift:2919-2997): softmax(q k^T /
//                   sqrt(128)) v in fp32, GQA.  Split-K over 64-key chunks ("flash decoding");
//                   one 256-thread block per (kv head, chunk) stages Q (all rows x heads of the
//                   group), K and V^T in LDS and runs QK^T and PV on v_mfma_f32_16x16x32_f16.
//                   Mask: committed positions inside the row's window [P-W+1, L-1]
//                   (AttentionMasks.swift:10-27) plus the row's ancestors and itself; a chain is
//                   the causal M-row pass.
//                   The block also finishes the projection's raw q and k rows as
//                   maple_qk_norm_rope + maple_write_kv_pair do (2794-2901): per-head RMSNorm(eps)
//                   * w, non-traditional half-split RoPE on the first rope_dim dims at the row's
//                   position L + depth(r) (angles from the pass's RoPE table).  Queries are
//                   finished by every block of the group (they are small); the pass's own keys
//                   are finished by the block whose chunk holds them, which also appends them
//                   (K finished, V as projected) at slot (L + r) % C.
// k_attn_combine    merges the chunk partials per (row, head) and writes the output in the qx
//                   format consumed by the o-projection.
#include "mj_device.h"
#include "mj_internal.h"

#define HD 128
#define AK 64     // keys per chunk
#define QSTR 136  // LDS row stride (halves) of Q and K tiles
#define VSTR 72   // LDS row stride (halves) of V^T and P tiles

// Chunks of a pass.  Keys are placed by absolute position: chunk c0 + c holds positions
// [AK (c0 + c), AK (c0 + c) + AK - 1], key lane = position % AK.  The committed window
// [lo, L - 1] is laid out that way; so are a chain pass's own rows (row r at position L + r).
// A tree pass's own rows (positions repeat across siblings) follow in chunks of their own, by
// row index.  With keys placed by position, a row's chunk partials and their merge order depend
// only on the row's position, not on the other rows of the pass: a chain verify row computes
// bit for bit what a one-row pass at its position computes.
struct ChunkGeom {
    int64_t lo, hi;  // positions placed by position: [lo, hi]
    int64_t c0;      // absolute index of the first chunk
    int n_abs, nch;  // chunks placed by position; all chunks
};

__host__ __device__ inline ChunkGeom chunk_geom(int window, int64_t L, int M, bool chain) {
    ChunkGeom g;
    g.lo = window > 0 ? (L - window + 1 > 0 ? L - window + 1 : 0) : 0;
    g.hi = chain ? L + M - 1 : L - 1;
    g.c0 = g.lo / AK;
    g.n_abs = g.hi >= g.lo ? (int)(g.hi / AK - g.c0 + 1) : 0;
    g.nch = g.n_abs + (chain ? 0 : (M + AK - 1) / AK);
    return g;
}

int attn_max_chunks(int window, int64_t L_max, int M) {
    // position-aligned chunks: one more than the keys span, one for a tree's own rows
    const int64_t keys = (window > 0 ? (int64_t)window - 1 : L_max) + M;
    return (int)((keys + AK - 1) / AK) + 2;
}

// DPP lane moves (no LDS round trip): quad_perm [1,0,3,2] (xor 1) 0xB1, [2,3,0,1] (xor 2)
// 0x4E; row_half_mirror 0x141, row_mirror 0x140; row_ror:n 0x120 + n (lane i of a row of 16
// takes lane i - n mod 16)
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_xor1(float v) { return dpp<0xB1>(v); }
__device__ __forceinline__ float quad_xor2(float v) { return dpp<0x4E>(v); }
// sum over each row of 16 lanes, every lane of the row gets it (the same bits in every lane:
// each step adds the same two values in either order)
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    return v;
}
// sum over each group of 8 lanes (the same bits in every lane of the group)
__device__ __forceinline__ float lane8_sum(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    return v;
}
// max / sum over lanes i, i ^ 16, i ^ 32, i ^ 48 (v_permlane16_swap: rows 2k + 1 of the first
// operand trade places with rows 2k of the second; v_permlane32_swap: the upper half of the
// first with the lower half of the second; with both operands v each returns the (lower,
// upper) pair of values, so every lane combines them in the same order)
__device__ __forceinline__ float xrow_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xrow_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
// lane i ^ X of a row of 16, X in {2, 4, 8}
template <int X>
__device__ __forceinline__ float row16_xor(float v, int lane) {
    static_assert(X == 2 || X == 4 || X == 8, "lane distance");
    if constexpr (X == 2) return dpp<0x4E>(v);
    if constexpr (X == 8) return dpp<0x128>(v);
    const float up = dpp<0x12C>(v), dn = dpp<0x124>(v);  // lanes i + 4, i - 4
    return (lane & 4) ? dn : up;
}

__device__ __forceinline__ void unpack8(const u4v v, float x[8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        x[2 * j] = h2f(v[j] & 0xFFFFu);
        x[2 * j + 1] = h2f(v[j] >> 16);
    }
}
__device__ __forceinline__ u4v pack8(const float x[8]) {
    u4v o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = (uint32_t)f2h(x[2 * j]) | ((uint32_t)f2h(x[2 * j + 1]) << 16);
    return o;
}

// RoPE of 8 dims d0 .. d0 + 7 (d0 a multiple of 8: the run lies on one side of half and of
// 2 half): dims below half take v cos - u sin, dims in [half, 2 half) v cos + u sin (u the
// partner dim d +/- half, angles cs[i]), later dims pass through (cos 1, sin 0).  Branch-free.
template <int HALF>
__device__ __forceinline__ void rope8(float v[8], const float u[8], const float2* cs, int d0) {
    const bool rot = d0 < 2 * HALF;
    const float sg = d0 < HALF ? -1.0f : 1.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float2 c = cs[i];
        const float cx = rot ? c.x : 1.0f, sy = rot ? sg * c.y : 0.0f;
        v[i] = v[i] * cx + u[i] * sy;
    }
}
// first angle of dims d0 .. (frequency d0 or d0 - half; 0 past 2 half, where nothing is read)
template <int HALF>
__device__ __forceinline__ int rope_f0(int d0) {
    return d0 < 2 * HALF ? (d0 < HALF ? d0 : d0 - HALF) : 0;
}

// Work of one block (kv head g, chunk c), 256 threads:
//   loads, every one issued before the first wait (all unconditional, at clamped addresses):
//     K: key t / 4, dims 32 (t % 4) ..      (the layout the own-key norm reduces over)
//     V: keys 4 (t % 16) .. + 3, dims 8 (t / 16) ..   (transposed in registers, 8-byte LDS rows)
//     Q: parts of 8 dims, four per thread (one round up to 16 rows)
//     the pass's RoPE table rows, staged in LDS once for the block's queries and own keys
//   barrier; q and the own keys finished (RMSNorm, RoPE) into LDS, own K / V appended; barrier
//   S^T = K Q^T on MFMA (A = 16 keys, B = 16 query vectors): lane (n, q) holds query vector n
//   against keys 16 kt + 4 q + r, so a query's mask, max and sum stay in its lane (plus two
//   cross-lane steps) and its probabilities are already the A operand of the PV product: that
//   product's k-slot 8 q + u takes key 32 j + 4 q + u (u < 4) or 32 j + 16 + 4 q + u - 4.
//   Scores are kept in log2 units (scale * log2 e), so p = exp2(s - m); the partial max is
//   stored in the same units.
#define LOG2E 1.44269504088896341f
// LDS of the RoPE table: M * half angles rounded up to whole 64-lane staging rounds
__host__ __device__ inline int tab_floats2(int M, int half) {
    return ((M * half / 2 + 63) / 64) * 64 * 2;
}
// HALF: rope_dim / 2 (0: no RoPE).  JR: finishing jobs (8 a vector) a thread requests before the
// first barrier; jobs past 256 JR go in further rounds, each a dependent load round trip, so
// passes with more vectors (a 17-row tree: 680 jobs) take JR = 3 and one round.
// NT: threads of a block, 256 or 512.  The K / V staging takes threads 0 .. 255; a pass of more
// than four query tiles (a 17-row tree: five) runs 512 threads, so that no wave takes two tiles
// and the finishing jobs spread over twice the threads.
template <int HALF, int JR, int NT>
__global__ __launch_bounds__(NT) void k_attn_chunk(AttnArgs a) {
    static_assert(NT == 256 || NT == 512, "block size");
    constexpr int NW = NT / 64;  // waves
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const bool kvt = NT == 256 || t < 256;  // stages K / V (wave-uniform)
    const int tk = t & 255;
    const int g = blockIdx.x / a.max_chunks, c = blockIdx.x % a.max_chunks;
    const StepDesc* sd = a.sd;
    const int64_t L = sd->L;
    const int M = a.M;
    const int gqa = a.nQ / a.nKV;
    const int nqv = M * gqa, nqt = (nqv + 15) / 16;
    const int qkvN = (a.nQ + 2 * a.nKV) * HD;
    constexpr int half = HALF;
    const ChunkGeom cg = chunk_geom(a.window, L, M, sd->chain != 0);
    // ring slot of position p (p - L is within the cache: |p - L| < C)
    const int64_t Lm = L % a.C;
    auto slot_of = [&](int64_t p) -> int64_t {
        int64_t sl = Lm + (p - L);
        sl += sl < 0 ? a.C : 0;
        sl -= sl >= a.C ? a.C : 0;
        return sl;
    };
    if (c >= cg.nch) return;  // whole block
    const bool by_pos = c < cg.n_abs;
    const int64_t cpos = (cg.c0 + c) * AK;  // position of key lane 0 (chunks placed by position)
    // key lane k of this chunk: -2 none, -1 committed (at position p), else own row (its
    // index; its position is L + depth[row])
    auto key_of = [&](int k, int64_t& p) -> int {
        if (by_pos) {
            p = cpos + k;
            if (p < cg.lo || p > cg.hi) return -2;
            return p < L ? -1 : (int)(p - L);
        }
        p = 0;
        const int ar = (c - cg.n_abs) * AK + k;
        return ar < M ? ar : -2;
    };
    // the pass's own rows fall in this block's chunk
    const bool own_chunk = by_pos ? cpos + AK - 1 >= L && cpos <= cg.hi : true;

    extern __shared__ uint16_t lds[];
    uint16_t* Qs = lds;                          // [nqt*16][QSTR]
    uint16_t* Ks = Qs + nqt * 16 * QSTR;         // [AK][QSTR]
    uint16_t* Vt = Ks + AK * QSTR;               // [HD][VSTR]
    float2* tab = (float2*)(Vt + HD * VSTR);     // [M][half] RoPE angles of the pass's rows
    int* kmeta = (int*)(tab + tab_floats2(M, half));  // [AK] key: (p - L) * 128 + (class + 2)
    int* rlo = kmeta + AK;                       // [MJ_ROWS] window start of a row, - L
    uint64_t* ranc = (uint64_t*)(rlo + MJ_ROWS);  // [MJ_ROWS] ancestor masks
    uint16_t* qnw_s = (uint16_t*)(ranc + MJ_ROWS);  // [HD] q norm weights
    uint16_t* knw_s = qnw_s + HD;                  // [HD] k norm weights
    int* s_abort = (int*)(knw_s + HD);

    // ---- K: key kk = tk / 4, dims 32 dq ..
    const int kk = tk >> 2, dq = tk & 3;
    int64_t kp;
    const int kcls = key_of(kk, kp);
    const bool kvalid = kcls != -2;
    const bool kown = kcls >= 0;
    const int ar = kown ? kcls : 0;  // pass row of an own key
    u4v kv[4];
    if (kvt) {
        const int64_t slot = kvalid && !kown ? slot_of(kp) : 0;
        const uint16_t* ks = kown ? a.qkv + (size_t)ar * qkvN + (a.nQ + g) * HD + 32 * dq
                                  : a.kc + ((size_t)g * a.C + slot) * HD + 32 * dq;
#pragma unroll
        for (int q = 0; q < 4; ++q) kv[q] = *(const u4v*)(ks + 8 * q);
    }
    // ---- V: keys 4 vg .. 4 vg + 3, dims 8 vd ..
    const int vg = tk & 15, vd = tk >> 4;
    u4v vv[4];
    int vcls[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int64_t p;
        vcls[j] = key_of(4 * vg + j, p);
        const int64_t slot = vcls[j] == -1 ? slot_of(p) : 0;
        const uint16_t* vs =
            vcls[j] >= 0 ? a.qkv + (size_t)vcls[j] * qkvN + (a.nQ + a.nKV + g) * HD + 8 * vd
                         : a.vc + ((size_t)g * a.C + slot) * HD + 8 * vd;
        if (kvt) vv[j] = *(const u4v*)vs;
    }
    // ---- vectors to finish (RMSNorm + RoPE): the block's queries (vector qv = r * gqa + j is
    // head g * gqa + j of row r) and the pass's own keys in this chunk (lanes ko0 .. ko1 - 1).
    // Job jb of a vector holds its parts pa and pa + X (8 dims each; X = half / 8 parts apart,
    // so a rotated pair of dims sits in one thread), 8 jobs a vector in 8 consecutive threads.
    constexpr int X = HALF >= 16 ? HALF / 8 : 8;
    int ko0 = 0, ko1 = 0;
    if (own_chunk) {
        ko0 = by_pos ? (int)(L - cpos > 0 ? L - cpos : 0) : 0;
        ko1 = by_pos ? (int)(cg.hi - cpos + 1 < AK ? cg.hi - cpos + 1 : AK)
                     : (M - (c - cg.n_abs) * AK < AK ? M - (c - cg.n_abs) * AK : AK);
    }
    const int njobs = 8 * (nqv + ko1 - ko0);
    u4v jxa[JR], jxb[JR];
    auto job_src = [&](int j, int& pa) -> const uint16_t* {
        const int vi = j >> 3, jb = j & 7;
        pa = (jb & (X - 1)) | ((jb & ~(X - 1)) << 1);
        if (vi < nqv)
            return a.qkv + (size_t)(vi / gqa) * qkvN + (g * gqa + vi % gqa) * HD;
        int64_t p;
        const int r2 = key_of(ko0 + vi - nqv, p);
        return a.qkv + (size_t)(r2 >= 0 ? r2 : 0) * qkvN + (a.nQ + g) * HD;
    };
#pragma unroll
    for (int jj = 0; jj < JR; ++jj) {
        const int j = t + NT * jj;
        int pa;
        const uint16_t* src = job_src(j < njobs ? j : njobs - 1, pa);
        jxa[jj] = *(const u4v*)(src + 8 * pa);
        jxb[jj] = *(const u4v*)(src + 8 * (pa + X));
    }
    // the norm weights into LDS (16 lanes each of wave 0)
    if (wv == 0 && lane < HD / 8) {
        __builtin_amdgcn_global_load_lds(a.q_norm_w + 8 * lane,
                                         (__attribute__((address_space(3))) void*)qnw_s, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(a.k_norm_w + 8 * lane,
                                         (__attribute__((address_space(3))) void*)knw_s, 16, 0, 0);
    }
    // ---- RoPE table rows (float4 = two angles), key and row metadata
    // the table goes straight into LDS (16 bytes a lane): pairs 2e, 2e + 1 of the [M][half]
    // angles, wave w taking pairs 64 w + lane, 64 (w + 4) + lane, ...
    const int ntab4 = M * half / 2, hd = half > 0 ? half : 1;
    for (int e0 = 64 * wv; e0 < ntab4; e0 += NT) {
        const int e = e0 + lane;
        if (e < ntab4)
            __builtin_amdgcn_global_load_lds(a.rope_cs + (2 * e / hd) * MJ_ROPE_F + 2 * e % hd,
                                             (__attribute__((address_space(3))) void*)(tab + 2 * e0),
                                             16, 0, 0);
    }
    int64_t mpos;
    const int mcls = key_of(t & (AK - 1), mpos);  // -2 invalid, -1 committed, >= 0 own row
    const int rdep = sd->depth[t < M ? t : M - 1];
    const uint64_t ranc_t = sd->anc[t < M ? t : M - 1];
    const int abort_v = a.abort ? *a.abort : 0;  // thread 0's copy decides for the block

    // ---- LDS: K rows (own keys raw for now), V^T, the table, metadata; the padding query
    // rows of the last tile (read by the MFMAs, masked after) are cleared
    for (int i = nqv * 16 + t; i < nqt * 16 * 16; i += NT)
        *(u4v*)(Qs + (i >> 4) * QSTR + 8 * (i & 15)) = (u4v){0u, 0u, 0u, 0u};
    if (kvt) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *(u4v*)(Ks + kk * QSTR + 32 * dq + 8 * q) = kvalid ? kv[q] : (u4v){0u, 0u, 0u, 0u};
        u4v w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = vcls[j] != -2 ? vv[j] : (u4v){0u, 0u, 0u, 0u};
        // dim 8 vd + i of keys 4 vg .. + 3: halves i of the four key vectors
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int sh = 16 * (i & 1);
            const uint32_t a0 = (w[0][i >> 1] >> sh) & 0xFFFFu, a1 = (w[1][i >> 1] >> sh) & 0xFFFFu;
            const uint32_t a2 = (w[2][i >> 1] >> sh) & 0xFFFFu, a3 = (w[3][i >> 1] >> sh) & 0xFFFFu;
            *(uint2*)(Vt + (8 * vd + i) * VSTR + 4 * vg) = make_uint2(a0 | (a1 << 16), a2 | (a3 << 16));
        }
    }
    if (t < AK) {
        // position - L: p - L in chunks placed by position, depth[row] for a tree's own rows
        const int64_t rel = by_pos ? mpos - L : (int64_t)sd->depth[mcls >= 0 ? mcls : 0];
        kmeta[t] = mcls == -2 ? (int)0x80000000 : (int)rel * 128 + (mcls + 2);
    }
    if (t < M) {
        rlo[t] = a.window > 0 ? rdep - a.window + 1 : INT32_MIN / 2;
        ranc[t] = ranc_t;
    }
    if (t == 0) *s_abort = abort_v;
    __syncthreads();
    if (*s_abort) return;  // block-uniform

    // ---- finish the vectors: RMSNorm over the vector's 8 jobs, RoPE of dims d < half against
    // d + half (maple_qk_norm_rope); queries into Qs, own keys into Ks and appended at slot
    // (L + r) % C with their V rows (maple_write_kv_pair).  No other block of this launch
    // reads those slots (the committed window never reaches them).
    for (int j0 = 0; j0 < njobs; j0 += NT * JR) {
#pragma unroll
        for (int jj = 0; jj < JR; ++jj) {
            const int j = j0 + t + NT * jj;
            if (j0 > 0) {
                int pa;
                const uint16_t* src = job_src(j < njobs ? j : njobs - 1, pa);
                jxa[jj] = *(const u4v*)(src + 8 * pa);
                jxb[jj] = *(const u4v*)(src + 8 * (pa + X));
            }
            const int vi = j >> 3, jb = j & 7;
            const int pa = (jb & (X - 1)) | ((jb & ~(X - 1)) << 1), pb = pa + X;
            const bool isq = vi < nqv;
            int64_t kpos2;
            const int kl = ko0 + vi - nqv;  // own key lane
            const int kr2 = isq ? 0 : key_of(kl & (AK - 1), kpos2);
            const int row = isq ? (vi < nqv ? vi / gqa : 0) : (kr2 >= 0 ? kr2 : 0);
            float xa[8], xb[8], wa[8], wb[8];
            unpack8(jxa[jj], xa);
            unpack8(jxb[jj], xb);
            const uint16_t* nw = isq ? qnw_s : knw_s;
            unpack8(*(const u4v*)(nw + 8 * pa), wa);
            unpack8(*(const u4v*)(nw + 8 * pb), wb);
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) ss += xa[i] * xa[i];
#pragma unroll
            for (int i = 0; i < 8; ++i) ss += xb[i] * xb[i];
            ss = lane8_sum(ss);
            const float scl = 1.0f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                xa[i] = xa[i] * scl * wa[i];
                xb[i] = xb[i] * scl * wb[i];
            }
            if constexpr (HALF > 0) {
                // dims 8 pa + i < half pair with 8 pa + i + half = 8 pb + i
                const bool rot = 8 * pa < half;
                const float2* cs = tab + row * half + (rot ? 8 * pa : 0);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float2 c2 = cs[i];
                    const float cx = rot ? c2.x : 1.0f, sy = rot ? c2.y : 0.0f;
                    const float ra = xa[i] * cx - xb[i] * sy, rb = xb[i] * cx + xa[i] * sy;
                    xa[i] = ra;
                    xb[i] = rb;
                }
            }
            const u4v oa = pack8(xa), ob = pack8(xb);
            if (j < njobs) {
                if (isq) {
                    *(u4v*)(Qs + vi * QSTR + 8 * pa) = oa;
                    *(u4v*)(Qs + vi * QSTR + 8 * pb) = ob;
                } else {
                    *(u4v*)(Ks + kl * QSTR + 8 * pa) = oa;
                    *(u4v*)(Ks + kl * QSTR + 8 * pb) = ob;
                    const size_t dst = ((size_t)g * a.C + slot_of(L + kr2)) * HD;
                    *(u4v*)(a.kc + dst + 8 * pa) = oa;
                    *(u4v*)(a.kc + dst + 8 * pb) = ob;
                }
            }
        }
    }
    if (own_chunk && kvt) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (vcls[j] >= 0)
                *(u4v*)(a.vc + ((size_t)g * a.C + slot_of(L + vcls[j])) * HD + 8 * vd) = vv[j];
    }
    // LDS-only barrier: the K / V appends above are read by later launches, not by this block
    // (it holds the finished keys in LDS), so they complete behind the attention work instead of
    // before it (__syncthreads would wait for the stores too)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    const float sc2 = a.scale * LOG2E;
    const int ln = lane & 15, lq = lane >> 4;
    const int iters = (nqt + NW - 1) / NW;
    for (int it = 0; it < iters; ++it) {
        const int qt = wv + NW * it;
        if (qt >= nqt) break;  // wave-uniform; no block barrier follows
        // S^T tiles: keys 16 kt + 4 lq + r against query vector 16 qt + ln
        u4v qb[4];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) qb[s4] = *(const u4v*)(Qs + (qt * 16 + ln) * QSTR + 32 * s4 + 8 * lq);
        f4 S[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            S[kt] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const u4v av = *(const u4v*)(Ks + (16 * kt + ln) * QSTR + 32 * s4 + 8 * lq);
                S[kt] = mfma16x16x32(as_h8(av), as_h8(qb[s4]), S[kt]);
            }
        }
        const int qv = qt * 16 + ln;
        const int row = qv < nqv ? qv / gqa : 0;
        const int lo_r = rlo[row];
        const uint64_t anc = ranc[row];
        float m = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            const int4 km = *(const int4*)(kmeta + 16 * kt + 4 * lq);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int e = r == 0 ? km.x : r == 1 ? km.y : r == 2 ? km.z : km.w;
                const int cls = (e & 127) - 2;  // -2 invalid, -1 committed, >= 0 own row
                const bool ok = (qv < nqv) & (e != (int)0x80000000) & ((e >> 7) >= lo_r) &
                                ((cls < 0) | (((anc >> (cls & 63)) & 1ull) != 0));
                const float sv = ok ? S[kt][r] * sc2 : -INFINITY;
                S[kt][r] = sv;
                m = fmaxf(m, sv);
            }
        }
        m = xrow_max(m);
        float l = 0.0f;
        u4v pa[2];  // A operands of the two PV products (fp16 pairs)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            float p[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                p[r] = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(S[kt][r] - m);
                l += p[r];
            }
            pa[kt >> 1][2 * (kt & 1)] = (uint32_t)f2h(p[0]) | ((uint32_t)f2h(p[1]) << 16);
            pa[kt >> 1][2 * (kt & 1) + 1] = (uint32_t)f2h(p[2]) | ((uint32_t)f2h(p[3]) << 16);
        }
        l = xrow_sum(l);
        // O = P V: B lane (d, lq) = V^T[d][32 j + 4 lq .. + 3] and [32 j + 16 + 4 lq .. + 3]
        f4 O[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) O[dt] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
                const uint16_t* vr = Vt + (16 * dt + ln) * VSTR + 32 * j + 4 * lq;
                const uint2 lo4 = *(const uint2*)vr, hi4 = *(const uint2*)(vr + 16);
                const u4v bv = {lo4.x, lo4.y, hi4.x, hi4.y};
                O[dt] = mfma16x16x32(as_h8(pa[j]), as_h8(bv), O[dt]);
            }
        }
        // lane (d, lq) holds O of query vectors 16 qt + 4 lq + r, dim 16 dt + ln
        const size_t pbase = ((size_t)g * a.max_chunks + c) * (size_t)(nqt * 16);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float* op = a.opart + (pbase + qt * 16 + 4 * lq + r) * HD;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) op[16 * dt + ln] = O[dt][r];
        }
        if (lq == 0) a.mlpart[pbase + qv] = make_float2(m, l);
    }
}

// One 256-thread block per (row, query head): wave w merges, in increasing order, the chunks
// whose absolute index is w mod 4 (lane = two dims), then the four wave sums are added in wave
// order and the row is written in qx order.  Every chunk of the pass holds a partial (a fully
// masked one has max -inf, sum 0, output 0 and adds exact zeros), so a row's merge depends only
// on the chunks that hold its keys.
__global__ __launch_bounds__(256) void k_attn_combine(AttnArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = blockIdx.x / a.nQ, hq = blockIdx.x % a.nQ;
    const int gqa = a.nQ / a.nKV;
    const int g = hq / gqa, qv = r * gqa + (hq % gqa);
    const size_t nq16 = (size_t)((a.M * gqa + 15) / 16) * 16;
    const ChunkGeom cg = chunk_geom(a.window, a.sd->L, a.M, a.sd->chain != 0);
    const int nch = cg.nch;
    const int cs = (int)(((int64_t)wv - cg.c0) & 3);  // this wave's first chunk
    const float2* ml = a.mlpart + (size_t)g * a.max_chunks * nq16 + qv;
    const float* op = a.opart + ((size_t)g * a.max_chunks * nq16 + qv) * HD + 2 * lane;
    // this wave's chunks cb + 4j, j < 4, requested at clamped indices (every lane loads; chunks
    // past the end are skipped below); two rounds (32 chunks) at once
    float2 m4[2][4], p4[2][4];
    const int clast = nch > 0 ? nch - 1 : 0;
    auto request = [&](int cb, float2* mm, float2* pp) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = min(cb + 4 * j, clast);
            mm[j] = ml[(size_t)c * nq16];
            pp[j] = *(const float2*)(op + (size_t)c * nq16 * HD);
        }
    };
    // the first two rounds, together with the chunk maxima (they do not need them)
    request(cs, m4[0], p4[0]);
    request(cs + 16, m4[1], p4[1]);
    // the maximum over the chunks (clamped indices: a repeated chunk leaves it unchanged)
    float mx = ml[(size_t)min(lane, clast) * nq16].x;
    for (int c = lane + 64; c < nch; c += 64) mx = fmaxf(mx, ml[(size_t)c * nq16].x);
    mx = wave_max(mx);
    float o0 = 0.0f, o1 = 0.0f, ls = 0.0f;
    for (int cb = cs, rd = 0; cb < nch; cb += 16, ++rd) {
        if (rd >= 2) request(cb, m4[0], p4[0]);
        const float2* mm = rd == 1 ? m4[1] : m4[0];
        const float2* pp = rd == 1 ? p4[1] : p4[0];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (cb + 4 * j >= nch) break;
            // log2 units
            const float w = mm[j].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mm[j].x - mx);
            ls += mm[j].y * w;
            o0 += w * pp[j].x;
            o1 += w * pp[j].y;
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
    // RoPE partners are found by lane moves: half = rope_dim / 2 in {16, 32, 64}
    if (a.rope_dim != 0 && a.rope_dim != 32 && a.rope_dim != 64 && a.rope_dim != 128)
        return hipErrorInvalidValue;
    // key positions relative to L are packed as (p - L) * 128 + class in an int
    if (a.C < 1 || a.C >= ((int64_t)1 << 23)) return hipErrorInvalidValue;
    const int gqa = a.nQ / a.nKV;
    const int nqt = (a.M * gqa + 15) / 16;
    const size_t lds = (size_t)(nqt * 16 * QSTR + AK * QSTR + HD * VSTR) * 2 +
                       (size_t)tab_floats2(a.M, a.rope_dim / 2) * 8 + AK * 4 + MJ_ROWS * (4 + 8) +
                       2 * HD * 2 + 16;
    // finishing jobs of the block that also holds the pass's own keys; more than four query
    // tiles take 512-thread blocks (two jobs a thread then cover up to 1024)
    const int jobs = 8 * (a.M * gqa + (a.M < AK ? a.M : AK));
    const bool wide = nqt > 4;
    const bool jr3 = jobs > 256 * 2;
    auto go = [&](auto k2, auto k3, auto w2) {
        const dim3 grid(a.nKV * a.max_chunks);
        if (wide)
            launch_timed(w2, grid, dim3(512), lds, st, a);
        else
            launch_timed(jr3 ? k3 : k2, grid, dim3(256), lds, st, a);
    };
    switch (a.rope_dim) {
        case 0: go(k_attn_chunk<0, 2, 256>, k_attn_chunk<0, 3, 256>, k_attn_chunk<0, 2, 512>); break;
        case 32: go(k_attn_chunk<16, 2, 256>, k_attn_chunk<16, 3, 256>, k_attn_chunk<16, 2, 512>); break;
        case 64: go(k_attn_chunk<32, 2, 256>, k_attn_chunk<32, 3, 256>, k_attn_chunk<32, 2, 512>); break;
        default: go(k_attn_chunk<64, 2, 256>, k_attn_chunk<64, 3, 256>, k_attn_chunk<64, 2, 512>); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_combine, dim3(a.M * a.nQ), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t set_attn_attributes() {
    hipError_t e = hipSuccess;
    const void* ks[] = {(const void*)k_attn_chunk<0, 2, 256>,  (const void*)k_attn_chunk<16, 2, 256>,
                        (const void*)k_attn_chunk<32, 2, 256>, (const void*)k_attn_chunk<64, 2, 256>,
                        (const void*)k_attn_chunk<0, 3, 256>,  (const void*)k_attn_chunk<16, 3, 256>,
                        (const void*)k_attn_chunk<32, 3, 256>, (const void*)k_attn_chunk<64, 3, 256>,
                        (const void*)k_attn_chunk<0, 2, 512>,  (const void*)k_attn_chunk<16, 2, 512>,
                        (const void*)k_attn_chunk<32, 2, 512>, (const void*)k_attn_chunk<64, 2, 512>};
    for (const void* k : ks)
        if (e == hipSuccess)
            e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    return e;
}
