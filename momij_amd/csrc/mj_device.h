// mj_device.h -- device helpers shared by the gfx950 kernels.
//
// 2-bit code expansion.  A uint32 word of the MLX layout holds codes c0..c15 (code i in bits
// [2i, 2i+1]).  unpack16() turns it into eight fp16 pairs without a per-code shift:
//     v[i] = (base_i + c_i, base_i + c_{i+8}),  base_i = 256, 64, 16, 4 for i % 4 = 0, 1, 2, 3,
// by masking two code positions straight into the fp16 mantissa of a constant whose ulp makes
// them count 1: 0x5C00 = 256.0 (code in mantissa bits 2-3), 0x5400 = 64.0 (bits 4-5), 0x4C00 =
// 16.0 (bits 6-7) and 0x4400 = 4.0 (bits 8-9).  Two shifted copies of the word (w << 2: codes
// 0-3 and 8-11; w >> 6: codes 4-7 and 12-15) cover all 16 codes: 10 VALU ops per 16 weights.
// The constant part is removed exactly after the dot product: sum_k (base_k + c_k) x_k -
// sum_k base_k x_k, with Bx = sum_k base_k x_k precomputed once per 64-element block of x.  The
// bases stay small enough (the fp32 partial sums within ~200x of the result) that the
// subtraction costs < 1e-4 relative.
//
// Activations feeding a 2-bit product are stored "permuted": inside each 16-element block
// the order is x0 x8 x1 x9 x2 x10 x3 x11 x4 x12 x5 x13 x6 x14 x7 x15, i.e. fp16 pair i is
// (x_i, x_{i+8}) and lines up with v[i].  Each 64-block also carries float2 {X, Bx} =
// {sum x, sum base*x}.  Together this is the "qx" activation format.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mj_internal.h"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

#define MJ_WAVE 64

__device__ __forceinline__ float h2f(uint16_t v) { return (float)__builtin_bit_cast(_Float16, v); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float hround(float f) { return (float)(_Float16)f; }

__device__ __forceinline__ void unpack16(uint32_t w, uint32_t v[8]) {
    const uint32_t s1 = w << 2, s2 = w >> 6;
    v[0] = (s1 & 0x000C000Cu) | 0x5C005C00u;
    v[1] = (s1 & 0x00300030u) | 0x54005400u;
    v[2] = (s1 & 0x00C000C0u) | 0x4C004C00u;
    v[3] = (s1 & 0x03000300u) | 0x44004400u;
    v[4] = (s2 & 0x000C000Cu) | 0x5C005C00u;
    v[5] = (s2 & 0x00300030u) | 0x54005400u;
    v[6] = (s2 & 0x00C000C0u) | 0x4C004C00u;
    v[7] = (s2 & 0x03000300u) | 0x44004400u;
}

// unpack16 with its masks and magic constants held in VGPRs (an AND-OR with a VGPR constant
// is one v_and_or_b32; with inline literals it is two instructions on this target).
struct UnpackK {
    uint32_t m[4], c[4];
};
__device__ __forceinline__ void unpack16k(uint32_t w, uint32_t v[8], const UnpackK& k) {
    const uint32_t s1 = w << 2, s2 = w >> 6;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = (s1 & k.m[i]) | k.c[i];
        v[i + 4] = (s2 & k.m[i]) | k.c[i];
    }
}

// base of qx pair i (i = 0..7 inside its 16-element block), as a float and as an fp16 pair
__device__ __forceinline__ float code_base(int i) { return (float)(256 >> (2 * (i & 3))); }
__device__ __forceinline__ uint32_t code_base2(int i) {
    constexpr uint32_t b2[4] = {0x5C005C00u, 0x54005400u, 0x4C004C00u, 0x44004400u};
    return b2[i & 3];
}
// bases of the plain pair (x_{2j}, x_{2j+1}) of an 8-aligned run of a row: (256, 64) for even
// j, (16, 4) for odd j
__device__ __forceinline__ uint32_t plain_base2(int j) { return (j & 1) ? 0x44004C00u : 0x54005C00u; }

// Value the optimiser cannot see through: keeps loop-invariant code expansion from being
// hoisted out of a loop (and held live across it) when registers are the scarce resource.
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}

// Pins a float at this point of the program: computations feeding it cannot be sunk past it
// (keeps unrolled accumulation chains from being deferred until every operand is live).
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }

// A wave-uniform value held in an SGPR the optimiser cannot see through.
__device__ __forceinline__ uint32_t opaque_s(uint32_t x) {
    asm volatile("" : "+s"(x));
    return x;
}

// the masks (SGPRs) and constants (VGPRs) of unpack16k: a v_and_or_b32 may read one SGPR, so
// each AND-OR stays one instruction while only the four constants take vector registers
__device__ __forceinline__ UnpackK unpack_consts() {
    return UnpackK{{opaque_s(0x000C000Cu), opaque_s(0x00300030u), opaque_s(0x00C000C0u),
                    opaque_s(0x03000300u)},
                   {opaque(0x5C005C00u), opaque(0x54005400u), opaque(0x4C004C00u), opaque(0x44004400u)}};
}

// fp16 pair (lo, hi) from two raw fp16 bit patterns
__device__ __forceinline__ uint32_t pack2(uint32_t lo16, uint32_t hi16) {
    return (lo16 & 0xFFFFu) | (hi16 << 16);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2v, a), __builtin_bit_cast(h2v, b), c,
                                  false);
}

// Permute one 16-element block held as 8 plain pairs u[j] = (x_{2j}, x_{2j+1}) into the qx
// order p[i] = (x_i, x_{i+8}).
__device__ __forceinline__ void perm16(const uint32_t u[8], uint32_t p[8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        p[2 * j] = (u[j] & 0xFFFFu) | (u[j + 4] << 16);
        p[2 * j + 1] = (u[j] >> 16) | (u[j + 4] & 0xFFFF0000u);
    }
}

// Position of plain element i (0..15) inside a permuted 16-block.
__device__ __forceinline__ int perm_pos(int i) { return i < 8 ? 2 * i : 2 * (i - 8) + 1; }

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
    Bx = dot2(v.x, plain_base2(0), Bx);
    Bx = dot2(v.y, plain_base2(1), Bx);
    Bx = dot2(v.z, plain_base2(2), Bx);
    Bx = dot2(v.w, plain_base2(3), Bx);
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
        X += __shfl_xor(X, m, MJ_WAVE);
        Bx += __shfl_xor(Bx, m, MJ_WAVE);
    }
    if ((lane & 7) == 0) xsum_row[k0 >> 6] = make_float2(X, Bx);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, MJ_WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, MJ_WAVE));
    return v;
}

// (value, index) argmax across the wave: larger value wins, lower index on ties.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, MJ_WAVE);
        const int oi = __shfl_xor(i, o, MJ_WAVE);
        if (ov > v || (ov == v && oi < i)) {
            v = ov;
            i = oi;
        }
    }
}

// Running log-sum-exp in log2 units: (m, s) stands for s * 2^m.  (-inf, 0) is empty.
__device__ __forceinline__ void lse_merge(float& m, float& s, float om, float os) {
    const float mn = fmaxf(m, om);
    if (mn == -INFINITY) return;
    s = s * __builtin_amdgcn_exp2f(m - mn) + os * __builtin_amdgcn_exp2f(om - mn);
    m = mn;
}

__device__ __forceinline__ f4 mfma16x16x4f32(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 mfma16x16x32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h8 as_h8(u4v v) { return __builtin_bit_cast(h8, v); }

__device__ __forceinline__ bool aborted(const int* flag) { return flag != nullptr && *flag != 0; }

// ------------------------------------------------------------------------------------------
// Canonical arithmetic for sampled acceptance.  The CPU oracle evaluates the identical IEEE
// operation sequence, so both produce the same bits: exp by Cody-Waite reduction and a
// degree-7 Taylor polynomial in fused multiply-adds, scaled by 2^n from exponent bits.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ float canon_expf(float x) {
#pragma clang fp contract(off)
    if (!(x >= -87.0f)) return 0.0f;
    const float n = __builtin_rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(-n, 0x1.62e400p-1f, x);
    r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0x1.000000p-1f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float two_n = __builtin_bit_cast(float, (uint32_t)((int)n + 127) << 23);
    return p * two_n;
}

// Philox4x32-10 (Salmon et al., SC'11).
__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
        c[1] = (uint32_t)p1;
        c[3] = (uint32_t)p0;
        c[0] = n0;
        c[2] = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

__device__ __forceinline__ float u01(uint32_t x) { return (float)(x >> 8) * 0x1p-24f; }

// RMSNorm of one 2048-element row held by a 256-thread block (thread t: elements 8t .. 8t+7,
// packed fp16 in hv), as k_rmsnorm_qx: out = half(x * (1 / sqrt(mean x^2 + eps)) * w), written
// plain and / or in qx order with its block sums (NormOut).  Every thread of the block must
// call it.
// RMSNorm of a 2048-wide row held as 8 halves a thread (256 threads), weights wv of this
// thread's 8 dims already loaded; writes the plain and / or qx-ordered output
__device__ __forceinline__ void norm_row_2048_w(const u4v hv, const u4v wv, const NormOut& no,
                                                int row) {
    const int t = threadIdx.x, lane = t & 63;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float a = h2f(hv[j] & 0xFFFFu), b = h2f(hv[j] >> 16);
        ss += a * a;
        ss += b * b;
    }
    ss = wave_sum(ss);
    __shared__ float red[4];
    if (lane == 0) red[t >> 6] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(tot / 2048.0f + no.eps);
    u4v o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float a = h2f(hv[j] & 0xFFFFu) * inv * h2f(wv[j] & 0xFFFFu);
        const float b = h2f(hv[j] >> 16) * inv * h2f(wv[j] >> 16);
        o[j] = (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16);
    }
    if (no.plain) *(u4v*)(no.plain + (size_t)row * 2048 + 8 * t) = o;
    if (no.xperm) emit_qx(o, lane, no.xperm + (size_t)row * 2048, no.xsum + (size_t)row * 32, 8 * t);
}
__device__ __forceinline__ void norm_row_2048(const u4v hv, const NormOut& no, int row) {
    norm_row_2048_w(hv, *(const u4v*)(no.w + 8 * threadIdx.x), no, row);
}
