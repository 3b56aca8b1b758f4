/*
 * momij_oracle.c -- CPU restatement of momij's speculative-decode verify step.
 *
 * TEST INFRASTRUCTURE ONLY (the parity reference and the timed CPU baseline).  The product library
 * libmomij_hip.so never links, loads or calls this code.  Built by oracle/Makefile with
 * -O3 -ffp-contract=off so that every a*b+c below rounds twice unless fmaf() is written.
 *
 * Citations are reference file:line under swift/Sources/MomijCore/ of penta2himajin/momij.
 * Parity of each function is pinned by tests/test_oracle_*.py (listed in momij_oracle.h).
 */
#include "momij_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* fp16 <-> fp32 (IEEE binary16, round to nearest even).                      */
/* WeightStore.swift:19-21 converts every checkpoint tensor to fp16; the      */
/* kernels read half and widen to float.                                      */
/* ------------------------------------------------------------------------- */
float or_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    float f;
    if (e == 0) {
        f = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);      /* NaN */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);     /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                       /* < 2^-14: subnormal */
        float v;
        memcpy(&v, &ax, 4);
        float s = v * 16777216.0f;                                /* exact: * 2^24 */
        uint32_t r = (uint32_t)nearbyintf(s);                     /* RNE */
        return (uint16_t)(sign | r);
    }
    uint32_t e = (ax >> 23) - 112u, m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13), rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

void or_h2f_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = or_h2f(in[i]);
}
void or_f2h_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = or_f2h(in[i]);
}

static inline float hround(float v) { return or_h2f(or_f2h(v)); }

/* ------------------------------------------------------------------------- */
/* a2: gqmm2_rows -- SeedlessMetal.swift:2145-2221.                           */
/*   y[mk, n] = half( sum_k (s[e,n,k/gs] * q[e,n,k] + b[e,n,k/gs]) * x[row, k] )  */
/*   e = inds[mk], row = lhs_per_expert ? mk : mk / ktop.                       */
/* The reference splits K into 512-wide blocks; simd lane l owns the 16        */
/* values [blk + 16 l, blk + 16 l + 16) and adds s*sum(q*x) + b*sum(x) per     */
/* chunk (qd2, 2157-2165), where sum(x) is built from half-precision 4-sums    */
/* (ld16_b2, 2145-2156: `x[i] + x[i+1] + ...` on half operands).  Per-lane     */
/* partials accumulate over blocks, then simd_sum (2217-2220).  Code k of row  */
/* n sits in bits [2(k%16), 2(k%16)+1] of uint32 word k/16 (LSB first).        */
/* ------------------------------------------------------------------------- */
void or_qmm2(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
             const uint16_t* biases, const int32_t* inds, uint16_t* y,
             int M, int ktop, int K, int N, int gs, int lhs_per_expert) {
    const int Kw = K / 16, Kg = K / gs;
    const int MK = M * ktop;
    for (int mk = 0; mk < MK; ++mk) {
        const int e = inds[mk];
        const uint16_t* xr = x + (size_t)(lhs_per_expert ? mk : mk / ktop) * K;
        /* x widened once; half 4-sums per 16-chunk as the reference forms them */
        float* xf = (float*)malloc(sizeof(float) * (size_t)K);
        float* csum = (float*)malloc(sizeof(float) * (size_t)(K / 16));
        for (int k = 0; k < K; ++k) xf[k] = or_h2f(xr[k]);
        for (int c = 0; c < K / 16; ++c) {
            float s = 0.0f;
            for (int i = 0; i < 16; i += 4) {
                float t = hround(xf[16 * c + i] + xf[16 * c + i + 1]);
                t = hround(t + xf[16 * c + i + 2]);
                t = hround(t + xf[16 * c + i + 3]);
                s += t;
            }
            csum[c] = s;
        }
#pragma omp parallel for schedule(static)
        for (int n = 0; n < N; ++n) {
            const uint32_t* wr = w + ((size_t)e * N + n) * Kw;
            const uint16_t* sr = scales + ((size_t)e * N + n) * Kg;
            const uint16_t* br = biases + ((size_t)e * N + n) * Kg;
            float lane[32];
            for (int l = 0; l < 32; ++l) lane[l] = 0.0f;
            for (int blk = 0; blk < K; blk += 512) {
                for (int l = 0; l < 32; ++l) {
                    const int k0 = blk + 16 * l;
                    if (k0 >= K) continue;
                    const uint32_t word = wr[k0 / 16];
                    float acc = 0.0f;
                    for (int j = 0; j < 16; ++j) {
                        const float q = (float)((word >> (2 * j)) & 3u);
                        acc += q * xf[k0 + j];
                    }
                    const float sc = or_h2f(sr[k0 / gs]), bi = or_h2f(br[k0 / gs]);
                    lane[l] += sc * acc + csum[k0 / 16] * bi;
                }
            }
            for (int off = 16; off > 0; off >>= 1)
                for (int l = 0; l < off; ++l) lane[l] = lane[l] + lane[l + off];
            y[(size_t)mk * N + n] = or_f2h(lane[0]);
        }
        free(xf);
        free(csum);
    }
}

/* ------------------------------------------------------------------------- */
/* a3: clamped SwiGLU -- SeedlessMetal.swift:2435-2450, MapleMoE.swift:4,35-39 */
/*   up = ug[:, :I], gate = ug[:, I:]  (WeightStore.swift:81-90 up||gate)       */
/*   act = half( silu(min(gate,7)) * clamp(up,-7,7) ),  silu(g) = g/(1+exp(-g)) */
/* ------------------------------------------------------------------------- */
void or_clamped_swiglu(const uint16_t* ug, uint16_t* act, int rows, int I) {
    for (int r = 0; r < rows; ++r)
        for (int j = 0; j < I; ++j) {
            float up = or_h2f(ug[(size_t)r * 2 * I + j]);
            float gate = or_h2f(ug[(size_t)r * 2 * I + I + j]);
            gate = fminf(gate, 7.0f);
            up = fminf(fmaxf(up, -7.0f), 7.0f);
            const float silu = gate / (1.0f + expf(-gate));
            act[(size_t)r * I + j] = or_f2h(silu * up);
        }
}

/* score_reduce -- SeedlessMetal.swift:2452-2470: y = half(sum_k down_k * score_k) */
void or_score_reduce(const uint16_t* down, const float* scores, uint16_t* y,
                     int M, int ktop, int H) {
    for (int m = 0; m < M; ++m)
        for (int h = 0; h < H; ++h) {
            float acc = 0.0f;
            for (int k = 0; k < ktop; ++k)
                acc += or_h2f(down[((size_t)m * ktop + k) * H + h]) * scores[m * ktop + k];
            y[(size_t)m * H + h] = or_f2h(acc);
        }
}

/* score_resid -- SeedlessMetal.swift:2474-2493: h = half(h + half(sum_k down_k*score_k)) */
void or_score_resid(const uint16_t* down, const float* scores, uint16_t* h,
                    int M, int ktop, int H) {
    for (int m = 0; m < M; ++m)
        for (int c = 0; c < H; ++c) {
            float acc = 0.0f;
            for (int k = 0; k < ktop; ++k)
                acc += or_h2f(down[((size_t)m * ktop + k) * H + c]) * scores[m * ktop + k];
            const size_t off = (size_t)m * H + c;
            h[off] = or_f2h(or_h2f(h[off]) + hround(acc));
        }
}

/* ------------------------------------------------------------------------- */
/* a4: RMSNorm -- SeedlessMetal.swift:2496-2526 (also MapleAttention.swift:48-51):  */
/*   out = half( x * rsqrt(mean(x^2) + eps) * w ),  fp32.                      */
/* ------------------------------------------------------------------------- */
void or_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* out, int M, int H, float eps) {
    for (int m = 0; m < M; ++m) {
        const uint16_t* xm = x + (size_t)m * H;
        float part[256];
        for (int t = 0; t < 256; ++t) part[t] = 0.0f;
        for (int i = 0; i < H; ++i) {
            const float v = or_h2f(xm[i]);
            part[i % 256] += v * v;
        }
        for (int s = 128; s > 0; s >>= 1)
            for (int t = 0; t < s; ++t) part[t] += part[t + s];
        const float inv = 1.0f / sqrtf(part[0] / (float)H + eps);
        for (int i = 0; i < H; ++i)
            out[(size_t)m * H + i] = or_f2h(or_h2f(xm[i]) * inv * or_h2f(w[i]));
    }
}

/* Router logits -- SeedlessMetal.swift:2574-2595: y[m,e] = sum_k W[e,k] * x[m,k] (fp32 out) */
void or_router_logits(const uint16_t* W, const uint16_t* x, float* logits, int M, int E, int H) {
    for (int m = 0; m < M; ++m)
        for (int e = 0; e < E; ++e) {
            float lane[32];
            for (int l = 0; l < 32; ++l) lane[l] = 0.0f;
            for (int k = 0; k < H; ++k)
                lane[k % 32] += or_h2f(W[(size_t)e * H + k]) * or_h2f(x[(size_t)m * H + k]);
            for (int off = 16; off > 0; off >>= 1)
                for (int l = 0; l < off; ++l) lane[l] += lane[l + off];
            logits[(size_t)m * E + e] = lane[0];
        }
}

/* ------------------------------------------------------------------------- */
/* Route -- SeedlessMetal.swift:2720-2791 (MLX form MapleMoE.swift:41-56):     */
/*   gates = softmax(logits) (max-subtracted, exp); top-k by LOGIT, descending, */
/*   lowest index wins ties (strict > in the tree, 2771-2773);                 */
/*   scores = gates[sel] / sum_k gates[sel]  (sequential sum, 2785-2789).       */
/* ------------------------------------------------------------------------- */
void or_route_topk(const float* logits, int32_t* inds, float* scores, int M, int E, int k) {
    for (int m = 0; m < M; ++m) {
        const float* lg = logits + (size_t)m * E;
        float mx = -INFINITY;
        for (int e = 0; e < E; ++e) mx = fmaxf(mx, lg[e]);
        float* g = (float*)malloc(sizeof(float) * (size_t)E);
        float* work = (float*)malloc(sizeof(float) * (size_t)E);
        float Z = 0.0f;
        for (int e = 0; e < E; ++e) {
            g[e] = expf(lg[e] - mx);
            Z += g[e];
        }
        for (int e = 0; e < E; ++e) {
            g[e] = g[e] / Z;
            work[e] = lg[e];
        }
        for (int j = 0; j < k; ++j) {
            int bi = 0;
            for (int e = 1; e < E; ++e)
                if (work[e] > work[bi]) bi = e;
            inds[(size_t)m * k + j] = bi;
            scores[(size_t)m * k + j] = g[bi];
            work[bi] = -INFINITY;
        }
        float ss = 0.0f;
        for (int j = 0; j < k; ++j) ss += scores[(size_t)m * k + j];
        for (int j = 0; j < k; ++j) scores[(size_t)m * k + j] = scores[(size_t)m * k + j] / ss;
        free(g);
        free(work);
    }
}

/* ------------------------------------------------------------------------- */
/* MoE block -- encodeMoEBlock SeedlessMetal.swift:576-609 / MapleMoE.swift:58-80: */
/*   xn = rms(x) ; logits ; top-k ; ug = gqmm2(xn, up||gate) ; act = swiglu(ug) ; */
/*   d = gqmm2(act, down, lhsPerExpert) ; y = [x +] half(sum_k d_k * score_k).   */
/* ------------------------------------------------------------------------- */
void or_moe_block(const or_moe_w* w, const uint16_t* x, uint16_t* y, int M, int flags,
                  int32_t* out_inds, float* out_scores) {
    const int H = w->H, I = w->I, E = w->E, k = w->top_k;
    uint16_t* xin = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)M * H);
    uint16_t* xn = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)M * H);
    float* logits = (float*)malloc(sizeof(float) * (size_t)M * E);
    uint16_t* ug = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)M * k * 2 * I);
    uint16_t* act = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)M * k * I);
    uint16_t* d = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)M * k * H);
    memcpy(xin, x, sizeof(uint16_t) * (size_t)M * H);
    if (flags & OR_MOE_PRENORM)
        or_rms_norm(xin, w->norm_w, xn, M, H, w->eps);
    else
        memcpy(xn, xin, sizeof(uint16_t) * (size_t)M * H);
    or_router_logits(w->router_w, xn, logits, M, E, H);
    or_route_topk(logits, out_inds, out_scores, M, E, k);
    or_qmm2(xn, w->up_gate_w, w->up_gate_s, w->up_gate_b, out_inds, ug, M, k, H, 2 * I, w->gs, 0);
    or_clamped_swiglu(ug, act, M * k, I);
    or_qmm2(act, w->down_w, w->down_s, w->down_b, out_inds, d, M, k, I, H, w->gs, 1);
    if (flags & OR_MOE_RESIDUAL) {
        memcpy(y, xin, sizeof(uint16_t) * (size_t)M * H);
        or_score_resid(d, out_scores, y, M, k, H);
    } else {
        or_score_reduce(d, out_scores, y, M, k, H);
    }
    free(xin);
    free(xn);
    free(logits);
    free(ug);
    free(act);
    free(d);
}

/* ------------------------------------------------------------------------- */
/* a5: qk-norm + RoPE -- SeedlessMetal.swift:2794-2847, inv_freq                */
/* SeedlessAttn.swift:110-117 (base^(-i/(rope/2)) in Float).  Per head:          */
/*   v_j = x_j * rsqrt(mean(x^2)+eps) * w_j ; for j < rope_dim, non-traditional  */
/*   half-split rotation by theta = pos * inv_freq[j mod rope/2].  Output half.  */
/* Positions are per row (verify row r sits at L + depth(r)).                    */
/* ------------------------------------------------------------------------- */
void or_rope_inv_freq(float* inv_freq, int rope_dim, float base) {
    const int half = rope_dim / 2 > 0 ? rope_dim / 2 : 1;
    for (int i = 0; i < half; ++i)
        inv_freq[i] = rope_dim > 0 ? powf(base, -(float)i / (float)half) : 1.0f;
}

static void norm_rope_head(const uint16_t* xh, const uint16_t* wh, const float* inv_freq,
                           float pos, int D, int rope_dim, float eps, uint16_t* oh) {
    float ss = 0.0f;
    for (int j = 0; j < D; ++j) {
        const float v = or_h2f(xh[j]);
        ss += v * v;
    }
    const float sc = 1.0f / sqrtf(ss / (float)D + eps);
    const int half = rope_dim / 2;
    for (int j = 0; j < D; ++j) {
        float v = or_h2f(xh[j]) * sc * or_h2f(wh[j]);
        if (rope_dim > 0 && j < rope_dim) {
            const int p = j < half ? j : j - half;
            const float th = pos * inv_freq[p];
            const float c = cosf(th), s = sinf(th);
            const int j2 = j < half ? j + half : j - half;
            const float u = or_h2f(xh[j2]) * sc * or_h2f(wh[j2]);
            v = j < half ? (v * c - u * s) : (v * c + u * s);
        }
        oh[j] = or_f2h(v);
    }
}

void or_qk_norm_rope(const uint16_t* qkv, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                     const float* inv_freq, const int64_t* pos, uint16_t* q_out, uint16_t* k_out,
                     int M, int nQ, int nKV, int D, int rope_dim, float eps) {
    const int row = (nQ + 2 * nKV) * D;
    for (int m = 0; m < M; ++m) {
        const float p = (float)pos[m];
        for (int hh = 0; hh < nQ; ++hh)
            norm_rope_head(qkv + (size_t)m * row + (size_t)hh * D, q_norm_w, inv_freq, p, D,
                           rope_dim, eps, q_out + ((size_t)m * nQ + hh) * D);
        for (int g = 0; g < nKV; ++g)
            norm_rope_head(qkv + (size_t)m * row + (size_t)(nQ + g) * D, k_norm_w, inv_freq, p,
                           D, rope_dim, eps, k_out + ((size_t)m * nKV + g) * D);
    }
}

/* ------------------------------------------------------------------------- */
/* Attention -- maple_sdpa_d128 math (SeedlessMetal.swift:2919-2997: q*scale,    */
/* fp32 softmax, GQA head/gqa) with the exact sliding-window mask of the MLX    */
/* path (AttentionMasks.swift:10-27: query at absolute position P attends keys  */
/* in [P-W+1, P]) extended to a draft tree: verify row r (position L+depth(r))  */
/* attends committed positions in [P-W+1, L-1] plus its ancestors and itself.  */
/* A chain (parents[r] = r-1) reduces to the causal M-row pass                   */
/* (SeedlessDecodeEngine.swift:264-327).                                        */
/* ------------------------------------------------------------------------- */
static void tree_depths(const int32_t* parents, int M, int* depth) {
    for (int r = 0; r < M; ++r) depth[r] = (parents == NULL || parents[r] < 0) ? (parents ? 0 : r)
                                                                             : depth[parents[r]] + 1;
}

static int is_anc_or_self(const int32_t* parents, int a, int r) {
    if (parents == NULL) return a <= r;
    while (r >= 0) {
        if (r == a) return 1;
        r = parents[r];
    }
    return 0;
}

void or_attention(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache,
                  int64_t C, int64_t L, const int32_t* parents, int M, int nQ, int nKV, int D,
                  int window, uint16_t* out) {
    int* depth = (int*)malloc(sizeof(int) * (size_t)M);
    tree_depths(parents, M, depth);
    const float scale = (float)pow((double)D, -0.5);
    const int gqa = nQ / nKV;
    const int64_t maxkeys = L + M;
    float* sc = (float*)malloc(sizeof(float) * (size_t)maxkeys);
    int64_t* slot = (int64_t*)malloc(sizeof(int64_t) * (size_t)maxkeys);
    float* qf = (float*)malloc(sizeof(float) * (size_t)D);
    float* o = (float*)malloc(sizeof(float) * (size_t)D);
    for (int r = 0; r < M; ++r) {
        const int64_t P = L + depth[r];
        const int64_t lo = window > 0 ? (P - window + 1 > 0 ? P - window + 1 : 0) : 0;
        int64_t nk = 0;
        for (int64_t p = lo; p < L; ++p) slot[nk++] = p % C;
        for (int a = 0; a < M; ++a)
            if (is_anc_or_self(parents, a, r) && L + depth[a] >= lo) slot[nk++] = (L + a) % C;
        for (int hh = 0; hh < nQ; ++hh) {
            const int g = hh / gqa;
            const uint16_t* qh = q + ((size_t)r * nQ + hh) * D;
            for (int d = 0; d < D; ++d) qf[d] = scale * or_h2f(qh[d]);
            float mx = -INFINITY;
            for (int64_t i = 0; i < nk; ++i) {
                const uint16_t* kp = kcache + ((size_t)g * C + (size_t)slot[i]) * D;
                float s = 0.0f;
                for (int d = 0; d < D; ++d) s += qf[d] * or_h2f(kp[d]);
                sc[i] = s;
                mx = fmaxf(mx, s);
            }
            float Z = 0.0f;
            for (int d = 0; d < D; ++d) o[d] = 0.0f;
            for (int64_t i = 0; i < nk; ++i) {
                const float e = expf(sc[i] - mx);
                Z += e;
                const uint16_t* vp = vcache + ((size_t)g * C + (size_t)slot[i]) * D;
                for (int d = 0; d < D; ++d) o[d] += e * or_h2f(vp[d]);
            }
            for (int d = 0; d < D; ++d)
                out[(size_t)r * nQ * D + (size_t)hh * D + d] = or_f2h(Z == 0.0f ? o[d] : o[d] / Z);
        }
    }
    free(depth);
    free(sc);
    free(slot);
    free(qf);
    free(o);
}

/* ------------------------------------------------------------------------- */
/* Attention block -- encodeAttnBlock SeedlessMetal.swift:926-1005 with the     */
/* input RMSNorm of encodeLayerBlock (1008-1048): xa = rms(h); qkv = gqmm2      */
/* (dense, Ktop=1, inds 0 -- SeedlessAttn.swift:159-164); qk-norm+RoPE; K/V      */
/* append at slot (L+r) % C (maple_write_kv_pair 2871-2901); SDPA; o-proj with  */
/* residual h = half(h + half(o)) (gqmm2_rows_fold_add epilogue 3488-3543).      */
/* ------------------------------------------------------------------------- */
void or_attn_block(const or_cfg* cfg, const or_attn_w* w, const float* inv_freq, uint16_t* h,
                   uint16_t* kcache, uint16_t* vcache, int64_t L, const int32_t* parents, int M) {
    const int H = cfg->H, nQ = cfg->nQ, nKV = cfg->nKV, D = cfg->D;
    const int qkvN = (nQ + 2 * nKV) * D;
    uint16_t* xa = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)M * H);
    uint16_t* qkv = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)M * qkvN);
    uint16_t* qo = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)M * nQ * D);
    uint16_t* ko = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)M * nKV * D);
    uint16_t* at = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)M * nQ * D);
    uint16_t* o = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)M * H);
    int32_t* zero = (int32_t*)calloc((size_t)M, sizeof(int32_t));
    int* depth = (int*)malloc(sizeof(int) * (size_t)M);
    int64_t* pos = (int64_t*)malloc(sizeof(int64_t) * (size_t)M);
    tree_depths(parents, M, depth);
    for (int r = 0; r < M; ++r) pos[r] = L + depth[r];
    or_rms_norm(h, w->norm_w, xa, M, H, cfg->eps);
    or_qmm2(xa, w->qkv_w, w->qkv_s, w->qkv_b, zero, qkv, M, 1, H, qkvN, cfg->gs, 0);
    or_qk_norm_rope(qkv, w->q_norm_w, w->k_norm_w, inv_freq, pos, qo, ko, M, nQ, nKV, D,
                    cfg->rope_dim, cfg->eps);
    for (int r = 0; r < M; ++r) {
        const int64_t s = (L + r) % cfg->C;
        for (int g = 0; g < nKV; ++g)
            for (int d = 0; d < D; ++d) {
                kcache[((size_t)g * cfg->C + (size_t)s) * D + d] = ko[((size_t)r * nKV + g) * D + d];
                vcache[((size_t)g * cfg->C + (size_t)s) * D + d] =
                    qkv[(size_t)r * qkvN + (size_t)(nQ + nKV) * D + (size_t)g * D + d];
            }
    }
    or_attention(qo, kcache, vcache, cfg->C, L, parents, M, nQ, nKV, D, cfg->window, at);
    or_qmm2(at, w->o_w, w->o_s, w->o_b, zero, o, M, 1, nQ * D, H, cfg->gs, 0);
    for (size_t i = 0; i < (size_t)M * H; ++i) h[i] = or_f2h(or_h2f(h[i]) + or_h2f(o[i]));
    free(xa);
    free(qkv);
    free(qo);
    free(ko);
    free(at);
    free(o);
    free(zero);
    free(depth);
    free(pos);
}

void or_layer_forward(const or_cfg* cfg, const or_layer_w* w, const float* inv_freq, uint16_t* h,
                      uint16_t* kcache, uint16_t* vcache, int64_t L, const int32_t* parents, int M,
                      int32_t* out_inds, float* out_scores) {
    or_attn_block(cfg, &w->attn, inv_freq, h, kcache, vcache, L, parents, M);
    or_moe_block(&w->moe, h, h, M, OR_MOE_PRENORM | OR_MOE_RESIDUAL, out_inds, out_scores);
}

/* ------------------------------------------------------------------------- */
/* KV commit after a tree verify.  The reference's reject rollback rewinds the  */
/* offset over append-only writes (rewindOffset / snapshotForChain,             */
/* SeedlessAttn.swift:219-225, 319-322, 540-586); a draft tree also has to move  */
/* the accepted path into consecutive positions so the cache reads as if the    */
/* path had been fed as a chain: the K and V rows written at slot               */
/* (L + path[i]) % C go to slot (L + i) % C, i = 0 .. n_path-1, every source    */
/* read before any destination is written.  Caches [nKV][C][D].                 */
/* ------------------------------------------------------------------------- */
void or_kv_commit(uint16_t* kcache, uint16_t* vcache, int nKV, int64_t C, int D, int64_t L,
                  const int32_t* path, int n_path) {
    uint16_t* rows = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)2 * nKV * n_path * D);
    for (int c = 0; c < 2; ++c) {
        uint16_t* cache = c == 0 ? kcache : vcache;
        for (int g = 0; g < nKV; ++g)
            for (int i = 0; i < n_path; ++i) {
                const int64_t src = (L + path[i]) % C;
                memcpy(rows + (((size_t)c * nKV + g) * n_path + i) * D,
                       cache + ((size_t)g * C + (size_t)src) * D, sizeof(uint16_t) * (size_t)D);
            }
    }
    for (int c = 0; c < 2; ++c) {
        uint16_t* cache = c == 0 ? kcache : vcache;
        for (int g = 0; g < nKV; ++g)
            for (int i = 0; i < n_path; ++i) {
                const int64_t dst = (L + i) % C;
                memcpy(cache + ((size_t)g * C + (size_t)dst) * D,
                       rows + (((size_t)c * nKV + g) * n_path + i) * D, sizeof(uint16_t) * (size_t)D);
            }
    }
    free(rows);
}

/* ------------------------------------------------------------------------- */
/* a7: lm_head -- maple_lm_head_argmax semantics (SeedlessMetal.swift:3005-3111)  */
/* with an fp16 weight: logits = sum_k w[v,k] * x[m,k].  Accumulated in double   */
/* here (closest to the exact value) and rounded once to float.                  */
/* Argmax: lowest id wins ties (3073, 3083-3084, 3108); banned ids skipped       */
/* (3038-3042).                                                                  */
/* ------------------------------------------------------------------------- */
void or_lm_head_logits(const uint16_t* x, const uint16_t* w, float* logits, int M, int K, int V) {
    float* xf = (float*)malloc(sizeof(float) * (size_t)M * K);
    or_h2f_array(x, xf, (size_t)M * K);
#pragma omp parallel for schedule(static)
    for (int v = 0; v < V; ++v) {
        float wf[K];
        for (int k = 0; k < K; ++k) wf[k] = or_h2f(w[(size_t)v * K + k]);
        for (int m = 0; m < M; ++m) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += (double)wf[k] * (double)xf[(size_t)m * K + k];
            logits[(size_t)m * V + v] = (float)acc;
        }
    }
    free(xf);
}

/* ------------------------------------------------------------------------- */
/* a7, the Maple head: maple_lm_head_argmax's 4-bit affine weight                */
/* (SeedlessMetal.swift:3005-3068): uint32 w[V][K/8] holds 8 codes, LSB first   */
/* (nib j = (pack >> 4j) & 15, 3046-3053); scale / bias fp16 [V][K/64], the     */
/* group of pack wk is wk >> 3 (3043-3044: group size 64); the weight is        */
/* float(nib) * sc + bi in fp32 (3055-3062) times x.  Accumulated in double     */
/* here and rounded once to float.                                             */
/* ------------------------------------------------------------------------- */
void or_lm_head_q4_logits(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                          const uint16_t* biases, float* logits, int M, int K, int V) {
    float* xf = (float*)malloc(sizeof(float) * (size_t)M * K);
    or_h2f_array(x, xf, (size_t)M * K);
    const int packs = K / 8, groups = K / 64;
#pragma omp parallel for schedule(static)
    for (int v = 0; v < V; ++v) {
        float* wf = (float*)malloc(sizeof(float) * (size_t)K);
        for (int wk = 0; wk < packs; ++wk) {
            const uint32_t pack = w[(size_t)v * packs + wk];
            const float sc = or_h2f(scales[(size_t)v * groups + (wk >> 3)]);
            const float bi = or_h2f(biases[(size_t)v * groups + (wk >> 3)]);
            for (int j = 0; j < 8; ++j) {
                const float q = (float)((pack >> (4 * j)) & 15u);
                const float qs = q * sc;
                wf[8 * wk + j] = qs + bi;
            }
        }
        for (int m = 0; m < M; ++m) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += (double)wf[k] * (double)xf[(size_t)m * K + k];
            logits[(size_t)m * V + v] = (float)acc;
        }
        free(wf);
    }
    free(xf);
}

void or_argmax_rows(const float* logits, int M, int V, const int32_t* banned, int n_banned,
                    int32_t* out_idx, float* out_best, float* out_second) {
    for (int m = 0; m < M; ++m) {
        float best = -INFINITY, second = -INFINITY;
        int bi = V;
        for (int v = 0; v < V; ++v) {
            int skip = 0;
            for (int b = 0; b < n_banned; ++b)
                if (banned[b] == v) skip = 1;
            if (skip) continue;
            const float s = logits[(size_t)m * V + v];
            if (s > best) {
                second = best;
                best = s;
                bi = v;
            } else if (s > second) {
                second = s;
            }
        }
        out_idx[m] = bi;
        if (out_best) out_best[m] = best;
        if (out_second) out_second[m] = second;
    }
}

/* ------------------------------------------------------------------------- */
/* a8: greedy acceptance -- verifyDraftChain SeedlessDecodeEngine.swift:1574-1603 */
/* (p = longest prefix with evals[i] == draft[i]; emit draft[..p] + evals[p]),   */
/* generalised to a tree: walk from row 0, step to the lowest-index child whose   */
/* token equals the current row's argmax, stop when none matches; the bonus is   */
/* the argmax of the deepest accepted row.  A chain gives the reference rule.    */
/* ------------------------------------------------------------------------- */
int or_accept_greedy(const int32_t* tokens, const int32_t* parents, const int32_t* argmax,
                     int n_rows, int32_t* out_path, int32_t* out_emit) {
    int cur = 0, acc = 0;
    out_path[0] = 0;
    for (;;) {
        int next = -1;
        for (int c = cur + 1; c < n_rows; ++c) {
            const int par = parents ? parents[c] : c - 1;
            if (par == cur && tokens[c] == argmax[cur]) {
                next = c;
                break;
            }
        }
        if (next < 0) break;
        out_emit[acc] = tokens[next];
        ++acc;
        out_path[acc] = next;
        cur = next;
    }
    out_emit[acc] = argmax[cur];
    return acc;
}

/* ------------------------------------------------------------------------- */
/* a9: sampled acceptance.                                                      */
/* ------------------------------------------------------------------------- */

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11 "Parallel random numbers: as */
/* easy as 1, 2, 3"); multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key bumps         */
/* 0x9E3779B9 / 0xBB67AE85.                                                        */
void or_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        c0 = hi1 ^ c1 ^ k0;
        c1 = lo1;
        c2 = hi0 ^ c3 ^ k1;
        c3 = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

/* 24 high bits -> [0, 1) */
float or_u01_from_u32(uint32_t x) { return (float)(x >> 8) * 0x1p-24f; }

/* One Philox block per verify row: ctr = (row, counter lo, counter hi, 0x6d6a6a76),
 * key = (seed lo, seed hi).  u[row][0] = accept test, u[row][1] = residual/bonus walk. */
void or_verify_uniforms(uint64_t seed, uint64_t counter, int rows, float* u) {
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    for (int r = 0; r < rows; ++r) {
        const uint32_t ctr[4] = {(uint32_t)r, (uint32_t)counter, (uint32_t)(counter >> 32),
                                 0x6d6a6a76u};
        uint32_t o[4];
        or_philox4x32_10(ctr, key, o);
        u[2 * r] = or_u01_from_u32(o[0]);
        u[2 * r + 1] = or_u01_from_u32(o[1]);
    }
}

/* SplitMix64 -- LogitsProcessor.swift:4-14 (seed 0 is replaced by 0xDEADBEEFCAFEBABE). */
uint64_t or_splitmix64_next(uint64_t* state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Float.random(in: 0..<1, using:) as read from the Swift standard library:
 * (next() & (2^24 - 1)) * 2^-24.  Parity unpinned (no Swift here). */
static float swift_rand01(uint64_t* st) {
    return (float)(or_splitmix64_next(st) & 0xFFFFFFull) * 0x1p-24f;
}

/* Canonical exp for x <= 0: Cody-Waite reduction by ln2 (hi/lo split), degree-7 Taylor
 * polynomial by Horner with fused multiply-adds, scale by 2^n built from exponent bits.
 * x < -87 returns 0 so that every non-zero result is a normal float.  The device code
 * evaluates the identical operation sequence, so both produce the same bits. */
float or_canon_expf(float x) {
    if (!(x >= -87.0f)) return 0.0f;
    const float n = rintf(x * 0x1.715476p+0f);
    float r = fmaf(-n, 0x1.62e400p-1f, x);
    r = fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;  /* 1/5040 */
    p = fmaf(p, r, 0x1.6c16c2p-10f);  /* 1/720 */
    p = fmaf(p, r, 0x1.111112p-7f);   /* 1/120 */
    p = fmaf(p, r, 0x1.555556p-5f);   /* 1/24 */
    p = fmaf(p, r, 0x1.555556p-3f);   /* 1/6 */
    p = fmaf(p, r, 0x1.000000p-1f);   /* 1/2 */
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const uint32_t bits = (uint32_t)((int)n + 127) << 23;
    float two_n;
    memcpy(&two_n, &bits, 4);
    return p * two_n;
}

#define CANON_CHUNK 16
#define CANON_BLOCK 64 /* chunks per block */

float or_canon_sum(const float* v, int n) {
    const int nch = (n + CANON_CHUNK - 1) / CANON_CHUNK;
    float total = 0.0f;
    for (int b0 = 0; b0 < nch; b0 += CANON_BLOCK) {
        float bs = 0.0f;
        const int b1 = b0 + CANON_BLOCK < nch ? b0 + CANON_BLOCK : nch;
        for (int c = b0; c < b1; ++c) {
            float cs = 0.0f;
            const int e = (c + 1) * CANON_CHUNK < n ? (c + 1) * CANON_CHUNK : n;
            for (int i = c * CANON_CHUNK; i < e; ++i) cs += v[i];
            bs += cs;
        }
        total += bs;
    }
    return total;
}

/* Hierarchical walk: first block whose running total reaches t, then the first chunk of
 * that block, then the first element; each level restarts from the prefix before it.
 * Falls back to the last index (SpeculativeSampling.swift:56, LogitsProcessor.swift:164). */
int or_canon_walk(const float* v, int n, float t) {
    const int nch = (n + CANON_CHUNK - 1) / CANON_CHUNK;
    float P = 0.0f;
    for (int b0 = 0; b0 < nch; b0 += CANON_BLOCK) {
        const int b1 = b0 + CANON_BLOCK < nch ? b0 + CANON_BLOCK : nch;
        float bs = 0.0f;
        for (int c = b0; c < b1; ++c) {
            float cs = 0.0f;
            const int e = (c + 1) * CANON_CHUNK < n ? (c + 1) * CANON_CHUNK : n;
            for (int i = c * CANON_CHUNK; i < e; ++i) cs += v[i];
            bs += cs;
        }
        const float Pn = P + bs;
        if (t <= Pn) {
            float Q = P;
            for (int c = b0; c < b1; ++c) {
                const int e = (c + 1) * CANON_CHUNK < n ? (c + 1) * CANON_CHUNK : n;
                float cs = 0.0f;
                for (int i = c * CANON_CHUNK; i < e; ++i) cs += v[i];
                const float Qn = Q + cs;
                if (t <= Qn) {
                    float R = Q;
                    for (int i = c * CANON_CHUNK; i < e; ++i) {
                        R = R + v[i];
                        if (t <= R) return i;
                    }
                    return e - 1;
                }
                Q = Qn;
            }
            const int last = b1 * CANON_CHUNK < n ? b1 * CANON_CHUNK : n;
            return last - 1;
        }
        P = Pn;
    }
    return n - 1;
}

/* Full-vocab speculative sampling in canonical arithmetic.  Per row:
 *   invT = 1/max(T,1e-5); sc_v = l_v*invT; mx = max sc; e_v = canon_exp(sc_v - mx);
 *   Z = canon_sum(e); p_v = e_v / Z   (LogitsProcessor.probabilities, 168-189)
 * Row i < D: accept iff q > 0 && p > 0 && u_i0 <= min(1, p/q)   (tryAccept 27-43)
 *   reject: residual r (point q: p with r_d = max(0, p_d - q); uniform q: max(p - q, 0)),
 *   S = canon_sum(r); token = canon_walk(r, u_i1 * S)   (44-57); S == 0 -> sample p.
 * All accepted: bonus = canon_walk(e_D, u_D0 * Z_D)   (walkDraft 92-98, samplePrepared 157-164). */
static void row_probs(const float* l, int V, float invT, float* e, float* Zout) {
    float mx = -INFINITY;
    for (int v = 0; v < V; ++v) mx = fmaxf(mx, l[v]);
    const float mxs = mx * invT;
    for (int v = 0; v < V; ++v) {
        const float s = l[v] * invT;
        e[v] = or_canon_expf(s - mxs);
    }
    *Zout = or_canon_sum(e, V);
}

int or_accept_sampled(const float* logits, int rows, int V, const int32_t* draft,
                      float temperature, int q_mode, const float* q_point,
                      const float* uniforms, int32_t* out_token) {
    const float invT = 1.0f / fmaxf(temperature, 1e-5f);
    float* e = (float*)malloc(sizeof(float) * (size_t)V);
    float* r = (float*)malloc(sizeof(float) * (size_t)V);
    const int D = rows - 1;
    int result = D;
    for (int i = 0; i < D; ++i) {
        float Z;
        row_probs(logits + (size_t)i * V, V, invT, e, &Z);
        const int d = draft[i];
        const float p = (d >= 0 && d < V) ? e[d] / Z : 0.0f;
        float q = q_mode == 1 ? 1.0f / (float)V : (q_point ? q_point[i] : 1.0f);
        q = fmaxf(0.0f, q);
        if (q > 0.0f && p > 0.0f) {
            const float ratio = p / q;
            if (uniforms[2 * i] <= fminf(1.0f, ratio)) continue;
        }
        for (int v = 0; v < V; ++v) {
            const float pv = e[v] / Z;
            r[v] = q_mode == 1 ? fmaxf(pv - q, 0.0f) : pv;
        }
        if (q_mode != 1 && d >= 0 && d < V && q > 0.0f) r[d] = fmaxf(0.0f, r[d] - q);
        const float S = or_canon_sum(r, V);
        if (S > 0.0f)
            *out_token = or_canon_walk(r, V, uniforms[2 * i + 1] * S);
        else
            *out_token = or_canon_walk(e, V, uniforms[2 * i + 1] * Z);
        result = i;
        break;
    }
    if (result == D) {
        float Z;
        row_probs(logits + (size_t)D * V, V, invT, e, &Z);
        *out_token = or_canon_walk(e, V, uniforms[2 * D] * Z);
    }
    free(e);
    free(r);
    return result;
}

/* LogitsProcessor.prepare (LogitsProcessor.swift:57-104, order 91-104) over a full-vocabulary
 * row, in place.  The seen set is the history tokens (unique, any order) plus the first n_extra
 * draft tokens; a token's count is its history count plus its occurrences among those drafts
 * (walkDraft adds each accepted draft to both, SpeculativeSampling.swift:86-87).  Each seen
 * token is penalised once: repetition (x > 0 ? x / r : x * r; off when |r - 1| <= 1e-6 or
 * r <= 0, 78-89), presence (x - pres; off at 0, 57-65), frequency (x - freq * count for
 * count > 0; off at 0, 67-76). */
static float penalize1(float x, int count, float rep, float pres, float freq) {
    if (fabsf(rep - 1.0f) > 1e-6f && rep > 0.0f) x = x > 0.0f ? x / rep : x * rep;
    if (pres != 0.0f) x = x - pres;
    if (freq != 0.0f && count > 0) x = x - freq * (float)count;
    return x;
}

void or_penalize_row(float* l, int V, const int32_t* hist_tok, const int32_t* hist_cnt,
                     int n_hist, const int32_t* extra, int n_extra, float rep, float pres,
                     float freq) {
    for (int j = 0; j < n_hist; ++j) {
        const int t = hist_tok[j];
        if (t < 0 || t >= V) continue;
        int c = hist_cnt[j];
        for (int d = 0; d < n_extra; ++d) c += extra[d] == t;
        l[t] = penalize1(l[t], c, rep, pres, freq);
    }
    for (int d = 0; d < n_extra; ++d) {
        const int t = extra[d];
        if (t < 0 || t >= V) continue;
        int first = 1, in_hist = 0, c = 0;
        for (int e = 0; e < d; ++e) first &= extra[e] != t;
        for (int j = 0; j < n_hist; ++j) in_hist |= hist_tok[j] == t;
        if (!first || in_hist) continue;
        for (int e = 0; e < n_extra; ++e) c += extra[e] == t;
        l[t] = penalize1(l[t], c, rep, pres, freq);
    }
}

/* LogitsProcessor.samplePrepared's nucleus + multinomial (LogitsProcessor.swift:137-164).
 * Tokens are ranked by e descending, the lower id first among equal e (the reference's unstable
 * sort leaves ties unordered).  The kept set is the shortest ranked prefix (at least one token)
 * whose mass reaches clamp(top_p, 0, 1) * Z, the masses summed exactly: each e as the integer
 * trunc(e * 2^40), the target as trunc(fl(tp * Z) * 2^40) (an order-free sum, so the device may
 * find the cut by a radix selection instead of a sort).  The sample is or_canon_walk over the
 * kept e in id order at u * (their or_canon_sum), or the top-ranked token when that sum is 0;
 * with the target above the whole mass every token is kept. */
typedef struct {
    float e;
    int32_t id;
} rank_item;

static int rank_cmp(const void* a, const void* b) {
    const rank_item* x = (const rank_item*)a;
    const rank_item* y = (const rank_item*)b;
    if (x->e != y->e) return x->e > y->e ? -1 : 1;
    return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

uint64_t or_nucleus_fixed(float e) { return (uint64_t)((double)e * 0x1p40); }

int or_nucleus_sample(const float* e, int V, float Z, float top_p, float u) {
    rank_item* it = (rank_item*)malloc(sizeof(rank_item) * (size_t)V);
    float* kept = (float*)malloc(sizeof(float) * (size_t)V);
    for (int v = 0; v < V; ++v) {
        it[v].e = e[v];
        it[v].id = v;
    }
    qsort(it, (size_t)V, sizeof(rank_item), rank_cmp);
    const float tp = top_p < 0.0f ? 0.0f : (top_p > 1.0f ? 1.0f : top_p);
    const uint64_t F = or_nucleus_fixed(tp * Z);
    int k = V - 1;
    uint64_t acc = 0;
    for (int i = 0; i < V; ++i) {
        acc += or_nucleus_fixed(it[i].e);
        if (acc >= F) {
            k = i;
            break;
        }
    }
    const float es = it[k].e;
    const int is = it[k].id;
    for (int v = 0; v < V; ++v) kept[v] = (e[v] > es || (e[v] == es && v <= is)) ? e[v] : 0.0f;
    const float S = or_canon_sum(kept, V);
    const int tok = S > 0.0f ? or_canon_walk(kept, V, u * S) : it[0].id;
    free(it);
    free(kept);
    return tok;
}

/* or_accept_sampled with LogitsProcessor's penalties and nucleus (walkDraft,
 * SpeculativeSampling.swift:65-99): row i's logits are penalised with the history plus drafts
 * 0 .. i-1; tryAccept's probabilities take no nucleus (27-59); the bonus row and a residual of
 * zero mass are sampled through samplePrepared, i.e. with the nucleus when top_p < 1 - 1e-6.
 * The residual's fallback and the bonus use u1 and u0 of their row, as or_accept_sampled. */
int or_accept_sampled_ex(const float* logits, int rows, int V, const int32_t* draft,
                         float temperature, float top_p, float rep, float pres, float freq,
                         const int32_t* hist_tok, const int32_t* hist_cnt, int n_hist,
                         int q_mode, const float* q_point, const float* uniforms,
                         int32_t* out_token) {
    const float invT = 1.0f / fmaxf(temperature, 1e-5f);
    const int nucleus = top_p < 1.0f - 1e-6f;
    float* l = (float*)malloc(sizeof(float) * (size_t)V);
    float* e = (float*)malloc(sizeof(float) * (size_t)V);
    float* r = (float*)malloc(sizeof(float) * (size_t)V);
    const int D = rows - 1;
    int result = D;
    for (int i = 0; i <= D; ++i) {
        memcpy(l, logits + (size_t)i * V, sizeof(float) * (size_t)V);
        or_penalize_row(l, V, hist_tok, hist_cnt, n_hist, draft, i, rep, pres, freq);
        float Z;
        row_probs(l, V, invT, e, &Z);
        if (i == D) {
            *out_token = nucleus ? or_nucleus_sample(e, V, Z, top_p, uniforms[2 * D])
                                 : or_canon_walk(e, V, uniforms[2 * D] * Z);
            break;
        }
        const int d = draft[i];
        const float p = (d >= 0 && d < V) ? e[d] / Z : 0.0f;
        float q = q_mode == 1 ? 1.0f / (float)V : (q_point ? q_point[i] : 1.0f);
        q = fmaxf(0.0f, q);
        if (q > 0.0f && p > 0.0f) {
            const float ratio = p / q;
            if (uniforms[2 * i] <= fminf(1.0f, ratio)) continue;
        }
        for (int v = 0; v < V; ++v) {
            const float pv = e[v] / Z;
            r[v] = q_mode == 1 ? fmaxf(pv - q, 0.0f) : pv;
        }
        if (q_mode != 1 && d >= 0 && d < V && q > 0.0f) r[d] = fmaxf(0.0f, r[d] - q);
        const float S = or_canon_sum(r, V);
        if (S > 0.0f)
            *out_token = or_canon_walk(r, V, uniforms[2 * i + 1] * S);
        else
            *out_token = nucleus ? or_nucleus_sample(e, V, Z, top_p, uniforms[2 * i + 1])
                                 : or_canon_walk(e, V, uniforms[2 * i + 1] * Z);
        result = i;
        break;
    }
    free(l);
    free(e);
    free(r);
    return result;
}

/* Literal restatement over candidate lists (no canonical order), used for the KATs of
 * SpeculativeSamplingTests.swift.  LogitsProcessor.probabilities 168-189, samplePrepared
 * 116-165 (no nucleus), SpeculativeSampling.tryAccept 27-59. */
static void cand_probs(const float* logits, int n, float T, float* p) {
    if (T <= 1e-5f) {
        int best = 0;
        float bv = -INFINITY;
        for (int i = 0; i < n; ++i)
            if (logits[i] > bv) {
                bv = logits[i];
                best = i;
            }
        for (int i = 0; i < n; ++i) p[i] = 0.0f;
        p[best] = 1.0f;
        return;
    }
    const float invT = 1.0f / fmaxf(T, 1e-5f);
    float mx = -INFINITY;
    for (int i = 0; i < n; ++i) mx = fmaxf(mx, logits[i] * invT);
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) {
        p[i] = expf(logits[i] * invT - mx);
        sum += p[i];
    }
    if (!(sum > 0.0f)) {
        for (int i = 0; i < n; ++i) p[i] = 1.0f / (float)n;
        return;
    }
    for (int i = 0; i < n; ++i) p[i] = p[i] / sum;
}

static int cand_sample(const int32_t* ids, const float* logits, int n, float T, uint64_t* rng) {
    if (T <= 1e-5f) {
        int best = 0;
        float bv = -INFINITY;
        for (int i = 0; i < n; ++i)
            if (logits[i] > bv) {
                bv = logits[i];
                best = i;
            }
        return ids[best];
    }
    const float invT = 1.0f / fmaxf(T, 1e-5f);
    float mx = -INFINITY;
    for (int i = 0; i < n; ++i) mx = fmaxf(mx, logits[i] * invT);
    float* ex = (float*)malloc(sizeof(float) * (size_t)n);
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) {
        ex[i] = expf(logits[i] * invT - mx);
        sum += ex[i];
    }
    int tok = ids[0];
    if (sum > 0.0f) {
        const float u = swift_rand01(rng) * sum;
        float acc = 0.0f;
        tok = ids[n - 1];
        for (int i = 0; i < n; ++i) {
            acc += ex[i];
            if (u <= acc) {
                tok = ids[i];
                break;
            }
        }
    }
    free(ex);
    return tok;
}

int or_try_accept(int draft_token, const int32_t* ids, const float* logits, int n,
                  float temperature, float draft_q, uint64_t* rng, int32_t* out_token) {
    float* p = (float*)malloc(sizeof(float) * (size_t)n);
    cand_probs(logits, n, temperature, p);
    int idx = -1;
    for (int i = 0; i < n; ++i)
        if (ids[i] == draft_token) {
            idx = i;
            break;
        }
    const float pd = idx >= 0 ? p[idx] : 0.0f;
    const float q = fmaxf(0.0f, draft_q);
    if (q > 0.0f && pd > 0.0f) {
        const float u = swift_rand01(rng);
        if (u <= fminf(1.0f, pd / q)) {
            *out_token = draft_token;
            free(p);
            return 1;
        }
    }
    if (idx >= 0 && q > 0.0f) p[idx] = fmaxf(0.0f, p[idx] - q);
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) sum += p[i];
    if (sum > 0.0f) {
        const float u = swift_rand01(rng) * sum;
        float acc = 0.0f;
        *out_token = ids[n - 1];
        for (int i = 0; i < n; ++i) {
            acc += p[i];
            if (u <= acc) {
                *out_token = ids[i];
                break;
            }
        }
    } else {
        *out_token = cand_sample(ids, logits, n, temperature, rng);
    }
    free(p);
    return 0;
}

/* walkDraft -- SpeculativeSampling.swift:65-99 without penalties; rows [n_draft+1][n_cand]. */
int or_walk_draft(const int32_t* draft, int n_draft, const int32_t* row_ids,
                  const float* row_logits, int n_cand, float temperature, uint64_t* rng,
                  int32_t* out_next) {
    for (int i = 0; i < n_draft; ++i) {
        int32_t tok;
        const int ok = or_try_accept(draft[i], row_ids + (size_t)i * n_cand,
                                     row_logits + (size_t)i * n_cand, n_cand, temperature, 1.0f,
                                     rng, &tok);
        if (!ok) {
            *out_next = tok;
            return i;
        }
    }
    *out_next = cand_sample(row_ids + (size_t)n_draft * n_cand,
                            row_logits + (size_t)n_draft * n_cand, n_cand, temperature, rng);
    return n_draft;
}

int or_walk_draft_greedy(const int32_t* draft, int n_draft, const int32_t* row_ids,
                         const float* row_logits, int n_cand, int32_t* out_next) {
    uint64_t st = 1;
    return or_walk_draft(draft, n_draft, row_ids, row_logits, n_cand, 0.0f, &st, out_next);
}

void or_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }

int or_max_threads(void) { return omp_get_max_threads(); }
