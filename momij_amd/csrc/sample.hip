// sample.hip -- full-vocabulary speculative sampling (rejection sampling) on the device.
//
// Rules: SpeculativeSampling.tryAccept / walkDraft (SpeculativeSampling.swift:27-99) with
// LogitsProcessor.probabilities / samplePrepared (LogitsProcessor.swift:116-189):
//   p = softmax(logits * (1/T));  accept draft d iff q > 0, p_d > 0 and u0 <= min(1, p_d / q);
//   on reject sample the residual (point q: p with p_d -> max(0, p_d - q); uniform q:
//   max(p - q, 0)) by a cumulative walk to u1 * sum; after a full accept sample the bonus from
//   the last row by a walk to u0 * sum of exps.
// LogitsProcessor options: penalties (prepare, LogitsProcessor.swift:57-104) on every row, the
// seen set and counts growing with the drafts accepted before it (walkDraft 86-87);
// samplePrepared's nucleus (137-154) for the bonus and for a residual of zero mass: tokens
// ranked by e descending, the lower id first on ties, kept up to the first ranked prefix whose
// blocked prefix sum reaches top_p * Z, sampled in id order (the ranking is a radix sort of
// the row's e bits).
// Every float operation below happens in a fixed order (chunks of 16 summed sequentially,
// blocks of 64 chunks summed sequentially, block totals summed sequentially; exp evaluated by
// canon_expf; IEEE divisions) so the CPU oracle reproduces each decision bit for bit.
#pragma clang fp contract(off)
#include <hipcub/hipcub.hpp>

#include "mj_device.h"
#include "mj_internal.h"

#define CH 16
#define BLK 64
#define MAX_CHUNKS 12288  // V <= 196608
#define RMB 32            // blocks a row's maximum is split over
#define DEC_STAGE 8192    // block sums the decision kernel stages in LDS (the rest it reads)

// Hand-off from the accept decisions to the residual walk: phase 1 = row fr was rejected and
// its residual still has to be summed (k_resid_sums) and walked (k_resid_walk).
struct SampleState {
    int phase, fr, d, pad;
    float q, Zr, pad2, pad3;
};
static_assert(sizeof(SampleState) == 32, "state fits its 8 floats");

struct SampleArgs {
    float* logits;         // [rows][V] (penalised in place)
    int rows, V;
    const int32_t* draft;  // [rows-1]
    float invT;
    int q_mode;            // 0 point, 1 uniform
    float q_uniform;       // 1/V
    const float* q_point;  // [rows-1] or nullptr (= 1)
    uint64_t seed, counter;
    float* rowmax;         // [rows]
    float* bsum;           // [rows][nblocks] block sums of e
    int nblocks;
    float* mpart;          // [rows][RMB] partial row maxima
    float* rbs;            // [nblocks] block sums of the residual of the rejected row
    struct SampleState* state;
    int32_t* out;          // [2] or nullptr
    StepResult* res;       // or nullptr
    const StepDesc* sd;    // when set: temperature, q, seed, counter, draft, options from it
    const int* abort;
    SampleOpts o;
    NucleusBuf nb;         // nb.st == nullptr: no nucleus
};

// Effective per-call parameters (from the step descriptor when one is given).
__device__ __forceinline__ SampleArgs resolve(SampleArgs a) {
    if (a.sd) {
        a.invT = __fdiv_rn(1.0f, fmaxf(a.sd->temperature, 1e-5f));
        a.q_mode = a.sd->q_mode;
        a.q_uniform = a.sd->q_uniform;
        a.q_point = a.sd->has_qpoint ? a.sd->q_point : nullptr;
        a.seed = a.sd->seed;
        a.counter = a.sd->counter;
        a.draft = a.sd->tokens + 1;
        a.o.top_p = a.sd->top_p;
        a.o.rep = a.sd->rep;
        a.o.pres = a.sd->pres;
        a.o.freq = a.sd->freq;
        a.o.n_hist = a.sd->n_hist;
    }
    return a;
}

__device__ __forceinline__ bool nucleus_on(const SampleArgs& a) {
    return a.nb.st != nullptr && a.o.top_p < 1.0f - 1e-6f;
}

// LogitsProcessor.prepare for one token: repetition, presence, frequency (in that order)
__device__ __forceinline__ float penalize1(float x, int count, float rep, float pres, float freq) {
    if (fabsf(rep - 1.0f) > 1e-6f && rep > 0.0f) x = x > 0.0f ? __fdiv_rn(x, rep) : x * rep;
    if (pres != 0.0f) x = x - pres;
    if (freq != 0.0f && count > 0) x = x - freq * (float)count;
    return x;
}

// Row i's penalties: every history token, then every draft d < i that is neither earlier among
// the drafts nor in the history, each once with its total count (history count + occurrences
// among drafts 0 .. i-1).  One block per row; each token is written by one thread.
__global__ __launch_bounds__(256) void k_penalize(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const bool rep_on = fabsf(a.o.rep - 1.0f) > 1e-6f && a.o.rep > 0.0f;
    if (!rep_on && a.o.pres == 0.0f && a.o.freq == 0.0f) return;
    const int i = blockIdx.x, t = threadIdx.x;
    float* l = a.logits + (size_t)i * a.V;
    for (int j = t; j < a.o.n_hist; j += 256) {
        const int tok = a.o.hist_tok[j];
        if (tok < 0 || tok >= a.V) continue;
        int c = a.o.hist_cnt[j];
        for (int d = 0; d < i; ++d) c += a.draft[d] == tok;
        l[tok] = penalize1(l[tok], c, a.o.rep, a.o.pres, a.o.freq);
    }
    for (int d = t; d < i; d += 256) {
        const int tok = a.draft[d];
        if (tok < 0 || tok >= a.V) continue;
        bool first = true;
        for (int e = 0; e < d; ++e) first = first && a.draft[e] != tok;
        int lo = 0, hi = a.o.n_hist;  // binary search of the ascending history
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (a.o.hist_tok[mid] < tok) lo = mid + 1; else hi = mid;
        }
        const bool in_hist = lo < a.o.n_hist && a.o.hist_tok[lo] == tok;
        if (!first || in_hist) continue;
        int c = 0;
        for (int e = 0; e < i; ++e) c += a.draft[e] == tok;
        l[tok] = penalize1(l[tok], c, a.o.rep, a.o.pres, a.o.freq);
    }
}

__device__ __forceinline__ void row_uniforms(const SampleArgs& a, int row, float& u0, float& u1) {
    uint32_t c[4] = {(uint32_t)row, (uint32_t)a.counter, (uint32_t)(a.counter >> 32), 0x6d6a6a76u};
    philox4x32_10(c, (uint32_t)a.seed, (uint32_t)(a.seed >> 32));
    u0 = u01(c[0]);
    u1 = u01(c[1]);
}

__device__ __forceinline__ float e_at(const SampleArgs& a, int row, int v, float mxs) {
    const float s = a.logits[(size_t)row * a.V + v] * a.invT;
    return canon_expf(s - mxs);
}

// residual mass at v of row `row` (p_v = e_v / Z)
__device__ __forceinline__ float r_at(const SampleArgs& a, int row, int v, float mxs, float Z,
                                      float q, int d) {
    const float pv = __fdiv_rn(e_at(a, row, v, mxs), Z);
    if (a.q_mode == 1) return fmaxf(pv - q, 0.0f);
    if (v == d && q > 0.0f) return fmaxf(0.0f, pv - q);
    return pv;
}

// Row maxima in RMB slices a row (a maximum is exact in any order): block (row, j) writes the
// maximum of its slice; the sums kernel folds the RMB partials.
__global__ __launch_bounds__(256) void k_rowmax(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const int row = blockIdx.x / RMB, j = blockIdx.x % RMB, t = threadIdx.x;
    const int span = (a.V + RMB - 1) / RMB;
    const int v0 = j * span, v1 = min(a.V, v0 + span);
    float m = -INFINITY;
    for (int v = v0 + t; v < v1; v += 256) m = fmaxf(m, a.logits[(size_t)row * a.V + v]);
    m = wave_max(m);
    __shared__ float sm[4];
    if ((t & 63) == 0) sm[t >> 6] = m;
    __syncthreads();
    if (t == 0) a.mpart[row * RMB + j] = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
}

// Block sums of e_v: one 64-thread block per (row, 1024-element block), lane = chunk.
__global__ __launch_bounds__(64) void k_sample_sums(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const int row = blockIdx.x / a.nblocks, b = blockIdx.x % a.nblocks;
    const int lane = threadIdx.x;
    const int nch = (a.V + CH - 1) / CH;
    const int chunk = b * BLK + lane;
    float mx = lane < RMB ? a.mpart[row * RMB + lane] : -INFINITY;
    mx = wave_max(mx);
    if (b == 0 && lane == 0) a.rowmax[row] = mx;
    const float mxs = mx * a.invT;
    float cs = 0.0f;
    if (chunk < nch) {
        const int e = min(chunk * CH + CH, a.V);
        for (int v = chunk * CH; v < e; ++v) cs = cs + e_at(a, row, v, mxs);
    }
    __shared__ float s[BLK];
    s[lane] = cs;
    __syncthreads();
    if (lane == 0) {
        float bs = 0.0f;
        for (int c = 0; c < BLK; ++c)
            if (b * BLK + c < nch) bs = bs + s[c];
        a.bsum[(size_t)row * a.nblocks + b] = bs;
    }
}

__device__ __forceinline__ void write_result(const SampleArgs& a, int acc, int tok) {
    if (a.out) {
        a.out[0] = acc;
        a.out[1] = tok;
    }
    if (a.res) {
        a.res->accepted = acc;
        a.res->token = tok;
        for (int i = 0; i <= acc; ++i) a.res->path[i] = i;
        for (int i = 0; i < acc; ++i) a.res->emit[i] = a.draft[i];
        a.res->emit[acc] = tok;
    }
}

// Walk of row `row` to tgt over its mass -- the residual (walk_resid: block sums in rbs) or e
// (block sums in bsum) -- block, then chunk (the chosen block's 64 chunk sums recomputed in the
// same order), then element; writes (fr, token).  Whole block (>= 64 threads).
__device__ void walk_write(const SampleArgs& a, int row, int fr, bool walk_resid, float tgt,
                           float mxs, float Zr, float q, int d) {
    const int t = threadIdx.x;
    const int nch = (a.V + CH - 1) / CH;
    __shared__ float sbs[MAX_CHUNKS / BLK];
    __shared__ float cs[BLK];
    __shared__ float ev[CH];
    __shared__ int s_bidx, s_cidx, s_tok;
    __shared__ float s_P, s_Q;
    // the row's block sums, requested together
    for (int b = t; b < a.nblocks; b += blockDim.x)
        sbs[b] = walk_resid ? a.rbs[b] : a.bsum[(size_t)row * a.nblocks + b];
    __syncthreads();
    if (t == 0) {
        float P = 0.0f;
        int blk = -1;
        for (int b = 0; b < a.nblocks; ++b) {
            const float Pn = P + sbs[b];
            if (tgt <= Pn) {
                blk = b;
                break;
            }
            P = Pn;
        }
        s_bidx = blk;
        s_P = P;
        s_tok = a.V - 1;
    }
    __syncthreads();
    const int blk = s_bidx;
    if (blk >= 0) {
        if (t < BLK) {
            const int c = blk * BLK + t;
            float sum = 0.0f;
            if (c < nch) {
                const int e = min(c * CH + CH, a.V);
                for (int v = c * CH; v < e; ++v)
                    sum = sum + (walk_resid ? r_at(a, row, v, mxs, Zr, q, d) : e_at(a, row, v, mxs));
            }
            cs[t] = sum;
        }
        __syncthreads();
        if (t == 0) {
            const int c0 = blk * BLK, c1 = min(c0 + BLK, nch);
            float Q = s_P;
            int cc = -1;
            for (int c = c0; c < c1; ++c) {
                const float Qn = Q + cs[c - c0];
                if (tgt <= Qn) {
                    cc = c;
                    break;
                }
                Q = Qn;
            }
            s_cidx = cc;
            s_Q = Q;
            if (cc < 0) s_tok = min(c1 * CH, a.V) - 1;
        }
        __syncthreads();
        const int cc = s_cidx;
        if (cc >= 0) {
            // the chunk's element values, each computed once, then the running total in order
            const int e = min(cc * CH + CH, a.V);
            if (t < CH && cc * CH + t < e) {
                const int v = cc * CH + t;
                ev[t] = walk_resid ? r_at(a, row, v, mxs, Zr, q, d) : e_at(a, row, v, mxs);
            }
            __syncthreads();
            if (t == 0) {
                float R = s_Q;
                int tok = e - 1;
                for (int v = cc * CH; v < e; ++v) {
                    R = R + ev[v - cc * CH];
                    if (tgt <= R) {
                        tok = v;
                        break;
                    }
                }
                s_tok = tok;
            }
            __syncthreads();
        }
    }
    if (t == 0) write_result(a, fr, s_tok);
}

// Single block: row totals and the sequential accept decisions.  A full accept samples the bonus
// here (or leaves it to the nucleus kernels); a reject hands row fr to k_resid_sums /
// k_resid_walk through the state.
__global__ __launch_bounds__(64) void k_sample_decide(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const int t = threadIdx.x;
    const int D = a.rows - 1;
    __shared__ float Z[MJ_ROWS];
    __shared__ float ed[MJ_ROWS];
    __shared__ float sbs[DEC_STAGE];
    __shared__ int s_fr;
    // every row's block sums and the drafts' e values, requested together; then each row's
    // total in block order
    const int per = a.nblocks;
    const int nst = min(a.rows * per, DEC_STAGE);
    for (int idx = t; idx < nst; idx += blockDim.x) sbs[idx] = a.bsum[idx];
    if (t < D) {
        const int d = a.draft[t];
        ed[t] = (d >= 0 && d < a.V) ? e_at(a, t, d, a.rowmax[t] * a.invT) : 0.0f;
    }
    __syncthreads();
    if (t < a.rows) {
        float z = 0.0f;
        for (int b = 0; b < per; ++b) {
            const int idx = t * per + b;
            z = z + (idx < DEC_STAGE ? sbs[idx] : a.bsum[idx]);
        }
        Z[t] = z;
    }
    __syncthreads();
    if (t == 0) {
        int fr = D;
        for (int i = 0; i < D; ++i) {
            const int d = a.draft[i];
            const float p = (d >= 0 && d < a.V) ? __fdiv_rn(ed[i], Z[i]) : 0.0f;
            float q = a.q_mode == 1 ? a.q_uniform : (a.q_point ? a.q_point[i] : 1.0f);
            q = fmaxf(0.0f, q);
            float u0, u1;
            row_uniforms(a, i, u0, u1);
            if (q > 0.0f && p > 0.0f && u0 <= fminf(1.0f, __fdiv_rn(p, q))) continue;
            fr = i;
            break;
        }
        s_fr = fr;
        if (fr < D) {
            float q = a.q_mode == 1 ? a.q_uniform : (a.q_point ? a.q_point[fr] : 1.0f);
            *a.state = SampleState{1, fr, a.draft[fr], 0, fmaxf(0.0f, q), Z[fr], 0.0f, 0.0f};
        } else {
            *a.state = SampleState{0, fr, -1, 0, 0.0f, Z[fr], 0.0f, 0.0f};
        }
    }
    __syncthreads();
    const int fr = s_fr;
    if (fr < D) return;  // the residual kernels finish (block-uniform)
    // the bonus: sample the last row by a walk to u0 * Z over e (samplePrepared)
    float u0, u1;
    row_uniforms(a, fr, u0, u1);
    if (nucleus_on(a)) {
        if (t == 0) *a.nb.st = NucState{1, fr, fr, u0, Z[fr]};
        return;  // block-uniform
    }
    if (t == 0 && a.nb.st) a.nb.st->need = 0;
    walk_write(a, fr, fr, false, u0 * Z[fr], a.rowmax[fr] * a.invT, Z[fr], 0.0f, -1);
}

// Residual block sums of the rejected row (same chunk / block order as the e sums): one 64-thread
// block per 1024-element block, lane = chunk.
__global__ __launch_bounds__(64) void k_resid_sums(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const SampleState st = *a.state;
    if (st.phase != 1) return;
    const int b = blockIdx.x, lane = threadIdx.x;
    const int nch = (a.V + CH - 1) / CH;
    const int chunk = b * BLK + lane;
    const float mxs = a.rowmax[st.fr] * a.invT;
    float cs = 0.0f;
    if (chunk < nch) {
        const int e = min(chunk * CH + CH, a.V);
        for (int v = chunk * CH; v < e; ++v) cs = cs + r_at(a, st.fr, v, mxs, st.Zr, st.q, st.d);
    }
    __shared__ float sc[BLK];
    sc[lane] = cs;
    __syncthreads();
    if (lane == 0) {
        float bs = 0.0f;
        for (int c = 0; c < BLK; ++c)
            if (b * BLK + c < nch) bs = bs + sc[c];
        a.rbs[b] = bs;
    }
}

// The rejected row's sample: the residual total S, then a walk to u1 * S over the residual, or,
// with no residual mass, samplePrepared of the row (nucleus kernels, or a walk to u1 * Z over e).
__global__ __launch_bounds__(64) void k_resid_walk(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const SampleState st = *a.state;
    if (st.phase != 1) return;
    const int t = threadIdx.x;
    __shared__ float s_S;
    __shared__ float srb[MAX_CHUNKS / BLK];
    for (int b = t; b < a.nblocks; b += blockDim.x) srb[b] = a.rbs[b];
    __syncthreads();
    if (t == 0) {
        float S = 0.0f;
        for (int b = 0; b < a.nblocks; ++b) S = S + srb[b];
        s_S = S;
    }
    __syncthreads();
    const float S = s_S;
    float u0, u1;
    row_uniforms(a, st.fr, u0, u1);
    const bool walk_resid = S > 0.0f;
    if (nucleus_on(a) && !walk_resid) {
        if (t == 0) *a.nb.st = NucState{1, st.fr, st.fr, u1, st.Zr};
        return;  // block-uniform
    }
    if (t == 0 && a.nb.st) a.nb.st->need = 0;
    walk_write(a, st.fr, st.fr, walk_resid, walk_resid ? u1 * S : u1 * st.Zr,
               a.rowmax[st.fr] * a.invT, st.Zr, st.q, st.d);
}

// ---- nucleus (samplePrepared, LogitsProcessor.swift:137-164) --------------------------------
// Canonical sum and walk of n values f(i) by a 1024-thread block, in or_canon_sum /
// or_canon_walk's order: chunks of CH in order, blocks of BLK chunks in order, block totals in
// order; the walk finds the first block, then chunk, then element whose running total reaches
// tgt (the last index of the level otherwise).  cs / bs hold the chunk and block sums of f
// (blk_sum fills them for blk_walk).
template <class F>
__device__ float blk_sum(F f, int n, float* cs, float* bs, float* s_out) {
    const int t = threadIdx.x;
    const int nch = (n + CH - 1) / CH, nbk = (nch + BLK - 1) / BLK;
    for (int c = t; c < nch; c += 1024) {
        float sum = 0.0f;
        const int e = min(c * CH + CH, n);
        for (int v = c * CH; v < e; ++v) sum = sum + f(v);
        cs[c] = sum;
    }
    __syncthreads();
    for (int b = t; b < nbk; b += 1024) {
        float sum = 0.0f;
        for (int c = b * BLK; c < min(b * BLK + BLK, nch); ++c) sum = sum + cs[c];
        bs[b] = sum;
    }
    __syncthreads();
    if (t == 0) {
        float S = 0.0f;
        for (int b = 0; b < nbk; ++b) S = S + bs[b];
        *s_out = S;
    }
    __syncthreads();
    return *s_out;
}

template <class F>
__device__ int blk_walk(F f, int n, float tgt, const float* cs, const float* bs, int* s_out) {
    if (threadIdx.x == 0) {
        const int nch = (n + CH - 1) / CH, nbk = (nch + BLK - 1) / BLK;
        int res = n - 1;
        float P = 0.0f;
        for (int b = 0; b < nbk; ++b) {
            const float Pn = P + bs[b];
            if (tgt <= Pn) {
                const int c0 = b * BLK, c1 = min(c0 + BLK, nch);
                res = min(c1 * CH, n) - 1;
                float Q = P;
                for (int c = c0; c < c1; ++c) {
                    const float Qn = Q + cs[c];
                    if (tgt <= Qn) {
                        const int e = min(c * CH + CH, n);
                        res = e - 1;
                        float R = Q;
                        for (int v = c * CH; v < e; ++v) {
                            R = R + f(v);
                            if (tgt <= R) {
                                res = v;
                                break;
                            }
                        }
                        break;
                    }
                    Q = Qn;
                }
                break;
            }
            P = Pn;
        }
        *s_out = res;
    }
    __syncthreads();
    return *s_out;
}

// e bits and ids of the nucleus row (e >= 0: its bits order as the values do)
__global__ __launch_bounds__(256) void k_nucleus_keys(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const NucState st = *a.nb.st;
    if (!st.need) return;
    const int v = blockIdx.x * 256 + threadIdx.x;
    if (v >= a.V) return;
    a.nb.keys[v] = __float_as_uint(e_at(a, st.row, v, a.rowmax[st.row] * a.invT));
    a.nb.ids[v] = v;
}

// After the ranking (ids_s / keys_s: e descending, lower id first among equal e): the kept
// prefix, its mass in id order, and the sample.
__global__ __launch_bounds__(1024) void k_nucleus_pick(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const NucState st = *a.nb.st;
    if (!st.need) return;
    __shared__ float cs[MAX_CHUNKS];
    __shared__ float bs[MAX_CHUNKS / BLK];
    __shared__ float s_f;
    __shared__ int s_i;
    const float mxs = a.rowmax[st.row] * a.invT;
    const float tp = a.o.top_p < 0.0f ? 0.0f : (a.o.top_p > 1.0f ? 1.0f : a.o.top_p);
    const uint32_t* ks = a.nb.keys_s;
    const auto ranked = [&](int i) { return __uint_as_float(ks[i]); };
    blk_sum(ranked, a.V, cs, bs, &s_f);
    const int k = blk_walk(ranked, a.V, tp * st.Z, cs, bs, &s_i);
    const float es = ranked(k);
    const int is = a.nb.ids_s[k];
    const auto kept = [&](int v) {
        const float e = e_at(a, st.row, v, mxs);
        return (e > es || (e == es && v <= is)) ? e : 0.0f;
    };
    const float S = blk_sum(kept, a.V, cs, bs, &s_f);
    const int tok = S > 0.0f ? blk_walk(kept, a.V, st.u * S, cs, bs, &s_i) : a.nb.ids_s[0];
    if (threadIdx.x == 0) write_result(a, st.acc, tok);
}

static size_t sort_tmp_bytes(int V) {
    size_t b = 0;
    hipError_t e = hipcub::DeviceRadixSort::SortPairsDescending(
        nullptr, b, (const uint32_t*)nullptr, (uint32_t*)nullptr, (const int32_t*)nullptr,
        (int32_t*)nullptr, V, 0, 32, (hipStream_t)0);
    return e == hipSuccess ? b : 0;
}

static size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t nucleus_bytes(int V) {
    return 4 * up256((size_t)V * 4) + up256(sort_tmp_bytes(V)) + up256(sizeof(NucState));
}

void nucleus_layout(void* base, int V, NucleusBuf& nb) {
    char* p = (char*)base;
    const size_t row = up256((size_t)V * 4);
    nb.keys = (uint32_t*)p;
    nb.ids = (int32_t*)(p + row);
    nb.keys_s = (uint32_t*)(p + 2 * row);
    nb.ids_s = (int32_t*)(p + 3 * row);
    nb.tmp = p + 4 * row;
    nb.tmp_bytes = sort_tmp_bytes(V);
    nb.st = (NucState*)(p + 4 * row + up256(nb.tmp_bytes));
}

hipError_t launch_accept_sampled(float* logits, int rows, int V, const int32_t* draft,
                                 float temperature, int q_mode, const float* q_point,
                                 uint64_t seed, uint64_t counter, const SampleOpts& o,
                                 const NucleusBuf* nb, float* rowmax, float* bsum, int32_t* out,
                                 StepResult* res, const StepDesc* sd, const int* abort,
                                 hipStream_t st) {
    SampleArgs a{};
    a.sd = sd;
    a.logits = logits;
    a.rows = rows;
    a.V = V;
    a.draft = draft;
    a.invT = 1.0f / fmaxf(temperature, 1e-5f);
    a.q_mode = q_mode;
    a.q_uniform = 1.0f / (float)V;
    a.q_point = q_point;
    a.seed = seed;
    a.counter = counter;
    a.rowmax = rowmax;
    a.nblocks = ((V + CH - 1) / CH + BLK - 1) / BLK;
    // the bsum buffer (sample_scratch_floats, 16-byte aligned): the hand-off state, block sums,
    // partial maxima, residual block sums
    a.state = (SampleState*)bsum;
    a.bsum = bsum + 8;
    a.mpart = a.bsum + (size_t)rows * a.nblocks;
    a.rbs = a.mpart + (size_t)rows * RMB;
    a.out = out;
    a.res = res;
    a.abort = abort;
    a.o = o;
    if (nb) a.nb = *nb;
    if (V > MAX_CHUNKS * CH || rows > MJ_ROWS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_penalize, dim3(rows), dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_rowmax, dim3(rows * RMB), dim3(256), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_sample_sums, dim3(rows * a.nblocks), dim3(64), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_sample_decide, dim3(1), dim3(64), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_resid_sums, dim3(a.nblocks), dim3(64), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_resid_walk, dim3(1), dim3(64), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess || !nb) return e;
    hipLaunchKernelGGL(k_nucleus_keys, dim3((V + 255) / 256), dim3(256), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    size_t tb = nb->tmp_bytes;
    e = hipcub::DeviceRadixSort::SortPairsDescending(nb->tmp, tb, nb->keys, nb->keys_s, nb->ids,
                                                      nb->ids_s, V, 0, 32, st);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_nucleus_pick, dim3(1), dim3(1024), 0, st, a);
    return hipGetLastError();
}

int sample_nblocks(int V) { return ((V + CH - 1) / CH + BLK - 1) / BLK; }

// floats of the buffer passed as bsum: 8 for the state, rows x nblocks block sums, rows x RMB
// partial maxima, nblocks residual block sums
size_t sample_scratch_floats(int rows, int V) {
    const size_t nb = (size_t)sample_nblocks(V);
    return 8 + (size_t)rows * nb + (size_t)rows * RMB + nb;
}
