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
// mass reaches top_p * Z, sampled in id order.  The masses are summed exactly, as integers
// trunc(e * 2^40), so no order is needed: the cut is found by a radix selection over the e bits
// (four 8-bit digit rounds of histograms of counts and masses), not by sorting the row.
// Every float operation below happens in a fixed order (chunks of 16 summed sequentially,
// blocks of 64 chunks summed sequentially, block totals summed sequentially; exp evaluated by
// canon_expf; IEEE divisions) so the CPU oracle reproduces each decision bit for bit.
#pragma clang fp contract(off)
#include "mj_device.h"
#include "mj_internal.h"

#define CH 16
#define BLK 64
#define MAX_CHUNKS 12288  // V <= 196608
#define RMB 32            // blocks a row's maximum is split over
#define DEC_STAGE (MJ_ROWS * (MAX_CHUNKS / BLK))  // every row's block sums, in LDS

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
    const float* head_max; // [rows] row maxima already known (no penalties), or nullptr
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
// among drafts 0 .. i-1).  One block per row; each token is written by one thread.  The drafts
// sit in LDS; a history entry counts its matches there and marks the drafts it equals (so a
// draft learns whether the history holds it without searching it); history entries and their
// logits are requested eight a thread at a time.
__global__ __launch_bounds__(256) void k_penalize(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const bool rep_on = fabsf(a.o.rep - 1.0f) > 1e-6f && a.o.rep > 0.0f;
    if (!rep_on && a.o.pres == 0.0f && a.o.freq == 0.0f) return;
    const int i = blockIdx.x, t = threadIdx.x;
    float* l = a.logits + (size_t)i * a.V;
    __shared__ int s_draft[MJ_ROWS];
    __shared__ int s_inh[MJ_ROWS];  // draft d equals a history token
    if (t < i) s_draft[t] = a.draft[t];
    if (t < MJ_ROWS) s_inh[t] = 0;
    __syncthreads();
    const int nh = a.o.n_hist;
    for (int j0 = t; j0 < nh; j0 += 256 * 8) {
        int tok[8], cnt[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int j = min(j0 + 256 * u, nh - 1);
            tok[u] = a.o.hist_tok[j];
            cnt[u] = a.o.hist_cnt[j];
        }
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const bool ok = j0 + 256 * u < nh && tok[u] >= 0 && tok[u] < a.V;
            x[u] = ok ? l[tok[u]] : 0.0f;
            for (int d = 0; d < i; ++d)
                if (s_draft[d] == tok[u] && j0 + 256 * u < nh) {
                    ++cnt[u];
                    s_inh[d] = 1;
                }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (j0 + 256 * u < nh && tok[u] >= 0 && tok[u] < a.V)
                l[tok[u]] = penalize1(x[u], cnt[u], a.o.rep, a.o.pres, a.o.freq);
    }
    __syncthreads();
    for (int d = t; d < i; d += 256) {
        const int tok = s_draft[d];
        if (tok < 0 || tok >= a.V || s_inh[d]) continue;
        bool first = true;
        for (int e = 0; e < d; ++e) first = first && s_draft[e] != tok;
        if (!first) continue;
        int c = 0;
        for (int e = 0; e < i; ++e) c += s_draft[e] == tok;
        l[tok] = penalize1(l[tok], c, a.o.rep, a.o.pres, a.o.freq);
    }
}

__device__ __forceinline__ void row_uniforms(const SampleArgs& a, int row, float& u0, float& u1) {
    uint32_t c[4] = {(uint32_t)row, (uint32_t)a.counter, (uint32_t)(a.counter >> 32), 0x6d6a6a76u};
    philox4x32_10(c, (uint32_t)a.seed, (uint32_t)(a.seed >> 32));
    u0 = u01(c[0]);
    u1 = u01(c[1]);
}

__device__ __forceinline__ float e_of(const SampleArgs& a, float x, float mxs) {
    const float s = x * a.invT;
    return canon_expf(s - mxs);
}

__device__ __forceinline__ float e_at(const SampleArgs& a, int row, int v, float mxs) {
    return e_of(a, a.logits[(size_t)row * a.V + v], mxs);
}

// residual mass at v given e_v (p_v = e_v / Z)
__device__ __forceinline__ float r_of(const SampleArgs& a, float e, int v, float Z, float q,
                                      int d) {
    const float pv = __fdiv_rn(e, Z);
    if (a.q_mode == 1) return fmaxf(pv - q, 0.0f);
    if (v == d && q > 0.0f) return fmaxf(0.0f, pv - q);
    return pv;
}

// Rows of 16-byte aligned logits (float4 requests) or not (one float a request).
__device__ __forceinline__ bool rows_aligned(const SampleArgs& a) {
    return ((a.V & 3) | ((uintptr_t)a.logits & 15)) == 0;
}

// The CH logits of chunk c of a row, requested together; indices past the row's end clamp to
// its last element (callers use only those below V).
__device__ __forceinline__ void chunk_logits(const SampleArgs& a, int row, int c, float x[CH]) {
    const float* rp = a.logits + (size_t)row * a.V;
    if (rows_aligned(a)) {
        const float4* p4 = (const float4*)rp;
        const int last = (a.V >> 2) - 1;
#pragma unroll
        for (int k = 0; k < CH / 4; ++k) {
            const float4 f = p4[min(c * (CH / 4) + k, last)];
            x[4 * k] = f.x;
            x[4 * k + 1] = f.y;
            x[4 * k + 2] = f.z;
            x[4 * k + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < CH; ++k) x[k] = rp[min(c * CH + k, a.V - 1)];
    }
}

// Chunk c's element values -- e, or the residual (resid) -- into x, and their sum in element
// order.
__device__ __forceinline__ float chunk_vals(const SampleArgs& a, int row, int c, bool resid,
                                            float mxs, float Z, float q, int d, float x[CH]) {
    chunk_logits(a, row, c, x);
    const int v0 = c * CH;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < CH; ++k) {
        float e = e_of(a, x[k], mxs);
        if (resid) e = r_of(a, e, v0 + k, Z, q, d);
        x[k] = e;
        if (v0 + k < a.V) s = s + e;
    }
    return s;
}

// n >= 1 floats from src into LDS by nt threads, eight requests a thread in flight.
__device__ __forceinline__ void stage_lds(float* dst, const float* src, int n, int t, int nt) {
    for (int base = t; base < n; base += nt * 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = src[min(base + nt * k, n - 1)];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (base + nt * k < n) dst[base + nt * k] = v[k];
    }
}

// One thread: p[0..n) (n >= 1) replaced by its running totals in order, p[b] = ((p_0 + p_1) +
// ...) + p_b from 0.0f; returns the total.
__device__ __forceinline__ float running_totals(float* p, int n) {
    float z = 0.0f;
    for (int b0 = 0; b0 < n; b0 += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = p[min(b0 + k, n - 1)];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (b0 + k < n) {
                z = z + v[k];
                p[b0 + k] = z;
            }
    }
    return z;
}

// First lane of the (whole, converged) wave whose `hit` holds, or -1.
__device__ __forceinline__ int wave_first(bool hit) {
    const uint64_t m = __ballot(hit);
    return m ? __ffsll((unsigned long long)m) - 1 : -1;
}

// Row maxima in RMB slices a row (a maximum is exact in any order): block (row, j) writes the
// maximum of its slice; the sums kernel folds the RMB partials.  A thread requests its whole
// share of the slice at once (indices clamp to the slice's last element, and a repeated element
// leaves a maximum unchanged).
#define RM_UNROLL 6  // float4 requests a thread: a slice of V / RMB <= 6144 floats in one round
__global__ __launch_bounds__(256) void k_rowmax(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const int row = blockIdx.x / RMB, j = blockIdx.x % RMB, t = threadIdx.x;
    const float* rp = a.logits + (size_t)row * a.V;
    float m = -INFINITY;
    if (rows_aligned(a)) {
        const int V4 = a.V >> 2, span = (V4 + RMB - 1) / RMB;
        const int v0 = j * span, v1 = min(V4, v0 + span);
        const float4* p4 = (const float4*)rp;
        for (int v = v0 + t; v < v1; v += 256 * RM_UNROLL) {
            float4 f[RM_UNROLL];
#pragma unroll
            for (int k = 0; k < RM_UNROLL; ++k) f[k] = p4[min(v + 256 * k, v1 - 1)];
#pragma unroll
            for (int k = 0; k < RM_UNROLL; ++k)
                m = fmaxf(m, fmaxf(fmaxf(f[k].x, f[k].y), fmaxf(f[k].z, f[k].w)));
        }
    } else {
        const int span = (a.V + RMB - 1) / RMB;
        const int v0 = j * span, v1 = min(a.V, v0 + span);
        for (int v = v0 + t; v < v1; v += 256 * 8) {
            float f[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) f[k] = rp[min(v + 256 * k, v1 - 1)];
#pragma unroll
            for (int k = 0; k < 8; ++k) m = fmaxf(m, f[k]);
        }
    }
    m = wave_max(m);
    __shared__ float sm[4];
    if ((t & 63) == 0) sm[t >> 6] = m;
    __syncthreads();
    if (t == 0) a.mpart[row * RMB + j] = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
}

// Block sums of e_v: one 64-thread block per (row, 1024-element block), lane = chunk.  The
// row maximum (the lm_head's, or folded from the partial maxima) and the chunk's logits are
// requested together (clamped indices: every lane loads, lanes past the end contribute nothing).
__global__ __launch_bounds__(64) void k_sample_sums(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const int row = blockIdx.x / a.nblocks, b = blockIdx.x % a.nblocks;
    const int lane = threadIdx.x;
    const int nch = (a.V + CH - 1) / CH;
    const int chunk = b * BLK + lane;
    float x[CH];
    chunk_logits(a, row, min(chunk, nch - 1), x);
    float mx;
    if (a.head_max)
        mx = a.head_max[row];
    else
        mx = wave_max(a.mpart[row * RMB + (lane & (RMB - 1))]);
    if (b == 0 && lane == 0) a.rowmax[row] = mx;
    const float mxs = mx * a.invT;
    const int v0 = chunk * CH;
    float cs = 0.0f;
#pragma unroll
    for (int k = 0; k < CH; ++k) {
        const float e = e_of(a, x[k], mxs);
        if (v0 + k < a.V) cs = cs + e;
    }
    __shared__ float s[BLK];
    s[lane] = chunk < nch ? cs : 0.0f;
    __syncthreads();
    if (lane == 0) {
        float bs = 0.0f;
        for (int c = 0; c < BLK; ++c)
            if (b * BLK + c < nch) bs = bs + s[c];
        a.bsum[(size_t)row * a.nblocks + b] = bs;
    }
}

// The outcome (acc drafts accepted, then tok), written by the 64 lanes of one wave: lane i
// writes path[i] and emit[i] (the accepted drafts are read together).
__device__ __forceinline__ void write_result(const SampleArgs& a, int acc, int tok) {
    const int i = threadIdx.x & 63;
    if (a.out && i == 0) {
        a.out[0] = acc;
        a.out[1] = tok;
    }
    if (a.res) {
        if (i == 0) {
            a.res->accepted = acc;
            a.res->token = tok;
        }
        if (i <= acc) {
            a.res->path[i] = i;
            a.res->emit[i] = i < acc ? a.draft[i] : tok;
        }
    }
}

// Walk of row `row` to tgt over its mass -- the residual (resid) or e -- given the running
// totals of its block sums (pref[b] = ((s_0 + s_1) + ...) + s_b, the totals a sequential walk
// forms): the first block whose running total reaches tgt (the last element if none), in it the
// first chunk (the block's 64 chunk sums recomputed in the same order, running on from the total
// before the block; the block's last element if none), then the first element of that chunk;
// writes (fr, token).  Block of 256 threads; the block's chunk sums and element values are
// computed once, and the running totals of a level are formed redundantly by every lane of
// wave 0 so that the first lane reaching tgt is found by one ballot.
__device__ void walk_write(const SampleArgs& a, int row, int fr, bool resid, float tgt,
                           const float* pref, float mxs, float Zr, float q, int d) {
    const int t = threadIdx.x;
    const int nch = (a.V + CH - 1) / CH, nb = a.nblocks;
    __shared__ __align__(16) float cs[BLK];
    __shared__ __align__(16) float ev[BLK][CH + 4];
    __shared__ int s_blk;
    if (t == 0) s_blk = nb;
    __syncthreads();
    if (t < nb && tgt <= pref[t]) atomicMin(&s_blk, t);  // nb <= MAX_CHUNKS / BLK <= 256
    __syncthreads();
    const int blk = s_blk;
    if (blk == nb) {  // block-uniform
        if (t < 64) write_result(a, fr, a.V - 1);
        return;
    }
    const int c0 = blk * BLK, n = min(BLK, nch - c0);
    const float P = blk > 0 ? pref[blk - 1] : 0.0f;
    if (t < BLK) {
        float x[CH];
        const float s = chunk_vals(a, row, min(c0 + t, nch - 1), resid, mxs, Zr, q, d, x);
        cs[t] = s;
        float4* e4 = (float4*)ev[t];
#pragma unroll
        for (int k = 0; k < CH / 4; ++k)
            e4[k] = make_float4(x[4 * k], x[4 * k + 1], x[4 * k + 2], x[4 * k + 3]);
    }
    __syncthreads();
    if (t >= 64) return;  // wave 0 finishes (wave-uniform)
    // chunk level: lane k keeps the running total after chunk k
    float Q = P, Qk = 0.0f;
#pragma unroll
    for (int k = 0; k < BLK; ++k) {
        Q = Q + cs[k];
        Qk = t == k ? Q : Qk;
    }
    const int ci = wave_first(t < n && tgt <= Qk);
    int tok;
    if (ci < 0) {
        tok = min((c0 + n) * CH, a.V) - 1;
    } else {
        const int cc = c0 + ci;
        const int ne = min(CH, a.V - cc * CH);
        float R = ci > 0 ? __shfl(Qk, ci - 1) : P, Rk = 0.0f;
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            R = R + ev[ci][k];
            Rk = t == k ? R : Rk;
        }
        const int ei = wave_first(t < ne && tgt <= Rk);
        tok = cc * CH + (ei < 0 ? ne - 1 : ei);
    }
    write_result(a, fr, tok);  // wave 0
}

// Single block: row totals (with their running totals kept for a walk) and the accept
// decisions, one row a lane; the first rejected row ends the chain.  A full accept samples the
// bonus here (or leaves it to the nucleus kernels); a reject hands row fr to k_resid_sums /
// k_resid_walk through the state.
__global__ __launch_bounds__(256) void k_sample_decide(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const int t = threadIdx.x;
    const int D = a.rows - 1;
    const int per = a.nblocks;
    __shared__ float Z[MJ_ROWS];
    __shared__ float pref[DEC_STAGE];  // row r's block sums at r * per, then their running totals
    __shared__ int s_fr;
    // the drafts' e values and every row's block sums, requested together
    int d = -1;
    float ed = 0.0f;
    if (t < D) {
        d = a.draft[t];
        if (d >= 0 && d < a.V)
            ed = e_of(a, a.logits[(size_t)t * a.V + d], a.rowmax[t] * a.invT);
    }
    stage_lds(pref, a.bsum, a.rows * per, t, 256);
    __syncthreads();
    if (t < a.rows) Z[t] = running_totals(pref + t * per, per);
    __syncthreads();
    if (t < 64) {  // wave 0: one draft a lane (D < MJ_ROWS == 64)
        bool rej = false;
        if (t < D) {
            const float p = (d >= 0 && d < a.V) ? __fdiv_rn(ed, Z[t]) : 0.0f;
            float q = a.q_mode == 1 ? a.q_uniform : (a.q_point ? a.q_point[t] : 1.0f);
            q = fmaxf(0.0f, q);
            float u0, u1;
            row_uniforms(a, t, u0, u1);
            rej = !(q > 0.0f && p > 0.0f && u0 <= fminf(1.0f, __fdiv_rn(p, q)));
        }
        const int f = wave_first(rej);
        const int fr = f < 0 ? D : f;
        if (t == 0) {
            s_fr = fr;
            if (fr < D) {
                float q = a.q_mode == 1 ? a.q_uniform : (a.q_point ? a.q_point[fr] : 1.0f);
                *a.state = SampleState{1, fr, a.draft[fr], 0, fmaxf(0.0f, q), Z[fr], 0.0f, 0.0f};
            } else {
                *a.state = SampleState{0, fr, -1, 0, 0.0f, Z[fr], 0.0f, 0.0f};
            }
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
    walk_write(a, fr, fr, false, u0 * Z[fr], pref + fr * per, a.rowmax[fr] * a.invT, Z[fr],
               0.0f, -1);
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
    float x[CH];
    const float cs = chunk_vals(a, st.fr, min(chunk, nch - 1), true, mxs, st.Zr, st.q, st.d, x);
    __shared__ float sc[BLK];
    sc[lane] = chunk < nch ? cs : 0.0f;
    __syncthreads();
    if (lane == 0) {
        float bs = 0.0f;
        for (int c = 0; c < BLK; ++c)
            if (b * BLK + c < nch) bs = bs + sc[c];
        a.rbs[b] = bs;
    }
}

// The rejected row's sample: the residual total S, then a walk to u1 * S over the residual, or,
// with no residual mass, samplePrepared of the row (nucleus kernels, or a walk to u1 * Z over e
// with the row's block sums).
__global__ __launch_bounds__(256) void k_resid_walk(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const SampleState st = *a.state;
    const int t = threadIdx.x;
    // the nucleus selection's first histogram starts empty (its kernel adds to it next)
    if (a.nb.st) {
        a.nb.hcnt[t] = 0u;
        a.nb.hmass[t] = 0ull;
    }
    if (st.phase != 1) return;
    __shared__ float s_S;
    __shared__ float pref[MAX_CHUNKS / BLK];
    stage_lds(pref, a.rbs, a.nblocks, t, 256);
    __syncthreads();
    if (t == 0) s_S = running_totals(pref, a.nblocks);
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
    if (!walk_resid) {  // block-uniform: the row's e block sums instead
        stage_lds(pref, a.bsum + (size_t)st.fr * a.nblocks, a.nblocks, t, 256);
        __syncthreads();
        if (t == 0) running_totals(pref, a.nblocks);
        __syncthreads();
    }
    walk_write(a, st.fr, st.fr, walk_resid, walk_resid ? u1 * S : u1 * st.Zr, pref,
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

// ---- nucleus cut by radix selection -------------------------------------------------------
// The e of the nucleus row are non-negative floats, so their bits order as their values.  Round
// r (0..3) histograms digit r (bits 31 - 8r .. 24 - 8r) of the keys that match the digits
// already chosen: a count and an exact mass (sum of trunc(e * 2^40)) per digit value.  Scanning a
// round's digits from the top, the cut lies in the first digit whose mass, added to the mass
// of the keys above it, reaches the target; after four rounds the cut key is known exactly,
// and among the keys equal to it (ties, taken in id order) the cut is the j-th, j the fewest
// that reach the target.  NUC_BLOCKS blocks of 256 threads cover up to NUC_BLOCKS * 2048 ids,
// block b ids [2048 b, 2048 b + 2048); the last round also keeps each block's digit counts so
// the j-th tie is found without another pass.
#define NUC_BLOCKS 96
#define NUC_PER_BLOCK 2048

__device__ __forceinline__ uint64_t nuc_fixed(float e) {
    return (uint64_t)(e * 0x1p40f);  // exact scaling, then truncation (e <= 1)
}

// The selection state after rounds 0 .. r - 1: the chosen digits (prefix) and the mass of the
// keys ranked above them; false when the target exceeds the row's whole mass (every key kept).
__device__ bool nuc_prefix(const NucleusBuf& nb, int r, uint64_t F, uint32_t& prefix,
                           uint64_t& above) {
    prefix = 0u;
    above = 0ull;
    for (int rr = 0; rr < r; ++rr) {
        const uint32_t* cnt = nb.hcnt + 256 * rr;
        const uint64_t* mass = nb.hmass + 256 * rr;
        int d = 255;
        for (; d >= 0; --d) {
            if (cnt[d] == 0u) continue;
            if (above + mass[d] >= F) break;
            above += mass[d];
        }
        if (d < 0) return false;
        prefix = (prefix << 8) | (uint32_t)d;
    }
    return true;
}

__device__ __forceinline__ uint64_t nuc_target(const SampleArgs& a, float Z) {
    const float tp = a.o.top_p < 0.0f ? 0.0f : (a.o.top_p > 1.0f ? 1.0f : a.o.top_p);
    return nuc_fixed(tp * Z);
}

// Round R of the selection; round 0 also computes the row's keys (e bits).
template <int R>
__global__ __launch_bounds__(256) void k_nucleus_round(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const int t = threadIdx.x, b = blockIdx.x;
    // the next round's histogram starts empty
    if constexpr (R < 3) {
        if (b == 0) {
            a.nb.hcnt[256 * (R + 1) + t] = 0u;
            a.nb.hmass[256 * (R + 1) + t] = 0ull;
        }
    }
    const NucState st = *a.nb.st;
    if (!st.need) return;
    __shared__ uint32_t s_cnt[256];
    __shared__ unsigned long long s_mass[256];
    s_cnt[t] = 0u;
    s_mass[t] = 0ull;
    uint32_t prefix = 0u;
    uint64_t above = 0ull;
    bool some = true;
    if constexpr (R > 0) some = nuc_prefix(a.nb, R, nuc_target(a, st.Z), prefix, above);
    __syncthreads();
    if (!some) return;  // block-uniform: every key is kept
    const float mxs = a.rowmax[st.row] * a.invT;
#pragma unroll
    for (int i = 0; i < NUC_PER_BLOCK / 256; ++i) {
        const int v = b * NUC_PER_BLOCK + 256 * i + t;
        if (v >= a.V) break;
        uint32_t key;
        if constexpr (R == 0) {
            key = __float_as_uint(e_at(a, st.row, v, mxs));
            a.nb.keys[v] = key;
        } else {
            key = a.nb.keys[v];
            if ((key >> (32 - 8 * R)) != prefix) continue;
        }
        const int d = (key >> (24 - 8 * R)) & 255;
        atomicAdd(&s_cnt[d], 1u);
        atomicAdd(&s_mass[d], (unsigned long long)nuc_fixed(__uint_as_float(key)));
    }
    __syncthreads();
    if (s_cnt[t] != 0u) {
        atomicAdd(a.nb.hcnt + 256 * R + t, s_cnt[t]);
        atomicAdd((unsigned long long*)(a.nb.hmass + 256 * R + t), s_mass[t]);
    }
    if constexpr (R == 3) a.nb.hblk[256 * b + t] = s_cnt[t];
}

// The cut (key and id), the kept mass in id order and the sample.
__global__ __launch_bounds__(1024) void k_nucleus_pick(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const NucState st = *a.nb.st;
    if (!st.need) return;
    __shared__ float cs[MAX_CHUNKS];
    __shared__ float bs[MAX_CHUNKS / BLK];
    __shared__ float s_f;
    __shared__ int s_i;
    __shared__ int s_wsum[16];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    uint32_t ck = 0u;   // the cut key
    int cid = a.V - 1;  // the cut id: with every key kept, the last
    uint64_t above = 0ull;
    const uint64_t F = nuc_target(a, st.Z);
    if (nuc_prefix(a.nb, 4, F, ck, above)) {
        // ties of the cut key, in id order: j of them reach the target (at least one)
        const uint64_t m = nuc_fixed(__uint_as_float(ck));
        const uint64_t need = F > above ? F - above : 0ull;
        const int j = need == 0ull ? 1 : (int)((need + m - 1) / m);
        // the block holding the j-th tie, and its rank there (every thread scans the counts)
        const int d = ck & 255;
        int b = 0, before = 0;
        for (; b < NUC_BLOCKS; ++b) {
            const int c = (int)a.nb.hblk[256 * b + d];
            if (before + c >= j) break;
            before += c;
        }
        const int jl = j - before;
        // two ids a thread of that block's range, counted by a block-wide prefix
        const int v0 = b * NUC_PER_BLOCK + 2 * t;
        const bool h0 = v0 < a.V && a.nb.keys[v0] == ck;
        const bool h1 = v0 + 1 < a.V && a.nb.keys[v0 + 1] == ck;
        const int c = (int)h0 + (int)h1;
        int incl = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o, MJ_WAVE);
            if (lane >= o) incl += y;
        }
        if (lane == 63) s_wsum[wv] = incl;
        __syncthreads();
        int off = 0;
        for (int w = 0; w < wv; ++w) off += s_wsum[w];
        const int ex = off + incl - c;
        if (c > 0 && ex < jl && jl <= ex + c) s_i = (h0 && ex + 1 == jl) ? v0 : v0 + 1;
        __syncthreads();
        cid = s_i;
    }
    const float mxs = a.rowmax[st.row] * a.invT;
    const uint32_t* keys = a.nb.keys;
    const auto kept = [&](int v) {
        const uint32_t k = keys[v];
        return (k > ck || (k == ck && v <= cid)) ? __uint_as_float(k) : 0.0f;
    };
    const float S = blk_sum(kept, a.V, cs, bs, &s_f);
    int tok;
    if (S > 0.0f) {
        tok = blk_walk(kept, a.V, st.u * S, cs, bs, &s_i);
    } else {  // the top-ranked token: the largest key, the lowest id among equal keys
        uint32_t bk = 0u;
        int bi = a.V;
        for (int v = t; v < a.V; v += 1024) {
            const uint32_t k = keys[v];
            if (k > bk || (k == bk && v < bi)) {
                bk = k;
                bi = v;
            }
        }
        if (t == 0) s_i = a.V;
        __syncthreads();
        for (int w = 0; w < 16; ++w) {  // fixed order: wave by wave through LDS
            __syncthreads();
            if (wv == w) {
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) {
                    const uint32_t ok = __shfl_xor(bk, o, MJ_WAVE);
                    const int oi = __shfl_xor(bi, o, MJ_WAVE);
                    if (ok > bk || (ok == bk && oi < bi)) {
                        bk = ok;
                        bi = oi;
                    }
                }
                if (lane == 0) {
                    const int pi = s_i;
                    const uint32_t pk = pi < a.V ? keys[pi] : 0u;
                    if (pi >= a.V || bk > pk || (bk == pk && bi < pi)) s_i = bi;
                }
            }
        }
        __syncthreads();
        tok = s_i < a.V ? s_i : 0;
    }
    if (t < 64) write_result(a, st.acc, tok);
}

static size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t nucleus_bytes(int V) {
    return up256((size_t)V * 4) + up256(4 * 256 * 4) + up256(4 * 256 * 8) +
           up256((size_t)NUC_BLOCKS * 256 * 4) + up256(sizeof(NucState));
}

void nucleus_layout(void* base, int V, NucleusBuf& nb) {
    char* p = (char*)base;
    nb.keys = (uint32_t*)p;
    p += up256((size_t)V * 4);
    nb.hcnt = (uint32_t*)p;
    p += up256(4 * 256 * 4);
    nb.hmass = (uint64_t*)p;
    p += up256(4 * 256 * 8);
    nb.hblk = (uint32_t*)p;
    p += up256((size_t)NUC_BLOCKS * 256 * 4);
    nb.st = (NucState*)p;
}

hipError_t launch_accept_sampled(float* logits, int rows, int V, const int32_t* draft,
                                 float temperature, int q_mode, const float* q_point,
                                 uint64_t seed, uint64_t counter, const SampleOpts& o,
                                 const NucleusBuf* nb, float* rowmax, float* bsum, int32_t* out,
                                 StepResult* res, const StepDesc* sd, const int* abort,
                                 hipStream_t st, const float* head_max) {
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
    a.head_max = head_max;
    if (V > MAX_CHUNKS * CH || V > NUC_BLOCKS * NUC_PER_BLOCK || rows > MJ_ROWS)
        return hipErrorInvalidValue;
    hipError_t e = hipSuccess;
    if (!head_max) {
        hipLaunchKernelGGL(k_penalize, dim3(rows), dim3(256), 0, st, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_rowmax, dim3(rows * RMB), dim3(256), 0, st, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_sample_sums, dim3(rows * a.nblocks), dim3(64), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_sample_decide, dim3(1), dim3(256), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_resid_sums, dim3(a.nblocks), dim3(64), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_resid_walk, dim3(1), dim3(256), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess || !nb) return e;
    hipLaunchKernelGGL(k_nucleus_round<0>, dim3(NUC_BLOCKS), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_nucleus_round<1>, dim3(NUC_BLOCKS), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_nucleus_round<2>, dim3(NUC_BLOCKS), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_nucleus_round<3>, dim3(NUC_BLOCKS), dim3(256), 0, st, a);
    e = hipGetLastError();
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
