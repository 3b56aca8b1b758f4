// sample.hip -- full-vocabulary speculative sampling (rejection sampling) on the device.
//
// Rules: SpeculativeSampling.tryAccept / walkDraft (SpeculativeSampling.swift:27-99) with
// LogitsProcessor.probabilities / samplePrepared (LogitsProcessor.swift:116-189):
//   p = softmax(logits * (1/T));  accept draft d iff q > 0, p_d > 0 and u0 <= min(1, p_d / q);
//   on reject sample the residual (point q: p with p_d -> max(0, p_d - q); uniform q:
//   max(p - q, 0)) by a cumulative walk to u1 * sum; after a full accept sample the bonus from
//   the last row by a walk to u0 * sum of exps.
// Every float operation below happens in a fixed order (chunks of 16 summed sequentially,
// blocks of 64 chunks summed sequentially, block totals summed sequentially; exp evaluated by
// canon_expf; IEEE divisions) so the CPU oracle reproduces each decision bit for bit.
#pragma clang fp contract(off)
#include "mj_device.h"
#include "mj_internal.h"

#define CH 16
#define BLK 64
#define MAX_CHUNKS 12288  // V <= 196608

struct SampleArgs {
    const float* logits;   // [rows][V]
    int rows, V;
    const int32_t* draft;  // [rows-1]
    float invT;
    int q_mode;            // 0 point, 1 uniform
    float q_uniform;       // 1/V
    const float* q_point;  // [rows-1] or nullptr (= 1)
    uint64_t seed, counter;
    float* rowmax;         // [rows]
    float* bsum;           // [rows][nblocks]
    int nblocks;
    int32_t* out;          // [2] or nullptr
    StepResult* res;       // or nullptr
    const StepDesc* sd;    // when set: temperature, q, seed, counter and draft come from it
    const int* abort;
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
    }
    return a;
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

__global__ __launch_bounds__(1024) void k_rowmax(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const int row = blockIdx.x, t = threadIdx.x;
    float m = -INFINITY;
    for (int v = t; v < a.V; v += 1024) m = fmaxf(m, a.logits[(size_t)row * a.V + v]);
    m = wave_max(m);
    __shared__ float sm[16];
    if ((t & 63) == 0) sm[t >> 6] = m;
    __syncthreads();
    if (t == 0) {
        float b = sm[0];
        for (int w = 1; w < 16; ++w) b = fmaxf(b, sm[w]);
        a.rowmax[row] = b;
    }
}

// Block sums of e_v: one 64-thread block per (row, 1024-element block), lane = chunk.
__global__ __launch_bounds__(64) void k_sample_sums(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const int row = blockIdx.x / a.nblocks, b = blockIdx.x % a.nblocks;
    const int lane = threadIdx.x;
    const int nch = (a.V + CH - 1) / CH;
    const int chunk = b * BLK + lane;
    const float mxs = a.rowmax[row] * a.invT;
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

// Single block: totals, sequential accept decisions, then the residual or bonus walk.
__global__ __launch_bounds__(1024) void k_sample_decide(SampleArgs a) {
    if (aborted(a.abort)) return;
    a = resolve(a);
    const int t = threadIdx.x;
    const int D = a.rows - 1;
    const int nch = (a.V + CH - 1) / CH;
    __shared__ float Z[MJ_ROWS];
    __shared__ float cs[MAX_CHUNKS];
    __shared__ float bs[MAX_CHUNKS / BLK];
    __shared__ int s_fr, s_blk, s_bidx, s_tok;
    __shared__ float s_t, s_P;
    if (t < a.rows) {
        float z = 0.0f;
        for (int b = 0; b < a.nblocks; ++b) z = z + a.bsum[(size_t)t * a.nblocks + b];
        Z[t] = z;
    }
    __syncthreads();
    if (t == 0) {
        int fr = D;
        for (int i = 0; i < D; ++i) {
            const int d = a.draft[i];
            const float mxs = a.rowmax[i] * a.invT;
            const float p = (d >= 0 && d < a.V) ? __fdiv_rn(e_at(a, i, d, mxs), Z[i]) : 0.0f;
            float q = a.q_mode == 1 ? a.q_uniform : (a.q_point ? a.q_point[i] : 1.0f);
            q = fmaxf(0.0f, q);
            float u0, u1;
            row_uniforms(a, i, u0, u1);
            if (q > 0.0f && p > 0.0f && u0 <= fminf(1.0f, __fdiv_rn(p, q))) continue;
            fr = i;
            break;
        }
        s_fr = fr;
    }
    __syncthreads();
    const int fr = s_fr;
    // which mass is walked: residual of row fr (mode 1), or e of row fr / D (mode 0)
    int row = fr, walk_resid = 0, d = -1;
    float q = 0.0f;
    const float mxs = a.rowmax[row] * a.invT;
    float tgt = 0.0f;
    if (fr < D) {
        d = a.draft[fr];
        q = a.q_mode == 1 ? a.q_uniform : (a.q_point ? a.q_point[fr] : 1.0f);
        q = fmaxf(0.0f, q);
        for (int c = t; c < nch; c += 1024) {
            float s = 0.0f;
            const int e = min(c * CH + CH, a.V);
            for (int v = c * CH; v < e; ++v) s = s + r_at(a, row, v, mxs, Z[row], q, d);
            cs[c] = s;
        }
        __syncthreads();
        for (int b = t; b < a.nblocks; b += 1024) {
            float s = 0.0f;
            for (int c = b * BLK; c < min(b * BLK + BLK, nch); ++c) s = s + cs[c];
            bs[b] = s;
        }
        __syncthreads();
        if (t == 0) {
            float S = 0.0f;
            for (int b = 0; b < a.nblocks; ++b) S = S + bs[b];
            float u0, u1;
            row_uniforms(a, row, u0, u1);
            s_t = S > 0.0f ? u1 * S : u1 * Z[row];
            s_blk = S > 0.0f ? 1 : 0;
        }
        __syncthreads();
        walk_resid = s_blk;
        tgt = s_t;
    } else {
        if (t == 0) {
            float u0, u1;
            row_uniforms(a, row, u0, u1);
            s_t = u0 * Z[row];
        }
        __syncthreads();
        tgt = s_t;
    }
    // block level
    if (t == 0) {
        float P = 0.0f;
        int blk = -1;
        for (int b = 0; b < a.nblocks; ++b) {
            const float bsv = walk_resid ? bs[b] : a.bsum[(size_t)row * a.nblocks + b];
            const float Pn = P + bsv;
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
        // chunk sums of the chosen block (e-walk recomputes them; residual has them)
        if (!walk_resid && t < BLK) {
            const int c = blk * BLK + t;
            float s = 0.0f;
            if (c < nch) {
                const int e = min(c * CH + CH, a.V);
                for (int v = c * CH; v < e; ++v) s = s + e_at(a, row, v, mxs);
            }
            cs[c < MAX_CHUNKS ? c : 0] = s;
        }
        __syncthreads();
        if (t == 0) {
            const int c0 = blk * BLK, c1 = min(c0 + BLK, nch);
            float Q = s_P;
            int tok = min(c1 * CH, a.V) - 1;
            for (int c = c0; c < c1; ++c) {
                const float Qn = Q + cs[c];
                if (tgt <= Qn) {
                    float R = Q;
                    const int e = min(c * CH + CH, a.V);
                    tok = e - 1;
                    for (int v = c * CH; v < e; ++v) {
                        R = R + (walk_resid ? r_at(a, row, v, mxs, Z[row], q, d)
                                            : e_at(a, row, v, mxs));
                        if (tgt <= R) {
                            tok = v;
                            break;
                        }
                    }
                    break;
                }
                Q = Qn;
            }
            s_tok = tok;
        }
        __syncthreads();
    }
    if (t == 0) {
        const int acc = fr;
        const int tok = s_tok;
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
}

hipError_t launch_accept_sampled(const float* logits, int rows, int V, const int32_t* draft,
                                 float temperature, int q_mode, const float* q_point,
                                 uint64_t seed, uint64_t counter, float* rowmax, float* bsum,
                                 int32_t* out, StepResult* res, const StepDesc* sd,
                                 const int* abort, hipStream_t st) {
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
    a.bsum = bsum;
    a.nblocks = ((V + CH - 1) / CH + BLK - 1) / BLK;
    a.out = out;
    a.res = res;
    a.abort = abort;
    hipLaunchKernelGGL(k_rowmax, dim3(rows), dim3(1024), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_sample_sums, dim3(rows * a.nblocks), dim3(64), 0, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_sample_decide, dim3(1), dim3(1024), 0, st, a);
    return hipGetLastError();
}

int sample_nblocks(int V) { return ((V + CH - 1) / CH + BLK - 1) / BLK; }
