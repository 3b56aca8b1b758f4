// moe_topk.h -- the router's per-row top-k (maple_route_top8, SeedlessMetal.swift:2720-2791):
// softmax with max subtraction, top-k by logit with the lowest index winning ties, weights
// renormalised over the k in rank order.  Shared by the route kernel and the up gather's fused
// routing prologue, so both give the same bits.
#pragma once
#include "mj_device.h"

// Wave-wide reductions for the top-k, in DPP lane moves instead of LDS-routed shuffles: xor 1
// and xor 2 inside each quad, the half-row and row mirrors (so every lane of a row of 16 holds
// the row's result), then the four rows' results combined from lanes 0, 16, 32 and 48.  Every
// lane returns the same value.
template <class T>
__device__ __forceinline__ T dpp_move(T v, int ctrl);
template <>
__device__ __forceinline__ float dpp_move<float>(float v, int ctrl) {
    const int x = __float_as_int(v);
    int r;
    switch (ctrl) {  // the control word has to be a constant
        case 0xB1: r = __builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false); break;
        case 0x4E: r = __builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false); break;
        case 0x141: r = __builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, false); break;
        default: r = __builtin_amdgcn_update_dpp(x, x, 0x140, 0xF, 0xF, false); break;
    }
    return __int_as_float(r);
}
template <>
__device__ __forceinline__ uint64_t dpp_move<uint64_t>(uint64_t v, int ctrl) {
    const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
    int a, b;
    switch (ctrl) {
        case 0xB1:
            a = __builtin_amdgcn_update_dpp(lo, lo, 0xB1, 0xF, 0xF, false);
            b = __builtin_amdgcn_update_dpp(hi, hi, 0xB1, 0xF, 0xF, false);
            break;
        case 0x4E:
            a = __builtin_amdgcn_update_dpp(lo, lo, 0x4E, 0xF, 0xF, false);
            b = __builtin_amdgcn_update_dpp(hi, hi, 0x4E, 0xF, 0xF, false);
            break;
        case 0x141:
            a = __builtin_amdgcn_update_dpp(lo, lo, 0x141, 0xF, 0xF, false);
            b = __builtin_amdgcn_update_dpp(hi, hi, 0x141, 0xF, 0xF, false);
            break;
        default:
            a = __builtin_amdgcn_update_dpp(lo, lo, 0x140, 0xF, 0xF, false);
            b = __builtin_amdgcn_update_dpp(hi, hi, 0x140, 0xF, 0xF, false);
            break;
    }
    return ((uint64_t)(uint32_t)b << 32) | (uint32_t)a;
}
__device__ __forceinline__ float lane_value(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ uint64_t lane_value(uint64_t v, int l) {
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((uint64_t)hi << 32) | lo;
}
template <class T, class Op>
__device__ __forceinline__ T wave_reduce_dpp(T v, Op op) {
    v = op(v, dpp_move(v, 0xB1));   // quad_perm [1,0,3,2]
    v = op(v, dpp_move(v, 0x4E));   // quad_perm [2,3,0,1]
    v = op(v, dpp_move(v, 0x141));  // row_half_mirror
    v = op(v, dpp_move(v, 0x140));  // row_mirror
    return op(op(lane_value(v, 0), lane_value(v, 16)), op(lane_value(v, 32), lane_value(v, 48)));
}

// Rank of lane's expert in a row of at most 64 (s_row: the row's logits padded with -inf to
// 64): experts ahead of it -- a larger logit, or an equal logit at a lower index.  The row is
// read as broadcast float4s issued together and "larger" counted from the sign of l - o (exact
// for distinct finite values, +0 for equal ones; -0 was folded into +0 when the row was
// staged).  Without ties the counts of the E experts are a permutation of 0..E-1; any other sum
// sends the row through the exact comparison rule.  Padding is -inf, which no real logit is
// below.
__device__ __forceinline__ int row_rank64(const float* s_row, int E) {
    const int lane = threadIdx.x & 63;
    const auto add_op = [](float x, float y) { return x + y; };
    const float l = s_row[lane];
    f4 o[16];
#pragma unroll
    for (int j4 = 0; j4 < 16; ++j4) o[j4] = *(const f4*)(s_row + 4 * j4);
    uint32_t gt = 0;
#pragma unroll
    for (int j4 = 0; j4 < 16; ++j4)
#pragma unroll
        for (int c = 0; c < 4; c += 2)
            gt += (__float_as_uint(l - o[j4][c]) >> 31) + (__float_as_uint(l - o[j4][c + 1]) >> 31);
    int rank = (int)gt;
    const float rsum = wave_reduce_dpp(lane < E ? (float)gt : 0.0f, add_op);
    if (rsum != 0.5f * (float)(E * (E - 1))) {
        rank = 0;
        for (int jj = 0; jj < E; ++jj) {
            const float oj = s_row[jj];
            rank += (int)(oj > l) + (int)(oj == l && jj < lane);
        }
    }
    return rank;
}

// Top-k of one row on one wave, lane holding experts lane + 64 i (i < NI; NI = 1 when E <= 64).
// s_row holds the row's logits padded with -inf to 64 NI.  Lanes < k return the rank-order
// expert and its softmax weight renormalised over the k (summed in rank order).  Ranking:
// higher logit first, the lower index on equal logits.
template <int NI>
__device__ __forceinline__ void row_topk(const float* s_row, int E, int k, int* s_ind,
                                         float* s_gate, int& ind, float& gate) {
    const int lane = threadIdx.x & 63;
    const auto fmax_op = [](float x, float y) { return fmaxf(x, y); };
    const auto add_op = [](float x, float y) { return x + y; };
    if constexpr (NI == 1) {
        const float l = s_row[lane];
        const int rank = row_rank64(s_row, E);
        const float mx = wave_reduce_dpp(l, fmax_op);
        const float g = lane < E ? expf(l - mx) : 0.0f;
        const float z = wave_reduce_dpp(g, add_op);
        if (lane < E && rank < k) {
            s_gate[rank] = g / z;
            s_ind[rank] = lane;
        }
    } else {
        // k rounds of a wave arg-max over (logit, -index) keys give the selection in rank order
        float lv[NI], mx = -INFINITY;
        uint64_t key[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int e = lane + 64 * i;
            lv[i] = s_row[e];
            mx = fmaxf(mx, lv[i]);
            uint32_t o = __float_as_uint(lv[i] + 0.0f);
            o = (o & 0x80000000u) ? ~o : (o | 0x80000000u);
            key[i] = e < E ? ((uint64_t)o << 32) | (uint32_t)(0xffffu - e) : 0;
        }
        mx = wave_reduce_dpp(mx, fmax_op);
        float z = 0.0f;
#pragma unroll
        for (int i = 0; i < NI; ++i) z += lane + 64 * i < E ? expf(lv[i] - mx) : 0.0f;
        z = wave_reduce_dpp(z, add_op);
        const auto umax_op = [](uint64_t x, uint64_t y) { return x > y ? x : y; };
        for (int j = 0; j < k; ++j) {
            uint64_t best = key[0];
#pragma unroll
            for (int i = 1; i < NI; ++i) best = key[i] > best ? key[i] : best;
            best = wave_reduce_dpp(best, umax_op);
            const int e = 0xffff - (int)(uint32_t)(best & 0xffffu);
#pragma unroll
            for (int i = 0; i < NI; ++i)
                if (key[i] == best) key[i] = 0;
            if (lane == 0) {
                s_gate[j] = expf(s_row[e] - mx) / z;
                s_ind[j] = e;
            }
        }
    }
    __builtin_amdgcn_wave_barrier();
    const f4 ga = *(const f4*)s_gate, gb = *(const f4*)(s_gate + 4);
    float ssum = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
        if (jj < k) ssum += jj < 4 ? ga[jj] : gb[jj - 4];  // in rank order
    if (lane < k) {
        gate = s_gate[lane] / ssum;
        ind = s_ind[lane];
    }
    __builtin_amdgcn_wave_barrier();
}

