// gather.hip -- 2-bit affine gather GEMM for verify passes on v_mfma_f32_16x16x32_f16.
//
// Semantics as k_qmv2 / k_gather (gqmm2_rows, SeedlessMetal.swift:2168-2221): per 64-input
// block, y += s * (sum q*x) + b * (sum x), fp32.
//
// Layout of the work: a block serves one expert (or the dense projection) and a strip of
// its output rows.  It stages the activation rows routed to that expert (qx order, up to 16
// per pass, read from the expert's pair list) in LDS once for all its waves.  Each wave owns
// a tile of 16 weight rows over one K-slice (KS slices per tile, summed through LDS at the
// end).  It issues every load of its weight tile (scales, biases, then the codes in 1 KB
// column groups, global -> LDS directly) before its first wait, and runs the MFMAs of a
// column group as soon as that group has landed.  Blocks of experts that no row picked exit
// at once, so only routed experts are read, each once per pass.
//
// Epilogues: STORE y = half(acc); ADD y = half(y + half(acc)) (o-proj residual,
// gqmm2_rows_fold_add 3488-3543); SWIGLU clamped SwiGLU of the up || gate row pair
// (maple_clamped_swiglu 2435-2450) written in qx order with its block sums.
#include <algorithm>
#include <type_traits>

#include "mj_device.h"
#include "mj_internal.h"
#include "moe_topk.h"

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane (wave-uniform lds)
__device__ __forceinline__ void load_lds16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds, 16, 0, 0);
}

// the same with a cache policy (16: sc1, device-coherent: sees stores of other XCDs made with
// sc1 once they have completed)
template <int CPOL>
__device__ __forceinline__ void load_lds16c(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds, 16, 0, CPOL);
}

// 4 bytes per lane, landing at lds + 4 * lane
__device__ __forceinline__ void load_lds4(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds, 4, 0, 0);
}

// Launch shape: R = 16 activation rows at most per pass (the MFMA M dimension), RA <= R rows
// staged in LDS per pass (a bucket with more rows takes several passes; `multi` says whether
// any can), K = 256 * KPL.  A block has WPB waves = TPB tiles of 16
// weight rows x KS K-slices: wave w owns tile w % TPB and K-slice w / TPB.
template <int KPL, int GS, int EPI, int WPB, int KS>
struct G5Shape {
    static constexpr int R = 16;
    static constexpr int K = KPL * 256;
    static constexpr int KB = K / 64;          // 64-blocks per row (= 16-byte code chunks per row)
    static constexpr int KBW = KB / KS;        // 64-blocks of one wave's K-slice
    static constexpr int TPB = WPB / KS;       // weight tiles per block
    static constexpr int XS = K + 8;           // LDS row stride of activations (halves)
    static constexpr int SCH = K / GS / 8;     // 16-byte scale chunks per weight row
    // K / GS == 4 (K = 512, group 128): a row's scales are 8 bytes, half a chunk; they are
    // staged 8 bytes a row and read as chunk 0 with its upper half zero
    static constexpr bool HSC = SCH == 0;
    static constexpr int SCW = HSC ? 1 : SCH / KS;  // ... per K-slice
    static constexpr int WCODE = 16 * KBW * 16;  // bytes of one wave's code tile
    static constexpr int WSB = 16 * SCW * 16;    // bytes of one wave's scales (and of its biases)
    static constexpr int WAVE_BYTES = WCODE + 2 * WSB;
    static constexpr int SS = KB + 2;          // LDS row stride of block sums (float2)
    static_assert(WAVE_BYTES >= 64 * 16, "a K-slice partial fits in its wave's tile area");
    static_assert(!HSC || (K / GS == 4 && KS == 1), "half-chunk scales: one K-slice of 4 groups");
    // K-slice partials: in a wave's own tile area when every bucket is one pass, else in their
    // own region (later passes reuse the tiles)
    static constexpr int RED = (KS - 1) * TPB * 64 * 16;
    // dbl: two sets of staged rows (persistent mode stages the next item's while this one
    // finishes)
    __host__ __device__ static size_t lds(int RA, bool multi, bool dbl = false) {
        return (size_t)WPB * WAVE_BYTES + (dbl ? 2 : 1) * ((size_t)RA * XS * 2 + (size_t)RA * SS * 8) +
               (multi ? RED : 0);
    }
};

// Weight tile of one wave: 16 rows x K codes with their scales and biases, fetched straight
// into LDS.  Scales and biases go first, then the codes in column groups: load j brings
// 64-blocks 4j .. 4j+3 of all 16 rows (16 runs of 64 bytes), so the MFMAs of group j start as
// soon as that load has landed while later groups are still streaming.  The code chunk
// (row r, block B) sits at slot 64 * (B / 4) + 4r + ((B % 4) ^ (r / 4)): lane (n, q) then reads
// word q of block B of row n from bank 16 (n % 4) + 4 ((B % 4) ^ (n / 4)) + q -- one 64-lane
// read touches every bank once.
//
// MFMA: A = 16 activation rows x 32 k (qx order, from LDS), B = word q of one 64-block of the
// 16 weight rows (lane (n, q)), so every MFMA stays inside one group of the scale and the
// block's partial sums D[4q+r][n] are scaled once, in fp32.  The affine remainder
// sum_B (b_B X_B - s_B Bx_B) is an fp32 MFMA chain over (block, term) pairs.

// s_waitcnt that waits for the vector-memory counter only (gfx9 encoding: expcnt and lgkmcnt
// left at their maximum)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier for LDS data only: this wave's LDS writes done (lgkmcnt 0) and at most N
// vector-memory loads still in flight (its LDS-DMA staging is older than those N), then
// s_barrier.  __syncthreads() would also drain every outstanding global load (its fence waits
// for vmcnt 0), i.e. the whole weight stream.  The "memory" clobber keeps LDS accesses on
// their side of it.
// 8-byte LDS store issued as inline assembly: the compiler would otherwise wait for every
// in-flight LDS-DMA load (it cannot prove the store misses their destinations) before it.  The
// ranges are disjoint by construction here; lds_barrier's lgkmcnt(0) orders the store.
__device__ __forceinline__ void lds_store_f2(float2* p, float2 v) {
    const uint32_t addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)p;
    const uint64_t bits = __builtin_bit_cast(uint64_t, v);
    asm volatile("ds_write_b64 %0, %1" ::"v"(addr), "v"(bits) : "memory");
}

template <int N>
__device__ __forceinline__ void lds_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Workgroup barrier that leaves vector-memory loads in flight: for LDS written with ds_write
// only (the next item's weight stream keeps landing meanwhile, in LDS nobody reads here).
__device__ __forceinline__ void lds_only_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// static LDS of the fused routing's slot records (persistent up || gate kernels)
// static LDS of the routing words of a launch that ranks up to FR rows itself
constexpr size_t g5_fused_rec_bytes(int FR) { return 64 * (4 + 8 + (FR > 16 ? 8 : 0)); }

// How one call of the tile-gather body fits into a launch.  MODE 0: the whole launch (the
// standalone kernels).  The fused MoE kernel calls the up || gate body (MODE 1) and then the down
// body (MODE 2) in every block; io carries the routing words from the first to the second.
struct FuseIO {
    uint32_t em = 0;   // lane t: rows that picked expert t (bit r)
    uint64_t er = 0;   // ... and expert t's rank in rows 0 .. 15 (3 bits at 3r)
    uint64_t er1 = 0;  // ... and in rows 16 .. 31 (3 bits at 3 (r - 16))
};

// FR: rows the fused routing ranks at most (16: two a wave, ranks in er; 32: four a wave, rows
// 16 .. 31's ranks in er1)
template <int KPL, int GS, int EPI, int WPB, int KS, bool PER, bool ROWA, bool FUS, int MODE,
          int FR = MJ_G5_FUSED_ROWS>
__device__ __forceinline__ void g5_body(GatherArgs a, int RA, int multi, FuseIO& io) {
    static_assert(FR == 16 || FR == 32, "fused routing rows");
    using S = G5Shape<KPL, GS, EPI, WPB, KS>;
    constexpr int R = S::R, K = S::K, KB = S::KB, KBW = S::KBW, TPB = S::TPB, XS = S::XS;
    constexpr int SCW = S::SCW;
    constexpr int NT = WPB * 64;
    constexpr int PPR = K / 8;                 // 16-byte parts per activation row
    static_assert(PPR % 64 == 0 && R % WPB == 0 && SCW >= 1 && SCW <= 4 && KBW % 4 == 0, "shape");

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int q = lane >> 4, n = lane & 15;
    const int tt = wv % TPB, kh = wv / TPB;   // weight tile and K-slice of this wave
    const int ncb = a.N / (16 * TPB);
    const int u = blockIdx.x / ncb;
    int cb = blockIdx.x % ncb;
    const bool own_sums = a.xsum == nullptr;  // block sums formed here from the staged rows

    // Persistent expert mode (PER): the work items are (routed-expert slot i / ncb, column
    // block i % ncb); block b takes items b, b + gridDim.x, ... until a slot with no pairs.
    // One load per lane brings a slot's record: pair j in lane j, the expert id and the pair
    // count in the high halves of lanes 0 and 1; the next item's record is fetched while the
    // current item computes.  Expert mode: block u serves expert u, whose ecnt[u] (row, slot)
    // pairs are listed at eplist[u * MJ_ROWS ..]; count and list are loaded together, and an
    // expert nobody picked ends here.  Bucket mode: block u serves the u-th expert of a Buckets
    // table.  Dense: rows 0 .. dense_rows-1 in groups of R, block u taking group u (the blocks
    // of a group stream the same weights, concurrently with the other groups' blocks).
    const int* plist = nullptr;
    int lpair = 0;  // expert modes: pair j of the list in lane j
    const bool dense_mode = !PER && a.ecnt == nullptr && a.bk == nullptr;
    const int rbase = dense_mode ? R * u : 0;  // dense: first row of the block's group
    int e = 0, np = dense_mode ? min(R, a.dense_rows - rbase) : a.dense_rows;
    int item = blockIdx.x;
    int rec_n = 0;  // the next item's record (persistent mode)
    extern __shared__ __align__(16) char g5lds[];

    // Fused routing (persistent up || gate product, rlogits set): every block ranks the router
    // logits itself -- the same top-k as the route kernel (row_topk) -- and keeps, per expert
    // t in lane t, the rows that picked it (em: bit r) and t's rank in each of them (er: 3 bits
    // a row).  A slot's record follows from these in registers: slots number the routed experts
    // in increasing id (as the route kernel's), a record lists its pairs (row * k + rank) by
    // row.  The last block also writes inds / scores and the global records for the down
    // product.
    struct FusedRoute {
        // per expert t, set by LDS atomics as the rows are ranked: the rows that picked t (bit
        // r) and t's rank in each (3 bits at 3r for rows 0 .. 15, at 3 (r - 16) in er1 beyond)
        uint32_t em[64];
        uint64_t er[64];
        uint64_t er1[FR > 16 ? 64 : 0];
    };
    // (an instantiation of its own, FUS: the routing code stays out of the other kernels)
    constexpr bool FUSABLE = FUS;
    static_assert(!FUS || (PER && EPI == EPI_SWIGLU), "fused routing: persistent up || gate");
    __shared__ __align__(16) std::conditional_t<FUSABLE, FusedRoute, char> s_fr;
    constexpr bool fused = FUS;
    static_assert(MODE == 0 || (MODE == 1 && FUS) || (MODE == 2 && PER && EPI == EPI_STORE),
                  "fused MoE phases: up || gate with routing, then down");
    // slot records from the routing words in registers: the ranking kernel itself, or the down
    // phase of the fused MoE launch (words handed over by its up phase)
    constexpr bool RREC = FUS || MODE == 2;
    uint32_t em = MODE == 2 ? io.em : 0u;
    uint64_t er = MODE == 2 ? io.er : 0ull;
    uint64_t er1 = MODE == 2 ? io.er1 : 0ull;
    // record of slot sl in the global records' form: pair j in lane j, expert id and pair count
    // in the high halves of lanes 0 and 1 (count 0 past the last routed expert)
    auto fused_rec = [&](int sl) -> int {
        const uint64_t on = __ballot(em != 0u);
        const int mys = __popcll(on & ((1ull << lane) - 1ull));
        const uint64_t hit = __ballot(em != 0u && mys == sl);
        if (hit == 0) return 0;
        const int ex = __builtin_ctzll(hit);
        const uint32_t rm = __builtin_amdgcn_readlane(em, ex);
        auto rl64 = [&](uint64_t w) {
            return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(w >> 32), ex) << 32) |
                   (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)w, ex);
        };
        const uint64_t rx0 = rl64(er), rx1 = FR > 16 ? rl64(er1) : 0ull;
        // lane r < FR (row r) sends its pair to lane "rows of ex before r"; the lanes that
        // send nothing send to lane 63, which no record entry uses (at most FR pairs)
        const int rr = lane & (FR - 1);
        const bool mine = lane < FR && ((rm >> rr) & 1u);
        const int pos = __popc(rm & ((1u << rr) - 1u));
        const int pr = rr * a.rk + (int)(((rr < 16 ? rx0 : rx1) >> (3 * (rr & 15))) & 7u);
        const int got = __builtin_amdgcn_ds_permute((mine ? pos : 63) * 4, pr);
        return got | (lane == 0 ? ex << 16 : lane == 1 ? __popc(rm) << 16 : 0);
    };
    if constexpr (FUSABLE) {
        static_assert(sizeof(FusedRoute) == g5_fused_rec_bytes(FR), "record bytes");
        static_assert(FR <= 4 * WPB, "at most four rows a wave");
        constexpr int RPW = (FR + WPB - 1) / WPB;  // rows a wave ranks
        if (fused) {
            const int M = a.rM, E = a.rE, k = a.rk;
            // row scratch in the weight tile area, free until the first item's loads
            float* s_row = (float*)g5lds + 64 * wv;                  // [WPB][64]
            float* s_gate = (float*)(g5lds + 256 * WPB) + 8 * wv;    // [WPB][8]
            int* s_ind = (int*)(g5lds + 288 * WPB) + 8 * wv;         // [WPB][8]
            // the wave's rows' logits (clamped row and expert: no branch waits) and the abort
            // flag requested together
            float v[RPW];
#pragma unroll
            for (int sr = 0; sr < RPW; ++sr)
                v[sr] = a.rlogits[min(wv + WPB * sr, M - 1) * E + min(lane, E - 1)];
            if (aborted(a.abort)) return;
            if (wv == 0) {
                s_fr.em[lane] = 0u;
                s_fr.er[lane] = 0ull;
                if constexpr (FR > 16) s_fr.er1[lane] = 0ull;
            }
            __syncthreads();  // (LDS only: the logits stay in flight)
            // expert t picked by row r at rank rk: its bits, ORed in from any wave
            auto mark = [&](int t, int r, int rk) {
                __hip_atomic_fetch_or(&s_fr.em[t], 1u << r, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_WORKGROUP);
                uint64_t* w = &s_fr.er[t];
                if constexpr (FR > 16) w = r < 16 ? w : &s_fr.er1[t];
                __hip_atomic_fetch_or(w, (uint64_t)rk << (3 * (r & 15)), __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_WORKGROUP);
            };
            const bool wr = blockIdx.x == gridDim.x - 1;  // writes inds / scores / records
#pragma unroll
            for (int sr = 0; sr < RPW; ++sr) {
                const int r = wv + WPB * sr;
                if (r >= M) break;
                s_row[lane] = lane < E ? v[sr] + 0.0f : -INFINITY;
                __builtin_amdgcn_wave_barrier();
                if (wr) {  // the selection with its weights
                    int ind = 0;
                    float gate = 0.0f;
                    row_topk<1>(s_row, E, k, s_ind, s_gate, ind, gate);
                    if (lane < k) {
                        mark(ind, r, lane);
                        a.rinds[r * k + lane] = ind;
                        a.rscores[r * k + lane] = gate;
                    }
                } else {  // the selection only: the ranks of row_topk, no weights
                    const int rank = row_rank64(s_row, E);
                    if (lane < E && rank < k) mark(lane, r, rank);
                }
                __builtin_amdgcn_wave_barrier();
            }
            __syncthreads();
            // lane t: the rows that picked expert t, and its rank in each
            em = s_fr.em[lane];
            er = s_fr.er[lane];
            if constexpr (FR > 16) er1 = s_fr.er1[lane];
            io.em = em;
            io.er = er;
            io.er1 = er1;
            if (wr && wv == 0) {
                const uint64_t on = __ballot(em != 0u);
                const int total = __popcll(on);
                if (em != 0u) {
                    int* gr = a.rsrec + __popcll(on & ((1ull << lane) - 1ull)) * MJ_ROWS;
                    const int cnt = __popc(em);
                    int c = 0;
#pragma unroll
                    for (int r = 0; r < FR; ++r) {
                        if ((em >> r) & 1u) {
                            gr[c] = (r * k + (int)(((r < 16 ? er : er1) >> (3 * (r & 15))) & 7u)) |
                                    (c == 0 ? lane << 16 : c == 1 ? cnt << 16 : 0);
                            ++c;
                        }
                    }
                    if (cnt == 1) gr[1] = 1 << 16;
                }
                if (lane >= total) {  // slots past the last routed expert: count 0
                    a.rsrec[lane * MJ_ROWS] = 0;
                    a.rsrec[lane * MJ_ROWS + 1] = 0;
                }
            }
            // the row scratch is free for the weight tiles: every wave is past the barrier above
        }
    }
    {
        const int ab = !fused && a.abort ? *a.abort : 0;  // fused: checked with the logits
        if constexpr (PER) {
            if constexpr (MODE == 2) {
                // blocks with one up item fewer come free first: they take the first down items
                // (slots in increasing order, the order the up items complete in)
                const int nS = __popcll(__ballot(em != 0u));
                const int G = (int)gridDim.x, rem = (nS * a.fup_ncb) % G;
                item = (int)blockIdx.x >= rem ? (int)blockIdx.x - rem : (int)blockIdx.x + (G - rem);
            }
            const int rec = RREC ? fused_rec(min(item / ncb, 63))
                                 : a.srec[min(item / ncb, 63) * MJ_ROWS + lane];
            e = __builtin_amdgcn_readlane(rec, 0) >> 16;
            np = item / ncb < 64 ? __builtin_amdgcn_readlane(rec, 1) >> 16 : 0;
            lpair = rec & 0xFFFF;
            cb = item % ncb;
        } else if (a.ecnt != nullptr) {
            e = u;
            np = a.ecnt[u];
            lpair = a.eplist[u * MJ_ROWS + lane];
        } else if (a.bk != nullptr) {
            const Buckets* bk = a.bk;
            const int cnt = bk->count, ee = bk->expert[u], s0 = bk->start[u], s1 = bk->start[u + 1];
            if (u >= cnt) return;  // whole block
            e = ee;
            np = s1 - s0;
            plist = bk->pair + s0;
        }
        if (ab || np <= 0) return;  // whole block
    }

    char* wreg = g5lds + (size_t)wv * S::WAVE_BYTES;      // this wave's weight tile
    char* wcode = wreg;
    uint16_t* wsc = (uint16_t*)(wreg + S::WCODE);          // [16][K/GS/KS] this K-slice
    uint16_t* wbi = (uint16_t*)(wreg + S::WCODE + S::WSB);
    // staged rows: one set, two in persistent mode (set buf serves the current item)
    // one row set; persistent mode keeps two pair lists (the next item's rows are staged once
    // every wave is done with the current ones, while the current epilogue still needs its pairs)
    constexpr int NBUF = PER ? 2 : 1;
    uint16_t* const xs0 = (uint16_t*)(g5lds + (size_t)WPB * S::WAVE_BYTES);  // [RA][XS] qx rows
    float2* const xsl0 = (float2*)(xs0 + RA * XS);  // [RA][SS] {sum x, sum base*x}
    char* red = (char*)(xsl0 + RA * S::SS);  // [KS-1][TPB][64] f4
    __shared__ int s_pair[NBUF][R];
    int buf = 0;
    auto xs_of = [&](int) { return xs0; };
    auto xsl_of = [&](int) { return xsl0; };

    // ---- activation rows of a pass, straight into LDS: rows < npass only (the rest feed
    // MFMA output rows that are discarded).  Wave w stages rows w, w + WPB, ...
    // residual add over dense rows: the first pass's residual values (rows 4q .. 4q + 3 of
    // output column n) are requested with the first rows, ahead of the weight stream, so the
    // epilogue does not wait on a dependent load (older than the weights, they change no wait
    // count)
    constexpr bool RES_PF = EPI == EPI_ADD && !PER;
    const bool res_pf = RES_PF && a.ecnt == nullptr && a.bk == nullptr && kh == 0;
    uint32_t resv[4] = {0u, 0u, 0u, 0u};
    auto stage_load = [&](int pb, int npass, int b, int lp, int npp, bool first = false) {
        uint16_t* xs = xs_of(b);
        float2* xsl = xsl_of(b);
        const int myr = min(pb + (lane < R ? lane : 0), npp - 1);
        const int prl =
            (PER || a.ecnt) ? __shfl(lp, myr, MJ_WAVE) : (plist ? plist[myr] : rbase + myr);
        if constexpr (RES_PF) {
            // (after the pair list: the wait for a list load would cover these too)
            if (first && res_pf) {
                // rows of the lane's outputs: q (a pass of at most 4 rows), else 4q .. 4q+3
                const int col = (cb * TPB + tt) * 16 + n;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int i = npass <= 4 ? q : 4 * q + r;
                    resv[r] = a.y[(size_t)(rbase + min(i, npass - 1)) * a.N + col];
                }
            }
        }
#pragma unroll
        for (int j = 0; j < R / WPB; ++j) {
            const int r = wv + WPB * j;
            const int pr = __builtin_amdgcn_readlane(prl, r);
            if (lane == 0) s_pair[b][r] = pr;
            if (r < npass) {
                const char* src = (const char*)(a.xperm + (size_t)(pr / a.x_div) * K);
#pragma unroll
                for (int i = 0; i < PPR / 64; ++i)
                    load_lds16c<MODE == 2 ? 16 : 0>(src + 1024 * i + 16 * lane,
                                                    (char*)(xs + r * XS) + 1024 * i);
                if (!own_sums && lane < KB / 2)
                    load_lds16((const char*)(a.xsum + (size_t)(pr / a.x_div) * KB) + 16 * lane,
                               xsl + r * S::SS);
            }
        }
    };
    // {sum x, sum base*x} of each (row, 64-block) from the staged rows (fixed order)
    auto own_block_sums = [&](int npass) {
        const uint16_t* xs = xs_of(buf);
        float2* xsl = xsl_of(buf);
        for (int idx = tid; idx < npass * KB; idx += NT) {
            const int r = idx % npass, b = idx / npass;
            const uint16_t* xr = xs + r * XS + 64 * b;
            float X = 0.0f, Bx = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const u4v v = *(const u4v*)(xr + 8 * c);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // qx pair (x_i, x_{i+8}) of a 16-block, i = (4c + j) % 8: base of code i
                    const float base = code_base(4 * c + j);
                    const float lo = h2f((uint16_t)v[j]), hi = h2f((uint16_t)(v[j] >> 16));
                    X += lo + hi;
                    Bx += base * (lo + hi);
                }
            }
            lds_store_f2(xsl + r * S::SS + b, make_float2(X, Bx));
        }
    };

    // ---- a wave's weight tile, coalesced into LDS: scales and biases, then the code groups
    const int I = a.N / 2;
    // scales (when `scales`) and code column groups j0 .. j1-1 of the tile
    auto issue_weights = [&](int ee, int cbb, bool scales = true, int j0 = 0, int j1 = S::KBW / 4) {
        auto tile_row = [&](int r) -> size_t {  // global row of tile row r
            if constexpr (EPI == EPI_SWIGLU) {
                const int j0 = (cbb * TPB + tt) * 8;
                return (size_t)ee * a.N + (r < 8 ? j0 + r : I + j0 + r - 8);
            } else {
                return (size_t)ee * a.N + (cbb * TPB + tt) * 16 + r;
            }
        };
        __builtin_amdgcn_sched_barrier(0);  // loads issued before stay ahead in the vmcnt queue
        if (!scales) {
        } else if constexpr (ROWA) {
            // row-alpha weights: one alpha per row (scale alpha, bias -alpha in every group);
            // tile rows 0..7 and 8..15 are each 8 consecutive rows, 16 bytes
            if (lane < 2) load_lds16((const char*)a.alpha + tile_row(8 * lane) * 2, wsc);
        } else if constexpr (S::HSC) {
            // 8 bytes of scales (and of biases) a row: lane l brings half l % 2 of row l / 2
            const char* sg = (const char*)a.s;
            const char* bg = (const char*)a.b;
            if (lane < 32) {
                load_lds4(sg + tile_row(lane >> 1) * 8 + 4 * (lane & 1), wsc);
                load_lds4(bg + tile_row(lane >> 1) * 8 + 4 * (lane & 1), wbi);
            }
        } else {
            const char* sg = (const char*)a.s;
            const char* bg = (const char*)a.b;
            if (lane < 16 * SCW) {
                const int r = lane / SCW, c = kh * SCW + lane % SCW;
                load_lds16(sg + tile_row(r) * (K / GS) * 2 + 16 * c, wsc);
                load_lds16(bg + tile_row(r) * (K / GS) * 2 + 16 * c, wbi);
            }
        }
        const char* wg = (const char*)a.w;
        const int r = lane >> 2, B4 = (lane & 3) ^ (r >> 2);
#pragma unroll
        for (int j = 0; j < KBW / 4; ++j)  // column group j: blocks kh*KBW + 4j .. +3
            if (j >= j0 && j < j1)
            load_lds16(wg + tile_row(r) * (K / 4) + 16 * (kh * KBW + 4 * j + B4),
                       wcode + 1024 * j);
        __builtin_amdgcn_sched_barrier(0);
    };
    // persistent mode: from the second item on, a wave's weights were issued as soon as its
    // MFMAs of the previous item were done (its tile is private to it), ahead of that item's
    // reduction and epilogue; the item's rows are staged after the block is done with the old
    // ones, so the item starts once everything it issued has landed
    bool early = false;
    // Fused MoE launch.  Up phase: an item's act values are stored device-coherent (sc1) into
    // act rows that the router launch filled with the marker 0xFFFF (a NaN, which the clamped
    // SwiGLU never produces: both its inputs are clamped to [-7, 7] first).  Down phase: an
    // item stages its rows at once and, once they have landed, checks them for the marker; rows
    // still marked are staged again.  The wait is bounded: the launch is sized so that every
    // block is resident, two a CU, and then every up item completes; a wait that runs out its
    // bound sets the fault word, which the host reports, and goes on, so the launch always ends.
    __shared__ int s_mark[WPB];
    // a half of the pass's staged rows still holds the marker (the same answer in every thread)
    auto rows_marked = [&](int npass) -> bool {
        const uint16_t* xs = xs_of(buf);
        bool bad = false;
        for (int idx = tid; idx < npass * (K / 8); idx += NT) {
            const int r = idx / (K / 8), c = idx - r * (K / 8);
            const u4v v = *(const u4v*)(xs + r * XS + 8 * c);
#pragma unroll
            for (int w = 0; w < 4; ++w)
                bad |= (v[w] & 0xFFFFu) == 0xFFFFu || (v[w] >> 16) == 0xFFFFu;
        }
        const bool wbad = __ballot(bad) != 0ull;
        if (lane == 0) s_mark[wv] = wbad ? 1 : 0;
        lds_only_barrier();
        int any = 0;
#pragma unroll
        for (int w = 0; w < WPB; ++w) any |= s_mark[w];
        return any != 0;
    };

  for (;;) {
    const int npass0 = min(RA, np);
    if (!early) {
        if constexpr (MODE == 2) {
            // the weights do not depend on the up phase: requested first, then the rows, checked
            // for the marker once they have landed
            issue_weights(e, cb);
            stage_load(0, npass0, buf, lpair, np, true);
            early = true;  // everything issued lands before the first pass
        } else {
            stage_load(0, npass0, buf, lpair, np, true);  // ahead of the weights (loads return in order)
            issue_weights(e, cb);
        }
    }
    const UnpackK uk = unpack_consts();
    const int xrow = min(n, RA - 1);
    const uint32_t* wq = (const uint32_t*)wcode + 16 * n + q;  // B: word q of row n's chunks

    // NR activation rows a lane's MFMA outputs hold.  A pass of at most 4 rows (NR = 1) places
    // staged row i at MFMA rows 4i .. 4i+3 (lane n reads row n / 4), so lane (n, q) holds row q
    // in each of its four outputs and scales and finishes one of them; more rows (NR = 4) sit at
    // MFMA rows 0 .. 15, lane (n, q) holding rows 4q .. 4q+3.  Each output is the same sum of the
    // same products either way.
    auto run_pass = [&](auto nr_t, int pb, int npass) {
        constexpr int NR = decltype(nr_t)::value;
        static_assert(NR == 1 || NR == 4, "rows a lane");
        const int xr = NR == 1 ? min(n >> 2, RA - 1) : xrow;
        constexpr int G = KBW / 4;  // code column groups, issued after the scale loads
        constexpr int NSB = ROWA ? 1 : 2;  // scale / bias loads of a tile
        // every wave's staged rows visible (this wave's were issued before its weights)
        if (pb == 0 && !early)
            lds_barrier<G + NSB>();
        else
            lds_barrier<0>();
        if constexpr (MODE == 2) {
            // act rows an up item has not finished yet: staged again until they have
            for (int it = 0; rows_marked(npass); ++it) {
                if (it >= a.fpolls) {
                    if (a.ffault != nullptr && tid == 0)
                        __hip_atomic_store(a.ffault, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    break;
                }
                if ((it & 63) == 63 && aborted(a.abort)) break;
                lds_only_barrier();  // every wave has read the marks before they are rewritten
                __builtin_amdgcn_s_sleep(8);
                stage_load(pb, npass, buf, lpair, np);
                lds_barrier<0>();
            }
        }
        if (own_sums) {
            own_block_sums(npass);
            lds_barrier<G + NSB>();
        }
        // persistent mode: the next item's record, fetched behind this item's weights (one
        // vector load younger than them: PF).  With fused routing the record is formed from
        // registers once the weights have landed; the load is then a stand-in that keeps the
        // queue's count, and its value is consumed (times zero) so that it stays
        // (the down phase of the fused launch forms every record from registers: no load)
        constexpr int PF = PER && MODE != 2 ? 1 : 0;
        if constexpr (PER && MODE != 2) {
            if (pb == 0) {
                const int* rp = fused ? (const int*)a.rlogits
                                      : a.srec + min((item + (int)gridDim.x) / ncb, 63) * MJ_ROWS + lane;
                rec_n = *rp;
            }
        }
        wait_vmcnt<G + PF>();      // scales and biases have landed
        u4v sv[SCW], bv[SCW];
        float alpha_n = 0.0f;  // row-alpha weights: alpha of weight row n
        if constexpr (ROWA) {
            alpha_n = h2f(wsc[n]);
        } else if constexpr (S::HSC) {
            const uint2 ts = *(const uint2*)(wsc + 4 * n), tb = *(const uint2*)(wbi + 4 * n);
            sv[0] = (u4v){ts.x, ts.y, 0u, 0u};
            bv[0] = (u4v){tb.x, tb.y, 0u, 0u};
        } else {
#pragma unroll
            for (int c = 0; c < SCW; ++c) {
                sv[c] = *(const u4v*)(wsc + (n * SCW + c) * 8);
                bv[c] = *(const u4v*)(wbi + (n * SCW + c) * 8);
            }
        }
        // + sum_B (b_B X_B - s_B Bx_B): fp32 MFMA chains over k = (block, term) pairs, issued
        // while the codes are still arriving (scales, biases and activation sums are in);
        // A = activation sums of block 2i + q/2 (term q & 1), B = bias / -scale of row n
        f4 corr[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) corr[c] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
        const float* xcs =
            (const float*)(xsl_of(buf) + xr * S::SS + kh * KBW + (q >> 1)) + (q & 1);
        // this lane's B values: the biases (term 0) or the negated scales (term 1), taken from
        // the fp16 half of block 2i + q/2's group (the sign flipped in the fp16 bits)
        const uint32_t sgn = (q & 1) ? 0x8000u : 0u;
        const uint32_t hsh = 16u * (uint32_t)(q >> 1);
        if constexpr (ROWA) {
            // bias -alpha and scale alpha: B = -alpha for both terms
#pragma unroll
            for (int i = 0; i < KBW / 2; ++i)
                corr[i & 3] = mfma16x16x4f32(xcs[4 * i], -alpha_n, corr[i & 3]);
        } else {
            u4v mv[SCW];
#pragma unroll
            for (int c = 0; c < SCW; ++c)
#pragma unroll
                for (int w = 0; w < 4; ++w) mv[c][w] = (q & 1) ? sv[c][w] : bv[c][w];
#pragma unroll
            for (int i = 0; i < KBW / 2; ++i) {
                const float xa_k = xcs[4 * i];  // block 2i + q/2
                uint32_t h;
                if constexpr (GS == 64) {  // group 2i + q/2: word i % 4 of chunk 2i / 8, half q/2
                    h = mv[(2 * i) / 8][i % 4] >> hsh;
                } else {  // group i
                    h = mv[i / 8][(i % 8) / 2] >> (16 * (i & 1));
                }
                const float wk = h2f((uint16_t)(h ^ sgn));
                corr[i & 3] = mfma16x16x4f32(xa_k, wk, corr[i & 3]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // A: activation row xr, quarter q, of this K-slice
        const uint16_t* xak = xs_of(buf) + xr * XS + 16 * q + 64 * kh * KBW;
        // the correction chain's sum starts the accumulator (its four partial chains are
        // then free); outputs r >= NR stay unused
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = (corr[0][r] + corr[1][r]) + (corr[2][r] + corr[3][r]);
        // row-alpha weights: every block has scale alpha, so the MFMA sums chain over the whole
        // slice and alpha scales them once
        f4 dacc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};  // even / odd blocks
        // persistent mode, last pass of the item: the next item (its record, and whether there
        // is one) and its weights.  In the fused launch (records formed from registers) the
        // scales and first half of the code groups are requested once this item's first half
        // is done (its scales are in registers, its first half's codes read), the rest after
        // its MFMAs; the item waits for its own groups first, so later waits count nothing new
        constexpr bool SPLIT = PER && (MODE == 1 || MODE == 2) && G >= 2;
        constexpr int GP = G / 2;  // code groups a part (four parts measured slower)
        bool stage_next = false;
        int np_next = 0;
        auto next_item = [&]() {
            if constexpr (PER) {
                const int nx = item + (int)gridDim.x;
                if constexpr (MODE == 2) {
                    rec_n = fused_rec(min(nx / ncb, 63));
                } else if (fused)
                    rec_n = fused_rec(min(nx / ncb, 63)) | (rec_n & (int)opaque(0u));
                np_next = __builtin_amdgcn_readlane(rec_n, 1) >> 16;
                stage_next = pb + RA >= np && nx / ncb < 64 && np_next > 0;
            }
        };
        // sum_B s_B * (sum q x)_B: per 64-block f16 MFMA sums, scaled in fp32, one column group
        // at a time as its codes arrive
        // fused launch: the wave computes at raised priority (s_setprio, the issue arbiter's
        // order among the CU's ready waves), so a wave whose tile has landed gets through its
        // groups, and to its next item's requests, ahead of waves still on the unpack of
        // theirs (launch 31.2 -> 30.1 us; through the epilogue as well: 30.4 us; a second
        // level for the second half: step 1.552 -> 1.548 ms)
        if constexpr (SPLIT) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int j = 0; j < G; ++j) {
          if (!(SPLIT && j >= GP && stage_next)) {
            if (j == 0) wait_vmcnt<G - 1 + PF>();
            if (j == 1) wait_vmcnt<(G >= 2 ? G - 2 : 0) + PF>();
            if (j == 2) wait_vmcnt<(G >= 3 ? G - 3 : 0) + PF>();
            if (j == 3) wait_vmcnt<(G >= 4 ? G - 4 : 0) + PF>();
            if (j == 4) wait_vmcnt<(G >= 5 ? G - 5 : 0) + PF>();
            if (j == 5) wait_vmcnt<(G >= 6 ? G - 6 : 0) + PF>();
            if (j == 6) wait_vmcnt<(G >= 7 ? G - 7 : 0) + PF>();
            if (j == 7) wait_vmcnt<PF>();
          }
            __builtin_amdgcn_sched_barrier(0);
            // LDS operands two blocks at a time (2 code words, 4 activation fragments), both
            // blocks' requested before the first is used
#pragma unroll
            for (int B2 = 4 * j; B2 < 4 * j + 4; B2 += 2) {
                uint32_t wd[2];
                u4v xv[2][2];
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    // word q of chunk slot 64 j + 4n + ((B % 4) ^ (n / 4)), B = B2 + b
                    wd[b] = wq[256 * j + 4 * (((B2 + b) & 3) ^ (n >> 2))];
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        xv[b][h] = *(const u4v*)(xak + 64 * (B2 + b) + 8 * h);
                }
#pragma unroll
              for (int b = 0; b < 2; ++b) {  // block kh * KBW + B
                const int B = B2 + b;
                uint32_t v[8];
                unpack16k(wd[b], v, uk);
                if constexpr (ROWA) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const u4v bq = {v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
                        dacc[b] = mfma16x16x32(as_h8(xv[b][h]), as_h8(bq), dacc[b]);
                    }
                } else {
                    f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const u4v bq = {v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
                        d = mfma16x16x32(as_h8(xv[b][h]), as_h8(bq), d);
                    }
                    const int g = B * 64 / GS;
                    const uint32_t sw = opaque(sv[g / 8][(g % 8) / 2]);
                    const float sc = h2f((uint16_t)(sw >> (16 * (g & 1))));
#pragma unroll
                    for (int r = 0; r < NR; ++r) acc[r] += sc * d[r];
                }
              }
            }
#pragma unroll
            for (int r = 0; r < NR; ++r) pin(acc[r]);
            if constexpr (SPLIT) {
                if ((j + 1) % GP == 0) {
                    if (j + 1 == GP) {
                        next_item();
                        if (stage_next) wait_vmcnt<0>();  // this item's remaining groups have landed
                    }
                    if (stage_next)
                        issue_weights(__builtin_amdgcn_readlane(rec_n, 0) >> 16,
                                      (item + (int)gridDim.x) % ncb, j + 1 == GP, j + 1 - GP, j + 1);
                    // priority 2 once the next item's first part is out (those waves are
                    // nearest their last requests), 0 after the last group
                    if (j + 1 == G)
                        __builtin_amdgcn_s_setprio(0);
                    else
                        __builtin_amdgcn_s_setprio(2);
                }
            }
        }
        if constexpr (ROWA) {
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[r] += alpha_n * (dacc[0][r] + dacc[1][r]);
        }
        // persistent mode, last pass of the item: this wave's tile is free, start the next
        // item's weights (the rest of them, split); its rows follow once every wave is done
        // with the current ones
        if constexpr (PER) {
            if constexpr (!SPLIT) {
                next_item();
                if (stage_next)
                    issue_weights(__builtin_amdgcn_readlane(rec_n, 0) >> 16, (item + (int)gridDim.x) % ncb);
            }
        }
        if constexpr (KS > 1) {
            // K-slices of a tile meet in LDS (a slice's partial goes into its own wave's tile
            // area, free once its MFMAs are done); slice 0 adds them in slice order
            auto slot = [&](int k2) -> f4* {
                return (f4*)((multi || PER) ? red + ((k2 - 1) * TPB + tt) * 1024
                                            : g5lds + (size_t)(k2 * TPB + tt) * S::WAVE_BYTES) +
                       lane;
            };
            if (kh > 0) *slot(kh) = (f4){acc[0], acc[1], acc[2], acc[3]};
            if (PER)
                lds_only_barrier();
            else
                lds_barrier<0>();
            if (kh == 0) {
#pragma unroll
                for (int k2 = 1; k2 < KS; ++k2) {
                    const f4 o = *slot(k2);
#pragma unroll
                    for (int r = 0; r < NR; ++r) acc[r] += o[r];
                }
            }
        }
        if constexpr (PER) {
            if (stage_next) {
                // every wave has read its rows (the K-slice barrier, or this one)
                if constexpr (KS == 1) lds_only_barrier();
                stage_load(0, min(RA, np_next), buf ^ 1, rec_n & 0xFFFF, np_next);
            }
        }
        // lane (n, q) now holds the outputs of activation rows 4q .. 4q+3 (NR = 4) or row q
        // (NR = 1) for weight row n
        if constexpr (EPI == EPI_SWIGLU) {
            // up row n < 8 pairs with gate row n + 8.  NR = 4: lanes n < 8 finish rows 4q, 4q + 1
            // and lanes n + 8 rows 4q + 2, 4q + 3, each taking the other half of its pair by a
            // swap; NR = 1: lanes n < 8 finish row q
            auto finish = [&](float up, float g, int i) {
                up = hround(up);
                g = hround(g);
                g = fminf(g, 7.0f);
                up = fminf(fmaxf(up, -7.0f), 7.0f);
                const float act = hround(g / (1.0f + expf(-g)) * up);
                const int j = (cb * TPB + tt) * 8 + (n & 7);
                uint16_t* dst = a.y + (size_t)s_pair[buf][i] * I + (j & ~15) + perm_pos(j & 15);
                if constexpr (MODE == 1)
                    __hip_atomic_store(dst, f2h(act), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else
                    *dst = f2h(act);
            };
            if constexpr (NR == 1) {
                const float recv = __shfl_xor(acc[0], 8, MJ_WAVE);
                if (kh == 0 && n < 8 && q < npass) finish(acc[0], recv, q);
            } else {
#pragma unroll
                for (int rr = 0; rr < 2; ++rr) {
                    const bool lo = n < 8;
                    const float recv = __shfl_xor(lo ? acc[rr + 2] : acc[rr], 8, MJ_WAVE);
                    const int r = lo ? rr : rr + 2;
                    const int i = 4 * q + r;
                    if (kh == 0 && i < npass) finish(lo ? acc[rr] : recv, lo ? recv : acc[rr + 2], i);
                }
            }
        } else {
            const int col = (cb * TPB + tt) * 16 + n;
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const int i = NR == 1 ? q : 4 * q + r;
                if (kh == 0 && i < npass) {
                    uint16_t* yp = a.y + (size_t)s_pair[buf][i] * a.N + col;
                    if constexpr (EPI == EPI_ADD) {
                        const uint16_t res = res_pf && pb == 0 ? (uint16_t)resv[r] : *yp;
                        *yp = f2h(h2f(res) + hround(acc[r]));
                    } else {
                        *yp = f2h(acc[r]);
                    }
                }
            }
        }
    };
    // a first pass of at most 4 rows (nearly every expert of a verify pass) takes the
    // one-row-a-lane form; later passes of a bucket with more rows than fit the general one
    if (npass0 <= 4)
        run_pass(std::integral_constant<int, 1>{}, 0, npass0);
    else
        run_pass(std::integral_constant<int, 4>{}, 0, npass0);
    for (int pb = RA; pb < np; pb += RA) {
        __syncthreads();  // the previous pass is done with LDS
        const int npass = min(RA, np - pb);
        stage_load(pb, npass, buf, lpair, np);
        run_pass(std::integral_constant<int, 4>{}, pb, npass);
    }
    if constexpr (!PER) break;
    item += gridDim.x;
    if (item / ncb >= 64) break;
    np = __builtin_amdgcn_readlane(rec_n, 1) >> 16;
    if (np <= 0) break;
    e = __builtin_amdgcn_readlane(rec_n, 0) >> 16;
    cb = item % ncb;
    lpair = rec_n & 0xFFFF;
    buf ^= 1;
    early = true;
  }
}

template <int KPL, int GS, int EPI, int WPB, int KS, bool PER = false, bool ROWA = false,
          bool FUS = false>
// four waves per SIMD: two 8-wave blocks (or one 16-wave block) per CU
__global__ __launch_bounds__(WPB * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_gather5(
    GatherArgs a, int RA, int multi) {
    FuseIO io;
    g5_body<KPL, GS, EPI, WPB, KS, PER, ROWA, FUS, 0>(a, RA, multi, io);
}

// Fused MoE launch (H = 2048, I = 1024): the up || gate product with its routing, then the down
// product, in the same persistent blocks.  A block that has finished its up items takes down
// items (blocks with fewer up items first, slots in increasing order) and stages an item's act
// rows once every up item of its slot has completed, so the up product's last round overlaps
// the down product, which needs no launch or record read of its own.
// FR: rows the launch ranks at most, 16 or 32 (the 32-row form ranks four rows a wave and
// carries a second rank word, which costs a 9-row pass about 1 us).
template <int GS, bool ROWA, int FR>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void k_moe_fused(
    GatherArgs up, GatherArgs dn, int ra_up, int ra_dn, int multi_up, int multi_dn) {
    FuseIO io;
    g5_body<8, GS, EPI_SWIGLU, 8, 2, true, ROWA, true, 1, FR>(up, ra_up, multi_up, io);
    __syncthreads();  // every wave is done with the up phase's LDS
    g5_body<4, GS, EPI_STORE, 8, 1, true, ROWA, false, 2, FR>(dn, ra_dn, multi_dn, io);
}

// dynamic LDS a tile-gather launch may take (the device has 160 KB per workgroup)
constexpr size_t G5_LDS_MAX = 159 * 1024;

// blocks of a persistent launch: two per CU (the LDS footprint allows two)
static int persistent_blocks() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
    }
    return 2 * cus;
}

template <int KPL, int GS, int EPI, int WPB, int KS, bool PER = false, bool ROWA = false>
static hipError_t launch_g5(const GatherArgs& a, int rows, int n_buckets, hipStream_t st) {
    using S = G5Shape<KPL, GS, EPI, WPB, KS>;
    const int ncb = a.N / (16 * S::TPB);
    // staged rows per pass: for the expert products as many as keep two blocks per CU (more
    // rows on one expert are rare and take extra passes); dense projections take up to 16
    const int want = rows < 1 ? 1 : rows;
    int RA = want < S::R ? want : S::R;
    const bool expert = a.ecnt != nullptr || a.srec != nullptr;
    // two blocks a CU for the expert products; static LDS: the pair lists (128 bytes) and, in
    // the persistent up || gate kernels, the fused routing's records
    const size_t stat = 256 + (PER && EPI == EPI_SWIGLU ? g5_fused_rec_bytes(MJ_G5_FUSED_ROWS) : 0);
    const size_t limit =
        (EPI == EPI_SWIGLU || EPI == EPI_STORE) && expert ? 80 * 1024 - stat : G5_LDS_MAX;
    while (RA > 1 && S::lds(RA, want > RA || PER) > limit) --RA;
    const bool multi = want > RA;
    int grid = n_buckets * ncb;
    if (PER && grid > persistent_blocks()) grid = persistent_blocks();
    if constexpr (PER && EPI == EPI_SWIGLU) {
        if (a.rlogits != nullptr) {
            launch_timed(k_gather5<KPL, GS, EPI, WPB, KS, PER, ROWA, true>, dim3(grid),
                         dim3(WPB * 64), S::lds(RA, multi || PER), st, a, RA, (int)multi);
            return hipGetLastError();
        }
    }
    launch_timed(k_gather5<KPL, GS, EPI, WPB, KS, PER, ROWA>, dim3(grid), dim3(WPB * 64),
                 S::lds(RA, multi || PER), st, a, RA, (int)multi);
    return hipGetLastError();
}

// Shapes the tile kernel covers: SWIGLU / ADD at K = 2048, STORE at K = 512, 1024 or 2048; N
// a multiple of the block's rows; group size 64 or 128.
bool gather3_supported(int epi, int K, int N, int gs) {
    if (gs != 64 && gs != 128) return false;
    switch (epi) {
        case EPI_SWIGLU: return K == 2048 && N % 64 == 0;
        case EPI_ADD: return K == 2048 && N % 64 == 0;
        case EPI_STORE: return (K == 512 || K == 1024 || K == 2048) && N % 64 == 0;
    }
    return false;
}

hipError_t launch_gather3(const GatherArgs& a, int epi, int max_rows_per_bucket, int n_buckets,
                          hipStream_t st) {
    if (!gather3_supported(epi, a.K, a.N, a.gs)) return hipErrorInvalidValue;
    int rows = max_rows_per_bucket;
    // expert products over routed-expert slot records (at most 64 experts): persistent
    const bool per = a.srec != nullptr;
    if (per && (n_buckets > 64 || (epi != EPI_SWIGLU && epi != EPI_STORE)))
        return hipErrorInvalidValue;
    // fused routing: the up || gate product ranks the router logits itself
    if (a.rlogits != nullptr &&
        (!per || epi != EPI_SWIGLU || a.rM < 1 || a.rM > MJ_G5_FUSED_ROWS || a.rE < 1 ||
         a.rE > 64 || a.rk < 1 || a.rk > 8 || a.rk > a.rE || a.x_div != a.rk ||
         a.rinds == nullptr || a.rscores == nullptr || a.rsrec == nullptr))
        return hipErrorInvalidValue;
    // row-alpha expert weights (scale alpha, bias -alpha in every group of a row): the
    // fold kernels read one alpha per row instead of the group scales and biases
    if (a.alpha != nullptr && (a.srec != nullptr || a.ecnt != nullptr) &&
        (epi == EPI_SWIGLU || epi == EPI_STORE)) {
#define MJ_G5A(KPL, E, KS64, KS128)                                                        \
    {                                                                                      \
        if (per)                                                                           \
            return a.gs == 64 ? launch_g5<KPL, 64, E, 8, KS64, true, true>(a, rows, n_buckets, st) \
                              : launch_g5<KPL, 128, E, 8, KS128, true, true>(a, rows, n_buckets, st); \
        return a.gs == 64 ? launch_g5<KPL, 64, E, 8, KS64, false, true>(a, rows, n_buckets, st)    \
                          : launch_g5<KPL, 128, E, 8, KS128, false, true>(a, rows, n_buckets, st); \
    }
        if (epi == EPI_SWIGLU) MJ_G5A(8, EPI_SWIGLU, 2, 2)
        if (a.K == 512) MJ_G5A(2, EPI_STORE, 1, 1)
        if (a.K == 1024) MJ_G5A(4, EPI_STORE, 1, 1)
        MJ_G5A(8, EPI_STORE, 2, 2)
#undef MJ_G5A
    }
#define MJ_G5(KPL, E, W, KS64, KS128)                                                      \
    if (per && (E == EPI_SWIGLU || E == EPI_STORE))                                         \
        return a.gs == 64 ? launch_g5<KPL, 64, E, W, KS64, true>(a, rows, n_buckets, st)    \
                          : launch_g5<KPL, 128, E, W, KS128, true>(a, rows, n_buckets, st); \
    return a.gs == 64 ? launch_g5<KPL, 64, E, W, KS64>(a, rows, n_buckets, st)              \
                      : launch_g5<KPL, 128, E, W, KS128>(a, rows, n_buckets, st);
    // dense projections (qkv, o-proj: a few MB at most) spread over many small blocks, four
    // waves of one 16-row tile (group 64) or two (group 128): the unpack work of a block is
    // then short, and the launch fills the chip.  More than 16 rows: one set of blocks per
    // 16-row group, running side by side (each re-reads the small weight matrix) instead of
    // one block unpacking its tile again for every further 16 rows.
    const bool dense = a.srec == nullptr && a.ecnt == nullptr && a.bk == nullptr;
    if (dense) {
        n_buckets = (a.dense_rows + 15) / 16;
        rows = rows < 16 ? rows : 16;
    }
    switch (epi) {
        case EPI_SWIGLU: MJ_G5(8, EPI_SWIGLU, 8, 2, 2)
        case EPI_ADD: MJ_G5(8, EPI_ADD, 4, 4, 2)
        case EPI_STORE:
            if (a.K == 512) { MJ_G5(2, EPI_STORE, 8, 1, 1) }
            if (a.K == 1024) { MJ_G5(4, EPI_STORE, 8, 1, 1) }
            if (dense) { MJ_G5(8, EPI_STORE, 4, 4, 2) }
            MJ_G5(8, EPI_STORE, 8, 2, 2)
    }
#undef MJ_G5
    return hipErrorInvalidValue;
}

// static LDS of the fused MoE kernel: both phases' pair lists and the routing words
constexpr size_t g5_fused_moe_stat(int FR) { return 256 + 256 + g5_fused_rec_bytes(FR); }

// rows staged a pass by the two phases, and the dynamic LDS of the launch (the form for `rows`)
template <int GS>
static size_t moe_fused_lds(int rows, int& ra_up, int& ra_dn) {
    using SU = G5Shape<8, GS, EPI_SWIGLU, 8, 2>;
    using SD = G5Shape<4, GS, EPI_STORE, 8, 1>;
    const int want = rows < 1 ? 1 : rows;
    const size_t limit = 80 * 1024 - g5_fused_moe_stat(want <= 16 ? 16 : 32);  // two blocks a CU
    ra_up = want < 16 ? want : 16;
    ra_dn = ra_up;
    while (ra_up > 1 && SU::lds(ra_up, true) > limit) --ra_up;
    while (ra_dn > 1 && SD::lds(ra_dn, true) > limit) --ra_dn;
    return std::max(SU::lds(ra_up, true), SD::lds(ra_dn, true));
}

// every block of the launch resident at once: two a CU at the largest footprint (32 rows),
// for both forms
template <int GS, bool ROWA>
static bool moe_fused_resident() {
    static int ok = -1;
    if (ok < 0) {
        int ra_up = 0, ra_dn = 0, n16 = 0, n32 = 0;
        const size_t lds16 = moe_fused_lds<GS>(16, ra_up, ra_dn);
        const size_t lds32 = moe_fused_lds<GS>(MJ_MOE_FUSED_ROWS, ra_up, ra_dn);
        ok = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n16, k_moe_fused<GS, ROWA, 16>, 512,
                                                          lds16) == hipSuccess &&
             hipOccupancyMaxActiveBlocksPerMultiprocessor(&n32, k_moe_fused<GS, ROWA, 32>, 512,
                                                          lds32) == hipSuccess &&
             n16 >= 2 && n32 >= 2;
    }
    return ok == 1;
}

template <int GS, bool ROWA>
static hipError_t launch_moe_fused_t(GatherArgs up, GatherArgs dn, int rows, hipStream_t st) {
    using SU = G5Shape<8, GS, EPI_SWIGLU, 8, 2>;
    const int want = rows < 1 ? 1 : rows;
    int ra_up = 0, ra_dn = 0;
    const size_t lds = moe_fused_lds<GS>(rows, ra_up, ra_dn);
    up.fup_ncb = up.N / (16 * SU::TPB);
    dn.fup_ncb = up.fup_ncb;
    if (want <= 16)
        launch_timed(k_moe_fused<GS, ROWA, 16>, dim3(persistent_blocks()), dim3(512), lds, st, up,
                     dn, ra_up, ra_dn, (int)(want > ra_up), (int)(want > ra_dn));
    else
        launch_timed(k_moe_fused<GS, ROWA, 32>, dim3(persistent_blocks()), dim3(512), lds, st, up,
                     dn, ra_up, ra_dn, (int)(want > ra_up), (int)(want > ra_dn));
    return hipGetLastError();
}

bool moe_fused_supported(int H, int I, int E, int gs, int M, bool rowa) {
    if (!(H == 2048 && I == 1024 && E <= 64 && (gs == 64 || gs == 128) && M >= 1 &&
          M <= MJ_MOE_FUSED_ROWS))
        return false;
    if (gs == 64) return rowa ? moe_fused_resident<64, true>() : moe_fused_resident<64, false>();
    return rowa ? moe_fused_resident<128, true>() : moe_fused_resident<128, false>();
}

hipError_t launch_moe_fused(const GatherArgs& up, const GatherArgs& dn, int rows, hipStream_t st) {
    const bool rowa = up.alpha != nullptr;
    if (!moe_fused_supported(up.K, dn.K, up.rE, up.gs, up.rM, rowa) || up.N != 2 * dn.K ||
        dn.N != up.K || up.rlogits == nullptr || up.srec == nullptr ||
        dn.srec == nullptr)
        return hipErrorInvalidValue;
    if (up.gs == 64)
        return rowa ? launch_moe_fused_t<64, true>(up, dn, rows, st)
                    : launch_moe_fused_t<64, false>(up, dn, rows, st);
    return rowa ? launch_moe_fused_t<128, true>(up, dn, rows, st)
                : launch_moe_fused_t<128, false>(up, dn, rows, st);
}

template <int KPL, int GS, int EPI, int WPB, int KS, bool PER = false, bool ROWA = false,
          bool FUS = false>
static hipError_t g5_attr() {
    return hipFuncSetAttribute((const void*)k_gather5<KPL, GS, EPI, WPB, KS, PER, ROWA, FUS>,
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)std::min(G5Shape<KPL, GS, EPI, WPB, KS>::lds(16, true),
                                             G5_LDS_MAX));
}

hipError_t set_gather3_attributes() {
    hipError_t e = hipSuccess;
#define MJ_A(KPL, E, W, KS64, KS128)                                 \
    if (e == hipSuccess) e = g5_attr<KPL, 64, E, W, KS64>();          \
    if (e == hipSuccess) e = g5_attr<KPL, 128, E, W, KS128>();        \
    if (e == hipSuccess) e = g5_attr<KPL, 64, E, W, KS64, true>();    \
    if (e == hipSuccess) e = g5_attr<KPL, 128, E, W, KS128, true>();
    MJ_A(8, EPI_SWIGLU, 8, 2, 2) MJ_A(8, EPI_ADD, 4, 4, 2) MJ_A(2, EPI_STORE, 8, 1, 1)
    MJ_A(4, EPI_STORE, 8, 1, 1) MJ_A(8, EPI_STORE, 8, 2, 2) MJ_A(8, EPI_STORE, 4, 4, 2)
#undef MJ_A
#define MJ_AA(KPL, E, KS64, KS128)                                              \
    if (e == hipSuccess) e = g5_attr<KPL, 64, E, 8, KS64, true, true>();        \
    if (e == hipSuccess) e = g5_attr<KPL, 128, E, 8, KS128, true, true>();      \
    if (e == hipSuccess) e = g5_attr<KPL, 64, E, 8, KS64, false, true>();       \
    if (e == hipSuccess) e = g5_attr<KPL, 128, E, 8, KS128, false, true>();
    MJ_AA(8, EPI_SWIGLU, 2, 2) MJ_AA(2, EPI_STORE, 1, 1) MJ_AA(4, EPI_STORE, 1, 1)
    // the fused MoE kernels
    {
        int ra_up = 0, ra_dn = 0;
        size_t most = 0;
        for (int rows : {16, MJ_MOE_FUSED_ROWS})
            most = std::max({most, moe_fused_lds<64>(rows, ra_up, ra_dn),
                             moe_fused_lds<128>(rows, ra_up, ra_dn)});
        const int lds = (int)std::min(most, G5_LDS_MAX);
        const void* ks[] = {(const void*)k_moe_fused<64, false, 16>, (const void*)k_moe_fused<64, true, 16>,
                            (const void*)k_moe_fused<128, false, 16>, (const void*)k_moe_fused<128, true, 16>,
                            (const void*)k_moe_fused<64, false, 32>, (const void*)k_moe_fused<64, true, 32>,
                            (const void*)k_moe_fused<128, false, 32>, (const void*)k_moe_fused<128, true, 32>};
        for (const void* k : ks)
            if (e == hipSuccess) e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    }
    // the fused-routing up || gate kernels
    if (e == hipSuccess) e = g5_attr<8, 64, EPI_SWIGLU, 8, 2, true, false, true>();
    if (e == hipSuccess) e = g5_attr<8, 128, EPI_SWIGLU, 8, 2, true, false, true>();
    if (e == hipSuccess) e = g5_attr<8, 64, EPI_SWIGLU, 8, 2, true, true, true>();
    if (e == hipSuccess) e = g5_attr<8, 128, EPI_SWIGLU, 8, 2, true, true, true>();
    MJ_AA(8, EPI_STORE, 2, 2)
#undef MJ_AA
    return e;
}
