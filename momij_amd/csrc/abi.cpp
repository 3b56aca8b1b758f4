// abi.cpp -- C ABI: context, device memory, and the op-level entry points.
//
// The context mirrors SeedlessMetal's process-global state (device, queue, stop buffer;
// SeedlessMetal.swift:23-104) as an explicit handle: one HIP stream, a device abort word and a
// scratch arena for the op-level calls.  Shape guards mirror SeedlessMetal.gqmm2's
// (SeedlessMetal.swift:336-338), widened to what the gfx950 kernels tile.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/momij_hip.h"
#include "mj_abi_internal.h"
#include "mj_internal.h"

// Scratch of mj_moe_block_noalloc: one statically allocated array per GPU, held until the
// process ends.  Host code never uses its name as an address (that is a host-side stand-in);
// the device address comes from hipGetSymbolAddress, once per device at mj_init.
static __device__ __align__(256) char scratch[MJ_MOE_NOALLOC_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};       // device address of `scratch`, per device
hipError_t g_scratch_err[kMaxDevices] = {};  // the lookup's result, per device
bool g_scratch_done[kMaxDevices] = {};

// with `device` current: look the array's address up once for this device
void resolve_static_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_done[device]) return;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_err[device] = e;
    g_scratch_dev[device] = e == hipSuccess ? p : nullptr;
    g_scratch_done[device] = true;
}
}  // namespace

TimedLaunch& timed_launch() {
    static thread_local TimedLaunch t;
    return t;
}

mj_status mj_fail(mj_ctx* ctx, mj_status st, const char* fmt, ...) {
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        ctx->err = buf;
    }
    return st;
}

mj_status mj_hip(mj_ctx* ctx, hipError_t e, const char* what) {
    if (e == hipSuccess) return MJ_OK;
    return mj_fail(ctx, MJ_HIP_ERROR, "%s: %s", what, hipGetErrorString(e));
}

mj_status mj_scratch_reserve(mj_ctx* ctx, size_t bytes) {
    if (bytes <= ctx->scratch_bytes) return MJ_OK;
    mj_status s = mj_hip(ctx, hipStreamSynchronize(ctx->stream), "scratch sync");
    if (s != MJ_OK) return s;
    if (ctx->scratch) hipFree(ctx->scratch);
    ctx->scratch = nullptr;
    ctx->scratch_bytes = 0;
    const size_t want = bytes + (bytes >> 2) + 4096;
    s = mj_hip(ctx, hipMalloc(&ctx->scratch, want), "scratch alloc");
    if (s != MJ_OK) return s;
    s = mj_hip(ctx, hipMemset(ctx->scratch, 0, want), "scratch clear");
    if (s != MJ_OK) return s;
    ctx->scratch_bytes = want;
    return MJ_OK;
}

void* Arena::take(size_t bytes) {
    off = (off + 255) & ~(size_t)255;
    void* p = base ? (char*)base + off : nullptr;
    off += bytes;
    return p;
}

// Both report each set once to the owning thread: the generation they have seen becomes the
// reference of the next mj_sync.
mj_status mj_abort_begin(mj_ctx* ctx, unsigned* gen) {
    *gen = ctx->abort_gen.load();
    if (!ctx->abort_host.load()) return MJ_OK;
    ctx->synced_gen = *gen;
    return mj_fail(ctx, MJ_ABORTED, "aborted by the abort word");
}

mj_status mj_abort_end(mj_ctx* ctx, unsigned gen) {
    const unsigned now = ctx->abort_gen.load();
    const bool ab = ctx->abort_host.load() || now != gen;
    ctx->synced_gen = now;
    if (ab) return mj_fail(ctx, MJ_ABORTED, "aborted by the abort word");
    // the kernels that set the fault word have completed: the caller has synchronised
    if (ctx->fault && __atomic_load_n(ctx->fault, __ATOMIC_ACQUIRE) != 0) {
        __atomic_store_n(ctx->fault, 0, __ATOMIC_RELEASE);
        return mj_fail(ctx, MJ_HIP_ERROR,
                       "fused MoE launch: a block's wait for the up product ran out its bound "
                       "(blocks not co-resident: another stream's kernels on the device?); the "
                       "results since the last synchronising call are invalid");
    }
    return MJ_OK;
}

extern "C" {

int mj_abi_version(void) { return MJ_ABI_VERSION; }

const char* mj_status_str(mj_status s) {
    switch (s) {
        case MJ_OK: return "ok";
        case MJ_NO_DEVICE: return "no device";
        case MJ_NOT_READY: return "not ready";
        case MJ_UNSUPPORTED_SHAPE: return "unsupported shape";
        case MJ_INVALID_ARG: return "invalid argument";
        case MJ_ABORTED: return "aborted";
        case MJ_HIP_ERROR: return "hip error";
        case MJ_CAPACITY: return "capacity exceeded";
        case MJ_OUT_OF_MEMORY: return "out of memory";
    }
    return "unknown";
}

mj_status mj_init(int device, mj_ctx** out) {
    if (!out) return MJ_INVALID_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0 || device < 0 || device >= n)
        return MJ_NO_DEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return MJ_NO_DEVICE;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return MJ_NO_DEVICE;
    if (hipSetDevice(device) != hipSuccess) return MJ_NO_DEVICE;
    resolve_static_scratch(device);
    mj_ctx* c = new mj_ctx();
    c->device = device;
    if (hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&c->ctl, hipStreamNonBlocking) != hipSuccess ||
        hipHostMalloc(&c->abort_src, 2 * sizeof(int), hipHostMallocDefault) != hipSuccess ||
        hipMalloc(&c->abort_dev, sizeof(int)) != hipSuccess ||
        hipMemset(c->abort_dev, 0, sizeof(int)) != hipSuccess ||
        hipHostMalloc(&c->fault, sizeof(int), hipHostMallocMapped | hipHostMallocCoherent) !=
            hipSuccess ||
        hipHostGetDevicePointer((void**)&c->fault_dev, c->fault, 0) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        mj_destroy(c);
        return MJ_HIP_ERROR;
    }
    c->abort_src[0] = 0;
    c->abort_src[1] = 1;
    *c->fault = 0;
    c->stream = c->own;
    *out = c;
    return MJ_OK;
}

mj_status mj_destroy(mj_ctx* ctx) {
    if (!ctx) return MJ_INVALID_ARG;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    if (ctx->ctl) hipStreamSynchronize(ctx->ctl);
    if (ctx->scratch) hipFree(ctx->scratch);
    if (ctx->abort_dev) hipFree(ctx->abort_dev);
    if (ctx->abort_src) hipHostFree(ctx->abort_src);
    if (ctx->fault) hipHostFree(ctx->fault);
    if (ctx->own) hipStreamDestroy(ctx->own);
    if (ctx->ctl) hipStreamDestroy(ctx->ctl);
    delete ctx;
    return MJ_OK;
}

const char* mj_last_error(const mj_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

mj_status mj_set_stream(mj_ctx* ctx, void* s) {
    if (!ctx) return MJ_INVALID_ARG;
    ctx->stream = s ? (hipStream_t)s : ctx->own;
    return MJ_OK;
}

void* mj_get_stream(const mj_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

// Any thread, at any time: the word is written by a copy on the context's control stream,
// never on the stream passes run (or are captured) on.  Errors of the copy are returned, not
// recorded in the context's message (the owning thread may be reading it).
mj_status mj_set_abort(mj_ctx* ctx, int flag) {
    if (!ctx) return MJ_INVALID_ARG;
    const int v = flag ? 1 : 0;
    std::lock_guard<std::mutex> lock(ctx->abort_mu);
    int prev = -1;
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (hipSetDevice(ctx->device) != hipSuccess) return MJ_HIP_ERROR;
    // set: the generation and the host mirror move before the device word can; clear: the
    // mirror follows the device word
    if (v) {
        ctx->abort_gen.fetch_add(1);
        ctx->abort_host.store(1);
    }
    hipError_t e = hipMemcpyAsync(ctx->abort_dev, ctx->abort_src + v, sizeof(int),
                                  hipMemcpyHostToDevice, ctx->ctl);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->ctl);
    if (e == hipSuccess && !v) ctx->abort_host.store(0);
    if (prev >= 0) hipSetDevice(prev);
    return e == hipSuccess ? MJ_OK : MJ_HIP_ERROR;
}

mj_status mj_set_wait_limit(mj_ctx* ctx, int polls) {
    if (!ctx || polls < 0) return MJ_INVALID_ARG;
    ctx->wait_polls = polls;
    return MJ_OK;
}

// Reports MJ_ABORTED when the word is set, or was set since the previous synchronising call:
// the work queued in between may have been skipped.
mj_status mj_sync(mj_ctx* ctx) {
    if (!ctx) return MJ_INVALID_ARG;
    mj_status s = mj_hip(ctx, hipStreamSynchronize(ctx->stream), "sync");
    if (s != MJ_OK) return s;
    return mj_abort_end(ctx, ctx->synced_gen);
}

mj_status mj_alloc(mj_ctx* ctx, size_t bytes, void** out) {
    if (!ctx || !out) return MJ_INVALID_ARG;
    *out = nullptr;
    return mj_hip(ctx, hipMalloc(out, bytes ? bytes : 1), "alloc");
}

mj_status mj_free(mj_ctx* ctx, void* p) {
    if (!ctx) return MJ_INVALID_ARG;
    if (!p) return MJ_OK;
    mj_status s = mj_hip(ctx, hipStreamSynchronize(ctx->stream), "free sync");
    if (s != MJ_OK) return s;
    return mj_hip(ctx, hipFree(p), "free");
}

mj_status mj_h2d(mj_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return MJ_INVALID_ARG;
    mj_status s = mj_hip(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream),
                         "h2d");
    if (s != MJ_OK) return s;
    return mj_hip(ctx, hipStreamSynchronize(ctx->stream), "h2d sync");
}

mj_status mj_d2h(mj_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return MJ_INVALID_ARG;
    mj_status s = mj_hip(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream),
                         "d2h");
    if (s != MJ_OK) return s;
    return mj_hip(ctx, hipStreamSynchronize(ctx->stream), "d2h sync");
}

mj_status mj_gather_qmm2(mj_ctx* ctx, const void* x, const uint32_t* w, const void* scales,
                         const void* biases, const int32_t* inds, void* y, int M, int ktop,
                         int K, int N, int gs, int lhs_per_expert, int epilogue) {
    if (!ctx) return MJ_INVALID_ARG;
    if (!x || !w || !scales || !biases || !inds || !y || M < 1 || ktop < 1)
        return mj_fail(ctx, MJ_INVALID_ARG, "gather_qmm2: null pointer or M/ktop < 1");
    if (K % 512 != 0 || N % 16 != 0 || K < 512 || N < 16 || (gs != 64 && gs != 128) ||
        M * ktop > MJ_MAX_PAIRS)
        return mj_fail(ctx, MJ_UNSUPPORTED_SHAPE,
                       "unsupported shape N=%d K=%d gs=%d (need K%%512==0, N%%16==0, gs 64|128, "
                       "M*ktop<=%d)", N, K, gs, MJ_MAX_PAIRS);
    if (epilogue != MJ_EPI_STORE && epilogue != MJ_EPI_ADD)
        return mj_fail(ctx, MJ_INVALID_ARG, "gather_qmm2: unknown epilogue %d", epilogue);
    if (epilogue == MJ_EPI_ADD && ktop != 1)
        return mj_fail(ctx, MJ_INVALID_ARG, "gather_qmm2: MJ_EPI_ADD needs ktop == 1");
    hipSetDevice(ctx->device);
    {
        mj_status sa = mj_hip(ctx, set_kernel_attributes(), "kernel attributes");
        if (sa != MJ_OK) return sa;
    }
    const int P = M * ktop;
    if (P == 1 && epilogue == MJ_EPI_STORE && (K == 512 || K == 1024 || K == 2048 || K == 4096)) {
        QmvArgs a{};
        a.x = (const uint16_t*)x;
        a.w = w;
        a.s = (const uint16_t*)scales;
        a.b = (const uint16_t*)biases;
        a.inds = inds;
        a.y = (uint16_t*)y;
        a.K = K;
        a.N = N;
        a.gs = gs;
        a.pairs = 1;
        a.lhs_per = 0;
        a.abort = ctx->abort_dev;
        return mj_hip(ctx, launch_qmv2(a, EPI_STORE, ctx->stream), "qmv2 launch");
    }
    const int rows_x = lhs_per_expert ? P : M;
    Arena ar;
    ar.take((size_t)rows_x * K * 2);
    ar.take((size_t)rows_x * (K / 64) * sizeof(float2));
    ar.take(sizeof(Buckets));
    mj_status s = mj_scratch_reserve(ctx, ar.off);
    if (s != MJ_OK) return s;
    ar = Arena{ctx->scratch, 0};
    uint16_t* xperm = (uint16_t*)ar.take((size_t)rows_x * K * 2);
    float2* xsum = (float2*)ar.take((size_t)rows_x * (K / 64) * sizeof(float2));
    Buckets* bk = (Buckets*)ar.take(sizeof(Buckets));
    s = mj_hip(ctx, launch_qx_prep((const uint16_t*)x, xperm, xsum, rows_x, K, ctx->abort_dev,
                                   ctx->stream), "qx prep");
    if (s != MJ_OK) return s;
    s = mj_hip(ctx, launch_bucket_inds(inds, P, bk, ctx->abort_dev, ctx->stream), "bucket");
    if (s != MJ_OK) return s;
    GatherArgs g{};
    g.xperm = xperm;
    g.xsum = xsum;
    g.w = w;
    g.s = (const uint16_t*)scales;
    g.b = (const uint16_t*)biases;
    g.bk = bk;
    g.y = (uint16_t*)y;
    g.K = K;
    g.N = N;
    g.gs = gs;
    g.x_div = lhs_per_expert ? 1 : ktop;
    g.abort = ctx->abort_dev;
    const int nb = P < MJ_MAX_EXPERTS ? P : MJ_MAX_EXPERTS;
    return mj_hip(ctx, launch_gather(g, epilogue == MJ_EPI_ADD ? EPI_ADD : EPI_STORE, P, nb,
                                     ctx->stream), "gather launch");
}

// Arguments and shape of an MoE block call (shared by mj_moe_block and its no-alloc variant).
static mj_status check_moe_args(mj_ctx* ctx, const mj_moe_weights* w, const void* x, void* y,
                                int M, int flags) {
    if (!w || !x || !y || M < 1 || M > MJ_MAX_ROWS)
        return mj_fail(ctx, MJ_INVALID_ARG, "moe_block: null pointer or M outside 1..%d",
                       MJ_MAX_ROWS);
    if (!w->router_w || !w->up_gate_w || !w->up_gate_s || !w->up_gate_b || !w->down_w ||
        !w->down_s || !w->down_b || ((flags & MJ_MOE_PRENORM) && !w->norm_w))
        return mj_fail(ctx, MJ_INVALID_ARG, "moe_block: null weight pointer");
    if (((uintptr_t)w->up_gate_alpha | (uintptr_t)w->down_alpha) % 16 != 0)
        return mj_fail(ctx, MJ_INVALID_ARG, "moe_block: row-alpha arrays must be 16-byte aligned");
    const int H = w->H, I = w->I, E = w->E, k = w->top_k, gs = w->gs;
    if (H % 2048 != 0 || H > 4096 || I % 512 != 0 || I > 4096 || E < k || E > MJ_MAX_EXPERTS ||
        k < 1 || k > 8 || (gs != 64 && gs != 128))
        return mj_fail(ctx, MJ_UNSUPPORTED_SHAPE,
                       "moe_block: unsupported shape H=%d I=%d E=%d top_k=%d gs=%d", H, I, E, k,
                       gs);
    return MJ_OK;
}

mj_status mj_moe_block(mj_ctx* ctx, const mj_moe_weights* w, const void* x, void* y, int M,
                       int flags, int32_t* out_inds, float* out_scores) {
    if (!ctx) return MJ_INVALID_ARG;
    mj_status s = check_moe_args(ctx, w, x, y, M, flags);
    if (s != MJ_OK) return s;
    hipSetDevice(ctx->device);
    s = mj_hip(ctx, set_kernel_attributes(), "kernel attributes");
    if (s != MJ_OK) return s;
    MoeScratch ms;
    s = moe_scratch(ctx, w->H, w->I, w->E, w->top_k, M, ms);
    if (s != MJ_OK) return s;
    return run_moe(ctx, w, (const uint16_t*)x, (uint16_t*)y, M, flags, ms,
                   out_inds ? out_inds : ms.inds, out_scores ? out_scores : ms.scores,
                   ctx->stream);
}

mj_status mj_moe_block_noalloc(mj_ctx* ctx, const mj_moe_weights* w, const void* x, void* y,
                               int M, int flags, int32_t* out_inds, float* out_scores) {
    if (!ctx) return MJ_INVALID_ARG;
    mj_status s = check_moe_args(ctx, w, x, y, M, flags);
    if (s != MJ_OK) return s;
    const int dev = ctx->device;
    void* base = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (dev >= 0 && dev < kMaxDevices && g_scratch_done[dev]) {
            if (g_scratch_err[dev] != hipSuccess)
                return mj_fail(ctx, MJ_HIP_ERROR, "moe_block_noalloc: static scratch address: %s",
                               hipGetErrorString(g_scratch_err[dev]));
            base = g_scratch_dev[dev];
        }
    }
    if (!base)
        return mj_fail(ctx, MJ_NOT_READY, "moe_block_noalloc: no static scratch on device %d",
                       dev);
    Arena count;
    MoeScratch ms;
    moe_scratch_layout(count, w->H, w->I, w->E, w->top_k, M, ms);
    if (count.off > MJ_MOE_NOALLOC_BYTES)
        return mj_fail(ctx, MJ_CAPACITY,
                       "moe_block_noalloc: scratch of %zu bytes for M=%d H=%d I=%d E=%d top_k=%d "
                       "exceeds MJ_MOE_NOALLOC_BYTES (%u)", count.off, M, w->H, w->I, w->E,
                       w->top_k, (unsigned)MJ_MOE_NOALLOC_BYTES);
    hipSetDevice(dev);
    s = mj_hip(ctx, set_kernel_attributes(), "kernel attributes");
    if (s != MJ_OK) return s;
    Arena real{base, 0};
    moe_scratch_layout(real, w->H, w->I, w->E, w->top_k, M, ms);
    return run_moe(ctx, w, (const uint16_t*)x, (uint16_t*)y, M, flags, ms,
                   out_inds ? out_inds : ms.inds, out_scores ? out_scores : ms.scores,
                   ctx->stream);
}

mj_status mj_selftest_mfma(mj_ctx* ctx, const void* A, const void* B, float* D) {
    if (!ctx || !A || !B || !D) return MJ_INVALID_ARG;
    hipSetDevice(ctx->device);
    return mj_hip(ctx, launch_selftest_mfma((const uint16_t*)A, (const uint16_t*)B, D,
                                            ctx->stream), "selftest launch");
}

}  // extern "C"

// ----------------------------------------------------------------------------------------
// MoE block orchestration (shared with the model pass).
// ----------------------------------------------------------------------------------------
void moe_scratch_layout(Arena& a, int H, int I, int E, int k, int M, MoeScratch& ms) {
    ms.xn = (uint16_t*)a.take((size_t)M * H * 2);
    ms.xperm = (uint16_t*)a.take((size_t)M * H * 2);
    ms.xsum = (float2*)a.take((size_t)M * (H / 64) * sizeof(float2));
    ms.logits = (float*)a.take((size_t)M * E * 4);
    ms.inds = (int32_t*)a.take((size_t)M * k * 4);
    ms.scores = (float*)a.take((size_t)M * k * 4);
    ms.bk = (Buckets*)a.take(sizeof(Buckets));
    ms.act = (uint16_t*)a.take((size_t)M * k * I * 2);
    ms.act_sum = (float2*)a.take((size_t)M * k * (I / 64) * sizeof(float2));
    ms.down = (uint16_t*)a.take((size_t)M * k * H * 2);
    ms.ecnt = (int*)a.take((size_t)E * 4);
    ms.eplist = (int*)a.take((size_t)E * MJ_MAX_ROWS * 4);
    ms.srec = (int*)a.take((size_t)64 * 64 * 4);
}

mj_status moe_scratch(mj_ctx* ctx, int H, int I, int E, int k, int M, MoeScratch& ms) {
    Arena count;
    moe_scratch_layout(count, H, I, E, k, M, ms);
    mj_status s = mj_scratch_reserve(ctx, count.off);
    if (s != MJ_OK) return s;
    Arena real{ctx->scratch, 0};
    moe_scratch_layout(real, H, I, E, k, M, ms);
    return MJ_OK;
}

// 1: passes that rank the routing inside the up product run both expert products as one
// launch (moe_fused_supported shapes); 0: two launches (kept for measurement).
#ifndef MJ_MOE_FUSED
#define MJ_MOE_FUSED 1
#endif

// Fewest rows that take the MFMA tile path (fewer: the VALU dot2 GEMV path, k_qmv2).  1: one
// row takes the tile path too, so that a verify row equals the one-row step bit for bit; the
// one-row A/B of the two paths is built with 2.
#ifndef MJ_TILE_MIN_ROWS
#define MJ_TILE_MIN_ROWS 1
#endif

mj_status run_moe(mj_ctx* ctx, const mj_moe_weights* w, const uint16_t* x, uint16_t* y, int M,
                  int flags, const MoeScratch& ms, int32_t* inds, float* scores, hipStream_t st,
                  Prof* prof, const NormOut* next) {
    const int H = w->H, I = w->I, E = w->E, k = w->top_k;
    const int* ab = ctx->abort_dev;
    const uint16_t* xn = x;
    mj_status s;
    const bool fused = route_supported(H, E, k);
    const bool up_tile = gather3_supported(EPI_SWIGLU, H, 2 * I, w->gs);
    const bool dn_tile = gather3_supported(EPI_STORE, I, H, w->gs);
    // tile path: the top-k launch also lists each expert's (row, slot) pairs for the gathers.
    // One row takes it too, so a row's result does not depend on how many rows share its pass
    // (a verify row equals the one-row decode step at its position, bit for bit).
    const bool tile = fused && M >= MJ_TILE_MIN_ROWS && M <= MJ_MAX_ROWS && up_tile && dn_tile;
    // the common expert shape, up to 32 rows over at most 64 experts: one launch ranks the
    // logits (its blocks build the slot records in LDS) and runs both products
    const bool moe_fused =
        MJ_MOE_FUSED && tile && E <= 64 &&
        (w->up_gate_alpha == nullptr) == (w->down_alpha == nullptr) &&
        moe_fused_supported(H, I, E, w->gs, M, w->up_gate_alpha != nullptr);
    // otherwise, up to 16 rows: the up || gate product still ranks the logits itself (one
    // launch fewer than a separate top-k)
    const bool topk_in_up = moe_fused || (tile && E <= 64 && M <= MJ_G5_FUSED_ROWS);
    if (fused) {
        RouteArgs ra{};
        ra.x = x;
        ra.norm_w = (flags & MJ_MOE_PRENORM) ? (const uint16_t*)w->norm_w : nullptr;
        ra.W = (const uint16_t*)w->router_w;
        ra.xn = (((M == 1 && !tile) || ms.want_plain) && (flags & MJ_MOE_PRENORM)) ? ms.xn : nullptr;
        ra.xperm = (M > 1 || tile) ? ms.xperm : nullptr;
        ra.xsum = (M > 1 || tile) ? ms.xsum : nullptr;
        ra.inds = inds;
        ra.scores = scores;
        ra.logits = ms.logits;
        // E <= 64: slot records for the persistent gathers; more experts: per-expert lists
        ra.srec = tile && E <= 64 ? ms.srec : nullptr;
        ra.ecnt = tile && E > 64 ? ms.ecnt : nullptr;
        ra.eplist = tile && E > 64 ? ms.eplist : nullptr;
        ra.M = M;
        ra.E = E;
        ra.k = k;
        ra.eps = w->eps;
        ra.abort = ab;
        ra.act_mark = moe_fused ? ms.act : nullptr;
        ra.act_n16 = moe_fused ? M * k * I / 8 : 0;
        s = mj_hip(ctx, launch_route_logits(ra, H, st), "route");
        if (s != MJ_OK) return s;
        if (!topk_in_up) {
            s = mj_hip(ctx, launch_route_topk(ra, st), "route top-k");
            if (s != MJ_OK) return s;
        }
        if (M == 1 && !tile && (flags & MJ_MOE_PRENORM)) xn = ms.xn;
    }
    if (M == 1 && !tile) {
        if (fused) {
        } else if (flags & MJ_MOE_PRENORM) {
            s = mj_hip(ctx, launch_rmsnorm_qx(x, (const uint16_t*)w->norm_w, w->eps, ms.xn,
                                              nullptr, nullptr, 1, H, ab, st), "rmsnorm");
            if (s != MJ_OK) return s;
            xn = ms.xn;
        }
        if (!fused) {
            s = mj_hip(ctx, launch_router((const uint16_t*)w->router_w, xn, ms.logits, 1, E, H,
                                          ab, st), "router");
            if (s != MJ_OK) return s;
            s = mj_hip(ctx, launch_topk_bucket(ms.logits, 1, E, k, inds, scores, nullptr, ab, st),
                       "topk");
            if (s != MJ_OK) return s;
        }
        QmvArgs up{};
        up.x = xn;
        up.w = w->up_gate_w;
        up.s = (const uint16_t*)w->up_gate_s;
        up.b = (const uint16_t*)w->up_gate_b;
        up.inds = inds;
        up.y = ms.act;
        up.K = H;
        up.N = 2 * I;
        up.gs = w->gs;
        up.pairs = k;
        up.lhs_per = 0;
        up.abort = ab;
        s = mj_hip(ctx, launch_qmv2(up, EPI_SWIGLU, st), "up qmv");
        if (s != MJ_OK) return s;
        QmvArgs dn = up;
        dn.x = ms.act;
        dn.w = w->down_w;
        dn.s = (const uint16_t*)w->down_s;
        dn.b = (const uint16_t*)w->down_b;
        dn.y = ms.down;
        dn.K = I;
        dn.N = H;
        dn.lhs_per = 1;
        s = mj_hip(ctx, launch_qmv2(dn, EPI_STORE, st), "down qmv");
        if (s != MJ_OK) return s;
    } else {
        if (!fused) {
            if (flags & MJ_MOE_PRENORM) {
                s = mj_hip(ctx, launch_rmsnorm_qx(x, (const uint16_t*)w->norm_w, w->eps, ms.xn,
                                                  ms.xperm, ms.xsum, M, H, ab, st), "rmsnorm");
                xn = ms.xn;
            } else {
                s = mj_hip(ctx, launch_qx_prep(x, ms.xperm, ms.xsum, M, H, ab, st), "qx prep");
            }
            if (s != MJ_OK) return s;
            s = mj_hip(ctx, launch_router((const uint16_t*)w->router_w, xn, ms.logits, M, E, H,
                                          ab, st), "router");
            if (s != MJ_OK) return s;
            s = mj_hip(ctx, launch_topk_bucket(ms.logits, M, E, k, inds, scores, ms.bk, ab, st),
                       "topk");
            if (s != MJ_OK) return s;
        } else if (!tile) {
            s = mj_hip(ctx, launch_bucket_inds(inds, M * k, ms.bk, ab, st), "bucket");
            if (s != MJ_OK) return s;
        }
        const int nb = M * k < E ? M * k : E;
        GatherArgs up{};
        up.xperm = ms.xperm;
        up.xsum = ms.xsum;
        up.w = w->up_gate_w;
        up.s = (const uint16_t*)w->up_gate_s;
        up.b = (const uint16_t*)w->up_gate_b;
        if (tile) {
            up.srec = E <= 64 ? ms.srec : nullptr;
            up.ecnt = E > 64 ? ms.ecnt : nullptr;
            up.eplist = E > 64 ? ms.eplist : nullptr;
        } else {
            up.bk = ms.bk;
        }
        up.alpha = tile ? (const uint16_t*)w->up_gate_alpha : nullptr;
        up.y = ms.act;
        up.ysum = ms.act_sum;
        up.K = H;
        up.N = 2 * I;
        up.gs = w->gs;
        up.x_div = k;
        up.abort = ab;
        if (topk_in_up) {
            up.rlogits = ms.logits;
            up.rM = M;
            up.rE = E;
            up.rk = k;
            up.rinds = inds;
            up.rscores = scores;
            up.rsrec = ms.srec;
        }
        if (!moe_fused) {
            if (prof) prof->begin(PROF_UP, st);
            s = mj_hip(ctx, launch_gather(up, EPI_SWIGLU, M, tile ? E : nb, st), "up gather");
            if (prof) prof->end(st);
            if (s != MJ_OK) return s;
        }
        // the tile kernel's SwiGLU epilogue writes act without block sums: the tile down
        // kernel forms them from its staged rows, any other down kernel gets them here
        if (up_tile && !dn_tile) {
            s = mj_hip(ctx, launch_qx_sums(ms.act, ms.act_sum, M * k, I, ab, st), "act sums");
            if (s != MJ_OK) return s;
        }
        GatherArgs dn = up;
        dn.rlogits = nullptr;  // the down product reads the records the up product wrote
        dn.xperm = ms.act;
        dn.xsum = dn_tile ? nullptr : ms.act_sum;
        dn.w = w->down_w;
        dn.s = (const uint16_t*)w->down_s;
        dn.b = (const uint16_t*)w->down_b;
        dn.alpha = tile ? (const uint16_t*)w->down_alpha : nullptr;
        dn.y = ms.down;
        dn.ysum = nullptr;
        dn.K = I;
        dn.N = H;
        dn.x_div = 1;
        if (moe_fused) {
            dn.rk = k;  // the down phase forms its records from the routing words too
            dn.fpolls = ctx->wait_polls;
            dn.ffault = ctx->fault_dev;
            if (prof) prof->begin(PROF_MOE, st);
            s = mj_hip(ctx, launch_moe_fused(up, dn, M, st), "fused MoE gathers");
            if (prof) prof->end(st);
            if (s != MJ_OK) return s;
        } else {
            if (prof) prof->begin(PROF_DOWN, st);
            s = mj_hip(ctx, launch_gather(dn, EPI_STORE, M, tile ? E : nb, st), "down gather");
            if (prof) prof->end(st);
            if (s != MJ_OK) return s;
        }
    }
    const uint16_t* resid = (flags & MJ_MOE_RESIDUAL) ? x : nullptr;
    if (next && H == 2048)
        return mj_hip(ctx, launch_combine_norm(ms.down, scores, resid, y, M, k, H, *next, ab, st),
                      "combine + norm");
    s = mj_hip(ctx, launch_score_combine(ms.down, scores, resid, y, M, k, H, ab, st), "combine");
    if (s != MJ_OK || !next) return s;
    return mj_hip(ctx, launch_rmsnorm_qx(y, next->w, next->eps, next->plain, next->xperm,
                                         next->xsum, M, H, ab, st), "next norm");
}
