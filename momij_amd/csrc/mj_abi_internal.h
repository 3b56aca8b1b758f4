// mj_abi_internal.h -- host-side state behind the C ABI handles.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../../include/momij_hip.h"
#include "mj_internal.h"

struct mj_ctx {
    int device = 0;
    hipStream_t own = nullptr;     // the context's own stream (default priority)
    hipStream_t stream = nullptr;  // stream in use (own, or a caller's)
    // Abort word (stopBuf).  abort_dev is what kernels read; only mj_set_abort writes it, with a
    // copy on `ctl`, a stream of its own that no pass runs or is captured on, so any thread may
    // set it while a pass is queued, running or being captured, and kernels that start after
    // the copy see it.  abort_host mirrors it (set before the device word, cleared after it);
    // abort_gen counts the sets.  A call reports MJ_ABORTED when the word was set at its entry
    // or at its end, or was set in between (the generation moved): whenever its kernels may
    // have seen the word set.
    int* abort_dev = nullptr;
    hipStream_t ctl = nullptr;
    int* abort_src = nullptr;      // pinned {0, 1}: the copies' sources
    std::atomic<int> abort_host{0};
    std::atomic<unsigned> abort_gen{0};
    unsigned synced_gen = 0;       // abort_gen the owning thread's last synchronising call saw
    std::mutex abort_mu;           // one set or clear at a time
    // Fault word of the fused MoE launch (pinned, mapped: device writes land in host memory):
    // a block whose wait for the up product's items ran out its bound of polls sets it, and the
    // next synchronising call reports MJ_HIP_ERROR and clears it.
    int* fault = nullptr;
    int* fault_dev = nullptr;
    int wait_polls = 1 << 17;      // that bound (mj_set_wait_limit)
    void* scratch = nullptr;       // op-level scratch arena
    size_t scratch_bytes = 0;
    std::string err;
};

// Bump allocator over a buffer (base == nullptr: size counting only).
struct Arena {
    void* base = nullptr;
    size_t off = 0;
    void* take(size_t bytes);
};

struct MoeScratch {
    uint16_t* xn;        // normed rows, plain [M][H]
    uint16_t* xperm;     // qx rows [M][H]
    float2* xsum;        // [M][H/64]
    float* logits;       // [M][E]
    int32_t* inds;       // [M][k]
    float* scores;       // [M][k]
    Buckets* bk;
    uint16_t* act;       // [M*k][I] (qx for M > 1, plain for M == 1)
    float2* act_sum;     // [M*k][I/64]
    uint16_t* down;      // [M*k][H]
    int* ecnt;           // pairs per expert [E]
    int* eplist;         // pair lists per expert [E][MJ_ROWS]
    int* srec;           // routed-expert slot records [64][64] (E <= 64)
    bool want_plain = false;  // also write the normed rows plain into xn (debug capture)
};

// Optional per-kernel-class event timing of eager passes (classes of mj_model_kernel_ms).
enum {
    PROF_UP = 0, PROF_DOWN = 1, PROF_HEAD = 2, PROF_ATTN = 3, PROF_DENSE = 4,
    PROF_TIMER = 5,  // brackets around a hold of PROF_TIMER_US: bracket - hold = timer cost
    PROF_MOE = 6,    // up || gate then down in one launch (the fused MoE kernel)
    PROF_CLASSES = 7
};
constexpr unsigned PROF_TIMER_US = 20;
struct Prof {
    hipEvent_t* pool = nullptr;
    int cap = 0, used = 0;
    int cls[1024];
    bool valid[1024];
    // arms the next timing-aware launch with the event pair of this slot
    void begin(int c, hipStream_t) {
        if (!pool || used + 2 > cap) return;
        cls[used / 2] = c;
        timed_launch() = TimedLaunch{pool[used], pool[used + 1], true};
    }
    void end(hipStream_t) {
        if (!pool || used + 2 > cap) return;
        TimedLaunch& t = timed_launch();
        valid[used / 2] = !t.armed;  // the launch consumed the events
        t.armed = false;
        used += 2;
    }
};

mj_status mj_fail(mj_ctx* ctx, mj_status st, const char* fmt, ...);
mj_status mj_hip(mj_ctx* ctx, hipError_t e, const char* what);
mj_status mj_scratch_reserve(mj_ctx* ctx, size_t bytes);
// The abort word around one synchronising call: begin at its entry (MJ_ABORTED, and nothing
// queued, if the word is set; *gen receives the generation), end after its wait.
mj_status mj_abort_begin(mj_ctx* ctx, unsigned* gen);
mj_status mj_abort_end(mj_ctx* ctx, unsigned gen);
// Scratch of an MoE block call laid out over an arena (base nullptr: size counting only).
void moe_scratch_layout(Arena& a, int H, int I, int E, int k, int M, MoeScratch& ms);
mj_status moe_scratch(mj_ctx* ctx, int H, int I, int E, int k, int M, MoeScratch& ms);
// next: also normalise the block's output y into these outputs (the following RMSNorm).
mj_status run_moe(mj_ctx* ctx, const mj_moe_weights* w, const uint16_t* x, uint16_t* y, int M,
                  int flags, const MoeScratch& ms, int32_t* inds, float* scores, hipStream_t st,
                  Prof* prof = nullptr, const NormOut* next = nullptr);
