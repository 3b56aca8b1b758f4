// Temporary: entry points not yet implemented report MJ_NOT_READY.
#include "mj_abi_internal.h"
extern "C" {
mj_status mj_attn_block(mj_ctx* ctx, const mj_attn_config*, const mj_attn_weights*, void*, void*,
                        void*, int64_t, const int32_t*, int) {
    return mj_fail(ctx, MJ_NOT_READY, "attn_block not built");
}
mj_status mj_lm_head_verify(mj_ctx* ctx, const void*, const void*, int, int, int, const int32_t*,
                            int, int32_t*, float*, float*) {
    return mj_fail(ctx, MJ_NOT_READY, "lm_head not built");
}
mj_status mj_accept_greedy(mj_ctx* ctx, const int32_t*, const int32_t*, const int32_t*, int,
                           int32_t*) {
    return mj_fail(ctx, MJ_NOT_READY, "accept not built");
}
mj_status mj_accept_sampled(mj_ctx* ctx, const float*, int, int, const int32_t*, float, int,
                            const float*, uint64_t, uint64_t, int32_t*) {
    return mj_fail(ctx, MJ_NOT_READY, "accept not built");
}
mj_status mj_model_create(mj_ctx* ctx, const mj_model_config*, const mj_layer_weights*,
                          const void*, const void*, const void*, mj_model**) {
    return mj_fail(ctx, MJ_NOT_READY, "model not built");
}
mj_status mj_model_destroy(mj_model*) { return MJ_NOT_READY; }
int64_t mj_model_offset(const mj_model*) { return -1; }
mj_status mj_model_rewind(mj_model*, int64_t) { return MJ_NOT_READY; }
mj_status mj_model_kv(mj_model*, int, void**, void**) { return MJ_NOT_READY; }
mj_status mj_prefill(mj_model*, const int32_t*, int, int, int32_t*) { return MJ_NOT_READY; }
mj_status mj_step_chain_feeds(mj_model*, const int32_t*, int, int32_t*) { return MJ_NOT_READY; }
mj_status mj_verify_greedy(mj_model*, int32_t, const int32_t*, int, const int32_t*, int32_t*,
                           int32_t*) {
    return MJ_NOT_READY;
}
mj_status mj_verify_sampled(mj_model*, int32_t, const int32_t*, int, float, int, const float*,
                            uint64_t, uint64_t, int32_t*, int32_t*) {
    return MJ_NOT_READY;
}
mj_status mj_model_set_capture(mj_model*, void*, int32_t*, float*) { return MJ_NOT_READY; }
mj_status mj_model_set_graphs(mj_model*, int) { return MJ_NOT_READY; }
float mj_model_last_pass_ms(const mj_model*) { return -1.0f; }
}
