// arfq_moe.hip -- top-k routing, expert grouping and the grouped SwiGLU MoE.
#include "arfq_common.h"
#include "arfq_internal.h"

extern "C" {

int arfq_moe_route(arfq_ctx *ctx, const float *, int64_t, int, int, int, int32_t *, float *) {
    if (!ctx) return ARFQ_E_INVALID;
    ctx->err = "moe_route: not implemented";
    return ARFQ_E_UNSUPPORTED;
}

int arfq_moe(arfq_ctx *ctx, const arfq_weight *, const arfq_weight *, const arfq_weight *,
             const float *, int64_t, int, int, const void *, int, float *) {
    if (!ctx) return ARFQ_E_INVALID;
    ctx->err = "moe: not implemented";
    return ARFQ_E_UNSUPPORTED;
}

int arfq_moe_ids(arfq_ctx *ctx, const arfq_weight *, const arfq_weight *, const arfq_weight *,
                 const int32_t *, const float *, int64_t, int, const void *, int, float *) {
    if (!ctx) return ARFQ_E_INVALID;
    ctx->err = "moe_ids: not implemented";
    return ARFQ_E_UNSUPPORTED;
}
}
