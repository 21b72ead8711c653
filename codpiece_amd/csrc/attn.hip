// attn.hip — tree-masked GQA attention over the f16 KV cache.
#include "cpv_internal.h"

extern "C" cpv_status cpv_attn(cpv_ctx* ctx, const float*, const uint16_t*, const uint16_t*, int64_t,
                               const int32_t*, int, int, int, int, float, float*)
{
    return cpv_fail(ctx, CPV_EUNSUPPORTED, "attn: not built yet");
}
