// sample.hip — speculative acceptance on the device.
#include "cpv_internal.h"

extern "C" cpv_status cpv_spec_accept(cpv_ctx* ctx, const float*, const float*, const int32_t*, int, int, int,
                                      const cpv_sampler_params*, int, const float*, uint64_t, const float*,
                                      const int32_t*, int, int32_t*, int32_t*)
{
    return cpv_fail(ctx, CPV_EUNSUPPORTED, "spec_accept: not built yet");
}
