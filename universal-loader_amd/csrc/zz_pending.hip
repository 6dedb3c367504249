// Entry points whose kernels are not written yet.
#include "ulspec_internal.h"
using namespace ulspec;
extern "C" ulspec_status ulspec_verify_attention(ulspec_ctx* ctx, const uint16_t*, const uint16_t*, const uint16_t*,
                                                 uint32_t, uint32_t, const int32_t*, uint32_t, uint32_t, uint32_t,
                                                 float, float*)
{
    ULSPEC_CHECK_CTX(ctx);
    return fail(ctx, ULSPEC_EUNSUPPORTED, "verify_attention: not built yet");
}
