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
extern "C" ulspec_status ulspec_accept(ulspec_ctx* ctx, const ulspec_sampling*, uint32_t, uint32_t, uint32_t,
                                       const float*, const float*, const int32_t*, const float*, int32_t*, int32_t*)
{
    ULSPEC_CHECK_CTX(ctx);
    return fail(ctx, ULSPEC_EUNSUPPORTED, "accept: not built yet");
}
extern "C" ulspec_status ulspec_sample(ulspec_ctx* ctx, const ulspec_sampling*, uint32_t, uint32_t, const float*,
                                       const float*, int32_t*)
{
    ULSPEC_CHECK_CTX(ctx);
    return fail(ctx, ULSPEC_EUNSUPPORTED, "sample: not built yet");
}
extern "C" ulspec_status ulspec_uniforms(ulspec_ctx* ctx, uint64_t, uint64_t, uint32_t, float*)
{
    ULSPEC_CHECK_CTX(ctx);
    return fail(ctx, ULSPEC_EUNSUPPORTED, "uniforms: not built yet");
}
