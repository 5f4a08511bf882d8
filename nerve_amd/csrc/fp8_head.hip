// FP8 output projection + argmax (a10, a11).
#include "common.h"
extern "C" nerve_hip_status nerve_hip_fp8_output_projection(nerve_hip_ctx* ctx, const char*, const void*, const void*,
                                                            const void*, void*, void*, void*, uint32_t, void*) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    return nh::fail(NERVE_HIP_UNSUPPORTED, "fp8_output_projection: not built yet");
}
extern "C" nerve_hip_status nerve_hip_argmax_f32(nerve_hip_ctx* ctx, const void*, uint32_t, uint32_t, void*, void*) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    return nh::fail(NERVE_HIP_UNSUPPORTED, "argmax_f32: not built yet");
}
