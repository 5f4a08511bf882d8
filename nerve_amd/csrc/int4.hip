// Group-scaled INT4 linear (a9).
#include "common.h"
extern "C" nerve_hip_status nerve_hip_int4_linear(nerve_hip_ctx* ctx, const char*, const void*, const void*, const void*,
                                                  const void*, const void*, void*, uint32_t, void*) {
    nerve_hip_status st = nh::enter(ctx);
    if (st) return st;
    return nh::fail(NERVE_HIP_UNSUPPORTED, "int4_linear: not built yet");
}
