// Internal interface of the router-logits kernels (cw_router.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cw {

// logits[t][e] = x[t] . W[e] (+ bias[e]); W is E x h, f32 (CW_F32) or f16 (CW_F16); h % 4 == 0
int router_logits(int wdtype, const void *w, int E, int h, const float *bias, const float *x, int T, float *logits,
                  hipStream_t s);

}  // namespace cw
