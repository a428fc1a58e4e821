// Host-side helpers shared by the library's translation units: status codes, the per-thread
// last-error message, argument checks and HIP error propagation.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/cwmoe.h"

namespace cw {

int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Launch-time HIP errors (a bad configuration, an invalid stream) become CW_EHIP.
int check_launch(const char *what);

inline bool is_weight_type(int dtype) {
    return dtype == CW_Q8_0 || dtype == CW_Q2_K || dtype == CW_Q4_K || dtype == CW_Q5_K || dtype == CW_Q6_K ||
           dtype == CW_IQ2_XXS || dtype == CW_IQ2_S || dtype == CW_IQ3_XXS || dtype == CW_IQ3_S || dtype == CW_IQ4_XS ||
           dtype == CW_MXFP4;
}

}  // namespace cw

#define CW_REQUIRE(cond, ...) \
    do { if (!(cond)) return ::cw::set_error(CW_EINVAL, __VA_ARGS__); } while (0)
