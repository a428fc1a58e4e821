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
// Byte offset of block b of row r in a matrix of MXFP4 rows held in groups of 16 (the layout of
// CW_MXFP4_R16): group g = r / 16 takes its 16 rows' bytes from 16 g row_bytes, as GGUF rows do;
// within it step c (blocks 4c .. 4c + cb - 1, cb = min(4, nblk - 4c)) holds the 16 rows' blocks of
// that step side by side, row after row: 272 cb bytes from 1,088 c. Blocks stay whole (17 bytes).
__host__ __device__ __forceinline__ int64_t rows16_offset(int64_t r, int b, int nblk) {
    const int c = b >> 2, cb = nblk - 4 * c < 4 ? nblk - 4 * c : 4;
    return (r >> 4) * 16 * (int64_t)nblk * 17 + (int64_t)c * 1088 + (r & 15) * 17 * cb + (b & 3) * 17;
}

// formats of expert matrices: the GGUF ones, and MXFP4 in row groups of 16
inline bool is_expert_type(int dtype) { return is_weight_type(dtype) || dtype == CW_MXFP4_R16; }
// bytes of a matrix of n rows: row groups of 16 hold whole groups
inline int64_t matrix_bytes(int dtype, int64_t n, int64_t row_bytes) {
    return (dtype == CW_MXFP4_R16 ? (n + 15) / 16 * 16 : n) * row_bytes;
}

}  // namespace cw

#define CW_REQUIRE(cond, ...) \
    do { if (!(cond)) return ::cw::set_error(CW_EINVAL, __VA_ARGS__); } while (0)
