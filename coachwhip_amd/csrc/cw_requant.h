// Internal interface of the shrink to Q2_K (cw_requant.hip) for the bank's fill.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cw {

constexpr int SHRINK_PIECES = 64;  // pieces per launch

struct ShrinkIndex {
    uint32_t i[SHRINK_PIECES];
};

// Piece y < n: blocks_per_piece super-blocks of src_dtype (Q3_K, Q4_K or Q5_K) at src + y *
// src_stride shrunk to Q2_K at dst + index.i[y] * dst_stride; shape (device, blocks_per_row *
// 256 column weights) or NULL.
int shrink_pieces(int src_dtype, const uint8_t *src, int64_t src_stride, const ShrinkIndex &index, int n, uint8_t *dst,
                  int64_t dst_stride, int64_t blocks_per_piece, const float *shape, int64_t blocks_per_row, hipStream_t s);

}  // namespace cw
