// Internal interface of the matvec kernels (cw_gemv.hip) for the C ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cw {

struct GemvArgs {
    const uint8_t *w0;        // bank (gate, or the only matrix)
    const uint8_t *w1;        // up bank (gate/up mode)
    int64_t slot_stride0, slot_stride1;
    int64_t row_bytes;        // bytes per row, same for w0 and w1
    int n, k, nsb;            // rows, weights per row, 32-weight sub-blocks per row
    int n_slots;              // ids >= n_slots are rejected (NaN output)
    const float *x;           // activations, rows of k
    int x_per_pick;           // x row = pick index (1) or pick / K (0)
    const uint32_t *ids;      // slot of each pick, or NULL (slot 0)
    const uint32_t *experts;  // expert id of each pick (bias lookup), or NULL
    int K;                    // picks per token
    float *out;
    int out_width;            // row stride of out (>= n; gate/up mode zero-pads up to it)
    int act;                  // gate/up mode: enum cw_act
    float alpha, limit;
    const float *b0, *b1;     // gate/up biases (E x n) or NULL
    const float *wts;         // down mode: routing weights (T x K)
    const float *bd;          // down mode: down bias (E x n) or NULL
    int tile;                 // down mode: rows per block (set by gemv_down)
};

int gemv_plain(int dtype, const GemvArgs &a, int picks, hipStream_t s);
int gemv_gateup(int dtype, const GemvArgs &a, int picks, hipStream_t s);
int gemv_down(int dtype, GemvArgs a, int tokens, hipStream_t s);
int dequantize(int dtype, const void *blocks, int64_t n_elems, float *out, hipStream_t s);
int max_gemv_k();

}  // namespace cw
