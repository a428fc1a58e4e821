// Internal interface of the matvec kernels (cw_gemv.hip) for the C ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cw {

struct GemvArgs {
    const uint8_t *w0;        // matrix, or bank of slot matrices
    int64_t slot_stride0;
    int64_t row_bytes;        // bytes per row
    int n, k, nsb;            // rows, weights per row, 32-weight sub-blocks per row
    int n_slots;              // ids >= n_slots are rejected (NaN output)
    const float *x;           // activations, rows of k
    int x_per_pick;           // x row = pick index (1) or pick / K (0)
    const uint32_t *ids;      // slot of each pick, or NULL (slot 0)
    int K;                    // picks per token
    float *out;
    int out_width;            // row stride of out (>= n)
};

int gemv_plain(int dtype, const GemvArgs &a, int picks, hipStream_t s);
// y[t] = W x[t] for t < m rows of x and one matrix (QMatMul at small m): x staged once per block
int gemv_dense(int dtype, const GemvArgs &a, int m, hipStream_t s);
int dequantize(int dtype, const void *blocks, int64_t n_elems, float *out, hipStream_t s);
int max_gemv_k();

}  // namespace cw
