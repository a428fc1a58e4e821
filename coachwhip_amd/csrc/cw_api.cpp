// C ABI entry points for formats, dense quantized matmul and the expert matvec, plus the
// library's error reporting. The MoE-layer, routing and activation entry points live in
// cw_moe.hip; the host bank bookkeeping in cw_slots.cpp.
#include <stdarg.h>
#include <stdlib.h>
#include <string.h>

#include "cw_common.h"
#include "cw_gemv.h"
#include "cw_mfma.h"

namespace cw {

static thread_local char g_err[512] = "";

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(CW_EHIP, "%s: %s", what, hipGetErrorString(e));
    return CW_OK;
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace cw

using namespace cw;

extern "C" {

const char *cw_version(void) { return "cwmoe 0.1 (gfx950)"; }

const char *cw_last_error(void) { return g_err; }

int cw_block_size(int dtype) {
    switch (dtype) {
    case CW_F32: case CW_F16: return 1;
    case CW_Q8_0: case CW_MXFP4: case CW_MXFP4_R16: return 32;
    case CW_Q2_K: case CW_Q3_K: case CW_Q4_K: case CW_Q5_K: case CW_Q6_K: case CW_IQ2_XXS: case CW_IQ2_S:
    case CW_IQ3_XXS: case CW_IQ3_S: case CW_IQ4_XS: return 256;
    default: return 0;
    }
}

int cw_type_size(int dtype) {
    switch (dtype) {
    case CW_F32: return 4;
    case CW_F16: return 2;
    case CW_Q8_0: return 34;
    case CW_Q2_K: return 84;
    case CW_Q3_K: return 110;
    case CW_Q4_K: return 144;
    case CW_Q5_K: return 176;
    case CW_Q6_K: return 210;
    case CW_IQ3_XXS: return 98;
    case CW_IQ4_XS: return 136;
    case CW_IQ2_XXS: return 66;
    case CW_IQ2_S: return 82;
    case CW_IQ3_S: return 110;
    case CW_MXFP4: case CW_MXFP4_R16: return 17;
    default: return 0;
    }
}

int cw_dequantize(int dtype, const void *blocks, int64_t n_elems, float *out, cw_stream_t stream) {
    if (!is_weight_type(dtype)) return set_error(CW_ENOTSUP, "dequantize: dtype %d is not supported", dtype);
    const int bs = cw_block_size(dtype);
    CW_REQUIRE(n_elems >= 0 && n_elems % bs == 0, "dequantize: %lld weights are not whole %d-weight blocks",
               (long long)n_elems, bs);
    if (n_elems == 0) return CW_OK;
    CW_REQUIRE(blocks && out, "dequantize: null pointer");
    CW_REQUIRE(aligned16(out), "dequantize: out must be 16-byte aligned");
    return dequantize(dtype, blocks, n_elems, out, (hipStream_t)stream);
}

// Rows of x from which cw_qmatmul runs as an MFMA GEMM instead of one matvec per row, where the
// two cross over on MI355X (graph-replayed, 2048x2048 Q8_0 and 4096x4096 Q4_K): a Q4_K matvec
// row costs ~11 us, the GEMM ~20 us at any small M; a Q8_0 row ~4.4 us against ~14 us.
// CWMOE_MM_MIN_ROWS overrides. (The reference switches to its simdgroup-matrix kernel above 8
// rows, vendor/candle-core/src/quantized/metal.rs:339-353.)
static int64_t mm_min_rows(int dtype) {
    const char *e = getenv("CWMOE_MM_MIN_ROWS");
    return e ? atoll(e) : dtype == CW_Q4_K ? 2 : 8;
}
static bool qmatmul_mfma(int dtype, int64_t k, int64_t m) {
    return m >= mm_min_rows(dtype) && cw::mfma_supported(dtype) && k % cw_block_size(dtype) == 0 && k % 32 == 0 &&
           (dtype == CW_Q8_0 || dtype == CW_MXFP4 || k % 256 == 0);
}

size_t cw_qmatmul_workspace_size(int dtype, int64_t n, int64_t k, int64_t m) {
    (void)n;
    if (!is_weight_type(dtype) || k <= 0 || m <= 0 || !qmatmul_mfma(dtype, k, m)) return 0;
    return cw::mfma_dense_workspace(dtype, m, n, k);
}

int cw_qmatmul(int dtype, const void *w, int64_t n, int64_t k, const float *x, int64_t m, float *y, void *ws,
               size_t ws_bytes, cw_stream_t stream) {
    if (!is_weight_type(dtype)) return set_error(CW_ENOTSUP, "qmatmul: dtype %d is not supported", dtype);
    const int bs = cw_block_size(dtype);
    CW_REQUIRE(n >= 0 && m >= 0 && k > 0, "qmatmul: n %lld, k %lld, m %lld", (long long)n, (long long)k, (long long)m);
    CW_REQUIRE(k % bs == 0, "qmatmul: k %lld is not whole %d-weight blocks", (long long)k, bs);
    CW_REQUIRE(n < (1ll << 31) && m < (1ll << 31), "qmatmul: n or m too large");
    if (k > max_gemv_k()) return set_error(CW_ENOTSUP, "qmatmul: k %lld exceeds %d", (long long)k, max_gemv_k());
    if (n == 0 || m == 0) return CW_OK;
    CW_REQUIRE(w && x && y, "qmatmul: null pointer");
    CW_REQUIRE(aligned16(x), "qmatmul: x must be 16-byte aligned");
    if (qmatmul_mfma(dtype, k, m))
        return cw::mfma_dense(dtype, (const uint8_t *)w, k / bs * cw_type_size(dtype), (int)n, (int)k, x, (int)m, y, ws,
                              ws_bytes, (hipStream_t)stream);
    GemvArgs a = {};
    a.w0 = (const uint8_t *)w;
    a.row_bytes = k / bs * cw_type_size(dtype);
    a.slot_stride0 = 0;
    a.n = (int)n;
    a.k = (int)k;
    a.nsb = (int)(k / 32);
    a.n_slots = 1;
    a.x = x;
    a.x_per_pick = 1;
    a.K = 1;
    a.out = y;
    a.out_width = (int)n;
    return gemv_dense(dtype, a, (int)m, (hipStream_t)stream);
}

int cw_matvec_id(int dtype, int64_t n, int64_t k, int64_t n_slots, int64_t slot_stride, const void *bank, const float *x,
                 int x_rows_per_expert, const uint32_t *ids, int K, int T, float *out, cw_stream_t stream) {
    if (!is_weight_type(dtype)) return set_error(CW_ENOTSUP, "matvec_id: dtype %d is not supported", dtype);
    const int bs = cw_block_size(dtype);
    CW_REQUIRE(n > 0 && k > 0 && n < (1ll << 31), "matvec_id: n %lld, k %lld", (long long)n, (long long)k);
    CW_REQUIRE(k % bs == 0, "matvec_id: k %lld is not whole %d-weight blocks", (long long)k, bs);
    CW_REQUIRE(K > 0 && T >= 0, "matvec_id: K %d, T %d", K, T);
    CW_REQUIRE(n_slots > 0 && n_slots < (1ll << 32), "matvec_id: %lld slots", (long long)n_slots);
    const int64_t row_bytes = k / bs * cw_type_size(dtype);
    CW_REQUIRE(slot_stride >= n * row_bytes, "matvec_id: slot stride %lld below the %lld-byte matrix",
               (long long)slot_stride, (long long)(n * row_bytes));
    if (k > max_gemv_k()) return set_error(CW_ENOTSUP, "matvec_id: k %lld exceeds %d", (long long)k, max_gemv_k());
    if (T == 0) return CW_OK;
    CW_REQUIRE(bank && x && ids && out, "matvec_id: null pointer");
    CW_REQUIRE(aligned16(x), "matvec_id: x must be 16-byte aligned");
    GemvArgs a = {};
    a.w0 = (const uint8_t *)bank;
    a.slot_stride0 = slot_stride;
    a.row_bytes = row_bytes;
    a.n = (int)n;
    a.k = (int)k;
    a.nsb = (int)(k / 32);
    a.n_slots = (int)(n_slots > 0x7fffffff ? 0x7fffffff : n_slots);
    a.x = x;
    a.x_per_pick = x_rows_per_expert ? 1 : 0;
    a.ids = ids;
    a.K = K;
    a.out = out;
    a.out_width = (int)n;
    return gemv_plain(dtype, a, T * K, (hipStream_t)stream);
}

}  // extern "C"
