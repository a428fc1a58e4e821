// The shrink to Q2_K: super-blocks of Q3_K, Q4_K or Q5_K re-encoded as Q2_K on the GPU, plain or
// with per-column importance weights.
//
// Restates crates/engine/src/requant.rs:113-304 (fit16, q2k_encode, q2k_encode_w and the six
// coachwhip_requant_* kernels). The reference runs one thread per 256-weight super-block with
// all 256 values in its registers; here 16 lanes share a super-block, lane j holding sub-block j
// (values 16j..16j+15), which is the unit fit16 works on:
//  1. each lane dequantizes its 16 values (candle's to_float arithmetic: a small integer times
//     an f32 product of f16 fields, minus another; the shader's dq_* readers give the same
//     values) and takes their min and max;
//  2. it runs fit16 (two weighted least-squares rounds) on its own;
//  3. the block's largest scale and min come from a butterfly over the 16 lanes, each lane
//     putting its scale and min on the 4-bit grid and rounding its 16 quants;
//  4. lane j's quants land in bytes 32(j/8) + 16(j%2) + i at bit 2((j%8)/2): the four lanes that
//     share those 16 bytes OR their words together through two shuffles, and one of them stores.
// Arithmetic is IEEE f32 in the shader's order, with no contraction into FMAs and correctly
// rounded division and square root, so the output bytes equal a CPU restatement's exactly.
#include "cw_common.h"
#include "cw_requant.h"

namespace cw {
namespace {

__device__ __forceinline__ float min_sel(float a, float b) { return b < a ? b : a; }
__device__ __forceinline__ float max_sel(float a, float b) { return b > a ? b : a; }
// clamp((int)v, 0, 3) and min(15, (int)v) with a saturating conversion (NaN gives 0)
__device__ __forceinline__ int level3(float v) { return v >= 3.f ? 3 : v >= 2.f ? 2 : v >= 1.f ? 1 : 0; }
__device__ __forceinline__ int level15(float v) { return v >= 15.f ? 15 : v >= 1.f ? (int)v : 0; }

__device__ __forceinline__ float f16_at(const uint8_t *p) {
    uint16_t h;
    __builtin_memcpy(&h, p, 2);
    return (float)__builtin_bit_cast(_Float16, h);
}

// sub-block j of 6-bit scale / min pairs packed in 12 bytes (vendor/candle-core/src/quantized/utils.rs:50-60)
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *q, int &d, int &m) {
    if (j < 4) {
        d = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// x[i] = value 16 g + i of a source super-block b (g = the lane's sub-block)
template <int SRC>
__device__ __forceinline__ void dequant16(const uint8_t *b, int g, float *x);

// Q3_K {hmask[32], qs[64], scales[12], d}: k_quants.rs:1514-1571
template <>
__device__ __forceinline__ void dequant16<CW_Q3_K>(const uint8_t *b, int g, float *x) {
#pragma clang fp contract(off)
    const int half = g >> 3, ss = (g >> 1) & 3, part = g & 1;
    const int lo = (b[96 + (g & 7)] >> (4 * (g >> 3))) & 0xF, hi = (b[104 + (g & 3)] >> (2 * (g >> 2))) & 3;
    const float dl = f16_at(b + 108) * ((float)(lo | (hi << 4)) - 32.0f);
    uint8_t q[16], h[16];
    __builtin_memcpy(q, b + 32 + 32 * half + 16 * part, 16);
    __builtin_memcpy(h, b + 16 * part, 16);
    const int hs = 4 * half + ss;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int v = ((q[i] >> (2 * ss)) & 3) - (((h[i] >> hs) & 1) ? 0 : 4);
        x[i] = dl * (float)v;
    }
}

// Q4_K {d, dmin, scales[12], qs[128]}: k_quants.rs:1821-1849
template <>
__device__ __forceinline__ void dequant16<CW_Q4_K>(const uint8_t *b, int g, float *x) {
#pragma clang fp contract(off)
    const int c = g >> 2, upper = (g >> 1) & 1;
    int s, m;
    scale_min_k4(2 * c + upper, b + 4, s, m);
    const float d1 = f16_at(b) * (float)s, m1 = f16_at(b + 2) * (float)m;
    uint8_t q[16];
    __builtin_memcpy(q, b + 16 + 32 * c + 16 * (g & 1), 16);
#pragma unroll
    for (int i = 0; i < 16; i++) x[i] = d1 * (float)(upper ? q[i] >> 4 : q[i] & 0xF) - m1;
}

// Q5_K {d, dmin, scales[12], qh[32], qs[128]}: k_quants.rs:2120-2152
template <>
__device__ __forceinline__ void dequant16<CW_Q5_K>(const uint8_t *b, int g, float *x) {
#pragma clang fp contract(off)
    const int c = g >> 2, upper = (g >> 1) & 1;
    int s, m;
    scale_min_k4(2 * c + upper, b + 4, s, m);
    const float d1 = f16_at(b) * (float)s, m1 = f16_at(b + 2) * (float)m;
    uint8_t q[16], h[16];
    __builtin_memcpy(q, b + 48 + 32 * c + 16 * (g & 1), 16);
    __builtin_memcpy(h, b + 16 + 16 * (g & 1), 16);
    const int hb = 2 * c + upper;
#pragma unroll
    for (int i = 0; i < 16; i++)
        x[i] = d1 * ((float)(upper ? q[i] >> 4 : q[i] & 0xF) + (((h[i] >> hb) & 1) ? 16.0f : 0.0f)) - m1;
}

// fit16, requant.rs:119-138
__device__ __forceinline__ void fit16(const float *x, const float *w, float &scale, float &mn) {
#pragma clang fp contract(off)
#pragma unroll
    for (int round = 0; round < 2; ++round) {
        float sw = 0.f, swl = 0.f, swll = 0.f, swx = 0.f, swlx = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int l = scale > 0.f ? level3((x[i] + mn) / scale + 0.5f) : 0;
            const float wi = w[i], fl = (float)l;
            sw += wi;
            swl += wi * fl;
            swll += wi * fl * fl;
            swx += wi * x[i];
            swlx += wi * fl * x[i];
        }
        const float det = sw * swll - swl * swl;
        if (det > 1e-12f) {
            const float a = (sw * swlx - swl * swx) / det;
            const float b = (swl * swlx - swll * swx) / det;
            if (a > 0.f && b >= 0.f) {
                scale = a;
                mn = b;
            }
        }
    }
}

// One super-block per 16 lanes (g = lane % 16 = this lane's sub-block): src is the source block,
// w the block's 256 column weights or NULL, y the 84-byte Q2_K block (stored when store is set;
// every lane takes part in the shuffles either way).
template <int SRC>
__device__ __forceinline__ void shrink_block(const uint8_t *src, const float *w_row, uint8_t *y, int g, bool store) {
#pragma clang fp contract(off)
    float x[16], w[16];
    dequant16<SRC>(src, g, x);
    if (w_row) {
        const float *ws = w_row + 16 * g;
#pragma unroll
        for (int i = 0; i < 16; i++) w[i] = sqrtf(max_sel(ws[i], 0.f)) + 1e-6f;
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) w[i] = 1.f;
    }
    float lo = x[0], hi = x[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) {
        lo = min_sel(lo, x[i]);
        hi = max_sel(hi, x[i]);
    }
    if (lo > 0.f) lo = 0.f;
    float sc = (hi - lo) / 3.f, mn = -lo;
    fit16(x, w, sc, mn);
    // the block's maxima, started from +0 as the shader's running maximum is
    float max_scale = max_sel(0.f, sc), max_min = max_sel(0.f, mn);
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) {
        max_scale = max_sel(max_scale, __shfl_xor(max_scale, o, 64));
        max_min = max_sel(max_min, __shfl_xor(max_min, o, 64));
    }
    const float inv_scale = max_scale > 0.f ? 15.f / max_scale : 0.f;
    const float inv_min = max_min > 0.f ? 15.f / max_min : 0.f;
    const int ls = level15(sc * inv_scale + 0.5f), lm = level15(mn * inv_min + 0.5f);
    const _Float16 dh = (_Float16)(max_scale / 15.f), mh = (_Float16)(max_min / 15.f);
    const float dj = (float)dh * (float)ls, mj = (float)mh * (float)lm;
    const int shift = 2 * ((g >> 1) & 3);
    uint32_t word[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t l = dj > 0.f ? (uint32_t)level3((x[i] + mj) / dj + 0.5f) : 0u;
        word[i >> 2] |= l << (8 * (i & 3) + shift);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        word[k] |= (uint32_t)__shfl_xor((int)word[k], 2, 64);
        word[k] |= (uint32_t)__shfl_xor((int)word[k], 4, 64);
    }
    if (!store) return;
    y[g] = (uint8_t)(ls | (lm << 4));
    if (shift == 0) {
        uint8_t *qs = y + 16 + 32 * (g >> 3) + 16 * (g & 1);
#pragma unroll
        for (int k = 0; k < 4; k++) __builtin_memcpy(qs + 4 * k, &word[k], 4);
    }
    if (g == 0) {
        const uint32_t dd = (uint32_t)__builtin_bit_cast(uint16_t, dh) | ((uint32_t)__builtin_bit_cast(uint16_t, mh) << 16);
        __builtin_memcpy(y + 80, &dd, 4);
    }
}

template <int SRC>
constexpr int src_bytes() { return SRC == CW_Q3_K ? 110 : SRC == CW_Q4_K ? 144 : 176; }

// n_blocks consecutive source blocks into n_blocks consecutive Q2_K blocks
template <int SRC>
__global__ __launch_bounds__(256) void k_requant_q2k(const uint8_t *src, int64_t n_blocks, const float *shape,
                                                     int64_t blocks_per_row, uint8_t *dst) {
    const int g = threadIdx.x & 15;
    const int64_t blk = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    // every lane joins the shuffles; lanes past the end work on the last block and store nothing
    const int64_t b = blk < n_blocks ? blk : n_blocks - 1;
    shrink_block<SRC>(src + b * src_bytes<SRC>(), shape ? shape + (b % blocks_per_row) * 256 : nullptr, dst + b * 84, g,
                      blk < n_blocks);
}

// Piece y (blockIdx.y) of a list: blocks_per_piece source blocks at src + y * src_stride into
// dst + index[y] * dst_stride (the bank's shrink of staged experts into their slots)
template <int SRC>
__global__ __launch_bounds__(256) void k_shrink_pieces(const uint8_t *src, int64_t src_stride, ShrinkIndex index, uint8_t *dst,
                                                       int64_t dst_stride, int64_t blocks_per_piece, const float *shape,
                                                       int64_t blocks_per_row) {
    const int g = threadIdx.x & 15;
    const int64_t blk = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int64_t b = blk < blocks_per_piece ? blk : blocks_per_piece - 1;
    const uint8_t *s = src + blockIdx.y * src_stride + b * src_bytes<SRC>();
    uint8_t *y = dst + (int64_t)index.i[blockIdx.y] * dst_stride + b * 84;
    shrink_block<SRC>(s, shape ? shape + (b % blocks_per_row) * 256 : nullptr, y, g, blk < blocks_per_piece);
}

}  // namespace

int shrink_pieces(int src_dtype, const uint8_t *src, int64_t src_stride, const ShrinkIndex &index, int n, uint8_t *dst,
                  int64_t dst_stride, int64_t blocks_per_piece, const float *shape, int64_t blocks_per_row, hipStream_t s) {
    if (n == 0 || blocks_per_piece == 0) return CW_OK;
    const dim3 grid((unsigned)((blocks_per_piece + 15) / 16), (unsigned)n), block(256);
    switch (src_dtype) {
    case CW_Q3_K: hipLaunchKernelGGL(k_shrink_pieces<CW_Q3_K>, grid, block, 0, s, src, src_stride, index, dst, dst_stride, blocks_per_piece, shape, blocks_per_row); break;
    case CW_Q4_K: hipLaunchKernelGGL(k_shrink_pieces<CW_Q4_K>, grid, block, 0, s, src, src_stride, index, dst, dst_stride, blocks_per_piece, shape, blocks_per_row); break;
    case CW_Q5_K: hipLaunchKernelGGL(k_shrink_pieces<CW_Q5_K>, grid, block, 0, s, src, src_stride, index, dst, dst_stride, blocks_per_piece, shape, blocks_per_row); break;
    default: return set_error(CW_ENOTSUP, "shrink: source type %d (Q3_K, Q4_K or Q5_K)", src_dtype);
    }
    return check_launch("k_shrink_pieces");
}

static int requant_q2k(int src_dtype, const void *src, int64_t n_blocks, const float *shape, int64_t blocks_per_row,
                       void *dst, hipStream_t s) {
    if (n_blocks == 0) return CW_OK;
    const dim3 grid((unsigned)((n_blocks + 15) / 16)), block(256);
    const uint8_t *in = (const uint8_t *)src;
    uint8_t *out = (uint8_t *)dst;
    switch (src_dtype) {
    case CW_Q3_K: hipLaunchKernelGGL(k_requant_q2k<CW_Q3_K>, grid, block, 0, s, in, n_blocks, shape, blocks_per_row, out); break;
    case CW_Q4_K: hipLaunchKernelGGL(k_requant_q2k<CW_Q4_K>, grid, block, 0, s, in, n_blocks, shape, blocks_per_row, out); break;
    case CW_Q5_K: hipLaunchKernelGGL(k_requant_q2k<CW_Q5_K>, grid, block, 0, s, in, n_blocks, shape, blocks_per_row, out); break;
    default: return set_error(CW_ENOTSUP, "requant: source type %d (Q3_K, Q4_K or Q5_K)", src_dtype);
    }
    return check_launch("k_requant_q2k");
}

}  // namespace cw

extern "C" int cw_requant_q2k(int src_dtype, const void *src, int64_t n_blocks, const float *shape,
                              int64_t blocks_per_row, void *dst, cw_stream_t stream) {
    CW_REQUIRE(n_blocks >= 0 && n_blocks < ((int64_t)1 << 35), "requant: %lld blocks", (long long)n_blocks);
    CW_REQUIRE(n_blocks == 0 || (src && dst), "requant: null pointer");
    CW_REQUIRE(!shape || (blocks_per_row > 0 && ((uintptr_t)shape & 3u) == 0),
               "requant: weights need blocks_per_row > 0 (got %lld) and 4-byte alignment", (long long)blocks_per_row);
    return cw::requant_q2k(src_dtype, src, n_blocks, shape, blocks_per_row, dst, (hipStream_t)stream);
}
