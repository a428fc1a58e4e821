// Device-side readers of the GGUF block formats on the expert path (gfx950).
//
// The unit every kernel works in is a 32-weight sub-block: one Q8_0 or MXFP4 block, or one
// eighth of a Q4_K / IQ super-block. For each format, Fmt::load() reads the bytes one
// sub-block needs straight from the raw row (gfx950 runs with unaligned access enabled, so the
// odd GGUF block strides of 17, 34, 66, 82, 84 and 110 bytes cost no extra instructions),
// Fmt::dequant() writes its 32 exact f32 values and Fmt::dot() returns their dot product with
// 32 f32 activations. Dequantization is an exact product of an f16 (or power-of-two) scale and
// small integers in every format here, so dequant() is bit-identical to the CPU dequantizers;
// dot() factors the scales out of the sum and differs from dequantize-then-dot only by f32
// rounding of the sum.
//
// Layout and arithmetic follow vendor/candle-core/src/quantized/k_quants.rs (Q8_0 766-782,
// Q2_K 1152-1190, Q4_K 1821-1849 with get_scale_min_k4 in quantized/utils.rs:50-60, Q5_K
// 2120-2152, Q6_K 2420-2451, MXFP4 638-691) and the Metal dequantizers in
// vendor/candle-metal-kernels/src/metal_src/quantized.metal (IQ2_XXS 6820-6843, IQ2_S 6918-6935,
// IQ3_XXS 6866-6891, IQ3_S 6893-6916, IQ4_XS 7000-7016).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "cw_grids.h"

namespace cw {

template <class F>
struct TableRegs;

// Lattice tables, copied to LDS by the kernels that read IQ formats.
static __constant__ uint64_t c_iq2xxs_grid[256] = {CW_IQ2XXS_GRID_VALUES};
static __constant__ uint64_t c_iq2s_grid[1024] = {CW_IQ2S_GRID_VALUES};
static __constant__ uint32_t c_iq3s_grid[512] = {CW_IQ3S_GRID_VALUES};
static __constant__ uint32_t c_iq3xxs_grid[256] = {CW_IQ3XXS_GRID_VALUES};
// kvalues_iq4nl_f (quantized.metal:4561-4563): the 16 non-linear levels of IQ4_XS
static __constant__ float c_kv_iq4nl[16] = {-127.f, -104.f, -83.f, -65.f, -49.f, -35.f, -22.f, -10.f,
                                            1.f,    13.f,   25.f,  38.f,  53.f,  69.f,  89.f,  113.f};

__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) { uint32_t v; __builtin_memcpy(&v, p, 4); return v; }
__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) { uint16_t v; __builtin_memcpy(&v, p, 2); return v; }
__device__ __forceinline__ uint2 ld_u64(const uint8_t *p) { uint2 v; __builtin_memcpy(&v, p, 8); return v; }
__device__ __forceinline__ uint4 ld_u128(const uint8_t *p) { uint4 v; __builtin_memcpy(&v, p, 16); return v; }

__device__ __forceinline__ float h2f(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)h)); }
__device__ __forceinline__ float ubyte(uint32_t w, int i) { return (float)((w >> (8 * i)) & 0xFFu); }
// x with its sign flipped when bit `bit` of `mask` is set
__device__ __forceinline__ float flip(float x, uint32_t mask, int bit) {
    return __uint_as_float(__float_as_uint(x) ^ (((mask >> bit) & 1u) << 31));
}
// ksigns_iq2xs[i] (quantized.metal:305): 7 sign bits plus a parity bit that makes the count even
__device__ __forceinline__ uint32_t ksign(uint32_t i7) { return i7 | ((__popc(i7) & 1u) << 7); }
// Byte masks of 8 sign bits: 0xFF (m) and 0x01 (b) in each byte whose bit is set. (g ^ m) + b
// negates those bytes of 8 unsigned lattice magnitudes (all >= 1, so no byte carries into the
// next), and the signed bytes convert to float in one instruction each (sign-extending byte
// selects): the dot then takes the same products as with the signs applied to x, one fewer
// instruction per weight.
__device__ __forceinline__ uint64_t sign_bytes(uint32_t s8, uint32_t v) {
    uint64_t m = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) m |= ((s8 >> k) & 1u) ? (uint64_t)v << (8 * k) : 0ull;
    return m;
}
// byte i of w as a signed value
__device__ __forceinline__ float sbyte(uint32_t w, int i) { return (float)(int8_t)(w >> (8 * i)); }
// 8 lattice magnitudes (two dwords) with the signs of mask entry mb (m low, m high, b low, b high)
__device__ __forceinline__ uint2 signed8(uint64_t g, uint4 mb) {
    return make_uint2(((uint32_t)g ^ mb.x) + mb.z, ((uint32_t)(g >> 32) ^ mb.y) + mb.w);
}

// 2^(e-128), with the f32 subnormals for e < 2 (k_quants.rs:642-649)
__device__ __forceinline__ float e8m0_half(uint32_t e) {
    return __uint_as_float(e < 2 ? (0x00200000u << e) : ((e - 1) << 23));
}
__device__ __forceinline__ float kv_mxfp4(uint32_t c) {
    uint32_t m = c & 7u;
    int mag = (int)(m < 4 ? m : ((2u | (m & 1u)) << ((m >> 1) - 1)));  // 4, 6, 8, 12 for 4..7
    // the reference table is i8, so code 8 is +0, not -0
    return (float)((c & 8u) ? -mag : mag);
}

// Sums of the two halves (16 values each) of a lane's 32 activations: computed once per lane and
// passed to the dots of formats with a minimum term (Q4_K, Q2_K), which subtract dmin * m * sum.
__device__ __forceinline__ void half_sums(const float *x, float *xs) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        a += x[i];
        b += x[16 + i];
    }
    xs[0] = a;
    xs[1] = b;
}

// ---------------------------------------------------------------------------------- Q8_0
struct FQ8_0 {
    static constexpr int BS = 32, TS = 34, LDS_BYTES = 0;
    static __device__ __forceinline__ uint64_t table_word(int) { return 0; }
    struct Raw { uint32_t d; uint4 q0, q1; };
    static __device__ __forceinline__ void fill_lds(void *, int, int) {}
    static __device__ __forceinline__ Raw load(const uint8_t *row, int sb) {
        const uint8_t *b = row + TS * sb;
        Raw r;
        r.d = ld_u16(b);
        r.q0 = ld_u128(b + 2);
        r.q1 = ld_u128(b + 18);
        return r;
    }
    static __device__ __forceinline__ int8_t q(const Raw &r, int j) {
        uint32_t w = j < 16 ? (&r.q0.x)[j >> 2] : (&r.q1.x)[(j - 16) >> 2];
        return (int8_t)(w >> (8 * (j & 3)));
    }
    static __device__ __forceinline__ void dequant(const Raw &r, const void *, float *y) {
        float d = h2f(r.d);
#pragma unroll
        for (int j = 0; j < 32; j++) y[j] = (float)q(r, j) * d;
    }
    static __device__ __forceinline__ float dot(const Raw &r, const void *, const float *x) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 32; j++) s = fmaf((float)q(r, j), x[j], s);
        return s * h2f(r.d);
    }
};

// get_scale_min_k4 (quantized/utils.rs:50-60) for sub-block j of a Q4_K / Q5_K super-block whose
// first 16 bytes (d, dmin, the 12 scale bytes) are hd
__device__ __forceinline__ uint32_t k4_sbyte(const uint4 &hd, int i) { return ((&hd.x)[1 + (i >> 2)] >> (8 * (i & 3))) & 0xFF; }
__device__ __forceinline__ void k4_sc_mn(const uint4 &hd, int j, uint32_t &sc, uint32_t &mn) {
    if (j < 4) {
        sc = k4_sbyte(hd, j) & 63;
        mn = k4_sbyte(hd, j + 4) & 63;
    } else {
        sc = (k4_sbyte(hd, j + 4) & 0xF) | ((k4_sbyte(hd, j - 4) >> 6) << 4);
        mn = (k4_sbyte(hd, j + 4) >> 4) | ((k4_sbyte(hd, j) >> 6) << 4);
    }
}

// ---------------------------------------------------------------------------------- Q4_K
struct FQ4_K {
    static constexpr int BS = 256, TS = 144, LDS_BYTES = 0;
    static __device__ __forceinline__ uint64_t table_word(int) { return 0; }
    // hd: d, dmin and the 12 scale bytes (the super-block's first 16 bytes, one load); sub-blocks
    // 2c and 2c+1 share the 32 bytes qs[32c..32c+32) (low and high nibbles). The 6-bit scale and
    // min are unpacked where they are used, so that load() only issues loads.
    struct Raw { uint4 hd; uint4 q0, q1; int j; };
    static __device__ __forceinline__ void fill_lds(void *, int, int) {}
    static __device__ __forceinline__ Raw load(const uint8_t *row, int sb) {
        const uint8_t *b = row + TS * (sb >> 3);
        const int j = sb & 7;
        Raw r;
        r.hd = ld_u128(b);
        const uint8_t *qs = b + 16 + 32 * (j >> 1);
        r.q0 = ld_u128(qs);
        r.q1 = ld_u128(qs + 16);
        r.j = j;
        return r;
    }
    static __device__ __forceinline__ void sc_mn(const Raw &r, uint32_t &sc, uint32_t &mn) { k4_sc_mn(r.hd, r.j, sc, mn); }
    static __device__ __forceinline__ uint32_t nib(const Raw &r, int l) {
        uint32_t w = l < 16 ? (&r.q0.x)[l >> 2] : (&r.q1.x)[(l - 16) >> 2];
        return (w >> (8 * (l & 3) + 4 * (r.j & 1))) & 0xFu;
    }
    static __device__ __forceinline__ void dequant(const Raw &r, const void *, float *y) {
        // y = (d*sc)*q - dmin*m: both products exact, one rounding (k_quants.rs:1834-1843)
        uint32_t sc, mn;
        sc_mn(r, sc, mn);
        float d1 = h2f(r.hd.x & 0xFFFF) * (float)sc, m1 = h2f(r.hd.x >> 16) * (float)mn;
#pragma unroll
        for (int l = 0; l < 32; l++) y[l] = d1 * (float)nib(r, l) - m1;
    }
    // sum of q * x: the 32 nibbles masked to bytes 4 at a time, each byte converted to f32 directly
    static __device__ __forceinline__ float qdot(const Raw &r, const float *x) {
        const uint32_t sh = 4 * (r.j & 1);
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t w = ((k < 4 ? (&r.q0.x)[k] : (&r.q1.x)[k - 4]) >> sh) & 0x0F0F0F0Fu;
#pragma unroll
            for (int i = 0; i < 4; i++) s = fmaf(ubyte(w, i), x[4 * k + i], s);
        }
        return s;
    }
    static constexpr bool HAS_MIN = true;
    // xs: the half sums of x (half_sums)
    static __device__ __forceinline__ float dot_s(const Raw &r, const void *, const float *x, const float *xs) {
        uint32_t sc, mn;
        sc_mn(r, sc, mn);
        return h2f(r.hd.x & 0xFFFF) * (float)sc * qdot(r, x) - h2f(r.hd.x >> 16) * (float)mn * (xs[0] + xs[1]);
    }
    static __device__ __forceinline__ float dot(const Raw &r, const void *lds, const float *x) {
        float xs[2];
        half_sums(x, xs);
        return dot_s(r, lds, x, xs);
    }
};

// ---------------------------------------------------------------------------------- Q2_K
// {scales[16], qs[64], d, dmin} (k_quants.rs:1152-1190; what the shrink writes): sub-block j is
// the 32 bytes qs[32(j/4) ..) at bit 2(j%4), its two halves of 16 weights scaled by scales[2j]
// and scales[2j+1] (low nibble: scale, high nibble: min).
struct FQ2_K {
    static constexpr int BS = 256, TS = 84, LDS_BYTES = 0;
    static __device__ __forceinline__ uint64_t table_word(int) { return 0; }
    struct Raw { uint32_t dd; uint32_t sc; uint4 q0, q1; int sh; };
    static __device__ __forceinline__ void fill_lds(void *, int, int) {}
    static __device__ __forceinline__ Raw load(const uint8_t *row, int sb) {
        const uint8_t *b = row + TS * (sb >> 3);
        const int j = sb & 7;
        Raw r;
        r.dd = ld_u32(b + 80);     // d | dmin << 16
        r.sc = ld_u16(b + 2 * j);  // scales[2j] | scales[2j+1] << 8
        const uint8_t *qs = b + 16 + 32 * (j >> 2);
        r.q0 = ld_u128(qs);
        r.q1 = ld_u128(qs + 16);
        r.sh = 2 * (j & 3);
        return r;
    }
    static __device__ __forceinline__ uint32_t q(const Raw &r, int l) {
        uint32_t w = l < 16 ? (&r.q0.x)[l >> 2] : (&r.q1.x)[(l - 16) >> 2];
        return (w >> (8 * (l & 3) + r.sh)) & 3u;
    }
    static __device__ __forceinline__ void dequant(const Raw &r, const void *, float *y) {
        // y = (d*sc)*q - dmin*m: both products exact, one rounding (k_quants.rs:1171-1185)
        const float d = h2f(r.dd & 0xFFFF), mn = h2f(r.dd >> 16);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t s = (r.sc >> (8 * h)) & 0xFFu;
            const float dl = d * (float)(s & 0xF), ml = mn * (float)(s >> 4);
#pragma unroll
            for (int l = 0; l < 16; l++) y[16 * h + l] = dl * (float)q(r, 16 * h + l) - ml;
        }
    }
    static constexpr bool HAS_MIN = true;
    // xs: the half sums of x (half_sums); the 2-bit fields masked to bytes 4 at a time
    static __device__ __forceinline__ float dot_s(const Raw &r, const void *, const float *x, const float *xs) {
        const float d = h2f(r.dd & 0xFFFF), mn = h2f(r.dd >> 16);
        float t = 0.f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t s = (r.sc >> (8 * h)) & 0xFFu;
            float sq = 0.f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t w = ((h == 0 ? (&r.q0.x)[k] : (&r.q1.x)[k]) >> r.sh) & 0x03030303u;
#pragma unroll
                for (int i = 0; i < 4; i++) sq = fmaf(ubyte(w, i), x[16 * h + 4 * k + i], sq);
            }
            t += d * (float)(s & 0xF) * sq - mn * (float)(s >> 4) * xs[h];
        }
        return t;
    }
    static __device__ __forceinline__ float dot(const Raw &r, const void *lds, const float *x) {
        float xs[2];
        half_sums(x, xs);
        return dot_s(r, lds, x, xs);
    }
};

// ---------------------------------------------------------------------------------- Q5_K
// {d, dmin, scales[12], qh[32], qs[128]} (k_quants.rs:2120-2152): sub-block j is the low (j even)
// or high (j odd) nibbles of qs[32(j/2) ..) plus 16 times bit j of qh[l], scaled as Q4_K:
// y = (d*sc)*q - dmin*m, the product exact (q < 32), one rounding.
struct FQ5_K {
    static constexpr int BS = 256, TS = 176, LDS_BYTES = 0;
    static __device__ __forceinline__ uint64_t table_word(int) { return 0; }
    struct Raw { uint4 hd; uint4 q0, q1; uint4 h0, h1; int j; };
    static __device__ __forceinline__ void fill_lds(void *, int, int) {}
    static __device__ __forceinline__ Raw load(const uint8_t *row, int sb) {
        const uint8_t *b = row + TS * (sb >> 3);
        const int j = sb & 7;
        Raw r;
        r.hd = ld_u128(b);
        r.h0 = ld_u128(b + 16);
        r.h1 = ld_u128(b + 32);
        const uint8_t *qs = b + 48 + 32 * (j >> 1);
        r.q0 = ld_u128(qs);
        r.q1 = ld_u128(qs + 16);
        r.j = j;
        return r;
    }
    // the 5-bit codes of weights 4k..4k+3 as bytes
    static __device__ __forceinline__ uint32_t codes4(const Raw &r, int k) {
        const uint32_t w = k < 4 ? (&r.q0.x)[k] : (&r.q1.x)[k - 4];
        const uint32_t h = k < 4 ? (&r.h0.x)[k] : (&r.h1.x)[k - 4];
        return ((w >> (4 * (r.j & 1))) & 0x0F0F0F0Fu) | (((h >> r.j) & 0x01010101u) << 4);
    }
    static __device__ __forceinline__ void dequant(const Raw &r, const void *, float *y) {
        uint32_t sc, mn;
        k4_sc_mn(r.hd, r.j, sc, mn);
        const float d1 = h2f(r.hd.x & 0xFFFF) * (float)sc, m1 = h2f(r.hd.x >> 16) * (float)mn;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t c = codes4(r, k);
#pragma unroll
            for (int i = 0; i < 4; i++) y[4 * k + i] = d1 * ubyte(c, i) - m1;
        }
    }
    static constexpr bool HAS_MIN = true;
    static __device__ __forceinline__ float dot_s(const Raw &r, const void *, const float *x, const float *xs) {
        uint32_t sc, mn;
        k4_sc_mn(r.hd, r.j, sc, mn);
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t c = codes4(r, k);
#pragma unroll
            for (int i = 0; i < 4; i++) s = fmaf(ubyte(c, i), x[4 * k + i], s);
        }
        return h2f(r.hd.x & 0xFFFF) * (float)sc * s - h2f(r.hd.x >> 16) * (float)mn * (xs[0] + xs[1]);
    }
    static __device__ __forceinline__ float dot(const Raw &r, const void *lds, const float *x) {
        float xs[2];
        half_sums(x, xs);
        return dot_s(r, lds, x, xs);
    }
};

// ---------------------------------------------------------------------------------- Q6_K
// {ql[128], qh[64], scales[16] (i8), d} (k_quants.rs:2420-2451): sub-block j = 4h + r (half h,
// quadrant r) is the low (r < 2) or high nibbles of ql[64h + 32(r&1) ..) plus 16 times bits
// 2r, 2r+1 of qh[32h + l], minus 32; its halves of 16 are scaled by d * scales[8h + 2r (+1)].
// y = (d*sc)*(q-32) is exact in f32.
struct FQ6_K {
    static constexpr int BS = 256, TS = 210, LDS_BYTES = 0;
    static __device__ __forceinline__ uint64_t table_word(int) { return 0; }
    struct Raw { uint4 q0, q1; uint4 h0, h1; uint32_t sc; uint32_t d; int r; };
    static __device__ __forceinline__ void fill_lds(void *, int, int) {}
    static __device__ __forceinline__ Raw load(const uint8_t *row, int sb) {
        const uint8_t *b = row + TS * (sb >> 3);
        const int j = sb & 7, h = j >> 2, q = j & 3;
        Raw r;
        const uint8_t *ql = b + 64 * h + 32 * (q & 1), *qh = b + 128 + 32 * h;
        r.q0 = ld_u128(ql);
        r.q1 = ld_u128(ql + 16);
        r.h0 = ld_u128(qh);
        r.h1 = ld_u128(qh + 16);
        r.sc = ld_u16(b + 192 + 8 * h + 2 * q);  // the scales of the two halves
        r.d = ld_u16(b + 208);
        r.r = q;
        return r;
    }
    // the 6-bit codes (before the -32) of weights 4k..4k+3 as bytes
    static __device__ __forceinline__ uint32_t codes4(const Raw &r, int k) {
        const uint32_t w = k < 4 ? (&r.q0.x)[k] : (&r.q1.x)[k - 4];
        const uint32_t h = k < 4 ? (&r.h0.x)[k] : (&r.h1.x)[k - 4];
        return ((w >> (4 * (r.r >> 1))) & 0x0F0F0F0Fu) | (((h >> (2 * r.r)) & 0x03030303u) << 4);
    }
    static __device__ __forceinline__ float scale(const Raw &r, int half) { return (float)(int8_t)(r.sc >> (8 * half)); }
    static __device__ __forceinline__ void dequant(const Raw &r, const void *, float *y) {
        const float d = h2f(r.d);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t c = codes4(r, k);
            const float ds = d * scale(r, k >> 2);
#pragma unroll
            for (int i = 0; i < 4; i++) y[4 * k + i] = ds * (float)((int)((c >> (8 * i)) & 0xFF) - 32);
        }
    }
    static constexpr bool HAS_MIN = true;
    // sum over each half of code * x, less 32 times the half's sum of x
    static __device__ __forceinline__ float dot_s(const Raw &r, const void *, const float *x, const float *xs) {
        float s[2] = {0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t c = codes4(r, k);
#pragma unroll
            for (int i = 0; i < 4; i++) s[k >> 2] = fmaf(ubyte(c, i), x[4 * k + i], s[k >> 2]);
        }
        return h2f(r.d) * (scale(r, 0) * (s[0] - 32.f * xs[0]) + scale(r, 1) * (s[1] - 32.f * xs[1]));
    }
    static __device__ __forceinline__ float dot(const Raw &r, const void *lds, const float *x) {
        float xs[2];
        half_sums(x, xs);
        return dot_s(r, lds, x, xs);
    }
};

// ---------------------------------------------------------------------------------- MXFP4
struct FMXFP4 {
    static constexpr int BS = 32, TS = 17, LDS_BYTES = 0;
    static __device__ __forceinline__ uint64_t table_word(int) { return 0; }
    struct Raw { uint32_t e; uint4 q; };
    static __device__ __forceinline__ void fill_lds(void *, int, int) {}
    static __device__ __forceinline__ Raw load(const uint8_t *row, int sb) {
        const uint8_t *b = row + TS * sb;
        Raw r;
        r.e = b[0];
        r.q = ld_u128(b + 1);
        return r;
    }
    // The doubled E2M1 values of byte j's two codes (low nibble first) by gfx950's scaled FP4
    // conversion (v_cvt_scalef32_pk_f32_fp4) with scale 2: exact, one instruction for two weights.
    // Code 8 gives -0 where the reference's i8 table has +0: dequant adds +0 to turn it into +0;
    // in dot it cannot show (the sum starts at +0, so no fma of a -0 product leaves a -0).
    static __device__ __forceinline__ float2 kv2(const Raw &r, int j) {
        const uint32_t w = (&r.q.x)[j >> 2];
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        f32x2 v;
        switch (j & 3) {
        case 0: v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 2.0f, 0); break;
        case 1: v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 2.0f, 1); break;
        case 2: v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 2.0f, 2); break;
        default: v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 2.0f, 3); break;
        }
        return make_float2(v.x, v.y);
    }
    static __device__ __forceinline__ void dequant(const Raw &r, const void *, float *y) {
        float d = e8m0_half(r.e);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const float2 v = kv2(r, j);
            y[j] = (v.x + 0.0f) * d;
            y[j + 16] = (v.y + 0.0f) * d;
        }
    }
    static __device__ __forceinline__ float dot(const Raw &r, const void *, const float *x) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const float2 v = kv2(r, j);
            s = fmaf(v.x, x[j], s);
            s = fmaf(v.y, x[j + 16], s);
        }
        return s * e8m0_half(r.e);
    }
};

// ---------------------------------------------------------------------------------- IQ2_XXS
struct FIQ2_XXS {
    // LDS: the 256-entry lattice, then for each 7-bit sign index its byte masks (sign_bytes of
    // ksign: m, then b)
    static constexpr int BS = 256, TS = 66, LDS_BYTES = 256 * 8 + 128 * 16;
    static __device__ __forceinline__ uint64_t table_word(int i) {
        if (i < 256) return c_iq2xxs_grid[i];
        const int e = (i - 256) >> 1;
        return sign_bytes(ksign((uint32_t)e), (i & 1) ? 0x01u : 0xFFu);
    }
    struct Raw { uint32_t d; uint32_t g; uint32_t s; };
    static __device__ __forceinline__ void fill_lds(void *lds, int tid, int nt) {
        uint64_t *t = (uint64_t *)lds;
        for (int i = tid; i < LDS_BYTES / 8; i += nt) t[i] = table_word(i);
    }
    static __device__ __forceinline__ Raw load(const uint8_t *row, int sb) {
        const uint8_t *b = row + TS * (sb >> 3);
        Raw r;
        r.d = ld_u16(b);
        uint2 v = ld_u64(b + 2 + 8 * (sb & 7));
        r.g = v.x;  // four grid indices (bytes)
        r.s = v.y;  // four 7-bit sign indices and the 4-bit scale in the top nibble
        return r;
    }
    static __device__ __forceinline__ void dequant(const Raw &r, const void *lds, float *y) {
        const uint64_t *grid = (const uint64_t *)lds;
        float dl = h2f(r.d) * (0.5f + (float)(r.s >> 28)) * 0.25f;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            uint64_t g = grid[(r.g >> (8 * l)) & 0xFF];
            uint32_t sg = ksign((r.s >> (7 * l)) & 127);
            uint32_t lo = (uint32_t)g, hi = (uint32_t)(g >> 32);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float gv = i < 4 ? ubyte(lo, i) : ubyte(hi, i - 4);
                y[8 * l + i] = dl * gv * ((sg >> i) & 1 ? -1.f : 1.f);
            }
        }
    }
    static __device__ __forceinline__ float dot(const Raw &r, const void *lds, const float *x) {
        const uint64_t *grid = (const uint64_t *)lds;
        const uint4 *masks = (const uint4 *)((const uint8_t *)lds + 256 * 8);
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint2 w = signed8(grid[(r.g >> (8 * l)) & 0xFF], masks[(r.s >> (7 * l)) & 127]);
#pragma unroll
            for (int i = 0; i < 8; i++) s = fmaf(i < 4 ? sbyte(w.x, i) : sbyte(w.y, i - 4), x[8 * l + i], s);
        }
        return s * (h2f(r.d) * (0.5f + (float)(r.s >> 28)) * 0.25f);
    }
};

// ---------------------------------------------------------------------------------- IQ2_S
struct FIQ2_S {
    // LDS: the 1024-entry lattice, then for each sign byte its byte masks (sign_bytes: m, then b)
    static constexpr int BS = 256, TS = 82, LDS_BYTES = 1024 * 8 + 256 * 16;
    static __device__ __forceinline__ uint64_t table_word(int i) {
        if (i < 1024) return c_iq2s_grid[i];
        const int e = (i - 1024) >> 1;
        return sign_bytes((uint32_t)e, (i & 1) ? 0x01u : 0xFFu);
    }
    struct Raw { uint32_t d; uint32_t qs; uint32_t sg; uint32_t qh; uint32_t sc; };
    static __device__ __forceinline__ void fill_lds(void *lds, int tid, int nt) {
        uint64_t *t = (uint64_t *)lds;
        for (int i = tid; i < LDS_BYTES / 8; i += nt) t[i] = table_word(i);
    }
    static __device__ __forceinline__ Raw load(const uint8_t *row, int sb) {
        const uint8_t *b = row + TS * (sb >> 3);
        const int ib = sb & 7;
        Raw r;
        r.d = ld_u16(b);
        r.qs = ld_u32(b + 2 + 4 * ib);        // low 8 bits of the four grid indices
        r.sg = ld_u32(b + 2 + 32 + 4 * ib);   // one sign byte per 8 weights
        r.qh = b[66 + ib];                    // 2 high index bits per group
        r.sc = b[74 + ib];                    // two 4-bit scales, one per 16 weights
        return r;
    }
    static __device__ __forceinline__ void dequant(const Raw &r, const void *lds, float *y) {
        const uint64_t *grid = (const uint64_t *)lds;
        float d = h2f(r.d);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            float dl = d * (0.5f + (float)((r.sc >> (4 * (t >> 1))) & 0xF)) * 0.25f;
            uint64_t g = grid[((r.qs >> (8 * t)) & 0xFF) | (((r.qh >> (2 * t)) & 3) << 8)];
            uint32_t sg = (r.sg >> (8 * t)) & 0xFF;
            uint32_t lo = (uint32_t)g, hi = (uint32_t)(g >> 32);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float gv = i < 4 ? ubyte(lo, i) : ubyte(hi, i - 4);
                y[8 * t + i] = dl * gv * ((sg >> i) & 1 ? -1.f : 1.f);
            }
        }
    }
    static __device__ __forceinline__ float dot(const Raw &r, const void *lds, const float *x) {
        const uint64_t *grid = (const uint64_t *)lds;
        const uint4 *masks = (const uint4 *)((const uint8_t *)lds + 1024 * 8);
        float s[2] = {0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint2 w = signed8(grid[((r.qs >> (8 * t)) & 0xFF) | (((r.qh >> (2 * t)) & 3) << 8)], masks[(r.sg >> (8 * t)) & 0xFF]);
#pragma unroll
            for (int i = 0; i < 8; i++) s[t >> 1] = fmaf(i < 4 ? sbyte(w.x, i) : sbyte(w.y, i - 4), x[8 * t + i], s[t >> 1]);
        }
        float d = h2f(r.d) * 0.25f;
        return d * ((0.5f + (float)(r.sc & 0xF)) * s[0] + (0.5f + (float)(r.sc >> 4)) * s[1]);
    }
};

// ---------------------------------------------------------------------------------- IQ3_S
struct FIQ3_S {
    static constexpr int BS = 256, TS = 110, LDS_BYTES = 512 * 4;
    static __device__ __forceinline__ uint64_t table_word(int i) {
        return (uint64_t)c_iq3s_grid[2 * i] | ((uint64_t)c_iq3s_grid[2 * i + 1] << 32);
    }
    // sc: the scales byte holding this sub-block's nibble at bit `sh` (unpacked where used, so that
    // load() only issues loads)
    struct Raw { uint32_t d; uint2 qs; uint32_t qh; uint32_t sg; uint32_t sc; uint32_t sh; };
    static __device__ __forceinline__ void fill_lds(void *lds, int tid, int nt) {
        uint32_t *t = (uint32_t *)lds;
        for (int i = tid; i < 512; i += nt) t[i] = c_iq3s_grid[i];
    }
    static __device__ __forceinline__ Raw load(const uint8_t *row, int sb) {
        const uint8_t *b = row + TS * (sb >> 3);
        const int ib = sb & 7;
        Raw r;
        r.d = ld_u16(b);
        r.qs = ld_u64(b + 2 + 8 * ib);            // low 8 bits of eight grid indices
        r.qh = b[66 + ib];                        // their 9th bits
        r.sg = ld_u32(b + 74 + 4 * ib);           // one sign bit per weight
        r.sc = b[106 + (ib >> 1)];
        r.sh = 4 * (ib & 1);
        return r;
    }
    static __device__ __forceinline__ uint32_t gidx(const Raw &r, int g) {
        uint32_t w = g < 4 ? r.qs.x : r.qs.y;
        return ((w >> (8 * (g & 3))) & 0xFF) | (((r.qh >> g) & 1) << 8);
    }
    static __device__ __forceinline__ void dequant(const Raw &r, const void *lds, float *y) {
        const uint32_t *grid = (const uint32_t *)lds;
        float dl = h2f(r.d) * (float)(1 + 2 * (int)((r.sc >> r.sh) & 0xF));
#pragma unroll
        for (int g = 0; g < 8; g++) {
            uint32_t gw = grid[gidx(r, g)];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                int v = 4 * g + i;
                y[v] = dl * ubyte(gw, i) * ((r.sg >> v) & 1 ? -1.f : 1.f);
            }
        }
    }
    static __device__ __forceinline__ float dot(const Raw &r, const void *lds, const float *x) {
        const uint32_t *grid = (const uint32_t *)lds;
        float s = 0.f;
#pragma unroll
        for (int g = 0; g < 8; g++) {
            uint32_t gw = grid[gidx(r, g)];
#pragma unroll
            for (int i = 0; i < 4; i++) s = fmaf(ubyte(gw, i), flip(x[4 * g + i], r.sg, 4 * g + i), s);
        }
        return s * (h2f(r.d) * (float)(1 + 2 * (int)((r.sc >> r.sh) & 0xF)));
    }
};

// ---------------------------------------------------------------------------------- IQ3_XXS
// {d, qs[64] grid indices, then one word per sub-block: four 7-bit sign indices and the 4-bit
// scale s on top} (quantized.metal:6866-6891): weights 8h..8h+7 of sub-block ib take grid entries
// qs[8ib + 2h], qs[8ib + 2h + 1] (4 values each) and the signs of index (word >> 7h) & 127;
// dl = d * (s + 0.5) * 0.5.
struct FIQ3_XXS {
    static constexpr int BS = 256, TS = 98, LDS_BYTES = 256 * 4;
    static __device__ __forceinline__ uint64_t table_word(int i) {
        return (uint64_t)c_iq3xxs_grid[2 * i] | ((uint64_t)c_iq3xxs_grid[2 * i + 1] << 32);
    }
    struct Raw { uint32_t d; uint2 q; uint32_t s; };
    static __device__ __forceinline__ void fill_lds(void *lds, int tid, int nt) {
        uint32_t *t = (uint32_t *)lds;
        for (int i = tid; i < 256; i += nt) t[i] = c_iq3xxs_grid[i];
    }
    static __device__ __forceinline__ Raw load(const uint8_t *row, int sb) {
        const uint8_t *b = row + TS * (sb >> 3);
        const int ib = sb & 7;
        Raw r;
        r.d = ld_u16(b);
        r.q = ld_u64(b + 2 + 8 * ib);
        r.s = ld_u32(b + 66 + 4 * ib);
        return r;
    }
    static __device__ __forceinline__ uint32_t gidx(const Raw &r, int g) { return ((g < 4 ? r.q.x : r.q.y) >> (8 * (g & 3))) & 0xFF; }
    static __device__ __forceinline__ float dl(const Raw &r) { return h2f(r.d) * (0.5f + (float)(r.s >> 28)) * 0.5f; }
    static __device__ __forceinline__ void dequant(const Raw &r, const void *lds, float *y) {
        const uint32_t *grid = (const uint32_t *)lds;
        const float d = dl(r);
#pragma unroll
        for (int h = 0; h < 4; h++) {
            const uint32_t sg = ksign((r.s >> (7 * h)) & 127);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint32_t gw = grid[gidx(r, 2 * h + t)];
#pragma unroll
                for (int i = 0; i < 4; i++) y[8 * h + 4 * t + i] = d * ubyte(gw, i) * ((sg >> (4 * t + i)) & 1 ? -1.f : 1.f);
            }
        }
    }
    static __device__ __forceinline__ float dot(const Raw &r, const void *lds, const float *x) {
        const uint32_t *grid = (const uint32_t *)lds;
        float s = 0.f;
#pragma unroll
        for (int h = 0; h < 4; h++) {
            const uint32_t sg = ksign((r.s >> (7 * h)) & 127);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint32_t gw = grid[gidx(r, 2 * h + t)];
#pragma unroll
                for (int i = 0; i < 4; i++) s = fmaf(ubyte(gw, i), flip(x[8 * h + 4 * t + i], sg, 4 * t + i), s);
            }
        }
        return s * dl(r);
    }
};

// ---------------------------------------------------------------------------------- IQ4_XS
// {d, scales_h (u16), scales_l[4], qs[128]} (quantized.metal:7000-7016): sub-block ib has the
// 6-bit scale ls (a scales_l nibble, 2 bits of scales_h on top), d_ib = d * (ls - 32), and its 32
// weights are the levels kvalues[nibble] of the low, then the high nibbles of qs[16ib ..). The
// 16 levels sit in LDS.
struct FIQ4_XS {
    static constexpr int BS = 256, TS = 136, LDS_BYTES = 16 * 4;
    static __device__ __forceinline__ uint64_t table_word(int i) {
        return (uint64_t)__float_as_uint(c_kv_iq4nl[2 * i]) | ((uint64_t)__float_as_uint(c_kv_iq4nl[2 * i + 1]) << 32);
    }
    struct Raw { uint2 hd; uint4 q; int ib; };
    static __device__ __forceinline__ void fill_lds(void *lds, int tid, int nt) {
        float *t = (float *)lds;
        for (int i = tid; i < 16; i += nt) t[i] = c_kv_iq4nl[i];
    }
    static __device__ __forceinline__ Raw load(const uint8_t *row, int sb) {
        const uint8_t *b = row + TS * (sb >> 3);
        Raw r;
        r.hd = ld_u64(b);  // d | scales_h << 16, scales_l[4]
        r.ib = sb & 7;
        r.q = ld_u128(b + 8 + 16 * r.ib);
        return r;
    }
    static __device__ __forceinline__ float dib(const Raw &r) {
        const uint32_t ls = ((r.hd.y >> (4 * r.ib)) & 0xF) | (((r.hd.x >> (16 + 2 * r.ib)) & 3) << 4);
        return h2f(r.hd.x & 0xFFFF) * (float)((int)ls - 32);
    }
    static __device__ __forceinline__ void dequant(const Raw &r, const void *lds, float *y) {
        const float *kv = (const float *)lds;
        const float d = dib(r);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t b = ((&r.q.x)[j >> 2] >> (8 * (j & 3))) & 0xFF;
            y[j] = d * kv[b & 0xF];
            y[16 + j] = d * kv[b >> 4];
        }
    }
    static __device__ __forceinline__ float dot(const Raw &r, const void *lds, const float *x) {
        const float *kv = (const float *)lds;
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t b = ((&r.q.x)[j >> 2] >> (8 * (j & 3))) & 0xFF;
            s = fmaf(kv[b & 0xF], x[j], s);
            s = fmaf(kv[b >> 4], x[16 + j], s);
        }
        return s * dib(r);
    }
};

// A block's share of a format's LDS table, held in registers between the global loads and the
// LDS stores, so the loads can be issued early and waited for late.
template <class F>
struct TableRegs {
    static constexpr int WORDS = F::LDS_BYTES / 8;
    static constexpr int PER = WORDS > 0 ? (WORDS + 255) / 256 : 1;
    uint64_t r[PER];
    __device__ __forceinline__ void load(int tid) {
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int i = tid + 256 * q;
            if constexpr (WORDS > 0) r[q] = F::table_word(i < WORDS ? i : WORDS - 1);  // clamped, not branched
        }
    }
    __device__ __forceinline__ void store(void *lds, int tid) const {
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int i = tid + 256 * q;
            if (i < WORDS) ((uint64_t *)lds)[i] = r[q];
        }
    }
};

// a format's dot with the lane's half sums of x precomputed (used only by formats with a minimum term)
template <class F, class = void>
struct HasMin { static constexpr bool value = false; };
template <class F>
struct HasMin<F, decltype((void)F::HAS_MIN)> { static constexpr bool value = F::HAS_MIN; };
template <class F>
__device__ __forceinline__ float dot_xs(const typename F::Raw &r, const void *lds, const float *x, const float *xs) {
    if constexpr (HasMin<F>::value) return F::dot_s(r, lds, x, xs);
    else return F::dot(r, lds, x);
}

}  // namespace cw
