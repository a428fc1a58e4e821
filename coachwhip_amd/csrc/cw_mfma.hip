// Grouped expert GEMMs on MFMA (gfx950, v_mfma_f32_16x16x32_f16) for the MoE layer's prefill.
//
// Picks are grouped by the slot they read (mfma_piles); a tile is up to MF_MT = 80 picks of one
// slot (5 MFMA blocks of 16) by RPB weight rows per matrix. A block has 16 waves for gate/up
// (8 on gate, 8 on up) and 8 for down and dense matmuls; each wave owns 16 weight rows and every
// pick block of the tile.
//
// Exactness: a weight is (f16 super-block scale) x (small integer code). The codes go through
// MFMA as fp16 integers, which they represent exactly: IQ2_XXS / IQ2_S codes (2s+1)*grid*sign
// are at most 31*43 = 1333, IQ3_XXS codes 8*(2s+1)*grid*sign multiples of 8 up to 8*31*62, IQ3_S
// codes (1+2s)*grid*sign at most 31*15 = 465, MXFP4 codes the doubled E2M1 values up to 12,
// IQ4_XS codes the non-linear levels (|v| <= 127, scaled per K-step like Q8_0). Products with fp16 activations are exact in the f32
// accumulators; the f32 scale of each super-block (d/8, d, or MXFP4's 2^(e-128) per 32) is
// applied to the partial sum of its K-steps. Activations are rounded to fp16 once, with a
// power-of-two scale per row (exact) so that no row overflows: that rounding (2^-11 relative)
// is the only approximation.
#include <atomic>
#include <type_traits>

#include "cw_common.h"
#include "cw_device.h"
#include "cw_mfma.h"
#include "cw_wave.h"

namespace cw {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pk_mul_u(uint32_t v, uint32_t sc2) {
    f16x2 a = __builtin_bit_cast(f16x2, v), b = __builtin_bit_cast(f16x2, sc2);
    return __builtin_bit_cast(uint32_t, a * b);
}
__device__ __forceinline__ uint4 scale4(uint4 v, uint32_t sc2) {
    return make_uint4(pk_mul_u(v.x, sc2), pk_mul_u(v.y, sc2), pk_mul_u(v.z, sc2), pk_mul_u(v.w, sc2));
}
// Signs of 8 fp16 codes (dword i holds weights 2i, 2i+1; sign bits clear): bit j of b negates
// weight j. With y = b | b << 15, y << (15 - 2i) has bit 2i of b at bit 15 and bit 2i+1 at bit
// 31; a bit-field insert takes exactly those two bits (bits 8 and up of b never reach them).
__device__ __forceinline__ uint32_t bfi_sign(uint32_t s, uint32_t g) { return (s & 0x80008000u) | (g & 0x7FFF7FFFu); }
__device__ __forceinline__ uint4 apply_signs(uint4 g, uint32_t b) {
    // an opaque b keeps the shifts as shifts: with b known to be small the compiler turns
    // (b | b << 15) << c into one quarter-rate 32-bit multiply per dword
    asm("" : "+v"(b));
    const uint32_t y = b | (b << 15);
    return make_uint4(bfi_sign(y << 15, g.x), bfi_sign(y << 13, g.y), bfi_sign(y << 11, g.z), bfi_sign(y << 9, g.w));
}
// fp16 pair of a small integer multiplier (exact below 2048)
__device__ __forceinline__ uint32_t splat_mult(uint32_t v) {
    const float m = (float)v;
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(m, m));
}

// ------------------------------------------------------------------------------ code tables
// Lattice entries as fp16 integers, built at compile time; a kernel copies the one its format
// needs into LDS. Signs are applied arithmetically (apply_signs), not through a table: a random
// 16-byte LDS lookup costs about as much LDS time as two conflict-free ones.
struct U4 { uint32_t x, y, z, w; };
template <int N> struct Tab { U4 v[N]; };

constexpr uint32_t f16_int(uint32_t v) {  // fp16 bits of a small non-negative integer (< 2048)
    if (v == 0) return 0;
    int e = 0;
    for (uint32_t t = v; t >= 2; t >>= 1) e++;
    return (uint32_t)((e + 15) << 10) | ((v << (10 - e)) & 0x3FFu);
}
constexpr U4 pack8(uint64_t bytes) {
    uint32_t h[8] = {};
    for (int b = 0; b < 8; b++) h[b] = f16_int((uint32_t)(bytes >> (8 * b)) & 0xFF);
    return U4{h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16};
}
constexpr Tab<256> make_iq2xxs_f16() {
    constexpr uint64_t g[256] = {CW_IQ2XXS_GRID_VALUES};
    Tab<256> t{};
    for (int i = 0; i < 256; i++) t.v[i] = pack8(g[i]);
    return t;
}
constexpr Tab<1024> make_iq2s_f16() {
    constexpr uint64_t g[1024] = {CW_IQ2S_GRID_VALUES};
    Tab<1024> t{};
    for (int i = 0; i < 1024; i++) t.v[i] = pack8(g[i]);
    return t;
}
constexpr Tab<256> make_iq3s_f16() {  // two 4-value entries per U4: entry 2i in x,y and 2i+1 in z,w
    constexpr uint32_t g[512] = {CW_IQ3S_GRID_VALUES};
    Tab<256> t{};
    for (int i = 0; i < 256; i++) {
        const U4 a = pack8((uint64_t)g[2 * i] | ((uint64_t)g[2 * i + 1] << 32));
        t.v[i] = a;
    }
    return t;
}
constexpr Tab<128> make_iq3xxs_f16() {  // two 4-value entries per U4: entry 2i in x,y and 2i+1 in z,w
    constexpr uint32_t g[256] = {CW_IQ3XXS_GRID_VALUES};
    Tab<128> t{};
    for (int i = 0; i < 128; i++) t.v[i] = pack8((uint64_t)g[2 * i] | ((uint64_t)g[2 * i + 1] << 32));
    return t;
}
static __constant__ Tab<256> c_iq2xxs_f16 = make_iq2xxs_f16();
static __constant__ Tab<1024> c_iq2s_f16 = make_iq2s_f16();
static __constant__ Tab<256> c_iq3s_f16 = make_iq3s_f16();
static __constant__ Tab<128> c_iq3xxs_f16 = make_iq3xxs_f16();

template <int N>
__device__ __forceinline__ void copy_tab(uint8_t *lds, const Tab<N> &t, int tid, int nt) {
    uint4 *d = (uint4 *)lds;
    const uint4 *src = (const uint4 *)&t;
    for (int i = tid; i < N; i += nt) d[i] = src[i];
}

// ------------------------------------------------------------------------------ formats
// Per format: TS bytes per block, SBK weights per scale unit, LDS table bytes, and the decode of
// one K-step (32 weights) of a row from the row's stage window in LDS (the bytes of 8 K-steps:
// one IQ super-block, or 8 MXFP4 blocks): lane group grp takes weights 8*grp..8*grp+7 of the
// step, as 8 fp16 integer codes times a per-lane multiplier.

__device__ __forceinline__ uint32_t lds_u8(const uint8_t *p) { return *p; }
__device__ __forceinline__ uint32_t lds_u16(const uint8_t *p) { uint16_t v; __builtin_memcpy(&v, p, 2); return v; }
__device__ __forceinline__ uint32_t lds_u32(const uint8_t *p) { uint32_t v; __builtin_memcpy(&v, p, 4); return v; }
// 8 bytes at any LDS address: three aligned dwords and a byte shift (a misaligned ds_read_b64
// measured ~2x slower for the whole stage)
__device__ __forceinline__ uint2 lds_u64(const uint8_t *p) {
    const uint32_t a = (uint32_t)(uintptr_t)p & 3;
    const uint32_t *q = (const uint32_t *)(p - a);
    const uint32_t d0 = q[0], d1 = q[1], d2 = q[2];
    return make_uint2(__builtin_amdgcn_alignbyte(d1, d0, a), __builtin_amdgcn_alignbyte(d2, d1, a));
}

// A row's stage window in LDS, with the dword address and byte shift of its 8-byte reads
// (which start ORG bytes into the window) worked out once per stage instead of per read
struct WinRef {
    const uint8_t *p;     // the window: the row's bytes of this stage
    const uint32_t *qa;   // p + ORG rounded down to a dword
    uint32_t sh;          // (p + ORG) & 3
    template <int ORG>
    static __device__ __forceinline__ WinRef at(const uint8_t *p) {
        const uint32_t o = (uint32_t)(uintptr_t)(p + ORG);
        return WinRef{p, (const uint32_t *)(p + ORG - (o & 3)), o & 3};
    }
    // 8 bytes at p + ORG + off, off a multiple of 4 (the shift stays sh)
    __device__ __forceinline__ uint2 u64(int off) const {
        const uint32_t *q = qa + off / 4;
        const uint32_t d0 = q[0], d1 = q[1], d2 = q[2];
        return make_uint2(__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh));
    }
    // 4 bytes at p + ORG + off, off a multiple of 4
    __device__ __forceinline__ uint32_t u32(int off) const {
        const uint32_t *q = qa + off / 4;
        return __builtin_amdgcn_alignbyte(q[1], q[0], sh);
    }
    // 4 bytes at p + ORG + off, any off
    __device__ __forceinline__ uint32_t u32x(int off) const {
        const uint32_t t = sh + (uint32_t)off;
        const uint32_t *q = qa + (t >> 2);
        return __builtin_amdgcn_alignbyte(q[1], q[0], t & 3);
    }
    // 8 bytes at p + ORG + off, any off
    __device__ __forceinline__ uint2 u64x(int off) const {
        const uint32_t t = sh + (uint32_t)off, a = t & 3;
        const uint32_t *q = qa + (t >> 2);
        const uint32_t d0 = q[0], d1 = q[1], d2 = q[2];
        return make_uint2(__builtin_amdgcn_alignbyte(d1, d0, a), __builtin_amdgcn_alignbyte(d2, d1, a));
    }
};

// Traits common to the formats: KST K-steps per stage; SCALE 0 = one f16 scale per super-block
// (read by scale()), 1 = MXFP4's power-of-two block scales, 2 = one f16 scale per 32-weight block
// (read by step_scale()).
struct MIQ2_XXS {
    static constexpr int TS = 66, SBK = 256, LDS = 256 * 16;
    static constexpr int KST = 8, SCALE = 0, ORG = 2;
    static __device__ void fill(uint8_t *lds, int tid, int nt) { copy_tab(lds, c_iq2xxs_f16, tid, nt); }
    struct Stage {
        __device__ __forceinline__ void load(const WinRef &, int) {}
    };
    // A fragment is the grid entry (one lookup) with the signs applied arithmetically: the 7 sign
    // bits of the lane's 8 weights plus their even parity as the 8th (ksigns_iq2xs), and the
    // multiplier 8*(2s+1) as one packed multiply, exact in fp16 with the grid values (at most
    // 43*248 = 1333*8); scale() takes the 8 back out. zero: the super-block scale is 0, so the
    // codes must not contribute (multiplier 0).
    struct Raw { uint2 q; };
    struct Look { uint4 g; };
    static __device__ __forceinline__ Raw raw(const WinRef &w, const Stage &, int kk, int) { return Raw{w.u64(8 * kk)}; }
    static __device__ __forceinline__ Look look(const Raw &r, const Stage &, int, int grp, const uint8_t *lds, bool) {
        return Look{((const uint4 *)lds)[(r.q.x >> (8 * grp)) & 0xFF]};
    }
    static __device__ __forceinline__ uint4 make(const Raw &r, const Look &l, const Stage &, int, int grp, bool zero) {
        const uint32_t s7 = (r.q.y >> (7 * grp)) & 127;
        const uint32_t b = s7 | ((__builtin_popcount(s7) & 1u) << 7);
        return scale4(apply_signs(l.g, b), splat_mult(zero ? 0u : ((r.q.y >> 28) << 4) | 8));
    }
    static __device__ __forceinline__ float scale(const uint8_t *win) { return h2f(lds_u16(win)) * (0.125f / 8); }
};

struct MIQ2_S {
    static constexpr int TS = 82, SBK = 256, LDS = 1024 * 16;
    static constexpr int KST = 8, SCALE = 0, ORG = 66;
    static __device__ void fill(uint8_t *lds, int tid, int nt) { copy_tab(lds, c_iq2s_f16, tid, nt); }
    // The lane's bits of qh[8] and scales[8] (bytes 66..81), read once per stage: qh bits 2grp,
    // 2grp+1 of byte kk at bits 8(kk&3) + 2(kk>>2) of qh; the scale nibble of byte kk for this
    // lane's half at bits 8(kk&3) + 4(kk>>2) of sc.
    struct Stage {
        uint32_t qh, sc;
        __device__ __forceinline__ void load(const WinRef &w, int grp) {
            const uint2 h = w.u64(0), c = w.u64(8);
            const int hs = 2 * grp, cs = 4 * (grp >> 1);
            qh = ((h.x >> hs) & 0x03030303u) | (((h.y >> hs) & 0x03030303u) << 2);
            sc = ((c.x >> cs) & 0x0F0F0F0Fu) | (((c.y >> cs) & 0x0F0F0F0Fu) << 4);
        }
    };
    // multiplier 8*(2s+1) for the 4-bit scale s, as (s << 4) | 8; scale() takes the 8 back out
    struct Raw { uint32_t qs, sgn; };
    struct Look { uint4 g; };
    static __device__ __forceinline__ Raw raw(const WinRef &w, const Stage &, int kk, int grp) {
        return Raw{lds_u8(w.p + 2 + 4 * kk + grp), lds_u8(w.p + 34 + 4 * kk + grp)};
    }
    static __device__ __forceinline__ Look look(const Raw &r, const Stage &st, int kk, int, const uint8_t *lds, bool) {
        const uint32_t qh = (st.qh >> (8 * (kk & 3) + 2 * (kk >> 2))) & 3;
        return Look{((const uint4 *)lds)[r.qs | (qh << 8)]};
    }
    static __device__ __forceinline__ uint4 make(const Raw &r, const Look &l, const Stage &st, int kk, int, bool zero) {
        const uint32_t s4 = (st.sc >> (8 * (kk & 3) + 4 * (kk >> 2))) & 0xF;
        return scale4(apply_signs(l.g, r.sgn), splat_mult(zero ? 0u : (s4 << 4) | 8));
    }
    static __device__ __forceinline__ float scale(const uint8_t *win) { return h2f(lds_u16(win)) * (0.125f / 8); }
};

struct MIQ3_S {
    static constexpr int TS = 110, SBK = 256, LDS = 512 * 8;
    static constexpr int KST = 8, SCALE = 0, ORG = 66;
    static __device__ void fill(uint8_t *lds, int tid, int nt) { copy_tab(lds, c_iq3s_f16, tid, nt); }  // entry i: 4 halves at byte 8*i
    // The lane's bits of qh[8] (bytes 66..73: bits 2grp, 2grp+1 of byte kk at bits 8(kk&3) +
    // 2(kk>>2)) and scales[4] (bytes 106..109), read once per stage (the read of the scales also
    // takes 4 bytes past the block, which stay unused)
    struct Stage {
        uint32_t qh, sc;
        __device__ __forceinline__ void load(const WinRef &w, int grp) {
            const uint2 h = w.u64(0);
            const int hs = 2 * grp;
            qh = ((h.x >> hs) & 0x03030303u) | (((h.y >> hs) & 0x03030303u) << 2);
            sc = w.u64(40).x;
        }
    };
    // multiplier 8*(2s+1), as (s << 4) | 8; scale() takes the 8 back out
    struct Raw { uint32_t qs, sgn; };
    struct Look { uint2 x, y; };
    static __device__ __forceinline__ Raw raw(const WinRef &w, const Stage &, int kk, int grp) {
        return Raw{lds_u16(w.p + 2 + 8 * kk + 2 * grp), lds_u8(w.p + 74 + 4 * kk + grp)};
    }
    static __device__ __forceinline__ Look look(const Raw &r, const Stage &st, int kk, int, const uint8_t *lds, bool) {
        const uint32_t qh = st.qh >> (8 * (kk & 3) + 2 * (kk >> 2));
        const uint2 *g = (const uint2 *)lds;
        return Look{g[(r.qs & 0xFF) | ((qh & 1) << 8)], g[(r.qs >> 8) | (((qh >> 1) & 1) << 8)]};
    }
    static __device__ __forceinline__ uint4 make(const Raw &r, const Look &l, const Stage &st, int kk, int, bool zero) {
        const uint32_t s4 = (st.sc >> (4 * kk)) & 0xF;
        return scale4(apply_signs(make_uint4(l.x.x, l.x.y, l.y.x, l.y.y), r.sgn), splat_mult(zero ? 0u : (s4 << 4) | 8));
    }
    static __device__ __forceinline__ float scale(const uint8_t *win) { return h2f(lds_u16(win)) * 0.125f; }
};

// MXFP4: one scale (e8m0) per 32 weights, so per K-step. The fragment carries the power of two
// 2^(e - base) relative to the largest exponent of the row's stage, and the accumulator is
// rescaled when that base changes; in fp16 the product code * 2^(e - base) is exact down to
// 2^-24 of the stage's largest block scale (smaller contributions round).

struct MMXFP4 {
    static constexpr int TS = 17, SBK = 32, LDS = 0;
    static constexpr int KST = 8, SCALE = 1, ORG = 1;
    static __device__ void fill(uint8_t *, int, int) {}
    struct Stage {
        __device__ __forceinline__ void load(const WinRef &, int) {}
    };
    static __device__ __forceinline__ uint32_t expo(const uint8_t *win, int kk) { return lds_u8(win + TS * kk); }
    // Lane group grp takes bytes 4grp..4grp+3 of the block, both nibbles of each: weights 4grp+i
    // and 4grp+i+16 (the low and high nibbles of byte 4grp+i) at fragment positions 2i, 2i+1.
    // The K order of a 32-weight step is thus permuted; the activations are packed in the same
    // order (pack_rows_f16 with perm, mfma_k_permuted), so every product pairs the same weight
    // and activation as in natural order.
    struct Raw { uint32_t q; uint32_t e; };
    struct Look {};
    static __device__ __forceinline__ Raw raw(const WinRef &w, const Stage &, int kk, int grp) {
        return Raw{w.u32x(TS * kk + 4 * grp), expo(w.p, kk)};
    }
    static __device__ __forceinline__ Look look(const Raw &, const Stage &, int, int, const uint8_t *, bool) { return Look{}; }
    // The fragment by gfx950's scaled FP4 conversion (v_cvt_scalef32_pk_f16_fp4: the two E2M1
    // values of one byte, low nibble first, times an f32 scale, to fp16), one conversion per byte
    // of the lane's dword: the scale 2^(de+1) gives the doubled E2M1 codes times 2^de, de = e - base
    // <= 0 the block's exponent against the stage's largest. Every product is exact in fp16 down
    // to 2^-24 of that largest block scale; below it, it rounds.
    static __device__ __forceinline__ uint32_t cvt2(uint32_t v, float sc, int sel) {
        f16x2 h;
        if (sel == 0)
            h = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 0);
        else if (sel == 1)
            h = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 1);
        else if (sel == 2)
            h = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 2);
        else
            h = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 3);
        return __builtin_bit_cast(uint32_t, h);
    }
    static __device__ __forceinline__ uint4 make_mx(const Raw &r, int, int de) {
        const float sc = de >= -127 ? __uint_as_float((uint32_t)(de + 128) << 23) : 0.f;
        return make_uint4(cvt2(r.q, sc, 0), cvt2(r.q, sc, 1), cvt2(r.q, sc, 2), cvt2(r.q, sc, 3));
    }
};

// 8 small unsigned byte values (v < 1024) of two dwords -> fp16 (1024 + v), by placing each byte
// under an 0x64 high byte
__device__ __forceinline__ uint4 bytes_plus_1024(uint32_t w0, uint32_t w1) {
    return make_uint4(__builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u),
                      __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u));
}
// x * mul + add on each fp16 pair (one rounding: exact when the result is a small integer)
__device__ __forceinline__ uint32_t pk_fma_u(uint32_t x, uint32_t mul, uint32_t add) {
    const f16x2 r = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, x), __builtin_bit_cast(f16x2, mul), __builtin_bit_cast(f16x2, add));
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint4 fma4(uint4 v, uint32_t mul, uint32_t add) {
    return make_uint4(pk_fma_u(v.x, mul, add), pk_fma_u(v.y, mul, add), pk_fma_u(v.z, mul, add), pk_fma_u(v.w, mul, add));
}
__device__ __forceinline__ uint32_t splat_f16f(float v) {
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)v);
    return h | (h << 16);
}

// Q8_0: codes are the int8 quants themselves (exact in fp16), one f16 scale per block (per K-step)
struct MQ8_0 {
    static constexpr int TS = 34, SBK = 32, LDS = 16;
    static constexpr int KST = 4, SCALE = 2, ORG = 2;
    static __device__ void fill(uint8_t *, int, int) {}
    struct Stage {
        __device__ __forceinline__ void load(const WinRef &, int) {}
    };
    // (q + 128) + 1024 from the byte pattern, then x - 1152 (or 0 when the block's scale is 0)
    struct Raw { uint2 q; float d; };
    struct Look {};
    static __device__ __forceinline__ Raw raw(const WinRef &w, const Stage &, int kk, int grp) {
        return Raw{w.u64x(TS * kk + 8 * grp), h2f(lds_u16(w.p + TS * kk))};
    }
    static __device__ __forceinline__ Look look(const Raw &, const Stage &, int, int, const uint8_t *, bool) { return Look{}; }
    static __device__ __forceinline__ float step_scale(const Raw &r) { return r.d; }
    static __device__ __forceinline__ uint4 make(const Raw &r, const Look &, const Stage &, int, int, bool zero) {
        const uint4 x = bytes_plus_1024(r.q.x ^ 0x80808080u, r.q.y ^ 0x80808080u);
        const uint32_t one = zero ? 0u : 0x3C003C00u, off = zero ? 0u : 0xE480E480u;  // 1.0, -1152.0
        return fma4(x, one, off);
    }
};

// Q4_K: y = d*sc*q - dmin*m per sub-block of 32 (k_quants.rs:1821-1849, get_scale_min_k4 in
// quantized/utils.rs:50-60).
struct MQ4_K {
    static constexpr int TS = 144, SBK = 256, LDS = 16;
    static constexpr int KST = 8, SCALE = 0, ORG = 16;
    static __device__ void fill(uint8_t *, int, int) {}
    // The minimum term is folded into the codes: y = s (a q - b) per weight, with the running
    // scale s = max(|d|, |dmin|) of the super-block, a = (d / s) sc and b = (dmin / s) m of the
    // sub-block (both within 63 in magnitude, so fp16 keeps them to 2^-11 of themselves, and the
    // code a q - b takes one rounding). One accumulator and one MFMA per weight fragment.
    static __device__ __forceinline__ float s_of(float d, float dm) { return fmaxf(fabsf(d), fabsf(dm)); }
    // the 12 scale bytes (4..15) of the super-block, and d and dmin over s, read once per stage
    struct Stage {
        uint32_t b[3];
        float fd, fm;
        __device__ __forceinline__ void load(const WinRef &w, int) {
            const uint2 lo = w.u64(-12);
            b[0] = lo.x;
            b[1] = lo.y;
            b[2] = w.u64(-4).x;
            const uint32_t dd = w.u32x(-16);  // d, then dmin
            const float d = h2f(dd & 0xFFFFu), dm = h2f(dd >> 16), s = s_of(d, dm);
            fd = s > 0.f ? d / s : 0.f;
            fm = s > 0.f ? dm / s : 0.f;
        }
        __device__ __forceinline__ uint32_t byte(int i) const { return (b[i >> 2] >> (8 * (i & 3))) & 0xFF; }
    };
    static __device__ __forceinline__ float scale(const uint8_t *win) { return s_of(h2f(lds_u16(win)), h2f(lds_u16(win + 2))); }
    // 6-bit scale and min of sub-block j
    static __device__ __forceinline__ void sc_m(const Stage &st, int j, uint32_t &sc, uint32_t &m) {
        if (j < 4) {
            sc = st.byte(j) & 63;
            m = st.byte(j + 4) & 63;
        } else {
            const uint32_t a = st.byte(j + 4), lo = st.byte(j - 4), hi = st.byte(j);
            sc = (a & 0xF) | ((lo >> 6) << 4);
            m = (a >> 4) | ((hi >> 6) << 4);
        }
    }
    // codes a q - b of sub-block kk (sub-blocks 2c, 2c+1 are the low and high nibbles of qs[32c..32c+32))
    struct Raw { uint2 q; };
    struct Look {};
    static __device__ __forceinline__ Raw raw(const WinRef &w, const Stage &, int kk, int grp) { return Raw{w.u64(32 * (kk >> 1) + 8 * grp)}; }
    static __device__ __forceinline__ Look look(const Raw &, const Stage &, int, int, const uint8_t *, bool) { return Look{}; }
    static __device__ __forceinline__ uint4 make(const Raw &r, const Look &, const Stage &stg, int kk, int, bool zero) {
        uint32_t sc, m;
        sc_m(stg, kk, sc, m);
        const float a = zero ? 0.f : stg.fd * (float)sc, b = zero ? 0.f : stg.fm * (float)m;
        const uint2 q = r.q;
        const int sh = 4 * (kk & 1);
        // q as fp16 (1024 + q less 1024: exact), then a q - b
        const uint4 x = fma4(bytes_plus_1024((q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu), splat_f16f(1.0f),
                             splat_f16f(-1024.0f));
        return fma4(x, splat_f16f(a), splat_f16f(-b));
    }
};

// Q2_K (what the shrink writes): y = d*(sc&15)*q - dmin*(sc>>4) per 16 weights (k_quants.rs:1152-1190).
// K-step kk is sub-block kk of 32 weights: bits 2(kk&3) of qs[32(kk>>2) ..), so lane group grp
// reads the 8 bytes qs[32(kk>>2) + 8grp ..) and its 8 weights share scale byte 2kk + (grp>>1).
// The minimum term folded into the codes as for Q4_K: y = s (a q - b), s = max(|d|, |dmin|),
// a = (d / s) (sc & 15), b = (dmin / s) (sc >> 4), both within 15 in magnitude.
struct MQ2_K {
    static constexpr int TS = 84, SBK = 256, LDS = 16;
    static constexpr int KST = 8, SCALE = 0, ORG = 16;
    static __device__ void fill(uint8_t *, int, int) {}
    // the 16 scale bytes (0..15) of the super-block, and d and dmin over s, read once per stage
    struct Stage {
        uint32_t b[4];
        float fd, fm;
        __device__ __forceinline__ void load(const WinRef &w, int) {
            const uint2 lo = w.u64(-16), hi = w.u64(-8);
            b[0] = lo.x;
            b[1] = lo.y;
            b[2] = hi.x;
            b[3] = hi.y;
            const uint32_t dd = w.u32x(64);  // d, then dmin
            const float d = h2f(dd & 0xFFFFu), dm = h2f(dd >> 16), s = MQ4_K::s_of(d, dm);
            fd = s > 0.f ? d / s : 0.f;
            fm = s > 0.f ? dm / s : 0.f;
        }
        // scale byte 2kk + (grp >> 1)
        __device__ __forceinline__ uint32_t byte(int kk, int grp) const {
            return (b[kk >> 1] >> (16 * (kk & 1) + 8 * (grp >> 1))) & 0xFF;
        }
    };
    static __device__ __forceinline__ float scale(const uint8_t *win) { return MQ4_K::s_of(h2f(lds_u16(win + 80)), h2f(lds_u16(win + 82))); }
    struct Raw { uint2 q; };
    struct Look {};
    static __device__ __forceinline__ Raw raw(const WinRef &w, const Stage &, int kk, int grp) { return Raw{w.u64(32 * (kk >> 2) + 8 * grp)}; }
    static __device__ __forceinline__ Look look(const Raw &, const Stage &, int, int, const uint8_t *, bool) { return Look{}; }
    static __device__ __forceinline__ uint4 make(const Raw &r, const Look &, const Stage &stg, int kk, int grp, bool zero) {
        const uint32_t sb = stg.byte(kk, grp);
        const float a = zero ? 0.f : stg.fd * (float)(sb & 0xF), b = zero ? 0.f : stg.fm * (float)(sb >> 4);
        const int sh = 2 * (kk & 3);
        const uint4 x = fma4(bytes_plus_1024((r.q.x >> sh) & 0x03030303u, (r.q.y >> sh) & 0x03030303u), splat_f16f(1.0f),
                             splat_f16f(-1024.0f));
        return fma4(x, splat_f16f(a), splat_f16f(-b));
    }
};


// IQ3_XXS: weights 8grp..8grp+7 of K-step kk are the grid entries qs[8kk + 2grp], qs[8kk + 2grp + 1]
// (4 values each) with the signs of index (w >> 7grp) & 127, w the sub-block's word at byte
// 66 + 4kk (scale nibble s on top). The multiplier 8*(2s+1), as (s << 4) | 8, keeps the codes
// (at most 8*31*62) exact in fp16; scale() takes the 8 and the 1/4 of dl = d*(2s+1)/4 back out.
struct MIQ3_XXS {
    static constexpr int TS = 98, SBK = 256, LDS = 256 * 8;
    static constexpr int KST = 8, SCALE = 0, ORG = 66;
    static __device__ void fill(uint8_t *lds, int tid, int nt) { copy_tab(lds, c_iq3xxs_f16, tid, nt); }  // entry i: 4 halves at byte 8*i
    struct Stage {
        __device__ __forceinline__ void load(const WinRef &, int) {}
    };
    struct Raw { uint32_t qs, w; };
    struct Look { uint2 x, y; };
    static __device__ __forceinline__ Raw raw(const WinRef &w, const Stage &, int kk, int grp) {
        return Raw{lds_u16(w.p + 2 + 8 * kk + 2 * grp), w.u32(4 * kk)};
    }
    static __device__ __forceinline__ Look look(const Raw &r, const Stage &, int, int, const uint8_t *lds, bool) {
        const uint2 *g = (const uint2 *)lds;
        return Look{g[r.qs & 0xFF], g[(r.qs >> 8) & 0xFF]};
    }
    static __device__ __forceinline__ uint4 make(const Raw &r, const Look &l, const Stage &, int, int grp, bool zero) {
        const uint32_t s7 = (r.w >> (7 * grp)) & 127;
        const uint32_t b = s7 | ((__builtin_popcount(s7) & 1u) << 7);
        return scale4(apply_signs(make_uint4(l.x.x, l.x.y, l.y.x, l.y.y), b), splat_mult(zero ? 0u : ((r.w >> 28) << 4) | 8));
    }
    static __device__ __forceinline__ float scale(const uint8_t *win) { return h2f(lds_u16(win)) * (0.25f / 8); }
};

// IQ4_XS: K-step kk is sub-block kk, with its own scale d*(ls - 32) (per K-step, as Q8_0). Lane
// group grp takes the low (grp < 2) or high nibbles of qs[16kk + 8(grp&1) ..); a nibble's level
// kvalues[n] (exact in fp16) comes from a byte table of kvalues + 128 by two byte permutes and a
// select on the nibble's top bit, then through the fp16 1024 + byte pattern less 1152.
struct MIQ4_XS {
    static constexpr int TS = 136, SBK = 256, LDS = 16;
    static constexpr int KST = 8, SCALE = 2, ORG = 0;
    static __device__ void fill(uint8_t *, int, int) {}
    // d | scales_h << 16 and scales_l[4]: the super-block's first 8 bytes, read once per stage
    struct Stage {
        uint32_t h0, h1;
        __device__ __forceinline__ void load(const WinRef &w, int) {
            const uint2 h = w.u64(0);
            h0 = h.x;
            h1 = h.y;
        }
    };
    struct Raw { uint2 q; float d; };
    struct Look {};
    static __device__ __forceinline__ Raw raw(const WinRef &w, const Stage &st, int kk, int grp) {
        const uint32_t ls = ((st.h1 >> (4 * kk)) & 0xF) | (((st.h0 >> (16 + 2 * kk)) & 3) << 4);
        return Raw{w.u64(8 + 16 * kk + 8 * (grp & 1)), h2f(st.h0 & 0xFFFF) * (float)((int)ls - 32)};
    }
    static __device__ __forceinline__ Look look(const Raw &, const Stage &, int, int, const uint8_t *, bool) { return Look{}; }
    static __device__ __forceinline__ float step_scale(const Raw &r) { return r.d; }
    // kvalues_iq4nl + 128 as bytes, entries 0..15 over four dwords
    static constexpr uint32_t T0 = 0x3F2D1801u, T1 = 0x766A5D4Fu, T2 = 0xA6998D81u, T3 = 0xF1D9C5B5u;
    static __device__ __forceinline__ uint32_t levels4(uint32_t n) {  // 4 nibbles (one per byte) -> 4 table bytes
        const uint32_t lo = __builtin_amdgcn_perm(T1, T0, n & 0x07070707u);
        const uint32_t hi = __builtin_amdgcn_perm(T3, T2, n & 0x07070707u);
        const uint32_t top = ((n >> 3) & 0x01010101u) * 0xFFu;
        return (hi & top) | (lo & ~top);
    }
    static __device__ __forceinline__ uint4 make(const Raw &r, const Look &, const Stage &, int, int grp, bool zero) {
        const int sh = 4 * (grp >> 1);
        const uint4 x = bytes_plus_1024(levels4((r.q.x >> sh) & 0x0F0F0F0Fu), levels4((r.q.y >> sh) & 0x0F0F0F0Fu));
        const uint32_t one = zero ? 0u : 0x3C003C00u, off = zero ? 0u : 0xE480E480u;  // 1.0, -1152.0
        return fma4(x, one, off);
    }
};

// A stage is KST K-steps (8: 256 weights of k; 4 for Q8_0). The window of a row for a stage
// holds the stage's bytes (an IQ, Q2_K or Q4_K super-block, or KST MXFP4 / Q8_0 blocks) from the
// 16-byte boundary at or below their start, in PCS pieces of 16 bytes. PCS is odd: the 16 rows of
// a fragment read their windows at a stride of 4*PCS dwords, and an even PCS put rows 8 (or 4)
// apart on the same LDS banks (config 4 prefill 1,302-1,310 -> 1,253-1,261 us, config 3 271-275 ->
// 267-268, the last piece a re-load nothing reads).
template <class MF>
struct Win {
    static constexpr int SEG = MF::SBK == 32 ? MF::KST * MF::TS : MF::TS;
    static constexpr int PCS = ((SEG + (MF::TS % 2 ? 15 : 14) + 15) / 16) | 1;
    static constexpr int BYTES = 16 * PCS;
};

// ------------------------------------------------------------------------------ kernels

template <int V> struct Ic { static constexpr int value = V; };

__device__ __forceinline__ f16x8 as_f16x8(uint4 v) { return __builtin_bit_cast(f16x8, v); }

// 16 bytes from global memory to LDS without passing through registers: lane l of the wave
// writes lds_base + 16*l (lds_base is the same for the whole wave).
// ASM: issued as inline asm instead of through __builtin_amdgcn_global_load_lds. The compiler
// counts the builtin as an LDS store that any later LDS read at a dynamic address (a table
// lookup) may alias, and puts an s_waitcnt vmcnt(0) before that read, so every prefetch is
// waited for right after it is issued. The kernel orders these loads itself: an explicit
// s_waitcnt on the issuing wave, then a barrier, before any wave reads the bytes, and a barrier
// between the last read of a buffer and the loads that overwrite it. Loads return in order, so
// the compiler's own vmcnt waits stay correct with these in flight (they only wait longer: a
// register spill's reload then waits for the prefetches before it, which is why the formats
// that spill keep the builtin).
template <bool ASM>
__device__ __forceinline__ void dma16(const void *g, uint8_t *lds_base) {
    if constexpr (ASM) {
        const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)lds_base);
        // M0 (the LDS base of the load) is reserved to the compiler, which may keep a value in it:
        // saved and restored around the load
        uint32_t keep;
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                     : "=&s"(keep) : "v"(g), "s"(m) : "memory");
    } else {
        __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)lds_base, 16, 0, 0);
    }
}

// Tile shape of the grouped GEMM: a block owns one M-tile (up to MF_MT = 80 picks of a slot, in
// 16-row pick blocks) and RPB weight rows per matrix. Each wave takes NB blocks of 16 rows of one
// matrix and every pick block: per K-step it reads one activation fragment per pick block,
// decodes NB weight fragments and issues up to MF_MB*NB MFMAs. The decode is the VALU's work, so
// the LDS holds code tables that take work off the VALU, and the activations are shared by all
// waves of the block.
template <class MF, int MODE>
struct GmShape {
    static constexpr int LDS_MAX = 160 * 1024;
    static constexpr int NM = MODE == 0 ? 2 : 1;
    static constexpr int NB = 1;
    // PF: K-step table lookups and activation fragments read one step ahead (two register sets).
    // ADMA: the stage loads issued as inline asm (dma16). Both for every format but MXFP4 (equal or
    // slower with either).
    static constexpr bool FAST = !std::is_same<MF, MMXFP4>::value;
    static constexpr bool PF = FAST, ADMA = FAST;
    // K-steps per activation buffer and buffers per stage. Q4_K's down and dense instances take 2:
    // the halved buffers make room for a second window buffer beside two blocks per CU.
    static constexpr int KA = std::is_same<MF, MQ4_K>::value && MODE != 0 ? 2 : 4, HPS = MF::KST / KA;
    static constexpr int A_HALF = KA * MF_MB * 64 * 16, A_BYTES = 2 * A_HALF;  // two activation buffers
    static constexpr int META_BYTES = MF_MT * 8;                     // scale and pick of each row of the tile
    static constexpr int FIXED = ((MF::LDS + 15) & ~15) + A_BYTES + META_BYTES;
    // Gate/up: 16 waves (one block per CU), where their windows fit beside the tables. Down and
    // dense: 8 waves, two blocks per CU where the LDS allows, so one block's item start and end
    // (with a short K: down's is 512) overlap the other's K-steps. A wave works on one matrix:
    // the first WPM waves on gate, the others on up (MODE 0), which keeps its registers to one
    // accumulator set.
    static constexpr int NW = MODE == 0 && FIXED + 16 * 16 * Win<MF>::BYTES <= LDS_MAX ? 16 : 8, NT = 64 * NW;
    static constexpr int WPM = NW / NM;                              // waves per matrix
    static constexpr int RPW = 16 * NB, RPB = WPM * RPW;
    static constexpr int W_BYTES = NM * RPB * Win<MF>::BYTES;       // one stage of weight windows
    // 8-wave blocks run two per CU where two fit. Two window buffers are taken where they fit
    // beside the rest (without costing the second block): the weights of stage st+1 then load
    // while stage st computes.
    static constexpr int BASE_BYTES = FIXED + W_BYTES;
    static constexpr int PER_CU = NW == 8 && 2 * BASE_BYTES <= LDS_MAX ? 2 : 1;  // resident blocks per CU
    static constexpr bool WDB = PER_CU * (BASE_BYTES + W_BYTES) <= LDS_MAX;
    static constexpr size_t lds_bytes() { return BASE_BYTES + (WDB ? W_BYTES : 0); }
    static_assert(BASE_BYTES <= LDS_MAX, "the GEMM's LDS does not fit");
    static_assert(MODE != 0 || MF_MT * RPB * 4 <= A_BYTES, "the gate/up exchange does not fit the activation buffers");
};

// MODE 0: gate and up with the activation, hidden rows written in pile order.
// MODE 1: down, one output row per pick (combined per token by k_combine, in pick order, so the
//         result does not depend on the order blocks finish in).
// MODE 2: a dense matmul, the same output as MODE 1 (pile_pick NULL: one row per position).
//
// Per stage of 8 K-steps, the block copies its activations and the weight bytes of its rows
// into LDS with direct global-to-LDS loads: activations in MFMA fragment order ([K-step][pick
// block][lane] x 16 bytes, so every fragment read is one conflict-free ds_read_b128), weights as
// one window of whole 16-byte pieces per row (each load instruction covers 1 KB of consecutive
// pieces, instead of a few bytes from each of 16 rows). Latency is hidden by the second block
// on the CU. A piece is loaded only when it holds a byte of the row's stage; an aligned 16-byte
// piece cannot cross a page boundary, so its other bytes are mapped memory too.
//
// Scales: the accumulator of a weight row carries a running scale. When a new scale unit starts
// (an IQ super-block, or an MXFP4 stage), the accumulator is multiplied by old/new scale and the
// unit's codes accumulate on top; the epilogue multiplies by the last scale. This keeps one
// accumulator per output instead of a partial sum per scale unit.
template <class MF, int MODE>
__global__ __launch_bounds__(1024, 4) void k_gmm(const MfArgs a) {
    using S = GmShape<MF, MODE>;
    using W = Win<MF>;
    constexpr int NB = S::NB, KST = MF::KST;
    constexpr int NM = 1;  // matrices per wave (a block has S::NM: gate/up waves are split)
    constexpr bool POW2 = MF::SCALE == 1, STEP = MF::SCALE == 2;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int split_last;  // split-K: this block finished its work item's last split
    uint8_t *tab = smem;
    uint8_t *As = smem + ((MF::LDS + 15) & ~15);
    uint8_t *Ws = As + S::A_BYTES;  // window buffer(s): stage st uses Ws + (WDB ? st & 1 : 0) * W_BYTES
    float *meta_sa = (float *)(Ws + (S::WDB ? 2 : 1) * S::W_BYTES);
    int *meta_pick = (int *)(meta_sa + MF_MT);
    const int n_nb = (a.n + S::RPB - 1) / S::RPB;
    // blocks go to the 8 XCDs round-robin; item b of each run of R*n_nb (R = run_tiles) takes
    // M-tile R*run + b%R and N-block b/R. With R = 8 an M-tile's N-blocks share an XCD (and its
    // L2 copy of the activations); with fewer tiles than 8, R < 8 spreads each tile's N-blocks
    // over R-strided XCDs instead of leaving XCDs idle.
    MF::fill(tab, threadIdx.x, S::NT);
    // Persistent blocks: block b takes work items b, b + gridDim.x, ... (gridDim.x is a multiple of
    // 8, so every item of a block maps to the block's XCD), and fills the code tables once.
    const int R = a.run_tiles, n_tiles = *a.n_tiles;
    for (int item = blockIdx.x; item < a.n_items; item += gridDim.x) {
        const int run = item / (R * n_nb), b = item - run * R * n_nb;
        const int mt = run * R + (b & (R - 1));
        if (mt >= n_tiles) continue;  // uniform across the block
        const int nblk = b / R;
        __syncthreads();  // the tables are in, and every wave is done with the previous item's LDS
        // lane values from an opaque copy of the thread index, so that nothing derived from them
        // is hoisted out of the item loop and kept in registers across items
        int tidi = threadIdx.x;
        asm("" : "+v"(tidi));
        const int tid = tidi, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), grp = lane >> 4, l16 = lane & 15;
        const MfTile tile = a.tiles[mt];
        const int mbs = (tile.m + 15) >> 4;

        // the epilogue's activation scale and pick index of tile row tid, fetched now and put in LDS
        // with the first stage
        float my_sa = 0.f;
        int my_pick = 0;
        if (tid < tile.m) {
            const int pos = tile.pos0 + tid;
            my_sa = a.ascale[a.rows ? a.rows[pos] : pos];
            my_pick = a.pile_pick ? a.pile_pick[pos] : pos;
        }

        // the activation row this lane copies: pick block `wave`, row l16, k-group grp
        const bool stager = wave < mbs;
        const int apos = tile.pos0 + min(16 * wave + l16, tile.m - 1);
        const uint16_t *asrc = a.a16 + (int64_t)(a.rows ? a.rows[apos] : apos) * a.lda + 8 * grp;

        // Row r of the block is row nblk*RPB + r % RPB of matrix r / RPB (rows past n read row 0).
        // Addresses are the block's matrix base (uniform) plus 32-bit offsets (a matrix is under
        // 4 GiB: checked at launch), so they need no 64-bit registers per row.
        const uint8_t *wb0 = a.w0 + (int64_t)tile.slot * a.s0;
        const uint8_t *wb1 = S::NM > 1 ? a.w1 + (int64_t)tile.slot * a.s1 : wb0;
        const int mw = S::NM > 1 ? wave / S::WPM : 0;  // this wave's matrix
        const int wrow = (wave - mw * S::WPM) * S::RPW;  // its first row within the matrix's N-block
        auto row_off = [&](int r, int m) -> uint32_t {  // byte offset of row r within matrix m
            const int n = nblk * S::RPB + (r - m * S::RPB);
            return (uint32_t)(n < a.n ? n : 0) * (uint32_t)a.row_bytes;
        };

        const int n_ks = a.k / 32, n_st = (n_ks + KST - 1) / KST;
        f32x4 acc[NM][NB][MF_MB];
        float rs[NM][NB];     // running scale (f16 scales) ...
        int rb[NM][NB];       // ... or running base exponent (MXFP4)
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int q = 0; q < NB; q++) {
                rs[m][q] = 1.f;
                rb[m][q] = 0;
#pragma unroll
                for (int mb = 0; mb < MF_MB; mb++) {
                    acc[m][q][mb] = f32x4{0, 0, 0, 0};
                    // the compiler must not treat the four elements as one value from here on: with
                    // that assumption it once fed later MFMAs three stale copies (wrong rows 1-3 of
                    // each 4-row group); the empty asm emits nothing
                    asm volatile("" : "+v"(acc[m][q][mb]));
                }
            }

        // The weight windows of stage st_w into buffer wbuf: every wave issues exactly NTW loads
        // (waves past the last piece repeat the first ones, writing the same bytes to the same place,
        // and pieces past a row's last one re-load that one into a slot nothing reads), so the
        // stage's wait can leave exactly the next stage's loads in flight. RPB*PCS is a multiple of
        // 64: a wave's pieces lie in one matrix and the matrix base stays scalar.
        constexpr int NP = S::NM * S::RPB * W::PCS, NTW = (NP + S::NT - 1) / S::NT;
        // A piece's row offset and its place in the row's window are the same in every stage: for
        // the formats with registers to spare (S::FAST) they are worked out once per tile (the
        // division by the window's piece count and the row's 32-bit multiply were most of the
        // stage's address arithmetic), the others recompute them per stage.
        uint32_t wp_off[NTW], wp_p[NTW];
        if constexpr (S::FAST) {
#pragma unroll
            for (int t = 0; t < NTW; t++) {
                const int i0 = tid + S::NT * t, i = i0 < NP ? i0 : i0 - NP;
                const int r = i / W::PCS;
                wp_p[t] = (uint32_t)(i - r * W::PCS);
                wp_off[t] = row_off(r, __builtin_amdgcn_readfirstlane(r / S::RPB));
            }
        }
        auto issue_w = [&](int st_w, uint8_t *wbuf, int tido) __attribute__((always_inline)) {
            const int nk_w = min(KST, n_ks - st_w * KST);
            const uint32_t seg_w = MF::SBK == 32 ? MF::TS * nk_w : MF::TS;  // bytes of a row in this stage
#pragma unroll
            for (int t = 0; t < NTW; t++) {
                const int i0 = tido + S::NT * t, i = i0 < NP ? i0 : i0 - NP;  // the wrap is uniform across the wave
                int m;
                uint32_t o, p;
                if constexpr (S::FAST) {
                    m = S::NM > 1 ? __builtin_amdgcn_readfirstlane(i / (S::RPB * W::PCS)) : 0;
                    o = wp_off[t];
                    p = wp_p[t];
                } else {
                    const int r = i / W::PCS;
                    p = (uint32_t)(i - r * W::PCS);
                    m = __builtin_amdgcn_readfirstlane(r / S::RPB);
                    o = row_off(r, m);
                }
                const uint8_t *mb = m == 0 ? wb0 : wb1;
                o += (uint32_t)(W::SEG * st_w);                                // the row's stage bytes
                const uint32_t mis = ((uint32_t)(uintptr_t)mb + o) & 15;      // ... from a 16-byte boundary
                const uint32_t pc = min(p, (mis + seg_w - 1) >> 4);
                // from the 16-byte boundary at or below the row's stage bytes, taken on the full
                // address (a slot whose base is not 16-byte aligned has mis > o for its row 0)
                const uint8_t *al = (const uint8_t *)(((uintptr_t)mb + o) & ~(uintptr_t)15);
                dma16<S::ADMA>(al + 16 * pc, wbuf + (i - (tido & 63)) * 16);
            }
        };
        // Activations of half-stage h (K-steps h*KA .. h*KA+KA-1, clamped to the row: a clamped load
        // fills a slot nothing reads) into buffer h & 1, by the waves that own a pick block.
        auto issue_a = [&](int h) __attribute__((always_inline)) {
            if (stager) {
#pragma unroll
                for (int kk = 0; kk < S::KA; kk++)
                    dma16<S::ADMA>(asrc + min(h * S::KA + kk, n_ks - 1) * 32, As + (h & 1) * S::A_HALF + ((kk * MF_MB + wave) * 64) * 16);
            }
        };
        // vmcnt(NTW) alone: every load but this wave's last NTW (the next stage's windows) is done
        constexpr int WAIT_BUT_W = (NTW & 15) | ((NTW >> 4) << 14) | (7 << 4) | (15 << 8);

        // Pipeline: the activations of the next half-stage load while this one computes (two
        // buffers), and where two window buffers fit, the next stage's windows load during the whole
        // stage. One barrier per half-stage both publishes its loads and frees the buffer they
        // replace; a single window buffer needs a second barrier before it is refilled.
        const int st_lo = a.split_st ? blockIdx.y * a.split_st : 0;
        const int st_hi = a.split_st ? min(n_st, st_lo + a.split_st) : n_st;
        issue_a(st_lo * S::HPS);
        if constexpr (S::WDB) issue_w(st_lo, Ws + (st_lo & 1) * S::W_BYTES, tid);
        for (int st = st_lo; st < st_hi; st++) {
            // Per-lane addressing is recomputed from an opaque copy of the thread index each stage
            // (a few integer operations) rather than kept in registers across the stage loop.
            int tido = tid;
            asm("" : "+v"(tido));
            const int l16o = tido & 15;
            const int nk = min(KST, n_ks - st * KST);              // K-steps in this stage
            uint8_t *const Wst = Ws + (S::WDB ? (st & 1) * S::W_BYTES : 0);
            if (st == st_lo && tid < MF_MT) {
                meta_sa[tid] = my_sa;
                meta_pick[tid] = my_pick;
            }
            if constexpr (!S::WDB) {
                if (st != st_lo) __syncthreads();  // every wave is done with the previous stage's windows
                issue_w(st, Wst, tido);
            }
            __builtin_amdgcn_s_waitcnt(0);  // this stage's windows and first activations
            __syncthreads();
            if (S::HPS >= 2)
                issue_a(S::HPS * st + 1);
            else if (st + 1 < st_hi)
                issue_a(st + 1);
            if constexpr (S::WDB)
                if (st + 1 < st_hi) issue_w(st + 1, Ws + ((st + 1) & 1) * S::W_BYTES, tido);

            // this lane's windows
            const uint8_t *win[NM][NB];
            WinRef wr[NM][NB];
            typename MF::Stage stg[NM][NB];
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int q = 0; q < NB; q++) {
                    // this lane's row within the block's windows, and its start in global memory mod 16
                    const int lrow = mw * S::RPB + wrow + 16 * q + l16o;
                    const uint32_t lmis = (uint32_t)(uintptr_t)(mw == 0 ? wb0 : wb1) + row_off(lrow, mw);
                    win[m][q] = Wst + lrow * W::BYTES + ((lmis + (uint32_t)(W::SEG * st)) & 15);
                    wr[m][q] = WinRef::at<MF::ORG>(win[m][q]);
                    stg[m][q].load(wr[m][q], grp);
                }

            bool zero[NM][NB];
            float ratio[NM][NB];  // running-scale moves of this stage (scale per super-block)
            if constexpr (STEP) {
#pragma unroll
                for (int m = 0; m < NM; m++)
#pragma unroll
                    for (int q = 0; q < NB; q++) zero[m][q] = false;
            } else if constexpr (POW2) {
#pragma unroll
                for (int m = 0; m < NM; m++)
#pragma unroll
                    for (int q = 0; q < NB; q++) {
                        zero[m][q] = false;
                        // the base is the largest block exponent of the item's stages so far: the
                        // accumulators only ever move down onto a larger base (moving them up onto a
                        // smaller one overflowed f32 for rows whose block scales span more than 2^127)
                        int base = st > st_lo ? rb[m][q] : 0;
#pragma unroll
                        for (int kk = 0; kk < KST; kk++)
                            if (kk < nk) base = max(base, (int)MF::expo(win[m][q], kk));
                        if (st > st_lo && base != rb[m][q]) {
#pragma unroll
                            for (int mb = 0; mb < MF_MB; mb++)
#pragma unroll
                                for (int i = 0; i < 4; i++) acc[m][q][mb][i] = ldexpf(acc[m][q][mb][i], rb[m][q] - base);
                        }
                        rb[m][q] = base;
                    }
            } else {
#pragma unroll
                for (int m = 0; m < NM; m++)
#pragma unroll
                    for (int q = 0; q < NB; q++) {
                        // the accumulators move onto the new scale at the start of the K-steps (only
                        // the tile's pick blocks); a zero scale keeps the old one (its codes do not count)
                        const float d = MF::scale(win[m][q]);
                        zero[m][q] = d == 0.f;
                        ratio[m][q] = d != 0.f ? rs[m][q] * __builtin_amdgcn_rcpf(d) : 1.f;
                        rs[m][q] = d != 0.f ? d : rs[m][q];
                    }
            }

            // The K-steps, with the tile's count of 16-pick MFMA blocks as a constant, software
            // pipelined so that no step waits on an LDS read it issued itself: the window bytes of a
            // step are requested two steps ahead, its table lookups and activation fragments one step
            // ahead (step kk issues those of kk+1 once its own fragment is decoded, and they arrive
            // while its MFMAs run). The first step of the second half-stage reads its activations
            // after the barrier that publishes them. A scheduling fence closes each step (without
            // it the compiler interleaves all eight steps and runs out of registers).
            auto ksteps = [&](auto mbs_c) __attribute__((always_inline)) {
                constexpr int MBS = decltype(mbs_c)::value;
                const int nke = MF::SBK == 32 ? nk : KST;  // super-block formats: every stage is whole
                typename MF::Raw rw[2][NM][NB];
                typename MF::Look lk[2][NM][NB];
                f16x8 av[2][MBS];
                auto issue_raw = [&](int kk) __attribute__((always_inline)) {
#pragma unroll
                    for (int m = 0; m < NM; m++)
#pragma unroll
                        for (int q = 0; q < NB; q++) rw[kk & 1][m][q] = MF::raw(wr[m][q], stg[m][q], kk, grp);
                };
                auto issue_look = [&](int kk) __attribute__((always_inline)) {
#pragma unroll
                    for (int m = 0; m < NM; m++)
#pragma unroll
                        for (int q = 0; q < NB; q++) lk[kk & 1][m][q] = MF::look(rw[kk & 1][m][q], stg[m][q], kk, grp, tab, zero[m][q]);
                };
                auto issue_av = [&](int kk) __attribute__((always_inline)) {
                    const uint8_t *Ak = As + ((S::HPS >= 2 ? kk / S::KA : st) & 1) * S::A_HALF + (kk % S::KA) * MF_MB * 64 * 16;
#pragma unroll
                    for (int mb = 0; mb < MBS; mb++) av[kk & 1][mb] = *(const f16x8 *)(Ak + (mb * 64 + lane) * 16);
                };
                if constexpr (!STEP && !POW2) {
#pragma unroll
                    for (int m = 0; m < NM; m++)
#pragma unroll
                        for (int q = 0; q < NB; q++) {
#pragma unroll
                            for (int mb = 0; mb < MBS; mb++) acc[m][q][mb] *= ratio[m][q];
                        }
                }
                issue_raw(0);
                if (1 < nke) issue_raw(1);
                if constexpr (S::PF) {
                    issue_look(0);
                    issue_av(0);
                }
#pragma unroll
                for (int kk = 0; kk < KST; kk++) {
                    if (kk >= nke) break;
                    if (S::HPS >= 2 && kk > 0 && kk % S::KA == 0) {
                        // a later part of the stage: its activations (loaded during the previous
                        // part) are in. Only the first part's wait can leave the next stage's
                        // windows in flight: later parts' activations were requested after them.
                        if (S::WDB && st + 1 < st_hi && kk == S::KA)
                            __builtin_amdgcn_s_waitcnt(WAIT_BUT_W);
                        else
                            __builtin_amdgcn_s_waitcnt(0);
                        __syncthreads();
                        if (kk / S::KA + 1 < S::HPS)
                            issue_a(S::HPS * st + kk / S::KA + 1);
                        else if (st + 1 < st_hi)
                            issue_a(S::HPS * (st + 1));
                        if constexpr (S::PF) issue_av(kk);
                    }
                    if constexpr (!S::PF) {
                        issue_look(kk);
                        issue_av(kk);
                    }
                    if constexpr (STEP) {
                        // a scale per K-step: move each accumulator onto it
#pragma unroll
                        for (int m = 0; m < NM; m++)
#pragma unroll
                            for (int q = 0; q < NB; q++) {
                                const float d = MF::step_scale(rw[kk & 1][m][q]);
                                zero[m][q] = d == 0.f;
                                if (d != 0.f) {
                                    const float ratio = __fdividef(rs[m][q], d);
#pragma unroll
                                    for (int mb = 0; mb < MBS; mb++) acc[m][q][mb] *= ratio;
                                    rs[m][q] = d;
                                }
                            }
                    }
                    f16x8 bf[NM][NB];
#pragma unroll
                    for (int m = 0; m < NM; m++)
#pragma unroll
                        for (int q = 0; q < NB; q++) {
                            if constexpr (POW2)
                                bf[m][q] = as_f16x8(MF::make_mx(rw[kk & 1][m][q], grp, (int)rw[kk & 1][m][q].e - rb[m][q]));
                            else
                                bf[m][q] = as_f16x8(MF::make(rw[kk & 1][m][q], lk[kk & 1][m][q], stg[m][q], kk, grp, zero[m][q]));
                        }
                    if (kk + 2 < KST && kk + 2 < nke) issue_raw(kk + 2);  // into the buffer step kk has just used
                    if (S::PF && kk + 1 < KST && kk + 1 < nke) {
                        issue_look(kk + 1);
                        if (!(S::HPS >= 2 && (kk + 1) % S::KA == 0)) issue_av(kk + 1);
                    }
#pragma unroll
                    for (int mb = 0; mb < MBS; mb++)
#pragma unroll
                        for (int m = 0; m < NM; m++)
#pragma unroll
                            for (int q = 0; q < NB; q++) {
                                acc[m][q][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[kk & 1][mb], bf[m][q], acc[m][q][mb], 0, 0, 0);
                            }
                    __builtin_amdgcn_sched_barrier(0);
                }
            };
            switch (mbs) {
            case 1: ksteps(Ic<1>{}); break;
            case 2: ksteps(Ic<2>{}); break;
            case 3: ksteps(Ic<3>{}); break;
            case 4: ksteps(Ic<4>{}); break;
            default: ksteps(Ic<5>{}); break;
            }
        }

        // epilogue: lane holds picks 16*mb + 4*grp + i (i < 4) of weight row n (block q)
        float fs[NB];
#pragma unroll
        for (int q = 0; q < NB; q++) fs[q] = POW2 ? ldexpf(1.0f, rb[0][q] - 128) : rs[0][q];
        auto value = [&](int q, int mb, int i, float sa) __attribute__((always_inline)) {
            return acc[0][q][mb][i] * fs[q] * sa;
        };
        if constexpr (MODE == 0) {
            // the up waves hand their values to the gate waves through LDS (the activation
            // buffers, free once every wave is past the last K-step)
            float *xu = (float *)As;
            __syncthreads();
            if (mw == 1) {
#pragma unroll
                for (int mb = 0; mb < MF_MB; mb++) {
                    if (mb >= mbs) break;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int r = 16 * mb + 4 * grp + i;
#pragma unroll
                        for (int q = 0; q < NB; q++) xu[r * S::RPB + wrow + 16 * q + l16] = value(q, mb, i, meta_sa[r]);
                    }
                }
            }
            __syncthreads();
            if (mw == 0) {
#pragma unroll
                for (int mb = 0; mb < MF_MB; mb++) {
                    if (mb >= mbs) break;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int r = 16 * mb + 4 * grp + i;
                        if (r >= tile.m) continue;
                        const int pos = tile.pos0 + r;
#pragma unroll
                        for (int q = 0; q < NB; q++) {
                            const int n = nblk * S::RPB + wrow + 16 * q + l16;
                            if (n >= a.n) continue;
                            // sigmoid(z) = 1 / (1 + 2^(-z log2 e)) on the hardware's exp2 and
                            // reciprocal (each within 1 ulp)
                            constexpr float LOG2E = 1.4426950408889634f;
                            float g = value(q, mb, i, meta_sa[r]), u = xu[r * S::RPB + wrow + 16 * q + l16], o;
                            if (a.act == CW_ACT_SILU) {
                                o = g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * LOG2E)) * u;
                            } else {
                                const int64_t e = tile.expert;  // every pick of the tile's
                                if (a.bias0) g += a.bias0[e * a.n + n];
                                if (a.bias1) u += a.bias1[e * a.n + n];
                                g = fminf(g, a.limit);
                                u = fminf(fmaxf(u, -a.limit), a.limit);
                                o = (u + 1.0f) * (g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-(g * a.alpha) * LOG2E)));
                            }
                            a.h[(int64_t)pos * a.ldh + n] = o;
                        }
                    }
                }
            }
        } else {
            const bool split = MODE == 2 && a.split_cnt;
#pragma unroll
            for (int mb = 0; mb < MF_MB; mb++) {
                if (mb >= mbs) break;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 16 * mb + 4 * grp + i;
                    if (r >= tile.m) continue;
                    const int pick = meta_pick[r];
#pragma unroll
                    for (int q = 0; q < NB; q++) {
                        const int n = nblk * S::RPB + wrow + 16 * q + l16;
                        if (n >= a.n) continue;
                        float *p = a.dn + blockIdx.y * a.split_stride + (int64_t)pick * a.n + n;
                        const float v = value(q, mb, i, meta_sa[r]);
                        if (split)
                            __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // at the coherence point
                        else
                            *p = v;
                    }
                }
            }
            if (split) {
                // The last of the item's splits to get here adds the partial rows in split order (as a
                // separate pass over all of them would): the partial stores are at the coherence
                // point once this thread's stores have completed, before the block's arrival.
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
                if (tid == 0)
                    split_last = __hip_atomic_fetch_add(a.split_cnt + item, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                                 (int)gridDim.y - 1;
                __syncthreads();
                if (split_last) {
                    // partial values read at the coherence point (buffer loads with the sc1 policy,
                    // the form of an agent-scope load), 8 splits in flight at a time
                    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
                        (void *)a.dn, (short)0, (int)(gridDim.y * a.split_stride * 4), 0x00020000);
                    const int cols = min(S::RPB, a.n - nblk * S::RPB), nsp = (int)gridDim.y;
                    for (int e = tid; e < tile.m * cols; e += S::NT) {
                        const int r = e / cols, n = nblk * S::RPB + (e - r * cols);
                        const int o = (int)((int64_t)meta_pick[r] * a.n + n);
                        float acc = 0.f;
                        for (int s0 = 0; s0 < nsp; s0 += 8) {
                            float v[8];
#pragma unroll
                            for (int u = 0; u < 8; u++)  // past the last split: 0 from the buffer's range, unused
                                v[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pr, 4 * (o + (s0 + u) * (int)a.split_stride), 0, 16));
#pragma unroll
                            for (int u = 0; u < 8; u++)
                                if (s0 + u < nsp) acc = (s0 + u == 0) ? v[u] : acc + v[u];
                        }
                        a.y[o] = acc;
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------ helpers

// sum of the first n entries of a small LDS array
__device__ __forceinline__ int wc_total(const int *w, int n) {
    int t = 0;
    for (int i = 0; i < n; i++) t += w[i];
    return t;
}

// Inclusive prefix sum across the wave (six shuffle steps)
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int u = __shfl_up(v, d);
        if (lane >= d) v += u;
    }
    return v;
}

// One block: histogram of slots, exclusive scans, scatter of picks into per-slot piles, tiles.
// Each thread reads its (up to) PILE_PER slots into registers before using any, so the loads
// overlap, and keeps them for the scatter; the order of picks inside a pile does not matter
// (every pick's outputs are computed independently of the other rows of its tile). Up to
// PILE_LDS picks, the scatter goes to LDS and the piles leave in coalesced stores (random 4-byte
// stores from one CU cost a memory transaction each).
constexpr int PILE_PER = 16, PILE_LDS = 12288;
__global__ __launch_bounds__(1024) void k_piles(const uint32_t *slots, const uint32_t *ids, int TK, int K, int n_slots,
                                                 int *pile_pick, int *pile_tok, MfTile *tiles, int *n_tiles) {
    __shared__ int cnt[1024], off[1024], cur[1024], rep[1024], wtot[16], wttot[16], wftot[16];
    __shared__ int staged[PILE_LDS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    cnt[tid] = 0;
    cur[tid] = 0;
    rep[tid] = 0;
    const bool one = TK <= 1024 * PILE_PER;  // the common case: every slot read once, kept in registers
    uint32_t v[PILE_PER];
#pragma unroll
    for (int q = 0; q < PILE_PER; q++) {
        const int i = q * 1024 + tid;
        v[q] = i < TK ? slots[i] : 0xFFFFFFFFu;
    }
    __syncthreads();
    for (int c0 = 0; c0 < TK; c0 += 1024 * PILE_PER) {
        if (c0) {
#pragma unroll
            for (int q = 0; q < PILE_PER; q++) {
                const int i = c0 + q * 1024 + tid;
                v[q] = i < TK ? slots[i] : 0xFFFFFFFFu;
            }
        }
#pragma unroll
        for (int q = 0; q < PILE_PER; q++)
            if (v[q] < (uint32_t)n_slots) {
                atomicAdd(&cnt[v[q]], 1);
                atomicMax(&rep[v[q]], c0 + q * 1024 + tid);  // a pick of the slot, for its expert id
            }
    }
    __syncthreads();
    // exclusive scans of the counts, the tile counts and the first tiles: per wave, then over the
    // 16 wave totals. The tile list holds every slot's first tile, then the later tiles of the
    // slots with more than MF_MT picks: the GEMMs hand out work items in list order, so the last
    // round of items, which only some blocks run, takes the (smaller) remainder tiles.
    const int c = tid < n_slots ? cnt[tid] : 0;
    const int tc = (c + MF_MT - 1) / MF_MT, fc = c > 0 ? 1 : 0;
    const int ic = wave_incl_scan(c, lane), itc = wave_incl_scan(tc, lane), ifc = wave_incl_scan(fc, lane);
    if (lane == 63) {
        wtot[wave] = ic;
        wttot[wave] = itc;
        wftot[wave] = ifc;
    }
    __syncthreads();
    int wc = 0, wtc = 0, wfc = 0, nf = 0;
    for (int w = 0; w < 16; w++) {
        if (w < wave) {
            wc += wtot[w];
            wtc += wttot[w];
            wfc += wftot[w];
        }
        nf += wftot[w];
    }
    const int my_off = wc + ic - c, my_toff = wtc + itc - tc, my_f = wfc + ifc - fc;
    if (tid == 1023) *n_tiles = my_toff + tc;
    off[tid] = my_off;
    if (tid < n_slots) {
        const int ex = ids && c > 0 ? (int)ids[rep[tid]] : tid;
        for (int q = 0; q < tc; q++)
            tiles[q == 0 ? my_f : nf + (my_toff - my_f) + q - 1] = MfTile{tid, my_off + q * MF_MT, min(MF_MT, c - q * MF_MT), ex};
    }
    __syncthreads();
    for (int c0 = 0; c0 < TK; c0 += 1024 * PILE_PER) {
        if (!one) {
#pragma unroll
            for (int q = 0; q < PILE_PER; q++) {
                const int i = c0 + q * 1024 + tid;
                v[q] = i < TK ? slots[i] : 0xFFFFFFFFu;
            }
        }
#pragma unroll
        for (int q = 0; q < PILE_PER; q++) {
            const int i = c0 + q * 1024 + tid;
            if (v[q] < (uint32_t)n_slots) {
                const int pos = off[v[q]] + atomicAdd(&cur[v[q]], 1);
                if (TK <= PILE_LDS) {
                    staged[pos] = i;
                } else {
                    pile_pick[pos] = i;
                    pile_tok[pos] = i / K;
                }
            }
        }
    }
    if (TK <= PILE_LDS) {
        __syncthreads();
        const int n = wtot[15] + wc_total(wtot, 15);  // picks that resolved to a slot
        for (int p = tid; p < n; p += 1024) {
            const int i = staged[p];
            pile_pick[p] = i;
            pile_tok[p] = i / K;
        }
    }
}

// One wave per row, the row held in registers (NV float4 per lane, k <= 256*NV): scale =
// 2^(15 - e) with max|x| in [2^(e-1), 2^e) keeps the row's largest value in [2^14, 2^15) of
// fp16; ascale receives 1/scale.
template <int NV, bool PERM>
__global__ __launch_bounds__(256) void k_pack_f16(const float *x, int rows, int k, int ldx, uint16_t *a16, float *ascale,
                                                  PackExtra e) {
    if (e.tiles && blockIdx.x == 0) {  // tile i of a dense matmul: rows MF_MT*i .., "slot" 0
        const int nt = (e.m + MF_MT - 1) / MF_MT;
        for (int i = threadIdx.x; i < nt; i += blockDim.x) e.tiles[i] = MfTile{0, i * MF_MT, min(MF_MT, e.m - i * MF_MT), 0};
        if (threadIdx.x == 0) *e.n_tiles = nt;
    }
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < e.n_zero; i += gridDim.x * blockDim.x) e.zero[i] = 0;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + (int64_t)row * ldx;
    float4 v[NV];
    float m = 0.f;
    // loads from clamped addresses (all in flight at once), the values past the row zeroed after
    if constexpr (PERM) {
        // positions c..c+3 of a 32-wide step take its elements 2t, 2t+16, 2t+1, 2t+17 (t = (c % 32) / 4)
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int c = min(4 * lane + 256 * i, k - 4);
            const float *b = xr + (c & ~31) + ((c & 31) >> 1);
            const float2 lo = *(const float2 *)b, hi = *(const float2 *)(b + 16);
            v[i] = make_float4(lo.x, hi.x, lo.y, hi.y);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NV; i++) v[i] = *(const float4 *)(xr + min(4 * lane + 256 * i, k - 4));
    }
#pragma unroll
    for (int i = 0; i < NV; i++)
        if (4 * lane + 256 * i >= k) v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < NV; i++) {
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    }
    m = wave_max(m);
    int ex = 0;
    if (m > 0.f && m < INFINITY) { frexpf(m, &ex); ex = 15 - ex; }
    const float sc = ldexpf(1.0f, ex);
    uint16_t *o = a16 + (int64_t)row * k;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = 4 * lane + 256 * i;
        if (c < k) {
            const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)(v[i].x * sc)) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(v[i].y * sc)) << 16);
            const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)(v[i].z * sc)) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(v[i].w * sc)) << 16);
            *(uint2 *)(o + c) = make_uint2(lo, hi);
        }
    }
    if (lane == 0) ascale[row] = ldexpf(1.0f, -ex);
}

// one thread per 4 outputs of a token: the weighted sum of its K picks' rows, bias added per pick,
// in pick order. A pick whose slot is out of range is in no pile and has no row: it contributes
// NaN, as it does on the matvec and decode paths. The picks go in chunks of CH, each chunk's
// slots, weights and expert ids loaded together, then its rows and bias rows (every pick has a
// row of dn, written or not, so those loads need no branch; past K a chunk reads pick K - 1
// again, unused).
template <int CH>
__global__ __launch_bounds__(256) void k_combine(const float *dn, const float *w, const float *bias, const uint32_t *ids,
                                                 const uint32_t *slots, uint32_t n_slots, int K, int H, float *out) {
    const int t = blockIdx.y, j = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (j >= H) return;
    const float nan = __int_as_float(0x7fc00000);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int e0 = 0; e0 < K; e0 += CH) {
        uint32_t sl[CH], id[CH];
        float we[CH];
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int64_t pick = (int64_t)t * K + min(e0 + c, K - 1);
            sl[c] = slots[pick];
            we[c] = w[pick];
            id[c] = bias ? ids[pick] : 0u;
        }
        float4 d[CH], b[CH];
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int64_t pick = (int64_t)t * K + min(e0 + c, K - 1);
            d[c] = *(const float4 *)(dn + pick * H + j);
            b[c] = bias ? *(const float4 *)(bias + (int64_t)id[c] * H + j) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int c = 0; c < CH; c++) {
            if (e0 + c >= K) break;
            float4 v = sl[c] < n_slots ? d[c] : make_float4(nan, nan, nan, nan);
            if (bias) {
                v.x += b[c].x; v.y += b[c].y; v.z += b[c].z; v.w += b[c].w;
            }
            const float wc = we[c];
            acc.x += v.x * wc; acc.y += v.y * wc; acc.z += v.z * wc; acc.w += v.w * wc;
        }
    }
    *(float4 *)(out + (int64_t)t * H + j) = acc;
}

__global__ void k_fill_zero(float *p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0.f;
}

// ------------------------------------------------------------------------------ launchers

bool mfma_supported(int dtype) {
    return dtype == CW_IQ2_XXS || dtype == CW_IQ2_S || dtype == CW_IQ3_S || dtype == CW_MXFP4 || dtype == CW_Q4_K || dtype == CW_Q8_0 ||
           dtype == CW_Q2_K || dtype == CW_IQ3_XXS || dtype == CW_IQ4_XS || dtype == CW_MXFP4_R16;
}

int max_tiles(int TK, int n_slots) { return (TK + MF_MT - 1) / MF_MT + (n_slots < TK ? n_slots : TK); }

int mfma_piles(const uint32_t *slots, const uint32_t *ids, int TK, int K, int n_slots, int *pile_pick, int *pile_tok, MfTile *tiles,
               int *n_tiles, hipStream_t s) {
    if (n_slots > 1024) return set_error(CW_ENOTSUP, "mfma: %d slots (1024 max)", n_slots);
    hipLaunchKernelGGL(k_piles, dim3(1), dim3(1024), 0, s, slots, ids, TK, K, n_slots, pile_pick, pile_tok, tiles, n_tiles);
    return check_launch("k_piles");
}

int pack_rows_f16(const float *x, int rows, int k, int ldx, uint16_t *a16, float *ascale, hipStream_t s,
                  const PackExtra *extra, bool perm) {
    if (rows == 0) return CW_OK;
    if (k % 4 || ldx % 4) return set_error(CW_ENOTSUP, "pack: row of %d (stride %d) is not whole float4s", k, ldx);
    if (perm && k % 32) return set_error(CW_ENOTSUP, "pack: a permuted row of %d is not whole 32-wide steps", k);
    const dim3 grid((rows + 3) / 4);
    const int nv = (k + 255) / 256;
    const PackExtra e = extra ? *extra : PackExtra{};
#define CW_PACK(N) \
    if (nv <= N) { \
        if (perm) hipLaunchKernelGGL((k_pack_f16<N, true>), grid, dim3(256), 0, s, x, rows, k, ldx, a16, ascale, e); \
        else hipLaunchKernelGGL((k_pack_f16<N, false>), grid, dim3(256), 0, s, x, rows, k, ldx, a16, ascale, e); \
        return check_launch("k_pack_f16"); \
    }
    CW_PACK(2) CW_PACK(4) CW_PACK(8) CW_PACK(12) CW_PACK(16) CW_PACK(32)
#undef CW_PACK
    return set_error(CW_ENOTSUP, "pack: rows of %d above 8192", k);
}

int combine_picks(const float *dn, const float *w, const float *bias, const uint32_t *ids, const uint32_t *slots, int n_slots,
                  int T, int K, int H, float *out, hipStream_t s) {
    if (T == 0) return CW_OK;
    if (H % 4) return set_error(CW_ENOTSUP, "combine: width %d is not a multiple of 4", H);
    const dim3 grid((H / 4 + 255) / 256, T);
    hipLaunchKernelGGL(k_combine<4>, grid, dim3(256), 0, s, dn, w, bias, ids, slots, (uint32_t)n_slots, K, H, out);
    return check_launch("k_combine");
}

int fill_zero(float *p, int64_t n, hipStream_t s) {
    if (n == 0) return CW_OK;
    int64_t b = (n + 255) / 256;
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)(b < 8192 ? b : 8192)), dim3(256), 0, s, p, n);
    return check_launch("k_fill_zero");
}

constexpr int MAX_DEVICES = 64;

static int current_device() {
    int dev = 0;
    return hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < MAX_DEVICES ? dev : 0;
}

// persistent GEMM blocks: per_cu per CU of the current device, a multiple of 8 (the XCD count)
static int64_t resident_blocks(int per_cu = 1) {
    static std::atomic<int> cus_of[MAX_DEVICES];
    const int dev = current_device();
    int cus = cus_of[dev].load(std::memory_order_relaxed);
    if (!cus) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) n = 256;
        cus = n / 8 * 8;
        cus_of[dev].store(cus, std::memory_order_relaxed);
    }
    return (int64_t)cus * per_cu;
}

template <class MF, int MODE>
static int launch(const MfArgs &a, int tiles_max, int splits, hipStream_t s) {
    using S = GmShape<MF, MODE>;
    if (a.k % MF::SBK) return set_error(CW_ENOTSUP, "mfma: k %d is not a multiple of %d", a.k, MF::SBK);
    if ((int64_t)a.n * a.row_bytes >= ((int64_t)1 << 32))
        return set_error(CW_ENOTSUP, "mfma: a matrix of %d rows of %lld bytes is 4 GiB or more", a.n, (long long)a.row_bytes);
    const int n_nb = (a.n + S::RPB - 1) / S::RPB;
    const int R = tiles_max >= 8 ? 8 : tiles_max >= 4 ? 4 : tiles_max >= 2 ? 2 : 1;
    const int64_t items = (int64_t)((tiles_max + R - 1) / R) * R * n_nb;
    if (items >= ((int64_t)1 << 31)) return set_error(CW_ENOTSUP, "mfma: %lld work items", (long long)items);
    const int64_t res = resident_blocks(S::PER_CU);
    const int64_t blocks = items < res ? (items + 7) / 8 * 8 : res;
    static std::atomic<bool> lds_set[MAX_DEVICES];  // dynamic LDS above 64 KB, opted into once per kernel and device
    const int dev = current_device();
    if (!lds_set[dev].load(std::memory_order_acquire)) {
        if (hipFuncSetAttribute((const void *)k_gmm<MF, MODE>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::lds_bytes()) != hipSuccess)
            return set_error(CW_EHIP, "mfma: cannot reserve %zu bytes of LDS", S::lds_bytes());
        lds_set[dev].store(true, std::memory_order_release);
    }
    MfArgs b = a;
    b.run_tiles = R;
    b.n_items = (int)items;
    hipLaunchKernelGGL((k_gmm<MF, MODE>), dim3((unsigned)blocks, (unsigned)splits), dim3(S::NT), S::lds_bytes(), s, b);
    return check_launch("k_gmm");
}

template <int MODE>
static int by_fmt(int dtype, const MfArgs &a, int tiles_max, int splits, hipStream_t s) {
    switch (dtype) {
    case CW_IQ2_XXS: return launch<MIQ2_XXS, MODE>(a, tiles_max, splits, s);
    case CW_IQ2_S: return launch<MIQ2_S, MODE>(a, tiles_max, splits, s);
    case CW_IQ3_S: return launch<MIQ3_S, MODE>(a, tiles_max, splits, s);
    case CW_MXFP4: return launch<MMXFP4, MODE>(a, tiles_max, splits, s);
    case CW_Q4_K: return launch<MQ4_K, MODE>(a, tiles_max, splits, s);
    case CW_Q8_0: return launch<MQ8_0, MODE>(a, tiles_max, splits, s);
    case CW_Q2_K: return launch<MQ2_K, MODE>(a, tiles_max, splits, s);
    case CW_IQ3_XXS: return launch<MIQ3_XXS, MODE>(a, tiles_max, splits, s);
    case CW_IQ4_XS: return launch<MIQ4_XS, MODE>(a, tiles_max, splits, s);
    default: return set_error(CW_ENOTSUP, "mfma: dtype %d has no MFMA path", dtype);
    }
}

static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

// the dense GEMM's N-block rows and stage size for a format (GmShape<MF, 2>)
template <class MF>
static void shape_of(int &rpb, int &kst, int &per_cu) {
    rpb = GmShape<MF, 2>::RPB;
    kst = MF::KST;
    per_cu = GmShape<MF, 2>::PER_CU;
}
static void dense_shape(int dtype, int &rpb, int &kst, int &per_cu) {
    switch (dtype) {
    case CW_IQ2_XXS: return shape_of<MIQ2_XXS>(rpb, kst, per_cu);
    case CW_IQ2_S: return shape_of<MIQ2_S>(rpb, kst, per_cu);
    case CW_IQ3_S: return shape_of<MIQ3_S>(rpb, kst, per_cu);
    case CW_MXFP4: return shape_of<MMXFP4>(rpb, kst, per_cu);
    case CW_Q8_0: return shape_of<MQ8_0>(rpb, kst, per_cu);
    case CW_Q2_K: return shape_of<MQ2_K>(rpb, kst, per_cu);
    case CW_IQ3_XXS: return shape_of<MIQ3_XXS>(rpb, kst, per_cu);
    case CW_IQ4_XS: return shape_of<MIQ4_XS>(rpb, kst, per_cu);
    default: return shape_of<MQ4_K>(rpb, kst, per_cu);
    }
}
// The split count S minimises the stages on the critical path: the launch's blocks (work items,
// padded as launch() pads them, times S) run in rounds of the resident blocks, and each block runs
// its items' ceil(n_st / S) stages one after another. (Filling the resident blocks exactly, as a
// first version did, left config 2's M = 512 at 768 blocks over 512 slots: 2 rounds of 6 stages
// where 1 round of 8 does.) Each 8 splits add a stage to the cost: the last split of a work item
// reads the partial rows 8 splits at a time (config 2 at M = 16: 16 splits of one stage measured
// 19.4 us, 8 splits of two 17.8). Ties go to fewer splits (less partial traffic).
static int dense_splits(int dtype, int64_t m, int64_t n, int64_t k, int &split_st) {
    int rpb, kst, per_cu;
    dense_shape(dtype, rpb, kst, per_cu);
    const int64_t tiles = (m + MF_MT - 1) / MF_MT, n_nb = (n + rpb - 1) / rpb;
    const int64_t R = tiles >= 8 ? 8 : tiles >= 4 ? 4 : tiles >= 2 ? 2 : 1;
    const int64_t items = (tiles + R - 1) / R * R * n_nb, res = resident_blocks(per_cu);
    const int64_t grid_x = items < res ? (items + 7) / 8 * 8 : res, per_block = (items + grid_x - 1) / grid_x;
    const int n_st = (int)((k / 32 + kst - 1) / kst);
    int best_s = 1;
    int64_t best = -1;
    for (int S = 1; S <= n_st; S++) {
        const int sst = (n_st + S - 1) / S;
        if ((n_st + sst - 1) / sst != S) continue;  // the same split as a smaller S
        if (S > 1 && (int64_t)S * m * n * 4 >= ((int64_t)1 << 31)) break;  // the partial rows stay under 2 GiB (32-bit offsets)
        const int64_t cost = (grid_x * S + res - 1) / res * per_block * sst + (S > 1 ? (S + 7) / 8 : 0);
        if (best < 0 || cost < best) {
            best = cost;
            best_s = S;
        }
    }
    split_st = (n_st + best_s - 1) / best_s;
    return best_s;
}

// work items of the dense GEMM's launch (M-tiles padded to the launch's run length, by N-blocks)
static int64_t dense_items(int dtype, int64_t m, int64_t n) {
    int rpb, kst, per_cu;
    dense_shape(dtype, rpb, kst, per_cu);
    const int64_t tiles = (m + MF_MT - 1) / MF_MT, n_nb = (n + rpb - 1) / rpb;
    const int64_t R = tiles >= 8 ? 8 : tiles >= 4 ? 4 : tiles >= 2 ? 2 : 1;
    return (tiles + R - 1) / R * R * n_nb;
}

size_t mfma_dense_workspace(int dtype, int64_t m, int64_t n, int64_t k) {
    int split_st;
    const int S = dense_splits(dtype, m, n, k, split_st);
    return al256(m * k * 2) + al256(m * 4) + al256((m + MF_MT - 1) / MF_MT * sizeof(MfTile)) + al256(4) +
           (S > 1 ? al256((size_t)S * m * n * 4) + al256((size_t)dense_items(dtype, m, n) * 4) : 0);
}

// Dense Q4_K QMatMul for 2..16 rows of x, one launch after the pack: block b takes weight rows
// 16b .. 16b+15 over the whole of k, its W waves a share of at most 2 super-blocks each (4 each
// measured 13.3 against 12.9 us for config 2 at M = 16: half the waves in flight), with all
// of a wave's loads (the rows' super-block headers and code bytes, and its activation fragments)
// issued at once: the persistent GEMM's per-stage window round trips and split-K partial rows
// cost ~12 us here for ~0.3 us of MFMA work. MFMA operands as in k_gmm: A = a token's 8 fp16
// activations (lane = token l16, K-group grp), B = a row's 8 codes sc*q (lane = row l16, K-group
// grp), and the minimum term as a second accumulator with codes -m; each super-block's sums are
// folded in f32 with the lane's row's d and dmin (a lane's 4 outputs share its row), the waves'
// partial tiles summed in LDS in wave order, then scaled by the token's activation scale.
constexpr int SKINNY_SB = 2;  // super-blocks per wave
template <int W>
__global__ __launch_bounds__(64 * W) void k_skinny_q4k(const uint8_t *w, int64_t row_bytes, int n, int k, const uint16_t *x16,
                                                       const float *xs, int m, float *y) {
    // a wave's 16 rows x SKINNY_SB super-blocks, copied as 16-byte chunks (row r's bytes at r * RB)
    constexpr int RB = SKINNY_SB * 144, NCH = 16 * RB / 16, NI = (NCH + 63) / 64;
    __shared__ __align__(16) uint8_t wl[W][NI * 1024];
    __shared__ float part[W][16 * 16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, grp = lane >> 4;
    const int nsb = k / 256, s0 = wave * nsb / W, s1 = (wave + 1) * nsb / W;  // this wave's super-blocks
    const uint16_t *xr = x16 + (int64_t)min(l16, m - 1) * k + 8 * grp;
    // every load at once, from clamped rows and super-blocks (those past s1 are not used): the
    // weight bytes as whole 16-byte chunks of each row's run of super-blocks straight into LDS
    // (per-lane 8-byte pieces of 16 rows measured slower), then the activation fragments
#pragma unroll
    for (int t = 0; t < NI; t++) {
        const int c = min(64 * t + lane, NCH - 1), r = c / (RB / 16), piece = c - r * (RB / 16), j = piece / 9;
        dma16<true>(w + (int64_t)min(blockIdx.x * 16 + r, n - 1) * row_bytes + 144 * min(s0 + j, nsb - 1) + 16 * (piece - 9 * j),
                    &wl[wave][1024 * t]);
    }
    uint4 head[SKINNY_SB];
    uint2 qs[SKINNY_SB][4];
    uint4 xf[SKINNY_SB][8];
#pragma unroll
    for (int j = 0; j < SKINNY_SB; j++) {
        const int sb = min(s0 + j, nsb - 1);
#pragma unroll
        for (int kk = 0; kk < 8; kk++) xf[j][kk] = *(const uint4 *)(xr + 256 * sb + 32 * kk);
    }
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(8 * SKINNY_SB) : "memory");  // the chunks have landed
#pragma unroll
    for (int j = 0; j < SKINNY_SB; j++) {
        const uint8_t *blk = &wl[wave][l16 * RB + 144 * j];
        head[j] = *(const uint4 *)blk;  // d, dmin, the 12 scale bytes
#pragma unroll
        for (int c = 0; c < 4; c++) qs[j][c] = *(const uint2 *)(blk + 16 + 32 * c + 8 * grp);
    }
    // nothing moves across this point: the scheduler would otherwise sink later super-blocks'
    // loads behind earlier MFMAs (to save registers), one memory round trip per super-block
    __builtin_amdgcn_sched_barrier(0);
    f32x4 fin = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < SKINNY_SB; j++) {
        // no branch on the wave's super-block count: a branch here kept the compiler from issuing
        // the later super-blocks' loads before the first one's MFMAs
        f32x4 acc = {0.f, 0.f, 0.f, 0.f}, accm = {0.f, 0.f, 0.f, 0.f};
        const uint32_t sb12[3] = {head[j].y, head[j].z, head[j].w};
        auto sbyte = [&](int i) { return (sb12[i >> 2] >> (8 * (i & 3))) & 0xFFu; };
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            uint32_t sc, mn;  // the 6-bit scale and min of sub-block kk (get_scale_min_k4)
            if (kk < 4) {
                sc = sbyte(kk) & 63;
                mn = sbyte(kk + 4) & 63;
            } else {
                sc = (sbyte(kk + 4) & 0xF) | ((sbyte(kk - 4) >> 6) << 4);
                mn = (sbyte(kk + 4) >> 4) | ((sbyte(kk) >> 6) << 4);
            }
            const int sh = 4 * (kk & 1);
            const uint2 q = qs[j][kk >> 1];
            const uint4 codes = fma4(bytes_plus_1024((q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu), splat_f16f((float)sc),
                                     splat_f16f(-1024.0f * (float)sc));
            const uint32_t mv = splat_f16f(-(float)mn);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(xf[j][kk]), as_f16x8(codes), acc, 0, 0, 0);
            accm = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(xf[j][kk]), as_f16x8(make_uint4(mv, mv, mv, mv)), accm, 0, 0, 0);
        }
        const bool live = s0 + j < s1;
        const float d = live ? h2f(head[j].x & 0xFFFF) : 0.f, dmin = live ? h2f(head[j].x >> 16) : 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) fin[i] += d * acc[i] + dmin * accm[i];
    }
    // lane: tokens 4*grp + i of weight row l16
#pragma unroll
    for (int i = 0; i < 4; i++) part[wave][(4 * grp + i) * 16 + l16] = fin[i];
    __syncthreads();
    for (int e = threadIdx.x; e < 256; e += 64 * W) {
        const int t = e >> 4, r = blockIdx.x * 16 + (e & 15);
        float v = 0.f;
#pragma unroll
        for (int q = 0; q < W; q++) v += part[q][e];
        if (t < m && r < n) y[(int64_t)t * n + r] = v * xs[t];
    }
}

// 2..16 rows of Q4_K x: the pack (fp16 activations and their scales), then k_skinny_q4k
static int dense_skinny_q4k(const uint8_t *w, int64_t row_bytes, int n, int k, const float *x, int m, float *y, uint16_t *x16,
                            float *xs, hipStream_t s) {
    int rc;
    if ((rc = pack_rows_f16(x, m, k, k, x16, xs, s, nullptr, false))) return rc;
    const int nsb = k / 256, waves = (nsb + SKINNY_SB - 1) / SKINNY_SB;
    const dim3 grid((unsigned)((n + 15) / 16));
    if (waves <= 1) hipLaunchKernelGGL(k_skinny_q4k<1>, grid, dim3(64), 0, s, w, row_bytes, n, k, x16, xs, m, y);
    else if (waves <= 2) hipLaunchKernelGGL(k_skinny_q4k<2>, grid, dim3(128), 0, s, w, row_bytes, n, k, x16, xs, m, y);
    else if (waves <= 4) hipLaunchKernelGGL(k_skinny_q4k<4>, grid, dim3(256), 0, s, w, row_bytes, n, k, x16, xs, m, y);
    else if (waves <= 8) hipLaunchKernelGGL(k_skinny_q4k<8>, grid, dim3(512), 0, s, w, row_bytes, n, k, x16, xs, m, y);
    else if (waves <= 16) hipLaunchKernelGGL(k_skinny_q4k<16>, grid, dim3(1024), 0, s, w, row_bytes, n, k, x16, xs, m, y);
    else return set_error(CW_ENOTSUP, "qmatmul: k %d above %d for the skinny Q4_K path", k, 16 * SKINNY_SB * 256);
    return check_launch("k_skinny_q4k");
}

int mfma_dense(int dtype, const uint8_t *w, int64_t row_bytes, int n, int k, const float *x, int m, float *y, void *ws,
               size_t ws_bytes, hipStream_t s) {
    const size_t need = mfma_dense_workspace(dtype, m, n, k);
    if (ws_bytes < need || !ws) return set_error(CW_EINVAL, "qmatmul: workspace of %zu bytes, %zu needed", ws_bytes, need);
    int split_st;
    const int S = dense_splits(dtype, m, n, k, split_st);
    uint8_t *p = (uint8_t *)ws;
    uint16_t *x16 = (uint16_t *)p; p += al256((size_t)m * k * 2);
    float *xs = (float *)p; p += al256((size_t)m * 4);
    // (its rows are copied as 16-byte chunks: a matrix off 16-byte alignment takes the GEMM below)
    if (dtype == CW_Q4_K && m <= 16 && ((uintptr_t)w & 15) == 0) return dense_skinny_q4k(w, row_bytes, n, k, x, m, y, x16, xs, s);
    MfTile *tiles = (MfTile *)p; p += al256((size_t)(m + MF_MT - 1) / MF_MT * sizeof(MfTile));
    int *n_tiles = (int *)p; p += al256(4);
    float *part = nullptr;
    int *cnt = nullptr;
    if (S > 1) {
        part = (float *)p;
        p += al256((size_t)S * m * n * 4);
        cnt = (int *)p;
    }
    // one launch packs x, writes the tile list and zeroes the split counters
    const PackExtra extra = {tiles, n_tiles, m, cnt, S > 1 ? (int)dense_items(dtype, m, n) : 0};
    int rc;
    if ((rc = pack_rows_f16(x, m, k, k, x16, xs, s, &extra, mfma_k_permuted(dtype)))) return rc;
    MfArgs a = {};
    a.w0 = w;
    a.s0 = 0;
    a.row_bytes = row_bytes;
    a.n = n;
    a.k = k;
    a.a16 = x16;
    a.ascale = xs;
    a.lda = k;
    a.tiles = tiles;
    a.n_tiles = n_tiles;
    a.K = 1;
    a.dn = S > 1 ? part : y;
    a.split_st = S > 1 ? split_st : 0;
    a.split_stride = (int64_t)m * n;
    a.split_cnt = cnt;
    a.y = y;
    return by_fmt<2>(dtype, a, (m + MF_MT - 1) / MF_MT, S, s);
}

int mfma_gateup(int dtype, const MfArgs &a, int tiles_max, hipStream_t s) { return by_fmt<0>(dtype, a, tiles_max, 1, s); }
int mfma_down(int dtype, const MfArgs &a, int tiles_max, hipStream_t s) { return by_fmt<1>(dtype, a, tiles_max, 1, s); }

}  // namespace cw
