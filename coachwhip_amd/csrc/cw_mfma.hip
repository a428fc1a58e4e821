// Grouped expert GEMMs on MFMA (gfx950, v_mfma_f32_16x16x32_f16) for the MoE layer's prefill.
//
// Picks are grouped by the slot they read (mfma_piles); a tile is up to 64 picks of one slot by
// 64 weight rows. Each of the 4 waves owns 16 weight rows and all 64 picks (4 MFMA blocks).
//
// Exactness: a weight is (f16 super-block scale) x (small integer code). The codes go through
// MFMA as fp16 integers, which they represent exactly: IQ2_XXS / IQ2_S codes (2s+1)*grid*sign
// are at most 31*43 = 1333, IQ3_S codes (1+2s)*grid*sign at most 31*15 = 465, MXFP4 codes the
// doubled E2M1 values up to 12. Products with fp16 activations are exact in the f32
// accumulators; the f32 scale of each super-block (d/8, d, or MXFP4's 2^(e-128) per 32) is
// applied to the partial sum of its K-steps. Activations are rounded to fp16 once, with a
// power-of-two scale per row (exact) so that no row overflows: that rounding (2^-11 relative)
// is the only approximation.
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
__device__ __forceinline__ uint32_t splat_f16(int v) {
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)v);
    return h | (h << 16);
}
__device__ __forceinline__ uint4 scale4(uint4 v, uint32_t sc2) {
    return make_uint4(pk_mul_u(v.x, sc2), pk_mul_u(v.y, sc2), pk_mul_u(v.z, sc2), pk_mul_u(v.w, sc2));
}
__device__ __forceinline__ uint4 xor4(uint4 a, uint4 b) { return make_uint4(a.x ^ b.x, a.y ^ b.y, a.z ^ b.z, a.w ^ b.w); }

// ------------------------------------------------------------------------------ code tables
// Lattice entries as fp16 integers and sign masks as fp16 sign bits, built at compile time; a
// kernel copies the ones its format needs into LDS.
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
constexpr U4 signs8(uint32_t s) {
    uint32_t w[4] = {};
    for (int i = 0; i < 4; i++) w[i] = (((s >> (2 * i)) & 1u) << 15) | (((s >> (2 * i + 1)) & 1u) << 31);
    return U4{w[0], w[1], w[2], w[3]};
}
constexpr uint32_t parity_signs(uint32_t i7) {  // ksigns_iq2xs: 7 bits plus an even-parity bit
    uint32_t p = i7 ^ (i7 >> 4);
    p ^= p >> 2;
    p ^= p >> 1;
    return i7 | ((p & 1u) << 7);
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
constexpr Tab<128> make_parity_signs() {
    Tab<128> t{};
    for (int i = 0; i < 128; i++) t.v[i] = signs8(parity_signs((uint32_t)i));
    return t;
}
constexpr Tab<256> make_signs() {
    Tab<256> t{};
    for (int i = 0; i < 256; i++) t.v[i] = signs8((uint32_t)i);
    return t;
}
static __constant__ Tab<256> c_iq2xxs_f16 = make_iq2xxs_f16();
static __constant__ Tab<1024> c_iq2s_f16 = make_iq2s_f16();
static __constant__ Tab<256> c_iq3s_f16 = make_iq3s_f16();
static __constant__ Tab<128> c_psigns = make_parity_signs();
static __constant__ Tab<256> c_signs = make_signs();

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

// Traits common to the formats: KST K-steps per stage; SCALE 0 = one f16 scale per super-block
// (read by scale()), 1 = MXFP4's power-of-two block scales, 2 = one f16 scale per 32-weight block
// (read by step_scale()); HAS_MIN = an f16 dmin per super-block and a 6-bit m per sub-block.
struct MIQ2_XXS {
    static constexpr int TS = 66, SBK = 256, LDS = 256 * 16 + 128 * 16;
    static constexpr int KST = 8, SCALE = 0;
    static constexpr bool HAS_MIN = false;
    static __device__ void fill(uint8_t *lds, int tid, int nt) {
        copy_tab(lds, c_iq2xxs_f16, tid, nt);
        copy_tab(lds + 256 * 16, c_psigns, tid, nt);
    }
    // zero: the super-block scale is 0, so the codes must not contribute
    static __device__ __forceinline__ uint4 frag(const uint8_t *win, int kk, int grp, const uint8_t *lds, bool zero) {
        const uint2 q = lds_u64(win + 2 + 8 * kk);
        const uint4 *g = (const uint4 *)lds, *sg = (const uint4 *)(lds + 256 * 16);
        const uint32_t gi = (q.x >> (8 * grp)) & 0xFF;
        const uint32_t si = (q.y >> (7 * grp)) & 127;
        const uint32_t sc = zero ? 0u : 2 * (q.y >> 28) + 1;
        return scale4(xor4(g[gi], sg[si]), splat_f16((int)sc));
    }
    static __device__ __forceinline__ float scale(const uint8_t *win) { return h2f(lds_u16(win)) * 0.125f; }
};

struct MIQ2_S {
    static constexpr int TS = 82, SBK = 256, LDS = 1024 * 16 + 256 * 16;
    static constexpr int KST = 8, SCALE = 0;
    static constexpr bool HAS_MIN = false;
    static __device__ void fill(uint8_t *lds, int tid, int nt) {
        copy_tab(lds, c_iq2s_f16, tid, nt);
        copy_tab(lds + 1024 * 16, c_signs, tid, nt);
    }
    static __device__ __forceinline__ uint4 frag(const uint8_t *win, int kk, int grp, const uint8_t *lds, bool zero) {
        const uint32_t qs = lds_u8(win + 2 + 4 * kk + grp), sgn = lds_u8(win + 34 + 4 * kk + grp);
        const uint32_t qh = lds_u8(win + 66 + kk), scb = lds_u8(win + 74 + kk);
        const uint4 *g = (const uint4 *)lds, *sg = (const uint4 *)(lds + 1024 * 16);
        const uint32_t gi = qs | (((qh >> (2 * grp)) & 3) << 8);
        const uint32_t sc = zero ? 0u : 2 * ((scb >> (4 * (grp >> 1))) & 0xF) + 1;
        return scale4(xor4(g[gi], sg[sgn]), splat_f16((int)sc));
    }
    static __device__ __forceinline__ float scale(const uint8_t *win) { return h2f(lds_u16(win)) * 0.125f; }
};

struct MIQ3_S {
    static constexpr int TS = 110, SBK = 256, LDS = 512 * 8 + 256 * 16;
    static constexpr int KST = 8, SCALE = 0;
    static constexpr bool HAS_MIN = false;
    static __device__ void fill(uint8_t *lds, int tid, int nt) {
        copy_tab(lds, c_iq3s_f16, tid, nt);   // entry i as 4 halves at byte 8*i
        copy_tab(lds + 512 * 8, c_signs, tid, nt);
    }
    static __device__ __forceinline__ uint4 frag(const uint8_t *win, int kk, int grp, const uint8_t *lds, bool zero) {
        const uint32_t qs = lds_u16(win + 2 + 8 * kk + 2 * grp), qh = lds_u8(win + 66 + kk);
        const uint32_t sgn = lds_u8(win + 74 + 4 * kk + grp), scb = lds_u8(win + 106 + (kk >> 1));
        const uint2 *g = (const uint2 *)lds;
        const uint4 *sg = (const uint4 *)(lds + 512 * 8);
        const uint32_t i0 = (qs & 0xFF) | (((qh >> (2 * grp)) & 1) << 8);
        const uint32_t i1 = (qs >> 8) | (((qh >> (2 * grp + 1)) & 1) << 8);
        const uint2 x = g[i0], y = g[i1];
        const uint32_t sc = zero ? 0u : 1 + 2 * ((scb >> (4 * (kk & 1))) & 0xF);
        return scale4(xor4(make_uint4(x.x, x.y, y.x, y.y), sg[sgn]), splat_f16((int)sc));
    }
    static __device__ __forceinline__ float scale(const uint8_t *win) { return h2f(lds_u16(win)); }
};

// MXFP4: one scale (e8m0) per 32 weights, so per K-step. The fragment carries the power of two
// 2^(e - base) relative to the largest exponent of the row's stage, and the accumulator is
// rescaled when that base changes; in fp16 the product code * 2^(e - base) is exact down to
// 2^-24 of the stage's largest block scale (smaller contributions round).
constexpr Tab<64> make_mxfp4_pairs() {  // fp16 pair of the doubled-E2M1 codes (lo, hi), index lo | hi << 4
    Tab<64> t{};
    const int kv[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    uint32_t w[256] = {};
    for (int i = 0; i < 256; i++) {
        uint32_t h[2] = {};
        for (int q = 0; q < 2; q++) {
            const int v = kv[(i >> (4 * q)) & 15];
            h[q] = f16_int((uint32_t)(v < 0 ? -v : v)) | (v < 0 ? 0x8000u : 0u);
        }
        w[i] = h[0] | (h[1] << 16);
    }
    for (int i = 0; i < 64; i++) t.v[i] = U4{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
    return t;
}
static __constant__ Tab<64> c_mxfp4_pairs = make_mxfp4_pairs();

struct MMXFP4 {
    static constexpr int TS = 17, SBK = 32, LDS = 1024;
    static constexpr int KST = 8, SCALE = 1;
    static constexpr bool HAS_MIN = false;
    static __device__ void fill(uint8_t *lds, int tid, int nt) { copy_tab(lds, c_mxfp4_pairs, tid, nt); }
    static __device__ __forceinline__ uint32_t expo(const uint8_t *win, int kk) { return lds_u8(win + TS * kk); }
    static __device__ __forceinline__ uint32_t pair(const uint32_t *tab, uint32_t w) {
        return tab[(w & 0xF) | ((w >> 4) & 0xF0)];
    }
    // lane group grp takes the low (grp < 2) or high nibbles of bytes 8*(grp&1)..+8; mult is the
    // splatted fp16 2^(e - base)
    static __device__ __forceinline__ uint4 frag_mx(const uint8_t *win, int kk, int grp, const uint8_t *lds, uint32_t mult) {
        const uint2 q = lds_u64(win + TS * kk + 1 + 8 * (grp & 1));
        const uint32_t *tab = (const uint32_t *)lds;
        const int sh = 4 * (grp >> 1);
        const uint32_t a = (q.x >> sh) & 0x0F0F0F0F, b = (q.y >> sh) & 0x0F0F0F0F;
        return scale4(make_uint4(pair(tab, a), pair(tab, a >> 16), pair(tab, b), pair(tab, b >> 16)), mult);
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
    static constexpr int KST = 4, SCALE = 2;
    static constexpr bool HAS_MIN = false;
    static __device__ void fill(uint8_t *, int, int) {}
    static __device__ __forceinline__ float step_scale(const uint8_t *win, int kk) { return h2f(lds_u16(win + TS * kk)); }
    // (q + 128) + 1024 from the byte pattern, then x - 1152 (or 0 when the block's scale is 0)
    static __device__ __forceinline__ uint4 frag(const uint8_t *win, int kk, int grp, const uint8_t *, bool zero) {
        const uint2 q = lds_u64(win + TS * kk + 2 + 8 * grp);
        const uint4 x = bytes_plus_1024(q.x ^ 0x80808080u, q.y ^ 0x80808080u);
        const uint32_t one = zero ? 0u : 0x3C003C00u, off = zero ? 0u : 0xE480E480u;  // 1.0, -1152.0
        return fma4(x, one, off);
    }
};

// Q4_K: y = d*sc*q - dmin*m per sub-block of 32 (k_quants.rs:1821-1849, get_scale_min_k4 in
// quantized/utils.rs:50-60). Codes sc*q (<= 945) are exact in fp16 with d as the running scale;
// the minimum term is a second product of the same activations with codes -m (<= 63) and dmin as
// its running scale.
struct MQ4_K {
    static constexpr int TS = 144, SBK = 256, LDS = 16;
    static constexpr int KST = 8, SCALE = 0;
    static constexpr bool HAS_MIN = true;
    static __device__ void fill(uint8_t *, int, int) {}
    static __device__ __forceinline__ float scale(const uint8_t *win) { return h2f(lds_u16(win)); }
    static __device__ __forceinline__ float dmin(const uint8_t *win) { return h2f(lds_u16(win + 2)); }
    // 6-bit scale and min of sub-block j
    static __device__ __forceinline__ void sc_m(const uint8_t *win, int j, uint32_t &sc, uint32_t &m) {
        const uint8_t *q = win + 4;
        if (j < 4) {
            sc = lds_u8(q + j) & 63;
            m = lds_u8(q + j + 4) & 63;
        } else {
            const uint32_t a = lds_u8(q + j + 4), lo = lds_u8(q + j - 4), hi = lds_u8(q + j);
            sc = (a & 0xF) | ((lo >> 6) << 4);
            m = (a >> 4) | ((hi >> 6) << 4);
        }
    }
    // codes sc*q of sub-block kk (sub-blocks 2c, 2c+1 are the low and high nibbles of qs[32c..32c+32))
    static __device__ __forceinline__ uint4 frag(const uint8_t *win, int kk, int grp, const uint8_t *, bool zero) {
        uint32_t sc, m;
        sc_m(win, kk, sc, m);
        if (zero) sc = 0;
        const uint2 q = lds_u64(win + 16 + 32 * (kk >> 1) + 8 * grp);
        const int sh = 4 * (kk & 1);
        const uint4 x = bytes_plus_1024((q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu);
        return fma4(x, splat_f16f((float)sc), splat_f16f(-1024.0f * (float)sc));
    }
    // codes -m for all 8 weights (the minimum term)
    static __device__ __forceinline__ uint4 min_frag(const uint8_t *win, int kk, bool zero) {
        uint32_t sc, m;
        sc_m(win, kk, sc, m);
        const uint32_t v = zero ? 0u : splat_f16f(-(float)m);
        return make_uint4(v, v, v, v);
    }
};

// fp16 bits of 2^x for x <= 0 (0 below the subnormal range), splatted to both halves
__device__ __forceinline__ uint32_t pow2_f16x2(int x) {
    const uint32_t h = x >= -14 ? (uint32_t)(x + 15) << 10 : (x >= -24 ? 1u << (x + 24) : 0u);
    return h | (h << 16);
}

// A stage is KST K-steps (8: 256 weights of k; 4 for Q8_0). The window of a row for a stage
// holds the stage's bytes (an IQ or Q4_K super-block, or KST MXFP4 / Q8_0 blocks) from the
// 16-byte boundary at or below their start, in PCS pieces of 16 bytes.
template <class MF>
struct Win {
    static constexpr int SEG = MF::SBK == 32 ? MF::KST * MF::TS : MF::TS;
    static constexpr int PCS = (SEG + (MF::TS % 2 ? 15 : 14) + 15) / 16;
    static constexpr int BYTES = 16 * PCS;
};

// ------------------------------------------------------------------------------ kernels

__device__ __forceinline__ f16x8 as_f16x8(uint4 v) { return __builtin_bit_cast(f16x8, v); }

// 16 bytes from global memory to LDS without passing through registers: lane l of the wave
// writes lds_base + 16*l (lds_base is the same for the whole wave)
__device__ __forceinline__ void dma16(const void *g, uint8_t *lds_base) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)lds_base, 16, 0, 0);
}

// Tile shape of the grouped GEMM: a block owns one M-tile (up to 64 picks of a slot, in 16-row
// pick blocks) and RPB weight rows per matrix. Each of the 4 waves takes NB blocks of 16 rows in
// each of its NM matrices (gate and up together for MODE 0, so the activation sees both) and
// every pick block: per K-step it reads one activation fragment per pick block, decodes NM*NB
// weight fragments and issues up to 4*NM*NB MFMAs.
template <class MF, int MODE>
struct GmShape {
    static constexpr int NM = MODE == 0 ? 2 : 1;
    // MODE 2 (dense matmul) uses narrower N-blocks than MODE 1 so one matrix still fills the chip
    static constexpr int NB = (MODE == 1 ? 4 : 2) / (MF::HAS_MIN ? 2 : 1);  // a second accumulator set for the minimum
    static constexpr int RPW = 16 * NB, RPB = 4 * RPW;
    static constexpr int A_BYTES = MF::KST * 4 * 64 * 16;           // one stage of activations
    static constexpr int W_BYTES = NM * RPB * Win<MF>::BYTES;       // one stage of weight windows
    static constexpr size_t lds_bytes() { return ((MF::LDS + 15) & ~15) + A_BYTES + W_BYTES; }
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
__global__ __launch_bounds__(256, 2) void k_gmm(const MfArgs a) {
    using S = GmShape<MF, MODE>;
    using W = Win<MF>;
    constexpr int NM = S::NM, NB = S::NB, KST = MF::KST;
    constexpr bool POW2 = MF::SCALE == 1, STEP = MF::SCALE == 2, MIN = MF::HAS_MIN;
    constexpr int NA = MIN ? NB : 1;  // accumulator sets of the minimum term
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t *tab = smem;
    uint8_t *As = smem + ((MF::LDS + 15) & ~15);
    uint8_t *Ws = As + S::A_BYTES;
    const int n_nb = (a.n + S::RPB - 1) / S::RPB;
    // blocks go to XCDs round-robin; block b of each run of 8*n_nb takes M-tile 8*run + b%8 and
    // N-block b/8, so an M-tile's N-blocks share an XCD (and its L2 copy of the activations)
    const int run = blockIdx.x / (8 * n_nb), b = blockIdx.x - run * 8 * n_nb;
    const int mt = run * 8 + (b & 7);
    if (mt >= *a.n_tiles) return;  // whole block exits before any barrier
    const int nblk = b >> 3;
    const MfTile tile = a.tiles[mt];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, grp = lane >> 4, l16 = lane & 15;
    const int mbs = (tile.m + 15) >> 4;
    MF::fill(tab, tid, 256);

    // the activation row this lane copies: pick block `wave`, row l16, k-group grp
    const bool stager = wave < mbs;
    const int apos = tile.pos0 + min(16 * wave + l16, tile.m - 1);
    const uint16_t *asrc = a.a16 + (int64_t)(a.rows ? a.rows[apos] : apos) * a.lda + 8 * grp;

    // row r of the block (r < NM*RPB: matrix r / RPB, row nblk*RPB + r % RPB; rows past n read row 0)
    auto row_ptr = [&](int r) -> const uint8_t * {
        const int m = r / S::RPB, n = nblk * S::RPB + (r - m * S::RPB);
        const int64_t roff = (int64_t)(n < a.n ? n : 0) * a.row_bytes;
        return (m == 0 ? a.w0 + (int64_t)tile.slot * a.s0 : a.w1 + (int64_t)tile.slot * a.s1) + roff;
    };

    const int n_ks = a.k / 32, n_st = (n_ks + KST - 1) / KST;
    f32x4 acc[NM][NB][4];
    f32x4 accm[NM][NA][4];  // minimum term (Q4_K)
    float rs[NM][NB];     // running scale (f16 scales) ...
    int rb[NM][NB];       // ... or running base exponent (MXFP4)
    float rsm[NM][NA];    // running dmin (Q4_K)
    uint32_t lrow[NM][NB];  // this lane's window row within the block's windows
    uintptr_t lptr[NM][NB]; // this lane's row in global memory (its alignment gives the shift)
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int q = 0; q < NB; q++) {
            rs[m][q] = 1.f;
            rb[m][q] = 0;
            lrow[m][q] = m * S::RPB + wave * S::RPW + 16 * q + l16;
            lptr[m][q] = (uintptr_t)row_ptr(lrow[m][q]);
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                acc[m][q][mb] = f32x4{0, 0, 0, 0};
                asm volatile("" : "+v"(acc[m][q][mb]));  // see accm below
            }
        }
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int q = 0; q < NA; q++) {
            rsm[m][q] = 1.f;
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                accm[m][q][mb] = f32x4{0, 0, 0, 0};
                // the compiler must not treat the four elements as one value from here on: with
                // that assumption it fed later MFMAs three stale copies (wrong rows 1-3 of each
                // 4-row group); the empty asm emits nothing
                asm volatile("" : "+v"(accm[m][q][mb]));
            }
        }

    const int st_lo = a.split_st ? blockIdx.y * a.split_st : 0;
    const int st_hi = a.split_st ? min(n_st, st_lo + a.split_st) : n_st;
    for (int st = st_lo; st < st_hi; st++) {
        if (st != st_lo) __syncthreads();  // every wave is done with the previous stage's LDS
        const int nk = min(KST, n_ks - st * KST);              // K-steps in this stage
        const int seg = MF::SBK == 32 ? MF::TS * nk : MF::TS;  // bytes of a row in this stage
        if (stager) {
#pragma unroll
            for (int kk = 0; kk < KST; kk++)
                if (kk < nk) dma16(asrc + (st * KST + kk) * 32, As + ((kk * 4 + wave) * 64) * 16);
        }
        constexpr int NP = NM * S::RPB * W::PCS;  // pieces of the block's windows, a multiple of 64
#pragma unroll
        for (int t = 0; t < (NP + 255) / 256; t++) {
            const int i = tid + 256 * t, r = i / W::PCS, p = i - r * W::PCS;
            if (i >= NP) break;  // uniform across the wave
            const uint8_t *o = row_ptr(r) + (int64_t)W::SEG * st;
            const uint8_t *base = (const uint8_t *)((uintptr_t)o & ~(uintptr_t)15);
            if (base + 16 * p < o + seg) dma16(base + 16 * p, Ws + (256 * t + 64 * wave) * 16);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();

        // this lane's windows
        const uint8_t *win[NM][NB];
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int q = 0; q < NB; q++)
                win[m][q] = Ws + lrow[m][q] * W::BYTES + ((lptr[m][q] + (uintptr_t)W::SEG * st) & 15);

        bool zero[NM][NB], zerom[NM][NA];
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
                    int base = 0;
#pragma unroll
                    for (int kk = 0; kk < KST; kk++)
                        if (kk < nk) base = max(base, (int)MF::expo(win[m][q], kk));
                    if (st > st_lo && base != rb[m][q]) {
#pragma unroll
                        for (int mb = 0; mb < 4; mb++)
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
                    const float d = MF::scale(win[m][q]);
                    zero[m][q] = d == 0.f;
                    if (d != 0.f) {
                        const float ratio = __fdividef(rs[m][q], d);
#pragma unroll
                        for (int mb = 0; mb < 4; mb++) acc[m][q][mb] *= ratio;
                        rs[m][q] = d;
                    }
                    if constexpr (MIN) {
                        const float dm = MF::dmin(win[m][q]);
                        zerom[m][q] = dm == 0.f;
                        if (dm != 0.f) {
                            const float ratio = __fdividef(rsm[m][q], dm);
#pragma unroll
                            for (int mb = 0; mb < 4; mb++) accm[m][q][mb] *= ratio;
                            rsm[m][q] = dm;
                        }
                    }
                }
        }

#pragma unroll
        for (int kk = 0; kk < KST; kk++) {
            if (kk >= nk) break;
            if constexpr (STEP) {
                // a scale per K-step: move each accumulator onto it
#pragma unroll
                for (int m = 0; m < NM; m++)
#pragma unroll
                    for (int q = 0; q < NB; q++) {
                        const float d = MF::step_scale(win[m][q], kk);
                        zero[m][q] = d == 0.f;
                        if (d != 0.f) {
                            const float ratio = __fdividef(rs[m][q], d);
#pragma unroll
                            for (int mb = 0; mb < 4; mb++) acc[m][q][mb] *= ratio;
                            rs[m][q] = d;
                        }
                    }
            }
            f16x8 bf[NM][NB], bm[NM][NA];
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int q = 0; q < NA; q++)
                    if constexpr (MIN) bm[m][q] = as_f16x8(MF::min_frag(win[m][q], kk, zerom[m][q]));
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int q = 0; q < NB; q++) {
                    if constexpr (POW2)
                        bf[m][q] = as_f16x8(MF::frag_mx(win[m][q], kk, grp, tab, pow2_f16x2((int)MF::expo(win[m][q], kk) - rb[m][q])));
                    else
                        bf[m][q] = as_f16x8(MF::frag(win[m][q], kk, grp, tab, zero[m][q]));
                }
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                if (mb >= mbs) break;
                const f16x8 av = *(const f16x8 *)(As + ((kk * 4 + mb) * 64 + lane) * 16);
#pragma unroll
                for (int m = 0; m < NM; m++)
#pragma unroll
                    for (int q = 0; q < NB; q++) {
                        acc[m][q][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bf[m][q], acc[m][q][mb], 0, 0, 0);
                        if constexpr (MIN) accm[m][q][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bm[m][q], accm[m][q][mb], 0, 0, 0);
                    }
            }
        }
    }

    // epilogue: lane holds picks 16*mb + 4*grp + i (i < 4) of weight row n (block q)
    float fs[NM][NB];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int q = 0; q < NB; q++) fs[m][q] = POW2 ? ldexpf(1.0f, rb[m][q] - 128) : rs[m][q];
#pragma unroll
    for (int mb = 0; mb < 4; mb++) {
        if (mb >= mbs) break;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 16 * mb + 4 * grp + i;
            if (r >= tile.m) continue;
            const int pos = tile.pos0 + r;
            const float sa = a.ascale[a.rows ? a.rows[pos] : pos];
            const int pick = a.pile_pick ? a.pile_pick[pos] : pos;
#pragma unroll
            for (int q = 0; q < NB; q++) {
                const int n = nblk * S::RPB + wave * S::RPW + 16 * q + l16;
                if (n >= a.n) continue;
                float v[NM];
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    v[m] = acc[m][q][mb][i] * fs[m][q];
                    if constexpr (MIN) v[m] += accm[m][q][mb][i] * rsm[m][q];
                    v[m] *= sa;
                }
                if constexpr (MODE == 0) {
                    float g = v[0], u = v[NM - 1], o;
                    if (a.act == CW_ACT_SILU) {
                        o = g / (1.0f + expf(-g)) * u;
                    } else {
                        const uint32_t e = a.ids[pick];
                        if (a.bias0) g += a.bias0[(int64_t)e * a.n + n];
                        if (a.bias1) u += a.bias1[(int64_t)e * a.n + n];
                        g = fminf(g, a.limit);
                        u = fminf(fmaxf(u, -a.limit), a.limit);
                        o = (u + 1.0f) * (g * (1.0f / (1.0f + expf(-(g * a.alpha)))));
                    }
                    a.h[(int64_t)pos * a.ldh + n] = o;
                } else {
                    a.dn[blockIdx.y * a.split_stride + (int64_t)pick * a.n + n] = v[0];
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------ helpers

// One block: histogram of slots, exclusive scans, scatter of picks into per-slot piles, tiles.
// Each thread reads its (up to) PILE_PER slots of a chunk into registers before using any, so
// the loads overlap; the order of picks inside a pile does not matter (every pick's outputs are
// computed independently of the other rows of its tile).
constexpr int PILE_PER = 16;
__global__ __launch_bounds__(1024) void k_piles(const uint32_t *slots, int TK, int K, int n_slots, int *pile_pick,
                                                 int *pile_tok, MfTile *tiles, int *n_tiles) {
    __shared__ int cnt[1024], off[1024], toff[1024], cur[1024];
    const int tid = threadIdx.x;
    cnt[tid] = 0;
    cur[tid] = 0;
    __syncthreads();
    for (int c0 = 0; c0 < TK; c0 += 1024 * PILE_PER) {
        uint32_t v[PILE_PER];
#pragma unroll
        for (int q = 0; q < PILE_PER; q++) {
            const int i = c0 + q * 1024 + tid;
            v[q] = i < TK ? slots[i] : 0xFFFFFFFFu;
        }
#pragma unroll
        for (int q = 0; q < PILE_PER; q++)
            if (v[q] < (uint32_t)n_slots) atomicAdd(&cnt[v[q]], 1);
    }
    __syncthreads();
    // inclusive scans of counts and tile counts (Hillis-Steele over 1024 entries)
    const int c = tid < n_slots ? cnt[tid] : 0;
    const int tc = (c + MF_MT - 1) / MF_MT;
    off[tid] = c;
    toff[tid] = tc;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        const int x = tid >= d ? off[tid - d] : 0, y = tid >= d ? toff[tid - d] : 0;
        __syncthreads();
        off[tid] += x;
        toff[tid] += y;
        __syncthreads();
    }
    const int my_off = off[tid] - c, my_toff = toff[tid] - tc;
    if (tid == 1023) *n_tiles = toff[1023];
    __syncthreads();
    off[tid] = my_off;
    __syncthreads();
    if (tid < n_slots)
        for (int q = 0; q < tc; q++) tiles[my_toff + q] = MfTile{tid, my_off + q * MF_MT, min(MF_MT, c - q * MF_MT), 0};
    for (int c0 = 0; c0 < TK; c0 += 1024 * PILE_PER) {
        uint32_t v[PILE_PER];
#pragma unroll
        for (int q = 0; q < PILE_PER; q++) {
            const int i = c0 + q * 1024 + tid;
            v[q] = i < TK ? slots[i] : 0xFFFFFFFFu;
        }
#pragma unroll
        for (int q = 0; q < PILE_PER; q++) {
            const int i = c0 + q * 1024 + tid;
            if (v[q] < (uint32_t)n_slots) {
                const int pos = off[v[q]] + atomicAdd(&cur[v[q]], 1);
                pile_pick[pos] = i;
                pile_tok[pos] = i / K;
            }
        }
    }
}

// One wave per row, the row held in registers (NV float4 per lane, k <= 256*NV): scale =
// 2^(15 - e) with max|x| in [2^(e-1), 2^e) keeps the row's largest value in [2^14, 2^15) of
// fp16; ascale receives 1/scale.
template <int NV>
__global__ __launch_bounds__(256) void k_pack_f16(const float *x, int rows, int k, int ldx, uint16_t *a16, float *ascale) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + (int64_t)row * ldx;
    float4 v[NV];
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int c = 4 * lane + 256 * i;
        v[i] = c < k ? *(const float4 *)(xr + c) : make_float4(0.f, 0.f, 0.f, 0.f);
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

// one thread per 4 outputs of a token: the weighted sum of its K picks' rows, bias added per pick
__global__ __launch_bounds__(256) void k_combine(const float *dn, const float *w, const float *bias, const uint32_t *ids, int K,
                                                 int H, float *out) {
    const int t = blockIdx.y, j = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (j >= H) return;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int e = 0; e < K; e++) {
        const int64_t pick = (int64_t)t * K + e;
        float4 d = *(const float4 *)(dn + pick * H + j);
        if (bias) {
            const float4 b = *(const float4 *)(bias + (int64_t)ids[pick] * H + j);
            d.x += b.x; d.y += b.y; d.z += b.z; d.w += b.w;
        }
        const float we = w[pick];
        acc.x += d.x * we; acc.y += d.y * we; acc.z += d.z * we; acc.w += d.w * we;
    }
    *(float4 *)(out + (int64_t)t * H + j) = acc;
}

__global__ void k_fill_zero(float *p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0.f;
}

// ------------------------------------------------------------------------------ launchers

bool mfma_supported(int dtype) {
    return dtype == CW_IQ2_XXS || dtype == CW_IQ2_S || dtype == CW_IQ3_S || dtype == CW_MXFP4 || dtype == CW_Q4_K || dtype == CW_Q8_0;
}

int max_tiles(int TK, int n_slots) { return (TK + MF_MT - 1) / MF_MT + (n_slots < TK ? n_slots : TK); }

int mfma_piles(const uint32_t *slots, int TK, int K, int n_slots, int *pile_pick, int *pile_tok, MfTile *tiles, int *n_tiles,
               hipStream_t s) {
    if (n_slots > 1024) return set_error(CW_ENOTSUP, "mfma: %d slots (1024 max)", n_slots);
    hipLaunchKernelGGL(k_piles, dim3(1), dim3(1024), 0, s, slots, TK, K, n_slots, pile_pick, pile_tok, tiles, n_tiles);
    return check_launch("k_piles");
}

int pack_rows_f16(const float *x, int rows, int k, int ldx, uint16_t *a16, float *ascale, hipStream_t s) {
    if (rows == 0) return CW_OK;
    if (k % 4 || ldx % 4) return set_error(CW_ENOTSUP, "pack: row of %d (stride %d) is not whole float4s", k, ldx);
    const dim3 grid((rows + 3) / 4);
    const int nv = (k + 255) / 256;
#define CW_PACK(N) \
    if (nv <= N) { hipLaunchKernelGGL(k_pack_f16<N>, grid, dim3(256), 0, s, x, rows, k, ldx, a16, ascale); return check_launch("k_pack_f16"); }
    CW_PACK(2) CW_PACK(4) CW_PACK(8) CW_PACK(12) CW_PACK(16) CW_PACK(32)
#undef CW_PACK
    return set_error(CW_ENOTSUP, "pack: rows of %d above 8192", k);
}

int combine_picks(const float *dn, const float *w, const float *bias, const uint32_t *ids, int T, int K, int H, float *out,
                  hipStream_t s) {
    if (T == 0) return CW_OK;
    if (H % 4) return set_error(CW_ENOTSUP, "combine: width %d is not a multiple of 4", H);
    hipLaunchKernelGGL(k_combine, dim3((H / 4 + 255) / 256, T), dim3(256), 0, s, dn, w, bias, ids, K, H, out);
    return check_launch("k_combine");
}

int fill_zero(float *p, int64_t n, hipStream_t s) {
    if (n == 0) return CW_OK;
    int64_t b = (n + 255) / 256;
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)(b < 8192 ? b : 8192)), dim3(256), 0, s, p, n);
    return check_launch("k_fill_zero");
}

template <class MF, int MODE>
static int launch(const MfArgs &a, int tiles_max, int splits, hipStream_t s) {
    using S = GmShape<MF, MODE>;
    if (a.k % MF::SBK) return set_error(CW_ENOTSUP, "mfma: k %d is not a multiple of %d", a.k, MF::SBK);
    const int n_nb = (a.n + S::RPB - 1) / S::RPB;
    const int64_t blocks = (int64_t)((tiles_max + 7) / 8) * 8 * n_nb;
    static bool lds_set = false;  // dynamic LDS above 64 KB is opted into once per kernel
    if (!lds_set) {
        if (hipFuncSetAttribute((const void *)k_gmm<MF, MODE>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::lds_bytes()) != hipSuccess)
            return set_error(CW_EHIP, "mfma: cannot reserve %zu bytes of LDS", S::lds_bytes());
        lds_set = true;
    }
    hipLaunchKernelGGL((k_gmm<MF, MODE>), dim3((unsigned)blocks, (unsigned)splits), dim3(256), S::lds_bytes(), s, a);
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
    default: return set_error(CW_ENOTSUP, "mfma: dtype %d has no MFMA path", dtype);
    }
}

// tile i of a dense matmul: rows 64i .. 64i + 63 of x, "slot" 0
__global__ void k_dense_tiles(MfTile *tiles, int *n_tiles, int m) {
    const int nt = (m + MF_MT - 1) / MF_MT;
    for (int i = threadIdx.x; i < nt; i += blockDim.x) tiles[i] = MfTile{0, i * MF_MT, min(MF_MT, m - i * MF_MT), 0};
    if (threadIdx.x == 0) *n_tiles = nt;
}

static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

// y[i] = sum over the S partial products, in split order
__global__ void k_sum_splits(const float *part, int S, int64_t n, float *y) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float acc = part[i];
        for (int s = 1; s < S; s++) acc += part[s * n + i];
        y[i] = acc;
    }
}

// the dense GEMM's N-block rows and stage size for a format (GmShape<MF, 2>)
static void dense_shape(int dtype, int &rpb, int &kst) {
    rpb = dtype == CW_Q4_K ? 64 : 128;
    kst = dtype == CW_Q8_0 ? 4 : 8;
}
// K splits: enough blocks to cover the chip twice, at least one stage each
static int dense_splits(int dtype, int64_t m, int64_t n, int64_t k, int &split_st) {
    int rpb, kst;
    dense_shape(dtype, rpb, kst);
    const int64_t blocks = (m + MF_MT - 1) / MF_MT * ((n + rpb - 1) / rpb);
    const int n_st = (int)((k / 32 + kst - 1) / kst);
    int S = (int)((512 + blocks - 1) / blocks);
    if (S > n_st) S = n_st;
    if (S < 1) S = 1;
    split_st = (n_st + S - 1) / S;
    return (n_st + split_st - 1) / split_st;
}

size_t mfma_dense_workspace(int dtype, int64_t m, int64_t n, int64_t k) {
    int split_st;
    const int S = dense_splits(dtype, m, n, k, split_st);
    return al256(m * k * 2) + al256(m * 4) + al256((m + MF_MT - 1) / MF_MT * sizeof(MfTile)) + al256(4) +
           (S > 1 ? al256((size_t)S * m * n * 4) : 0);
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
    MfTile *tiles = (MfTile *)p; p += al256((size_t)(m + MF_MT - 1) / MF_MT * sizeof(MfTile));
    int *n_tiles = (int *)p; p += al256(4);
    float *part = S > 1 ? (float *)p : nullptr;
    hipLaunchKernelGGL(k_dense_tiles, dim3(1), dim3(256), 0, s, tiles, n_tiles, m);
    int rc = check_launch("k_dense_tiles");
    if (rc) return rc;
    if ((rc = pack_rows_f16(x, m, k, k, x16, xs, s))) return rc;
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
    if ((rc = by_fmt<2>(dtype, a, (m + MF_MT - 1) / MF_MT, S, s))) return rc;
    if (S == 1) return CW_OK;
    const int64_t total = (int64_t)m * n, blocks = (total + 255) / 256;
    hipLaunchKernelGGL(k_sum_splits, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s, part, S, total, y);
    return check_launch("k_sum_splits");
}

int mfma_gateup(int dtype, const MfArgs &a, int tiles_max, hipStream_t s) { return by_fmt<0>(dtype, a, tiles_max, 1, s); }
int mfma_down(int dtype, const MfArgs &a, int tiles_max, hipStream_t s) { return by_fmt<1>(dtype, a, tiles_max, 1, s); }

}  // namespace cw
