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

constexpr int A_LD = 256 + 8;   // halves per staged activation row (padding breaks LDS bank conflicts)

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
// Per format: TS bytes per block, SBK weights per scale unit, LDS table bytes, the per-lane raw
// data of one scale unit, the fp16 fragment (8 codes) of K-step ks for lane group grp (weights
// 8*grp..8*grp+7 of the step's 32), and the unit's f32 scale.

struct MIQ2_XXS {
    static constexpr int TS = 66, SBK = 256, LDS = 256 * 16 + 128 * 16;
    struct Raw { uint32_t d; uint2 q[8]; };
    static __device__ void fill(uint8_t *lds, int tid, int nt) {
        copy_tab(lds, c_iq2xxs_f16, tid, nt);
        copy_tab(lds + 256 * 16, c_psigns, tid, nt);
    }
    static __device__ __forceinline__ void load(Raw &r, const uint8_t *row, int u) {
        const uint8_t *b = row + (int64_t)TS * u;
        r.d = ld_u16(b);
#pragma unroll
        for (int i = 0; i < 8; i++) r.q[i] = ld_u64(b + 2 + 8 * i);
    }
    static __device__ __forceinline__ uint4 frag(const Raw &r, int ks, int grp, const uint8_t *lds) {
        const uint4 *g = (const uint4 *)lds, *sg = (const uint4 *)(lds + 256 * 16);
        const uint32_t gi = (r.q[ks].x >> (8 * grp)) & 0xFF;
        const uint32_t si = (r.q[ks].y >> (7 * grp)) & 127;
        const uint32_t sc = 2 * (r.q[ks].y >> 28) + 1;
        return scale4(xor4(g[gi], sg[si]), splat_f16((int)sc));
    }
    static __device__ __forceinline__ float scale(const Raw &r) { return h2f(r.d) * 0.125f; }
};

struct MIQ2_S {
    static constexpr int TS = 82, SBK = 256, LDS = 1024 * 16 + 256 * 16;
    struct Raw { uint32_t d; uint32_t qs[8]; uint32_t sg[8]; uint2 qh; uint2 sc; };
    static __device__ void fill(uint8_t *lds, int tid, int nt) {
        copy_tab(lds, c_iq2s_f16, tid, nt);
        copy_tab(lds + 1024 * 16, c_signs, tid, nt);
    }
    static __device__ __forceinline__ void load(Raw &r, const uint8_t *row, int u) {
        const uint8_t *b = row + (int64_t)TS * u;
        r.d = ld_u16(b);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            r.qs[i] = ld_u32(b + 2 + 4 * i);
            r.sg[i] = ld_u32(b + 34 + 4 * i);
        }
        r.qh = ld_u64(b + 66);
        r.sc = ld_u64(b + 74);
    }
    static __device__ __forceinline__ uint32_t byte8(uint2 v, int i) { return ((i < 4 ? v.x : v.y) >> (8 * (i & 3))) & 0xFF; }
    static __device__ __forceinline__ uint4 frag(const Raw &r, int ks, int grp, const uint8_t *lds) {
        const uint4 *g = (const uint4 *)lds, *sg = (const uint4 *)(lds + 1024 * 16);
        const uint32_t qh = byte8(r.qh, ks);
        const uint32_t gi = ((r.qs[ks] >> (8 * grp)) & 0xFF) | (((qh >> (2 * grp)) & 3) << 8);
        const uint32_t si = (r.sg[ks] >> (8 * grp)) & 0xFF;
        const uint32_t sc = 2 * ((byte8(r.sc, ks) >> (4 * (grp >> 1))) & 0xF) + 1;
        return scale4(xor4(g[gi], sg[si]), splat_f16((int)sc));
    }
    static __device__ __forceinline__ float scale(const Raw &r) { return h2f(r.d) * 0.125f; }
};

struct MIQ3_S {
    static constexpr int TS = 110, SBK = 256, LDS = 512 * 8 + 256 * 16;
    struct Raw { uint32_t d; uint32_t qs[8]; uint2 qh; uint32_t sg[8]; uint32_t sc; };
    static __device__ void fill(uint8_t *lds, int tid, int nt) {
        copy_tab(lds, c_iq3s_f16, tid, nt);   // entry i as 4 halves at byte 8*i
        copy_tab(lds + 512 * 8, c_signs, tid, nt);
    }
    static __device__ __forceinline__ void load(Raw &r, const uint8_t *row, int u) {
        const uint8_t *b = row + (int64_t)TS * u;
        r.d = ld_u16(b);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            r.qs[i] = 0;  // filled per lane group below
            r.sg[i] = ld_u32(b + 74 + 4 * i);
        }
        r.qh = ld_u64(b + 66);
        r.sc = ld_u32(b + 106);
    }
    // the two grid bytes of lane group grp in sub-block i sit at 2 + 8*i + 2*grp
    static __device__ __forceinline__ void load_grp(Raw &r, const uint8_t *row, int u, int grp) {
        const uint8_t *b = row + (int64_t)TS * u;
#pragma unroll
        for (int i = 0; i < 8; i++) r.qs[i] = ld_u16(b + 2 + 8 * i + 2 * grp);
    }
    static __device__ __forceinline__ uint4 frag(const Raw &r, int ks, int grp, const uint8_t *lds) {
        const uint2 *g = (const uint2 *)lds;
        const uint4 *sg = (const uint4 *)(lds + 512 * 8);
        const uint32_t qh = ((ks < 4 ? r.qh.x : r.qh.y) >> (8 * (ks & 3))) & 0xFF;
        const uint32_t i0 = (r.qs[ks] & 0xFF) | (((qh >> (2 * grp)) & 1) << 8);
        const uint32_t i1 = (r.qs[ks] >> 8) | (((qh >> (2 * grp + 1)) & 1) << 8);
        const uint2 a = g[i0], c = g[i1];
        const uint32_t si = (r.sg[ks] >> (8 * grp)) & 0xFF;
        const uint32_t sc = 1 + 2 * ((r.sc >> (4 * ks)) & 0xF);   // nibble ks of the 4 scale bytes
        return scale4(xor4(make_uint4(a.x, a.y, c.x, c.y), sg[si]), splat_f16((int)sc));
    }
    static __device__ __forceinline__ float scale(const Raw &r) { return h2f(r.d); }
};

struct MMXFP4 {
    static constexpr int TS = 17, SBK = 32, LDS = 16;
    struct Raw { uint32_t e; uint2 q; };
    static __device__ void fill(uint8_t *, int, int) {}
    static __device__ __forceinline__ void load(Raw &r, const uint8_t *row, int u) {
        r.e = 0;
        r.q = make_uint2(0, 0);
        (void)row; (void)u;
    }
    // lane group grp takes the low (grp < 2) or high nibbles of bytes 8*(grp&1)..+8
    static __device__ __forceinline__ void load_grp(Raw &r, const uint8_t *row, int u, int grp) {
        const uint8_t *b = row + (int64_t)TS * u;
        r.e = b[0];
        r.q = ld_u64(b + 1 + 8 * (grp & 1));
    }
    static __device__ __forceinline__ uint32_t pair(uint32_t w, int b) {
        // doubled-E2M1 codes in bytes b and b+1 of w, as two fp16 integers
        const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)kv_mxfp4((w >> (8 * b)) & 0xF));
        const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)kv_mxfp4((w >> (8 * b + 8)) & 0xF));
        return lo | (hi << 16);
    }
    static __device__ __forceinline__ uint4 frag(const Raw &r, int ks, int grp, const uint8_t *) {
        (void)ks;
        const int sh = 4 * (grp >> 1);
        const uint32_t a = (r.q.x >> sh) & 0x0F0F0F0F, b = (r.q.y >> sh) & 0x0F0F0F0F;
        return make_uint4(pair(a, 0), pair(a, 2), pair(b, 0), pair(b, 2));
    }
    static __device__ __forceinline__ float scale(const Raw &r) { return e8m0_half(r.e); }
};

template <class MF, typename = void>
struct has_grp_load { static constexpr bool value = false; };
template <class MF>
struct has_grp_load<MF, decltype((void)&MF::load_grp, void())> { static constexpr bool value = true; };

// ------------------------------------------------------------------------------ kernels

__device__ __forceinline__ f16x8 as_f16x8(uint4 v) { return __builtin_bit_cast(f16x8, v); }

// MODE 0: gate and up (two matrices) with the activation, hidden rows written in pile order.
// MODE 1: down, the pick's routing weight (and bias) applied, accumulated into out[token].
// A block owns one M-tile (up to 64 picks of a slot) and NTB consecutive N-tiles of 64 weight
// rows; k streams through LDS in chunks of 256 (8 K-steps). Latency is hidden by occupancy
// (several blocks per CU).
template <class MF, int MODE, int NTB>
__global__ __launch_bounds__(256) void k_mfma(const MfArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t *tab = smem;
    _Float16 *As = (_Float16 *)(smem + ((MF::LDS + 15) & ~15));
    constexpr int UPC = 256 / MF::SBK;   // scale units per chunk
    constexpr int KPU = MF::SBK / 32;    // K-steps per scale unit
    const int n_nt = (a.n + MF_NT - 1) / MF_NT;
    const int groups = (n_nt + NTB - 1) / NTB;
    // blocks go to XCDs round-robin; block b of each run of 8*groups takes M-tile 8*run + b%8
    // and N-group b/8, so an M-tile's N-groups share an XCD and every XCD gets valid tiles
    const int run = blockIdx.x / (8 * groups), b = blockIdx.x - run * 8 * groups;
    const int mt = run * 8 + (b & 7);
    if (mt >= *a.n_tiles) return;  // whole block exits before any barrier
    const int nt_begin = (b >> 3) * NTB, nt_end = min(nt_begin + NTB, n_nt);
    const MfTile tile = a.tiles[mt];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, grp = lane >> 4, l16 = lane & 15;
    MF::fill(tab, tid, 256);
    const int n_ks = a.k / 32;

    for (int nt = nt_begin; nt < nt_end; nt++) {
        const int n = nt * MF_NT + wave * 16 + l16;   // this lane's weight row
        const bool nv = n < a.n;
        const uint8_t *r0 = a.w0 + (int64_t)tile.slot * a.s0 + (int64_t)(nv ? n : 0) * a.row_bytes;
        const uint8_t *r1 = MODE == 0 ? a.w1 + (int64_t)tile.slot * a.s1 + (int64_t)(nv ? n : 0) * a.row_bytes : r0;
        f32x4 acc0[4], acc1[4];
#pragma unroll
        for (int mb = 0; mb < 4; mb++) { acc0[mb] = f32x4{0, 0, 0, 0}; acc1[mb] = f32x4{0, 0, 0, 0}; }
        for (int c0 = 0; c0 < n_ks; c0 += 8) {
            const int nks = min(8, n_ks - c0);
            __syncthreads();  // previous chunk's readers are done
            for (int idx = tid; idx < MF_MT * 32; idx += 256) {
                const int r = idx >> 5, c = idx & 31;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (r < tile.m && c < nks * 4) {
                    const int pos = tile.pos0 + r;
                    const int src = a.rows ? a.rows[pos] : pos;
                    v = *(const uint4 *)(a.a16 + (int64_t)src * a.lda + (int64_t)c0 * 32 + c * 8);
                }
                *(uint4 *)(As + r * A_LD + c * 8) = v;
            }
            typename MF::Raw raw0[UPC], raw1[UPC];
#pragma unroll
            for (int u = 0; u < UPC; u++) {
                const int unit = c0 / KPU + u;
                if (u * KPU < nks) {
                    MF::load(raw0[u], r0, unit);
                    if constexpr (has_grp_load<MF>::value) MF::load_grp(raw0[u], r0, unit, grp);
                    if constexpr (MODE == 0) {
                        MF::load(raw1[u], r1, unit);
                        if constexpr (has_grp_load<MF>::value) MF::load_grp(raw1[u], r1, unit, grp);
                    }
                }
            }
            __syncthreads();
#pragma unroll
            for (int u = 0; u < UPC; u++) {
                if (u * KPU >= nks) break;
                f32x4 p0[4], p1[4];
#pragma unroll
                for (int mb = 0; mb < 4; mb++) { p0[mb] = f32x4{0, 0, 0, 0}; p1[mb] = f32x4{0, 0, 0, 0}; }
#pragma unroll
                for (int ks = 0; ks < KPU; ks++) {
                    const int kk = u * KPU + ks;
                    const f16x8 b0 = as_f16x8(MF::frag(raw0[u], ks, grp, tab));
                    f16x8 b1;
                    if constexpr (MODE == 0) b1 = as_f16x8(MF::frag(raw1[u], ks, grp, tab));
#pragma unroll
                    for (int mb = 0; mb < 4; mb++) {
                        const f16x8 av = as_f16x8(*(const uint4 *)(As + (16 * mb + l16) * A_LD + kk * 32 + 8 * grp));
                        p0[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b0, p0[mb], 0, 0, 0);
                        if constexpr (MODE == 0) p1[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b1, p1[mb], 0, 0, 0);
                    }
                }
                const float s0 = MF::scale(raw0[u]);
                const float s1 = MODE == 0 ? MF::scale(raw1[u]) : 0.f;
#pragma unroll
                for (int mb = 0; mb < 4; mb++) {
                    acc0[mb] += s0 * p0[mb];
                    if constexpr (MODE == 0) acc1[mb] += s1 * p1[mb];
                }
            }
        }

        // epilogue: lane holds rows 16*mb + 4*grp + i (i < 4) of weight row n
        if (!nv) continue;
#pragma unroll
        for (int mb = 0; mb < 4; mb++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = 16 * mb + 4 * grp + i;
                if (r >= tile.m) continue;
                const int pos = tile.pos0 + r;
                const int src = a.rows ? a.rows[pos] : pos;
                const float sa = a.ascale[src];
                const int pick = a.pile_pick[pos];
                if constexpr (MODE == 0) {
                    float g = acc0[mb][i] * sa, u = acc1[mb][i] * sa, o;
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
                    float v = acc0[mb][i] * sa;
                    if (a.bias_d) v += a.bias_d[(int64_t)a.ids[pick] * a.n + n];
                    atomicAdd(a.out + (int64_t)(pick / a.K) * a.n + n, a.w[pick] * v);
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------ helpers

// One block: histogram of slots, exclusive scans, scatter of picks into per-slot piles, tiles.
__global__ __launch_bounds__(1024) void k_piles(const uint32_t *slots, int TK, int K, int n_slots, int *pile_pick,
                                                 int *pile_tok, MfTile *tiles, int *n_tiles) {
    __shared__ int cnt[1024], off[1024], toff[1024], cur[1024];
    const int tid = threadIdx.x;
    for (int s = tid; s < 1024; s += blockDim.x) { cnt[s] = 0; cur[s] = 0; }
    __syncthreads();
    for (int i = tid; i < TK; i += blockDim.x) {
        const uint32_t s = slots[i];
        if (s < (uint32_t)n_slots) atomicAdd(&cnt[s], 1);
    }
    __syncthreads();
    // inclusive scans of counts and tile counts (Hillis-Steele over 1024 entries)
    int c = tid < n_slots ? cnt[tid] : 0;
    int tc = (c + MF_MT - 1) / MF_MT;
    off[tid] = c;
    toff[tid] = tc;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        const int a = tid >= d ? off[tid - d] : 0, b = tid >= d ? toff[tid - d] : 0;
        __syncthreads();
        off[tid] += a;
        toff[tid] += b;
        __syncthreads();
    }
    const int my_off = off[tid] - c, my_toff = toff[tid] - tc;
    if (tid == 1023) *n_tiles = toff[1023];
    __syncthreads();
    off[tid] = my_off;
    __syncthreads();
    if (tid < n_slots)
        for (int q = 0; q < tc; q++) tiles[my_toff + q] = MfTile{tid, my_off + q * MF_MT, min(MF_MT, c - q * MF_MT), 0};
    for (int i = tid; i < TK; i += blockDim.x) {
        const uint32_t s = slots[i];
        if (s < (uint32_t)n_slots) {
            const int pos = off[s] + atomicAdd(&cur[s], 1);
            pile_pick[pos] = i;
            pile_tok[pos] = i / K;
        }
    }
}

// one wave per row: scale = 2^(14 - floor(log2 max|x|)) keeps the row's largest value in
// [2^14, 2^15) of fp16; ascale receives 1/scale
__global__ __launch_bounds__(256) void k_pack_f16(const float *x, int rows, int k, int ldx, uint16_t *a16, float *ascale) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + (int64_t)row * ldx;
    float m = 0.f;
    for (int c = lane; c < k; c += 64) m = fmaxf(m, fabsf(xr[c]));
    m = wave_max(m);
    int ex = 0;
    if (m > 0.f && m < INFINITY) { frexpf(m, &ex); ex = 15 - ex; }  // m in [2^(e-1), 2^e)
    const float sc = ldexpf(1.0f, ex);
    uint16_t *o = a16 + (int64_t)row * k;
    for (int c = lane; c < k; c += 64) o[c] = __builtin_bit_cast(uint16_t, (_Float16)(xr[c] * sc));
    if (lane == 0) ascale[row] = ldexpf(1.0f, -ex);
}

__global__ void k_fill_zero(float *p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0.f;
}

// ------------------------------------------------------------------------------ launchers

bool mfma_supported(int dtype) { return dtype == CW_IQ2_XXS || dtype == CW_IQ2_S || dtype == CW_IQ3_S || dtype == CW_MXFP4; }

int max_tiles(int TK, int n_slots) { return (TK + MF_MT - 1) / MF_MT + (n_slots < TK ? n_slots : TK); }

int mfma_piles(const uint32_t *slots, int TK, int K, int n_slots, int *pile_pick, int *pile_tok, MfTile *tiles, int *n_tiles,
               hipStream_t s) {
    if (n_slots > 1024) return set_error(CW_ENOTSUP, "mfma: %d slots (1024 max)", n_slots);
    hipLaunchKernelGGL(k_piles, dim3(1), dim3(1024), 0, s, slots, TK, K, n_slots, pile_pick, pile_tok, tiles, n_tiles);
    return check_launch("k_piles");
}

int pack_rows_f16(const float *x, int rows, int k, int ldx, uint16_t *a16, float *ascale, hipStream_t s) {
    if (rows == 0) return CW_OK;
    hipLaunchKernelGGL(k_pack_f16, dim3((rows + 3) / 4), dim3(256), 0, s, x, rows, k, ldx, a16, ascale);
    return check_launch("k_pack_f16");
}

int fill_zero(float *p, int64_t n, hipStream_t s) {
    if (n == 0) return CW_OK;
    int64_t b = (n + 255) / 256;
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)(b < 8192 ? b : 8192)), dim3(256), 0, s, p, n);
    return check_launch("k_fill_zero");
}

template <class MF, int MODE, int NTB>
static int launch_v(const MfArgs &a, int tiles_max, hipStream_t s) {
    const size_t shmem = ((MF::LDS + 15) & ~15) + (size_t)MF_MT * A_LD * 2;
    const int n_nt = (a.n + MF_NT - 1) / MF_NT;
    const int64_t blocks = (int64_t)((tiles_max + 7) / 8) * 8 * ((n_nt + NTB - 1) / NTB);
    hipLaunchKernelGGL((k_mfma<MF, MODE, NTB>), dim3((unsigned)blocks), dim3(256), shmem, s, a);
    return check_launch("k_mfma");
}

template <class MF, int MODE>
static int launch(const MfArgs &a, int tiles_max, hipStream_t s) {
    if (a.k % 32) return set_error(CW_ENOTSUP, "mfma: k %d is not a multiple of 32", a.k);
    // short rows (down's k = expert FFN) do little work per N-tile: a block takes four
    if (a.k <= 1024) return launch_v<MF, MODE, 4>(a, tiles_max, s);
    return launch_v<MF, MODE, 1>(a, tiles_max, s);
}

template <int MODE>
static int by_fmt(int dtype, const MfArgs &a, int tiles_max, hipStream_t s) {
    switch (dtype) {
    case CW_IQ2_XXS: return launch<MIQ2_XXS, MODE>(a, tiles_max, s);
    case CW_IQ2_S: return launch<MIQ2_S, MODE>(a, tiles_max, s);
    case CW_IQ3_S: return launch<MIQ3_S, MODE>(a, tiles_max, s);
    case CW_MXFP4: return launch<MMXFP4, MODE>(a, tiles_max, s);
    default: return set_error(CW_ENOTSUP, "mfma: dtype %d has no MFMA path", dtype);
    }
}

int mfma_gateup(int dtype, const MfArgs &a, int tiles_max, hipStream_t s) { return by_fmt<0>(dtype, a, tiles_max, s); }
int mfma_down(int dtype, const MfArgs &a, int tiles_max, hipStream_t s) { return by_fmt<1>(dtype, a, tiles_max, s); }

}  // namespace cw
