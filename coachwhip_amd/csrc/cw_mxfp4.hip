// MXFP4 grouped GEMMs (the MoE layer's prefill, cw_matmul_id_grouped) on gfx950's block-scaled
// MFMA (v_mfma_scale_f32_16x16x128_f8f6f4).
//
// The weights go to the matrix cores as GGUF stores them: a lane's A operand is one MXFP4 block,
// its 16 code bytes unchanged (E2M1 codes, low nibble first) with the block's E8M0 byte as the
// lane's scale. The MFMA's A operand takes K index 32g + e from nibble e of lane group g, and a
// block's byte i holds weight i (low nibble) and weight i + 16 (high nibble): nibble e is weight
// (e >> 1) + 16 (e & 1) of the block. The activations are arranged to meet that order.
//
// Activations are f32 rows packed once per call (k_pack_fp6x3) into three FP6 (E2M3) terms per
// value: term t codes the residual the earlier terms left, each 32-value block with its own E8M0
// scale per term. The B operand of a lane is 32 FP6 codes (6 bits each, code e at bits 6e..6e+5
// of six dwords) with the lane's scale, and FP4 x FP6 issues at the FP4 rate, so the three terms
// cost 48 cycles per 16x16x128 product where fp16 MFMA needs 64, and nothing is decoded on the
// VALU. A term's scale puts the largest magnitude left in its block in (3.75, 7.5], where E2M3
// steps are at most 0.5, so what it leaves is at most 1/15 of what it started from: after three
// terms at most 1/3375 (2^-11.7) of the block's largest value (the fp16 path rounds each value to
// 2^-11 of itself).
//
// Packed activations: per row, 304 bytes per 128-wide K step (4 blocks of 32 values, the last
// step zero-filled past the row): term t of block g is 24 bytes of codes, dwords 0..3 at 96 t +
// 16 g and dwords 4, 5 at 96 t + 64 + 8 g, and the block's three scale bytes (term t at bits 8t)
// are the dword at 288 + 4 g. A lane's B operand is then one 16-byte and one 8-byte aligned load
// that land in its six operand registers, and the four lanes of a token read consecutive bytes.
#include <stdlib.h>

#include <atomic>
#include <type_traits>

#include "cw_common.h"
#include "cw_mfma.h"

namespace cw {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------------------ the pack

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef uint32_t u32x6 __attribute__((ext_vector_type(6)));

// The three-term record of one 32-value block (lo[i] = value i, hi[i] = value 16 + i) into block
// g of the step record at dst. Each term is scaled by the power of two that puts the block's
// largest remaining magnitude in (3.75, 7.5], where FP6 E2M3 (sign, 2 exponent bits with bias 1,
// 3 mantissa bits: steps of 1/8 below 2, 1/4 below 4, 1/2 up to 7.5) is exact to half a step.
// gfx950 converts a term in one instruction (`v_cvt_scalef32_2xpk16_fp6_f32`: code 2i of the
// 192-bit record from lo[i], code 2i + 1 from hi[i], each value divided by the scale and rounded
// to the nearest E2M3 value, ties to even), which is the record's element order: element e meets
// nibble e of the weight block, weight position (e >> 1) + 16 (e & 1). The residual subtracts the
// term's value as decoded by `v_cvt_scalef32_pk32_f32_fp6` (code times the scale), exactly: a
// value minus its rounding to 3 mantissa bits is representable.
__device__ __forceinline__ void fp6x3_record(f32x16 lo, f32x16 hi, uint8_t *dst, int g) {
    uint32_t sc = 0;
#pragma unroll
    for (int t = 0; t < 3; t++) {
        float m = 0.f;
#pragma unroll
        for (int e = 0; e < 16; e++) m = fmaxf(m, fmaxf(fabsf(lo[e]), fabsf(hi[e])));
        int ex = 0;
        if (m > 0.f) frexpf(m, &ex);  // m = f * 2^ex, f in [0.5, 1)
        int kk = m > 0.f ? ex - 3 : -127;
        if (m > ldexpf(7.5f, kk)) kk++;
        kk = min(max(kk, -127), 127);
        sc |= (uint32_t)(kk + 127) << (8 * t);
        const float scl = ldexpf(1.0f, kk);
        const u32x6 w = __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(lo, hi, scl);
        *(uint4 *)(dst + 96 * t + 16 * g) = make_uint4(w[0], w[1], w[2], w[3]);
        *(uint2 *)(dst + 96 * t + 64 + 8 * g) = make_uint2(w[4], w[5]);
        if (t < 2) {
            const f32x32 q = __builtin_amdgcn_cvt_scalef32_pk32_f32_fp6(w, scl);  // element 2i: lo[i], 2i + 1: hi[i]
#pragma unroll
            for (int e = 0; e < 16; e++) {
                lo[e] -= q[2 * e];
                hi[e] -= q[2 * e + 1];
            }
        }
    }
    *(uint32_t *)(dst + 288 + 4 * g) = sc;
}
// a zero record (codes and scale bytes 0), for blocks past a row
__device__ __forceinline__ void fp6x3_zero(uint8_t *dst, int g) {
#pragma unroll
    for (int t = 0; t < 3; t++) {
        *(uint4 *)(dst + 96 * t + 16 * g) = make_uint4(0u, 0u, 0u, 0u);
        *(uint2 *)(dst + 96 * t + 64 + 8 * g) = make_uint2(0u, 0u);
    }
    *(uint32_t *)(dst + 288 + 4 * g) = 0u;
}

// One lane per (row, 32-value block).
__global__ __launch_bounds__(256) void k_pack_fp6x3(const float *x, int rows, int k, int ldx, uint8_t *out) {
    const int nb = k / 32, nbp = (nb + 3) & ~3;  // blocks, and block records per row (whole steps)
    const int64_t n = (int64_t)rows * nbp;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const int64_t row = i / nbp;
        const int j = (int)(i - row * nbp);
        uint8_t *dst = out + row * (int64_t)(nbp / 4) * 304 + (j >> 2) * 304;
        const int g = j & 3;
        if (j >= nb) {  // past the row: zero codes and scale bytes
            fp6x3_zero(dst, g);
            continue;
        }
        const float4 *src = (const float4 *)(x + row * ldx + 32 * j);
        f32x16 lo, hi;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float4 f = src[c], h = src[4 + c];
            lo[4 * c] = f.x;
            lo[4 * c + 1] = f.y;
            lo[4 * c + 2] = f.z;
            lo[4 * c + 3] = f.w;
            hi[4 * c] = h.x;
            hi[4 * c + 1] = h.y;
            hi[4 * c + 2] = h.z;
            hi[4 * c + 3] = h.w;
        }
        fp6x3_record(lo, hi, dst, g);
    }
}

// ------------------------------------------------------------------------------ the GEMM

// 16 bytes from global memory (base + off, base a wave-uniform 16-byte aligned address) to LDS,
// lane l writing lds_base + 16 l. Issued as inline asm: the kernel counts its vector memory
// operations itself (a running count, and the count after each batch it will need) and waits for
// exactly the ones it needs, which the compiler, not seeing loads it did not issue, could not do.
// It takes a uniform 64-bit base and 32-bit lane offsets, so that no lane holds a 64-bit address.
// lds_base is an LDS address, the same for the whole wave.
__device__ __forceinline__ void gx_dma16(const uint8_t *base, uint32_t off, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(base),
                 "s"(__builtin_amdgcn_readfirstlane(lds_base)) : "memory", "m0");
}
// the same for 4 bytes (base 4-byte aligned; lane l writes lds_base + 4 l)
__device__ __forceinline__ void gx_dma4(const uint8_t *base, uint32_t off, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" : : "v"(off), "s"(base),
                 "s"(__builtin_amdgcn_readfirstlane(lds_base)) : "memory", "m0");
}
// s_waitcnt vmcnt(n) for n in {0, 3, 4, 5} (a stage's wait: the window loads of one stage in flight)
__device__ __forceinline__ void gx_wait_stage(int n) {
    if (n == 5) asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
    else if (n == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else if (n == 3) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
// s_waitcnt vmcnt(n) for a run-time n (the instruction takes an immediate; above 63 it waits for
// more than asked, never less)
__device__ __forceinline__ void gx_wait_vm(int n) {
#define CW_VM(N) case N: asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory"); break;
#define CW_VM8(B) CW_VM(B) CW_VM(B + 1) CW_VM(B + 2) CW_VM(B + 3) CW_VM(B + 4) CW_VM(B + 5) CW_VM(B + 6) CW_VM(B + 7)
    switch (n < 0 ? 0 : n > 63 ? 63 : n) {
        CW_VM8(0) CW_VM8(8) CW_VM8(16) CW_VM8(24) CW_VM8(32) CW_VM8(40) CW_VM8(48) CW_VM8(56)
    }
#undef CW_VM8
#undef CW_VM
}

// A block has 8 waves: 4 row groups of RW weight rows (of each matrix: gate and up for MODE 0) by
// 2 halves of the tile's 16-token blocks. A stage is one 128-wide K step. The weight bytes of a
// stage go to LDS by direct loads, three stages ahead (three buffers). From GGUF rows (L = 0) a
// row's window is the 6 16-byte pieces holding its 4 blocks (68 bytes at any offset): for the
// gpt-oss shape 384 short runs 1,530 bytes apart per stage. From rows in groups of 16 (L = 1,
// CW_MXFP4_R16: a group's blocks of one stage side by side) a stage is 24 runs of 1,088 bytes,
// 16-byte aligned, which HBM serves faster (a loads-only microbenchmark of config 4's gate/up
// windows on MI355X: 190 against 273 us; with the MFMAs and activation loads: 278 against 352),
// and lands in LDS as rows of 68 bytes (17 cb for a last stage of cb < 4 blocks), each matrix's
// groups from whole 1 KB loads of their own. The activation operands of a
// stage (token block t: its 16 tokens' 304-byte step records, whole) go to LDS by direct loads
// too, two stages ahead (two buffers), issued by the first waves. Each wave reads the operands of
// the next stage from LDS while it computes the current one: a token block's activation operands
// right after that block's MFMAs, the weight operands at the end of the stage, so that their
// latency hides behind the matrix work. One barrier per stage publishes every wave's loads (each
// wave first waits for exactly its own).
template <int MODE, int L = 0>
struct GxShape {
    static constexpr int NW = 8, NT = 64 * NW;
    static constexpr int NM = MODE == 0 ? 2 : 1;      // matrices (gate, up) per block
    static constexpr int RW = MODE == 0 ? 48 : 96;    // rows per row group per matrix
    static constexpr int FR = RW / 16;                // fragments per wave per matrix
    static constexpr int NF = NM * FR;                // fragments per wave
    static constexpr int RPB = 4 * RW;                // rows per matrix per block
    static constexpr int PCS = 6;                     // pieces per row window (L = 0)
    static constexpr int WROWS = NM * RPB;
    // L = 1: GPM row groups of 16 per matrix, 68 pieces each per full stage, a matrix's MI window
    // loads in an LDS region of its own
    static constexpr int GPM = RPB / 16;
    static constexpr int MI = (GPM * 68 + 63) / 64;
    static constexpr int W_INST = L ? NM * MI : WROWS * PCS / 64;  // window loads per stage (wave instructions)
    static constexpr int NJW = (W_INST + NW - 1) / NW;
    static constexpr int W_BYTES = W_INST * 1024;
    static constexpr int WDEPTH = 3;
    // a token block's operands of a stage: its 16 tokens' 304-byte step records side by side
    // (4,864 bytes), padded to the five 1 KB direct loads that bring them
    static constexpr int TB_BYTES = 5 * 1024;
    static constexpr int A_BYTES = MF_MB * TB_BYTES;
    // gate/up: the item's bias rows (gate, then up: RPB floats each) for the epilogue
    static constexpr int BIAS_OFF = WDEPTH * W_BYTES + 2 * A_BYTES;
    static constexpr int BIAS_BYTES = MODE == 0 ? NM * RPB * 4 : 0;
    static constexpr size_t LDS = (size_t)BIAS_OFF + BIAS_BYTES;
    // gate/up's hidden-row staging: rows of RPB floats 4 apart in banks (a 16-byte write per lane
    // of 16 tokens hits 64 distinct banks)
    static constexpr int HST = RPB + 4;
    static_assert(RPB * PCS % 64 == 0, "a window load lies in one matrix");
    static_assert(RPB % 16 == 0, "an N-block is whole row groups");
    static_assert(LDS <= 160 * 1024, "the scaled GEMM's LDS does not fit");
};


// One work item (M-tile x N-block) of one wave, NTB of the tile's token blocks from tb0; L is the
// weights' layout (0: GGUF rows, 1: rows in groups of 16).
template <int MODE, int NTB, int L>
__device__ __forceinline__ void gx_item(const MfArgs &a, const MfTile &tile, int nb, int mbs, int tb0, int wave, int lane,
                                        uint8_t *smem, uint32_t lds0) {
    using S = GxShape<MODE, L>;
    constexpr int NB = NTB > 0 ? NTB : 1;
    const int grp = lane >> 4, l16 = lane & 15, rg = wave & 3;
    const int nblk = a.k / 32, n_st = (nblk + 3) / 4;
    uint8_t *const Wb = smem;
    uint8_t *const Ab = smem + S::WDEPTH * S::W_BYTES;
    const uint32_t Al = lds0 + S::WDEPTH * S::W_BYTES;

    const uint8_t *wb0 = a.w0 + (int64_t)tile.slot * a.s0;
    const uint8_t *wb1 = S::NM > 1 ? a.w1 + (int64_t)tile.slot * a.s1 : wb0;
    // L = 0: rounded down to 16 bytes; L = 1: the matrices are 16-byte aligned (the launch checks)
    const uint8_t *wa0 = (const uint8_t *)((uintptr_t)wb0 & ~(uintptr_t)15);
    const uint8_t *wa1 = (const uint8_t *)((uintptr_t)wb1 & ~(uintptr_t)15);
    const uint32_t wm0 = (uint32_t)(uintptr_t)wb0 & 15u, wm1 = (uint32_t)(uintptr_t)wb1 & 15u;
    const int ngr = (a.n + 15) >> 4;  // L = 1: the matrix's row groups
    // window loads: wave instruction wi = wave + 8 j covers pieces 64 wi .. 64 wi + 63 (L = 0), or
    // of its matrix m = wi / MI pieces 64 (wi - m MI) .. + 63 (L = 1: in a stage of cb blocks piece
    // p is piece p % 17 cb of group p / 17 cb; pieces past the N-block's last bring its last again,
    // into the region's padding, and groups past the matrix bring its last group). L = 1 keeps the
    // offsets of a full stage (wo, plus 1,088 bytes per stage) and of a last stage of fewer blocks
    // (wp, whole).
    uint32_t wo[S::NJW], wp[S::NJW];
#pragma unroll
    for (int j = 0; j < S::NJW; j++) {
        if constexpr (L == 0) {
            const int pi = 64 * min(wave + 8 * j, S::W_INST - 1) + lane, row = pi / S::PCS;
            wp[j] = (uint32_t)(pi - row * S::PCS);
            const int n = nb * S::RPB + row % S::RPB;
            wo[j] = (uint32_t)(n < a.n ? n : 0) * (uint32_t)a.row_bytes;
        } else {
            const int wi = min(wave + 8 * j, S::W_INST - 1), m = wi / S::MI;
            const int lp = min(64 * (wi - m * S::MI) + lane, S::GPM * 68 - 1), gw = lp / 68;
            const int g = min(nb * S::GPM + gw, ngr - 1);
            wo[j] = (uint32_t)g * 16u * (uint32_t)a.row_bytes + 16u * (uint32_t)(lp - 68 * gw);
            const int cbl = nblk - 4 * (n_st - 1), ppg = 17 * cbl;  // the last stage's blocks
            const int lq = min(64 * (wi - m * S::MI) + lane, S::GPM * ppg - 1), gq = lq / ppg;
            const int gl = min(nb * S::GPM + gq, ngr - 1);
            wp[j] = (uint32_t)gl * 16u * (uint32_t)a.row_bytes + 1088u * (uint32_t)(n_st - 1) + 16u * (uint32_t)(lq - ppg * gq);
        }
    }
    // L = 0: this lane's rows' offsets from 16-byte alignment
    uint32_t lmis[S::NF];
#pragma unroll
    for (int f = 0; f < S::NF; f++) {
        const int mm = f / S::FR, n = nb * S::RPB + rg * S::RW + 16 * (f % S::FR) + l16;
        lmis[f] = L ? 0u : ((mm ? wm1 : wm0) + (uint32_t)(n < a.n ? n : 0) * (uint32_t)a.row_bytes) & 15u;
    }
    // activation staging: wave w < mbs stages token block w (lane = its K-group and token)
    // wave w < mbs stages token block w: a stage's 16 records of 304 bytes are 304 16-byte
    // pieces, piece p (token p / 19, its piece p % 19) brought by lane p % 64 of load p / 64 (the
    // last load's lanes past piece 303 bring that piece again, into the block's padding)
    const bool stager = wave < mbs;
    uint32_t xo[5] = {0, 0, 0, 0, 0};
    if (stager) {
#pragma unroll
        for (int c = 0; c < 5; c++) {
            const int p = min(64 * c + lane, 303), tk = p / 19;
            const int pos = tile.pos0 + min(16 * wave + tk, tile.m - 1);
            xo[c] = (uint32_t)(a.rows ? a.rows[pos] : pos) * (uint32_t)a.ap_row + 16u * (uint32_t)(p - 19 * tk);
        }
    }

    // Loads are counted per wave: in stage s a wave issues the activation loads of s + 2 (5 if it
    // stages a token block), then nw window loads of s + 3 (nw is 4 or 5, by wave). Before the
    // barrier of stage st, a wave needs its windows of st + 1 (requested in st - 2) and its
    // activations of st + 1 (requested in st - 1): only the windows of st + 2 may stay in flight.
    const int nw = (S::W_INST - wave + 7) / 8;
    int issued = 0;                    // this wave's loads in the item (it starts drained)
    int m_w0 = 0, m_a0 = 0;            // the count after stage 0's window and activation loads
    // window loads of stage st into buffer st % 3 (this wave's share)
    auto issue_w = [&](int st) __attribute__((always_inline)) {
        const int buf = st % S::WDEPTH;
        const uint32_t Wd = lds0 + buf * S::W_BYTES;
        if constexpr (L == 1) {
            const int cb = min(4, nblk - 4 * st);  // blocks per row in this stage
#pragma unroll
            for (int j = 0; j < S::NJW; j++) {
                const int wi = wave + 8 * j;
                if (wi < S::W_INST) {
                    const bool m1 = S::NM > 1 && wi >= S::MI;
                    gx_dma16(m1 ? wa1 : wa0, cb == 4 ? wo[j] + 1088u * (uint32_t)st : wp[j], Wd + wi * 1024);
                    issued++;
                }
            }
            if (st == 0) m_w0 = issued;
            return;
        }
        const uint32_t seg = 17u * (uint32_t)min(4, nblk - 4 * st);  // bytes of a row in this stage
#pragma unroll
        for (int j = 0; j < S::NJW; j++) {
            const int wi = wave + 8 * j;
            if (wi < S::W_INST) {
                const bool m1 = S::NM > 1 && wi >= S::W_INST / 2;
                // the row's bytes of stage st start at o past the aligned base
                const uint32_t o = wo[j] + 68u * (uint32_t)st + (m1 ? wm1 : wm0);
                const uint32_t pc = min(wp[j], ((o & 15u) + seg - 1) >> 4);
                gx_dma16(m1 ? wa1 : wa0, (o & ~15u) + 16 * pc, Wd + wi * 1024);
                issued++;
            }
        }
        if (st == 0) m_w0 = issued;
    };
    // a stager's token block of stage st into activation buffer st % 2 (five 1 KB direct loads)
    auto issue_x = [&](int st) __attribute__((always_inline)) {
        if (stager) {
            const uint32_t d = Al + (st & 1) * S::A_BYTES + wave * S::TB_BYTES;
#pragma unroll
            for (int c = 0; c < 5; c++) gx_dma16(a.ap, xo[c] + 304u * (uint32_t)st, d + 1024 * c);
            issued += 5;
        }
        if (st == 0) m_a0 = issued;
    };

    // operands in registers: each token block's activations of the stage being computed, the raw
    // weight dwords (5 around the block, and its E8M0 byte) of the next stage
    i32x8 bo[NB][3];  // an FP6 operand is dwords 0..5; the instruction ignores 6 and 7
    int bsc[NB];
    uint32_t ra[S::NF][5], re[S::NF];
    auto read_b = [&](int t, int st) __attribute__((always_inline)) {
        // this lane's token's record: per term 16 code bytes of its K-group at 96 j + 16 grp and 8
        // at 96 j + 64 + 8 grp, its scale dword at 288 + 4 grp (bank-conflict free: records are 76
        // dwords apart)
        const uint8_t *r = Ab + (st & 1) * S::A_BYTES + (tb0 + t) * S::TB_BYTES + 304 * l16;
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const i32x4 l = *(const i32x4 *)(r + 96 * j + 16 * grp);
            const i32x2 h = *(const i32x2 *)(r + 96 * j + 64 + 8 * grp);
            bo[t][j] = __builtin_shufflevector(l, __builtin_shufflevector(h, h, 0, 1, -1, -1), 0, 1, 2, 3, 4, 5, -1, -1);
        }
        bsc[t] = *(const int *)(r + 288 + 4 * grp);
    };
    // LDS offset of the E8M0 byte of this lane's block of fragment f in stage st's window
    auto aoff = [&](int f, int st) __attribute__((always_inline)) -> uint32_t {
        if constexpr (L == 1) {
            const int lr = rg * S::RW + 16 * (f % S::FR) + l16, cb = min(4, nblk - 4 * st);
            return (uint32_t)((f / S::FR) * S::MI * 1024) + (uint32_t)lr * (17u * (uint32_t)cb) + 17u * grp;
        }
        const int lrow = (f / S::FR) * S::RPB + rg * S::RW + 16 * (f % S::FR) + l16;
        return (uint32_t)lrow * (S::PCS * 16) + ((lmis[f] + 4u * (uint32_t)st) & 15u) + 17u * grp;
    };
    auto read_a = [&](int st) __attribute__((always_inline)) {
        const uint8_t *Wd = Wb + (st % S::WDEPTH) * S::W_BYTES;
#pragma unroll
        for (int f = 0; f < S::NF; f++) {
            const uint32_t off = aoff(f, st), cb = off + 1;
            const uint32_t *q = (const uint32_t *)(Wd + (cb & ~3u));
#pragma unroll
            for (int i = 0; i < 5; i++) ra[f][i] = q[i];
            re[f] = Wd[off];
        }
    };

    f32x4v acc[S::NF][NB];
#pragma unroll
    for (int f = 0; f < S::NF; f++)
#pragma unroll
        for (int t = 0; t < NB; t++) acc[f][t] = f32x4v{0.f, 0.f, 0.f, 0.f};

    // activations of stages 0 and 1 and windows of 0, 1 and 2 requested, then the operands of
    // stage 0 read
    issue_x(0);
    issue_w(0);
    if (n_st > 1) issue_x(1);
    if (n_st > 1) issue_w(1);
    // gate/up: the bias rows of the tile's expert into LDS (waves 0..5, 64 rows each), with the
    // windows of stage 1 (complete by the first stage's wait; rows past n bring row n - 1)
    if constexpr (MODE == 0) {
        if (a.act != CW_ACT_SILU && wave < 2 * S::RPB / 64) {
            const int m = wave / (S::RPB / 64), r0 = 64 * (wave - m * (S::RPB / 64));
            const float *b = m ? a.bias1 : a.bias0;
            if (b) {
                const int n = min(nb * S::RPB + r0 + lane, a.n - 1);
                gx_dma4((const uint8_t *)(b + (int64_t)tile.expert * a.n), (uint32_t)n * 4u,
                        lds0 + S::BIAS_OFF + (m * S::RPB + r0) * 4);
                issued++;
            }
        }
    }
    if (n_st > 2) issue_w(2);
    gx_wait_vm(issued - (m_w0 > m_a0 ? m_w0 : m_a0));  // this wave's loads of stage 0
    __syncthreads();                                    // everyone's
    if constexpr (NTB > 0) {
#pragma unroll
        for (int t = 0; t < NTB; t++) read_b(t, 0);
        read_a(0);
    }
    // Per stage st (its operands in registers): the activation loads of st + 2 and the window loads
    // of st + 3 go out, and the MFMAs of st run with the reads of st + 1's operands between them.
    for (int st = 0; st < n_st; st++) {
        const bool more = st + 1 < n_st;
        // this wave's loads of st + 1: its windows (requested two stages ago), then its
        // activations (one stage ago, before the windows of st + 2, which stay in flight)
        if (more) gx_wait_stage(st + 2 < n_st ? nw : 0);
        // everyone's loads of st + 1 are in; window buffer st % 3 and activation buffer st % 2
        // (read during st - 1) are free
        __syncthreads();
        if (st + 2 < n_st) issue_x(st + 2);
        if (st + 3 < n_st) issue_w(st + 3);
        if constexpr (NTB > 0) {
            const bool live = 4 * st + grp < nblk;  // past the row's last block
            // the stage read next (unconditionally, so that no register keeps two values: the last
            // stage reads itself again, unused)
            const int sn = more ? st + 1 : st;
            i32x8 av[S::NF];
            int sa[S::NF];
#pragma unroll
            for (int f = 0; f < S::NF; f++) {
                const uint32_t sh = (aoff(f, st) + 1u) & 3u;
                // past the row the codes are whatever the window holds: the activations there are
                // zero and the scale is 1, so the products are 0
                const i32x4 w4 = {(int)__builtin_amdgcn_alignbyte(ra[f][1], ra[f][0], sh),
                                  (int)__builtin_amdgcn_alignbyte(ra[f][2], ra[f][1], sh),
                                  (int)__builtin_amdgcn_alignbyte(ra[f][3], ra[f][2], sh),
                                  (int)__builtin_amdgcn_alignbyte(ra[f][4], ra[f][3], sh)};
                // an FP4 operand is dwords 0..3; the instruction ignores 4..7
                av[f] = __builtin_shufflevector(w4, w4, 0, 1, 2, 3, -1, -1, -1, -1);
                sa[f] = (int)(live ? (re[f] & 0xFFu) : 127u);
            }
#pragma unroll
            for (int t = 0; t < NTB; t++) {
                const int sb = bsc[t];
#pragma unroll
                for (int j = 0; j < 3; j++) {
#pragma unroll
                    for (int f = 0; f < S::NF; f++) {
                        if (j == 0) acc[f][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[f], bo[t][0], acc[f][t], 4, 2, 0, sa[f], 0, sb);
                        if (j == 1) acc[f][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[f], bo[t][1], acc[f][t], 4, 2, 0, sa[f], 1, sb);
                        if (j == 2) acc[f][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[f], bo[t][2], acc[f][t], 4, 2, 0, sa[f], 2, sb);
                    }
                }
                // the block's operands of st + 1 go into its registers once its MFMAs are issued
                // (the scheduling barrier keeps the compiler from hoisting the reads, which would
                // need a second register set)
                __builtin_amdgcn_sched_barrier(0);
                read_b(t, sn);
            }
            __builtin_amdgcn_sched_barrier(0);
            read_a(sn);
        }
    }

    // epilogue: lane holds weight rows 16 f' + 4 grp + i (i < 4) of token 16 (tb0 + t) + l16
    gx_wait_vm(0);
    // hidden rows packed in the block (k_gmx): staged in LDS as [tile row][HST] f32, once every
    // wave is done with the buffers
    const bool stage_h = MODE == 0 && a.hp != nullptr;
    if constexpr (NTB > 0) {
        if constexpr (MODE == 0) {
            // the bias of this lane's rows (gate and up rows n .. n + 3 of fragment f), staged in
            // LDS by the prologue
            const bool swiglu = a.act != CW_ACT_SILU;
            float bg[S::FR][4], bu[S::FR][4];
#pragma unroll
            for (int f = 0; f < S::FR; f++) {
                const int c = rg * S::RW + 16 * f + 4 * grp;  // the row's column in the block
#pragma unroll
                for (int m = 0; m < 2; m++) {
                    const float *b = m ? a.bias1 : a.bias0;
                    float *v = m ? bu[f] : bg[f];
                    v[0] = v[1] = v[2] = v[3] = 0.f;
                    if (!swiglu || !b) continue;
                    const float4 q = *(const float4 *)(smem + S::BIAS_OFF + (m * S::RPB + c) * 4);
                    v[0] = q.x;
                    v[1] = q.y;
                    v[2] = q.z;
                    v[3] = q.w;
                }
            }
            // hidden rows packed in the block (k_gmx): staged in LDS as [tile row][HST] f32, once
            // every wave is done with the buffers
            if (stage_h) __syncthreads();
            // sigmoid(z) = 1 / (1 + 2^(-z log2 e)) on the hardware's exp2 and reciprocal (each
            // within 1 ulp)
            constexpr float LOG2E = 1.4426950408889634f;
#pragma unroll
            for (int t = 0; t < NTB; t++) {
                const int rr = 16 * (tb0 + t) + l16;
                if (rr >= tile.m) continue;
                const int pos = tile.pos0 + rr;
#pragma unroll
                for (int f = 0; f < S::FR; f++) {
                    const int n = nb * S::RPB + rg * S::RW + 16 * f + 4 * grp;
                    float o[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        float g = acc[f][t][i], u = acc[S::FR + f][t][i];
                        if (!swiglu) {
                            o[i] = g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * LOG2E)) * u;
                        } else {
                            g += bg[f][i];
                            u += bu[f][i];
                            g = fminf(g, a.limit);
                            u = fminf(fmaxf(u, -a.limit), a.limit);
                            o[i] = (u + 1.0f) * (g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-(g * a.alpha) * LOG2E)));
                        }
                        if (n + i >= a.n) o[i] = 0.f;  // past the row: its packed values are 0
                    }
                    if (stage_h) {
                        // row rr of the tile at column n - nb * RPB (an index from the LDS base,
                        // never a pointer formed below it: a generic address below the shared
                        // aperture is taken for a global one)
                        *(float4 *)((float *)smem + rr * S::HST + (n - nb * S::RPB)) = make_float4(o[0], o[1], o[2], o[3]);
                    } else {
                        float *const hrow = a.h + (int64_t)pos * a.ldh + n;
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            if (n + i < a.n) hrow[i] = o[i];
                    }
                }
            }
        } else {
            // each token's pick (its output row), every load issued before any is used
            int pk[NB];
#pragma unroll
            for (int t = 0; t < NTB; t++) {
                const int rr = min(16 * (tb0 + t) + l16, tile.m - 1), pos = tile.pos0 + rr;
                pk[t] = a.pile_pick ? a.pile_pick[pos] : pos;
            }
#pragma unroll
            for (int t = 0; t < NTB; t++) {
                if (16 * (tb0 + t) + l16 >= tile.m) continue;
#pragma unroll
                for (int f = 0; f < S::FR; f++) {
                    const int n = nb * S::RPB + rg * S::RW + 16 * f + 4 * grp;
                    float *dst = a.dn + (int64_t)pk[t] * a.n + n;
                    if (n + 4 <= a.n && (a.n & 3) == 0) {
                        *(float4 *)dst = make_float4(acc[f][t][0], acc[f][t][1], acc[f][t][2], acc[f][t][3]);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            if (n + i < a.n) dst[i] = acc[f][t][i];
                    }
                }
            }
        }
    } else if (stage_h) {
        __syncthreads();  // the block's barrier before the staging, with no rows of its own
    }
}

// MODE 0: gate and up with the activation, hidden rows written in pile order (ldh floats).
// MODE 1: one output row per pick (dn, pick order), combined per token afterwards.
template <int MODE, int L>
__global__ __launch_bounds__(512, 1) void k_gmx(const MfArgs a) {
    using S = GxShape<MODE, L>;
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)smem;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_nb = (a.n + S::RPB - 1) / S::RPB;
    const int R = a.run_tiles, n_tiles = *a.n_tiles;
    // blocks go to the 8 XCDs round-robin; item b of each run of R*n_nb (R = run_tiles) takes
    // M-tile R*run + b%R and N-block b/R, so an M-tile's N-blocks share an XCD and its L2
    for (int item = blockIdx.x; item < a.n_items; item += gridDim.x) {
        const int run = item / (R * n_nb), b = item - run * R * n_nb;
        const int mt = run * R + (b & (R - 1));
        if (mt >= n_tiles) continue;  // uniform across the block
        const int nb = b / R;
        __syncthreads();  // every wave is done with the previous item's buffers
        const MfTile tile = a.tiles[mt];
        const int mbs = (tile.m + 15) >> 4, half = wave >> 2, n0 = (mbs + 1) >> 1;
        const int tb0 = half ? n0 : 0, ntb = half ? mbs - n0 : n0;
        switch (ntb) {
        case 0: gx_item<MODE, 0, L>(a, tile, nb, mbs, tb0, wave, lane, smem, lds0); break;
        case 1: gx_item<MODE, 1, L>(a, tile, nb, mbs, tb0, wave, lane, smem, lds0); break;
        case 2: gx_item<MODE, 2, L>(a, tile, nb, mbs, tb0, wave, lane, smem, lds0); break;
        default: gx_item<MODE, 3, L>(a, tile, nb, mbs, tb0, wave, lane, smem, lds0); break;
        }
        if constexpr (MODE == 0) {
            if (a.hp) {
                // the tile's hidden values of this N-block, one thread per (tile row, 32-value
                // block), into the down GEMM's FP6 records; rows' records past the GEMM's blocks
                // (zeros) come with the last N-block
                __syncthreads();
                constexpr int NBL = S::RPB / 32;
                const float *hb = (const float *)smem;
                for (int e = threadIdx.x; e < tile.m * NBL; e += S::NT) {
                    const int r = e / NBL, bl = e - r * NBL, jb = nb * NBL + bl;
                    if (jb >= a.hp_blocks) continue;
                    const float4 *src = (const float4 *)(hb + r * S::HST + 32 * bl);
                    f32x16 lo, hi;
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const float4 f = src[c], h = src[4 + c];
                        lo[4 * c] = f.x;
                        lo[4 * c + 1] = f.y;
                        lo[4 * c + 2] = f.z;
                        lo[4 * c + 3] = f.w;
                        hi[4 * c] = h.x;
                        hi[4 * c + 1] = h.y;
                        hi[4 * c + 2] = h.z;
                        hi[4 * c + 3] = h.w;
                    }
                    fp6x3_record(lo, hi, a.hp + (int64_t)(tile.pos0 + r) * a.hp_row + (jb >> 2) * 304, jb & 3);
                }
                const int from = n_nb * NBL, cnt = a.hp_blocks - from;
                if (nb == n_nb - 1 && cnt > 0) {
                    for (int e = threadIdx.x; e < tile.m * cnt; e += S::NT) {
                        const int r = e / cnt, jb = from + (e - r * cnt);
                        fp6x3_zero(a.hp + (int64_t)(tile.pos0 + r) * a.hp_row + (jb >> 2) * 304, jb & 3);
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------ launchers

int pack_rows_fp6(const float *x, int rows, int k, int ldx, uint8_t *out, hipStream_t s) {
    if (rows == 0) return CW_OK;
    if (k % 32) return set_error(CW_ENOTSUP, "pack fp6: rows of %d are not whole 32-value blocks", k);
    const int64_t n = (int64_t)rows * (((k / 32) + 3) & ~3), blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_pack_fp6x3, dim3((unsigned)(blocks < 16384 ? blocks : 16384)), dim3(256), 0, s, x, rows, k, ldx, out);
    return check_launch("k_pack_fp6x3");
}

size_t fp6_rows_bytes(int64_t rows, int64_t k) { return (size_t)rows * (size_t)((k + 127) / 128) * 304; }

static int gx_device() {
    int dev = 0;
    return hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 ? dev : 0;
}

template <int MODE, int L>
static int gx_launch(const MfArgs &a, int tiles_max, hipStream_t s) {
    using S = GxShape<MODE, L>;
    if (a.k % 32 || a.k <= 128) return set_error(CW_ENOTSUP, "mxfp4 gemm: k %d is not whole blocks over two steps", a.k);
    // lane offsets are 32-bit: from a matrix's 16-byte aligned base, and into the packed rows
    if ((int64_t)(a.n + 15) / 16 * 16 * a.row_bytes + 256 >= ((int64_t)1 << 32))
        return set_error(CW_ENOTSUP, "mxfp4 gemm: a matrix of %d rows of %lld bytes is 4 GiB or more", a.n, (long long)a.row_bytes);
    if (L == 1 && (((uintptr_t)a.w0 | (uintptr_t)a.s0) & 15 || (MODE == 0 && ((uintptr_t)a.w1 | (uintptr_t)a.s1) & 15)))
        return set_error(CW_EINVAL, "mxfp4 gemm: matrices in row groups of 16 must start on 16-byte boundaries");
    if (MODE == 0 && a.hp && (size_t)MF_MT * S::HST * 4 > (size_t)S::BIAS_OFF)
        return set_error(CW_ENOTSUP, "mxfp4 gemm: the hidden rows' staging does not fit");
    if (a.ap_rows * a.ap_row >= ((int64_t)1 << 32))
        return set_error(CW_ENOTSUP, "mxfp4 gemm: %lld packed activation rows are 4 GiB or more", (long long)a.ap_rows);
    static std::atomic<int> cus_of[64];
    static std::atomic<bool> lds_set[64];
    const int dev = gx_device();
    int cus = cus_of[dev].load(std::memory_order_relaxed);
    if (!cus) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) n = 256;
        cus = n / 8 * 8;
        cus_of[dev].store(cus, std::memory_order_relaxed);
    }
    if (!lds_set[dev].load(std::memory_order_acquire)) {
        if (hipFuncSetAttribute((const void *)k_gmx<MODE, L>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::LDS) != hipSuccess)
            return set_error(CW_EHIP, "mxfp4 gemm: cannot reserve %zu bytes of LDS", S::LDS);
        lds_set[dev].store(true, std::memory_order_release);
    }
    const int n_nb = (a.n + S::RPB - 1) / S::RPB;
    const int R = tiles_max >= 8 ? 8 : tiles_max >= 4 ? 4 : tiles_max >= 2 ? 2 : 1;
    const int64_t items = (int64_t)((tiles_max + R - 1) / R) * R * n_nb;
    if (items >= ((int64_t)1 << 31)) return set_error(CW_ENOTSUP, "mxfp4 gemm: %lld work items", (long long)items);
    const int64_t blocks = items < cus ? (items + 7) / 8 * 8 : cus;
    MfArgs b = a;
    b.run_tiles = R;
    b.n_items = (int)items;
    hipLaunchKernelGGL((k_gmx<MODE, L>), dim3((unsigned)blocks), dim3(S::NT), S::LDS, s, b);
    return check_launch("k_gmx");
}

int mxfp4_gateup(const MfArgs &a, int tiles_max, hipStream_t s) {
    return a.layout ? gx_launch<0, 1>(a, tiles_max, s) : gx_launch<0, 0>(a, tiles_max, s);
}
int mxfp4_down(const MfArgs &a, int tiles_max, hipStream_t s) {
    return a.layout ? gx_launch<1, 1>(a, tiles_max, s) : gx_launch<1, 0>(a, tiles_max, s);
}

// ------------------------------------------------------------------------------ the row-group layout

// One thread per (row, block) of each matrix: block b of GGUF row r to rows16_offset(r, b); rows
// past n up to the group's end get zero blocks (scale 2^-127, codes 0: products 0).
__global__ __launch_bounds__(256) void k_rows16(const uint8_t *src, int64_t src_stride, uint8_t *dst, int64_t dst_stride,
                                                int64_t n_mats, int n, int nblk) {
    const int rows = (n + 15) / 16 * 16;
    const int64_t per = (int64_t)rows * nblk, total = n_mats * per;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t mat = i / per, e = i - mat * per;
        const int r = (int)(e / nblk), b = (int)(e - (int64_t)r * nblk);
        uint8_t *d = dst + mat * dst_stride + rows16_offset(r, b, nblk);
        if (r < n) {
            const uint8_t *q = src + mat * src_stride + ((int64_t)r * nblk + b) * 17;
#pragma unroll
            for (int k = 0; k < 17; k++) d[k] = q[k];
        } else {
#pragma unroll
            for (int k = 0; k < 17; k++) d[k] = 0;
        }
    }
}

int rows16_repack(const uint8_t *src, int64_t src_stride, uint8_t *dst, int64_t dst_stride, int64_t n_mats, int n, int k,
                  hipStream_t s) {
    const int nblk = k / 32;
    const int64_t total = n_mats * (int64_t)((n + 15) / 16 * 16) * nblk;
    if (total == 0) return CW_OK;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(k_rows16, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, s, src, src_stride, dst,
                       dst_stride, n_mats, n, nblk);
    return check_launch("k_rows16");
}

// The scaled path is the default for MXFP4; CWMOE_MXFP4_F16=1 selects the fp16 MFMA path instead
// (for comparisons). Read at each call: a workspace size and the call it is for must agree, so the
// variable must not change between them.
bool mxfp4_scaled() {
    const char *e = getenv("CWMOE_MXFP4_F16");
    return !(e && atoi(e) == 1);
}

}  // namespace cw
