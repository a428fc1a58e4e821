// Internal interface of the MFMA grouped-GEMM path (cw_mfma.hip): prefill of the MoE layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cw {

constexpr int MF_MB = 5;            // MFMA blocks of 16 picks per tile
constexpr int MF_MT = 16 * MF_MB;   // picks per tile: 80 keeps the piles of a 1,500-token batch over
                                    // 256 experts (about 47 picks each) at one tile per expert

// A tile: m picks of one slot's pile from pile position pos0, and the expert they were routed to
// (every pick of a pile reads one slot, so one expert; the slot itself when the piles were built
// without the picks' expert ids).
struct MfTile {
    int slot, pos0, m, expert;
};

struct MfArgs {
    // weights: one matrix (or a gate/up pair) per slot
    const uint8_t *w0, *w1;
    int64_t s0, s1;            // slot strides
    int64_t row_bytes;
    int n, k;                  // weight rows, weights per row
    // activations: fp16 rows of k (lda halves) with a power-of-two scale per row
    const uint16_t *a16;
    const float *ascale;
    int lda;
    const int *rows;           // activation row of each pile position, or NULL (position itself)
    // piles
    const MfTile *tiles;
    const int *n_tiles;
    int run_tiles;             // M-tiles per run of work items (1, 2, 4 or 8; set by the launch)
    int n_items;               // work items (M-tile, N-block) of the launch (set by the launch)
    const int *pile_pick;      // pick index (t*K + j) of each pile position
    int K;
    // epilogues
    int act;
    float alpha, limit;
    const float *bias0, *bias1;   // gate/up bias (E x n)
    const uint32_t *ids;          // expert of each pick (bias lookup)
    float *h;                     // gate/up: hidden rows in pile order (ldh floats)
    int ldh;
    float *dn;                    // down: one row of n per pick, in pick order (t*K + j)
    // split-K (dense matmul): block row blockIdx.y takes stages [y*split_st, (y+1)*split_st) and
    // writes its partial rows at dn + y*split_stride; 0 = no split. The last split of a work item
    // to finish (split_cnt[item], zero at launch) adds the partial rows in split order into y.
    int split_st;
    int64_t split_stride;
    int *split_cnt;
    float *y;
    // MXFP4 on the scaled MFMA: activations packed by pack_rows_fp6 (ap_rows rows of ap_row bytes)
    const uint8_t *ap;
    int64_t ap_row, ap_rows;
    // gate/up on the scaled MFMA: the hidden rows packed as the down GEMM's FP6 activations (hp,
    // hp_row bytes per pile position, hp_blocks 32-value block records per row) instead of f32 h
    uint8_t *hp;
    int64_t hp_row;
    int hp_blocks;
    // the weights' layout on the scaled MFMA: 0 GGUF rows (CW_MXFP4), 1 rows in groups of 16
    // (CW_MXFP4_R16)
    int layout;
};

// Work a pack launch also does for the dense matmul that follows it: the tile list of m rows, and
// the split counters zeroed.
struct PackExtra {
    MfTile *tiles;
    int *n_tiles;
    int m;
    int *zero;
    int n_zero;
};

bool mfma_supported(int dtype);
// formats whose MFMA fragments take each 32-wide K step in a permuted order (MXFP4: a byte's two
// nibbles side by side); their activations are packed with pack_rows_f16(..., perm = true)
inline bool mfma_k_permuted(int dtype) { return dtype == CW_MXFP4; }
// one block: expert piles of the (slot) picks, and the tile list
int mfma_piles(const uint32_t *slots, const uint32_t *ids, int TK, int K, int n_slots, int *pile_pick, int *pile_tok, MfTile *tiles,
               int *n_tiles, hipStream_t s);
int max_tiles(int TK, int n_slots);
// rows x k f32 -> fp16 rows (ld = k) with per-row power-of-two scales
int pack_rows_f16(const float *x, int rows, int k, int ldx, uint16_t *a16, float *ascale, hipStream_t s,
                  const PackExtra *extra = nullptr, bool perm = false);
int fill_zero(float *p, int64_t n, hipStream_t s);
int mfma_gateup(int dtype, const MfArgs &a, int tiles_max, hipStream_t s);
int mfma_down(int dtype, const MfArgs &a, int tiles_max, hipStream_t s);
// y (m x n) = x (m x k) . W^T for one quantized matrix, through the same GEMM (fp16 activations)
size_t mfma_dense_workspace(int dtype, int64_t m, int64_t n, int64_t k);
int mfma_dense(int dtype, const uint8_t *w, int64_t row_bytes, int n, int k, const float *x, int m, float *y, void *ws,
               size_t ws_bytes, hipStream_t s);
// out[t] = sum_j w[t*K+j] * (dn[t*K+j] + bias[ids[t*K+j]]), picks in order (H a multiple of 4); a
// pick with slots[t*K+j] >= n_slots contributes NaN (it has no row)
int combine_picks(const float *dn, const float *w, const float *bias, const uint32_t *ids, const uint32_t *slots, int n_slots,
                  int T, int K, int H, float *out, hipStream_t s);

// MXFP4 grouped GEMMs on the block-scaled MFMA (cw_mxfp4.hip): the weights as stored (E2M1 codes
// and E8M0 block scales), the activations as three FP6 terms with E8M0 scales per 32 values.
bool mxfp4_scaled();
// a matrix of k weights per row runs on the scaled MFMA (MXFP4, at least two 128-wide K steps)
// (MXFP4 in row groups of 16 has no other path)
inline bool mxfp4_scaled_for(int dtype, int64_t k) {
    return k > 128 && k % 32 == 0 && ((dtype == CW_MXFP4 && mxfp4_scaled()) || dtype == CW_MXFP4_R16);
}
size_t fp6_rows_bytes(int64_t rows, int64_t k);
int pack_rows_fp6(const float *x, int rows, int k, int ldx, uint8_t *out, hipStream_t s);
int mxfp4_gateup(const MfArgs &a, int tiles_max, hipStream_t s);
int mxfp4_down(const MfArgs &a, int tiles_max, hipStream_t s);
// n_mats MXFP4 matrices of n GGUF rows of k weights (src_stride bytes apart) into the row-group
// layout of CW_MXFP4_R16 (dst_stride bytes apart, each (n + 15) / 16 * 16 rows)
int rows16_repack(const uint8_t *src, int64_t src_stride, uint8_t *dst, int64_t dst_stride, int64_t n_mats, int n, int k,
                  hipStream_t s);

}  // namespace cw
