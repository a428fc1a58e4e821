/* TEST INFRASTRUCTURE ONLY.
 *
 * CPU oracle for the quantized mixture-of-experts expert path: a plain-C restatement of the
 * reference's CPU arithmetic, used by tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline leg as the checker. Nothing in the product links or calls this library.
 *
 * Every function cites the reference file:line it restates (paths relative to the reference
 * checkout root). Parity status of each function is listed in oracle/README.md.
 */
#ifndef CW_ORACLE_H
#define CW_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids: vendor/candle-core/src/quantized/mod.rs:314-339, plus 21 (IQ3_S), 22 (IQ2_S). */
enum { OR_F32 = 0, OR_F16 = 1, OR_Q8_0 = 8, OR_Q2_K = 10, OR_Q3_K = 11, OR_Q4_K = 12, OR_Q5_K = 13,
       OR_Q6_K = 14, OR_Q8_K = 15, OR_IQ2_XXS = 16, OR_IQ3_XXS = 18, OR_IQ3_S = 21, OR_IQ2_S = 22,
       OR_IQ4_XS = 23, OR_MXFP4 = 39 };

int or_block_size(int dtype);   /* weights per block, 0 if unknown */
int or_type_size(int dtype);    /* bytes per block, 0 if unknown */

float or_f16_to_f32(uint16_t h);  /* IEEE widening (half 2.7.1 f16::to_f32) */
uint16_t or_f32_to_f16(float f);  /* round-to-nearest-even narrowing (half f16::from_f32) */
float or_e8m0_half(uint8_t e);    /* k_quants.rs:642-649 */

/* Dequantize n weights (n a multiple of the block size) into f32. 0 on success, -1 on a bad
 * dtype or size. */
int or_dequantize(int dtype, const void *blocks, int64_t n, float *out);

/* The GPU shrink, crates/engine/src/requant.rs:113-304: n_blocks super-blocks of Q3_K, Q4_K or
 * Q5_K re-encoded as Q2_K (84 bytes each). Each block is dequantized (the values of candle's
 * to_float, which the shader's dq_q3/dq_q4/dq_q5 equal exactly), then each sub-block of 16 is
 * fitted by fit16 (two weighted least-squares rounds from the min/max start), the 16 scales and
 * mins are put on 4 bits against the block's largest, and the quants rounded to 2 bits. With
 * shape != NULL (run_shaped) the weight of value i of a block is sqrt(max(shape[col], 0)) + 1e-6
 * for its column col = (block % blocks_per_row) * 256 + i; else every weight is 1. All
 * arithmetic is IEEE f32 in the order the shader writes it; minimum and maximum are taken as
 * "replace when strictly smaller / larger". 0 on success, -1 on a bad source type. */
int or_requant_q2k(int src_dtype, const void *src, int64_t n_blocks, const float *shape,
                   int64_t blocks_per_row, void *dst);

/* y[m][n] = sum_k dequant(W)[n][k] * x[m][k] in f64 (W is n rows of k weights). */
int or_qmatmul_f64(int dtype, const void *w, int64_t n, int64_t k, const float *x, int64_t m,
                   double *y);

/* Router: softmax over E (candle-nn softmax_last_dim semantics: max, exp, sequential sum,
 * divide), stable descending sort, top K best first, weights renormalised when norm != 0.
 * crates/engine/src/experts.rs:2364-2372, vendor/candle-core/src/sort.rs:40-53. */
void or_route(const float *logits, int T, int E, int K, int norm, uint32_t *ids, float *w);
/* Probabilities only (T x E), same arithmetic as or_route. */
void or_softmax(const float *logits, int T, int E, float *probs);
/* crates/engine/src/experts.rs:676-680: expert ids by score, best first, ties by id. */
void or_rank(const float *scores, int n, uint32_t *ids);

/* h = silu(g) * u in f32: vendor/candle-core/src/op.rs:757-759 and experts.rs:2391. */
void or_silu_mul(const float *g, const float *u, float *h, int64_t n);
/* gpt-oss clamped SwiGLU, experts.rs:2392-2404: rows of width `width`, row r uses biases of
 * expert ids[r]; the output rows are `pad` wide (zeros past width) when pad > width. */
void or_clamped_swiglu(const float *g, const float *u, const float *gate_b, const float *up_b,
                       const uint32_t *ids, int64_t rows, int width, int pad, float alpha,
                       float limit, float *h);
/* out[t][j] = sum_e w[t][e] * down[t][e][j]: crates/engine/src/fuse_kernel.rs:277-291. */
void or_weighted_sum(const float *down, const float *w, int T, int K, int H, float *out);
/* slots[i] = table[ids[i]]; NO_SLOT (0xffffffff) -> 0 and missing++: gpu_sync.rs:49-66. */
void or_resolve(const uint32_t *ids, const uint32_t *table, int n, uint32_t *slots,
                uint32_t *missing);

/* MoeMatvec (experts.rs:2183-2309): out[t][j][:] = W[slot ids[t][j]] . x_row in f64, with
 * x_row = x[t] (rows_per_expert == 0) or x[t*K + j]. Slot s's matrix starts at
 * bank + s * slot_stride bytes. */
int or_matvec_id(int dtype, int64_t n, int64_t k, int64_t n_slots, int64_t slot_stride,
                 const void *bank, const float *x, int rows_per_expert, const uint32_t *ids,
                 int K, int T, double *out);

/* The resident MoE layer (experts.rs:2562-2614) and the bank variant (3003-3015). */
typedef struct {
    int n_experts, top_k, hidden, inter;
    int norm;                 /* renormalise the top-k weights */
    int act;                  /* 0 = silu(gate)*up, 1 = clamped SwiGLU with biases */
    float alpha, limit;       /* clamped SwiGLU constants (model_gptoss.rs:16-17) */
    int pad;                  /* width down reads (>= inter), 0 = inter */
    int dtype[3];             /* gate, up, down */
    const void *w[3];         /* slot-major matrices: gate/up [slots][inter][hidden], down [slots][hidden][pad] */
    int64_t slot_stride[3];   /* bytes per slot */
    const float *bias[3];     /* (E x width) or NULL */
    const uint32_t *slot_table; /* expert -> slot, NULL = identity */
    int n_slots;
} or_moe_desc;

/* out[T][hidden] in f64; ids/w (T x K) receive the routing. Returns the number of picks that
 * had no slot (resolved to slot 0), or -1 on a bad argument. */
int or_moe_layer(const or_moe_desc *d, const float *x, const float *logits, int T, double *out,
                 uint32_t *ids, float *w);

/* candle's CPU activation quantizers and block dots (the timed CPU baseline's numerics). */
void or_quantize_q8_0(const float *x, int64_t n, void *blocks);  /* k_quants.rs:784-821 */
void or_quantize_q8_k(const float *x, int64_t n, void *blocks);  /* k_quants.rs:2495-2534 */
/* candle generic vec_dot of one weight row against one quantized activation row:
 * Q8_0 x Q8_0 k_quants.rs:855-874, Q4_K x Q8_K 1612-1692, MXFP4 x Q8_0 738-759. */
float or_vec_dot(int dtype, int64_t k, const void *wrow, const void *xq);
/* candle CPU QMatMul (generic matmul, k_quants.rs:2551-2670): quantize x, then vec_dot per
 * (row, column). Threads: 0 = all available. */
int or_candle_matmul(int dtype, const void *w, int64_t n, int64_t k, const float *x, int64_t m,
                     float *y, int threads);

void or_set_threads(int n);
int or_get_threads(void);

/* candle's x86 repacked QMatMul (repack.rs:219-283, repack_x86.rs), in cw_candle_x86.c: the
 * weights packed once into tiles of 16 rows, activations quantized to Q8_K per call, units of
 * 16 rows x up to 4 activation rows over the threads. */
int or_x86_level(void);   /* 2 AVX-512 VNNI, 1 AVX-VNNI, 0 AVX2 + FMA, -1 none (repack_x86.rs:905-928) */
/* whether candle takes this path for (dtype, m, n, k) on this host (repack_x86.rs:43-60) */
int or_x86_select(int dtype, int64_t m, int64_t n, int64_t k);
int64_t or_x86_packed_bytes(int dtype, int64_t n, int64_t k);  /* 0: not a packed case */
int or_x86_pack(int dtype, const void *w, int64_t n, int64_t k, void *packed);
/* y[m][n]; simd 1 = AVX-512 VNNI unit when the host has it, 0 = the plain-C unit (same bits);
 * threads 0 = all available */
int or_x86_matmul(int dtype, const void *packed, int64_t n, int64_t k, const float *x, int64_t m,
                  float *y, int simd, int threads);

#ifdef __cplusplus
}
#endif
#endif
