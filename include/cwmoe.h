/*
 * cwmoe.h — C ABI of the MI355X (gfx950) quantized mixture-of-experts expert path.
 *
 * This is the drop-in boundary for the reference engine's quantized matmul and MoE-layer
 * custom ops. Each entry point below names the reference interface it replaces (paths are
 * relative to the reference checkout: vendor/candle-* are the vendored candle crates,
 * crates/engine is the coachwhip engine crate).
 *
 * Conventions, kept from the reference (vendor/candle-core/src/custom_op.rs:8-95 and the
 * Metal launchers in vendor/candle-metal-kernels/src/kernels/quantized.rs):
 *  - Weights are raw GGUF blocks exactly as stored in the file (no repacking); `dtype` is the
 *    GGUF type id (vendor/candle-core/src/quantized/mod.rs:314-339, plus 21 = IQ3_S and
 *    22 = IQ2_S, which the reference's shaders implement).
 *  - A weight matrix is `n` rows of `k` weights, rows along the output dimension, blocks along
 *    k (GGUF order). Expert banks hold `n_slots` such matrices `slot_stride` bytes apart.
 *  - Activations and outputs are contiguous f32; routing ids are u32. Strides are in bytes.
 *  - All pointers are device pointers unless stated. Every call is asynchronous on `stream`
 *    (a hipStream_t; NULL = the default stream) and never synchronizes the device.
 *  - No entry point allocates device memory: scratch comes from a caller-owned workspace
 *    whose size the matching *_workspace_size query returns (the role of
 *    crates/engine/src/arena.rs:15-33).
 *  - Errors are returned, never thrown: CW_OK, CW_ENOTSUP (a capability probe said no; the
 *    caller may fall back, as mv_id.rs:156-179 does with Ok(false)), CW_EINVAL (shape, stride
 *    or argument error, as candle::bail! in crates/engine/src/experts.rs:2204-2217), CW_EHIP
 *    (the HIP runtime failed). cw_last_error() describes the last failure on this thread.
 *  - Calls on distinct streams may run concurrently when they use distinct workspaces (a call
 *    keeps all its scratch in the workspace it is given), with one exception: a one-token
 *    cw_moe_layer call (T = 1) is one persistent launch sized to fill the device, whose blocks
 *    meet at a device-wide barrier. It must not overlap other work on the device: blocks that
 *    cannot be scheduled make the barrier give up (outputs NaN, counted in the workspace's status
 *    word and by cw_device_errors) instead of hanging.
 */
#ifndef CWMOE_H
#define CWMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *cw_stream_t; /* hipStream_t */

/* CW_EFULL: a bank cannot place the experts asked for now (more than its slots, or too few
 * slots free); nothing changed, and the caller reads those experts another way. */
enum cw_status { CW_OK = 0, CW_ENOTSUP = 1, CW_EINVAL = 2, CW_EHIP = 3, CW_EFULL = 4 };

/* GGUF type ids of the weight formats this library reads. */
enum cw_dtype {
    CW_F32 = 0,
    CW_F16 = 1,
    CW_Q8_0 = 8,     /* {f16 d; i8 qs[32]}: 34 B per 32 weights */
    CW_Q2_K = 10,    /* {u8 scales[16]; u8 qs[64]; f16 d, dmin}: 84 B per 256 (the shrink's output) */
    CW_Q3_K = 11,    /* {u8 hmask[32]; u8 qs[64]; u8 scales[12]; f16 d}: 110 B per 256 (shrink input) */
    CW_Q4_K = 12,    /* {f16 d, dmin; u8 scales[12]; u8 qs[128]}: 144 B per 256 */
    CW_Q5_K = 13,    /* {f16 d, dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]}: 176 B per 256 */
    CW_Q6_K = 14,    /* {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}: 210 B per 256 */
    CW_IQ2_XXS = 16, /* {f16 d; u16 qs[32]}: 66 B per 256 */
    CW_IQ3_XXS = 18, /* {f16 d; u8 qs[64]; u32 scales_and_signs[8]}: 98 B per 256 */
    CW_IQ3_S = 21,   /* {f16 d; u8 qs[64], qh[8], signs[32], scales[4]}: 110 B per 256 */
    CW_IQ2_S = 22,   /* {f16 d; u8 qs[64], qh[8], scales[8]}: 82 B per 256 */
    CW_IQ4_XS = 23,  /* {f16 d; u16 scales_h; u8 scales_l[4]; u8 qs[128]}: 136 B per 256 */
    CW_MXFP4 = 39,   /* {u8 e8m0; u8 qs[16]}: 17 B per 32 */
    /* Not a GGUF type: CW_MXFP4 blocks with each matrix's rows in groups of 16, the group's blocks
     * of each 4-block step side by side (16 runs of 17 cb bytes, cb = blocks of the step), a group
     * in the bytes its 16 GGUF rows take, the last group padded with zero rows. Made by
     * cw_repack_rows16; read by the expert paths (cw_moe_layer, cw_matmul_id_grouped), whose
     * GEMMs and decode load a step of each group as one run instead of one short run per row. */
    CW_MXFP4_R16 = 295
};

enum cw_act { CW_ACT_SILU = 0, CW_ACT_CLAMPED_SWIGLU = 1 };

#define CW_NO_SLOT 0xFFFFFFFFu /* crates/engine/src/gpu_sync.rs:20 */

/* ---- library ---------------------------------------------------------------------------- */

/* Version string and the last error message of the calling thread. */
const char *cw_version(void);
const char *cw_last_error(void);

/* Weights per block and bytes per block of a dtype; 0 when the dtype is not supported.
 * Replaces GgmlDType::block_size / type_size (vendor/candle-core/src/quantized/mod.rs:420-460). */
int cw_block_size(int dtype);
int cw_type_size(int dtype);

/* ---- formats ---------------------------------------------------------------------------- */

/* out[i] = the f32 value of weight i, for n_elems weights (a multiple of the block size).
 * Bit-exact with the CPU dequantizers (every in-scope dequantization is an exact product).
 * Replaces QTensor::dequantize / QMetalStorage::dequantize
 * (vendor/candle-core/src/quantized/metal.rs:40-139) and the Metal dequantize_* functions
 * (vendor/candle-metal-kernels/src/metal_src/quantized.metal:6691-7017). */
int cw_dequantize(int dtype, const void *blocks, int64_t n_elems, float *out, cw_stream_t stream);

/* ---- dense quantized matmul ------------------------------------------------------------- */

/* y[m][n] = x[m][k] . W[n][k]^T for a quantized W; the QMatMul::forward contract
 * (vendor/candle-core/src/quantized/mod.rs:1206-1345 with the Metal dispatch of
 * quantized/metal.rs:359-470, call_quantized_matmul_mv_t / _mm_t in
 * vendor/candle-metal-kernels/src/kernels/quantized.rs:32-43, 198-213).
 * From 2 rows of x (Q4_K) or 8 rows (the other formats) the product runs as an MFMA GEMM on
 * fp16-rounded activations (rel-L2 about 3e-4 against f64) and needs the workspace; below that
 * it is one f32 matvec per row. ws may be NULL when cw_qmatmul_workspace_size returns 0. */
size_t cw_qmatmul_workspace_size(int dtype, int64_t n, int64_t k, int64_t m);
int cw_qmatmul(int dtype, const void *w, int64_t n, int64_t k, const float *x, int64_t m,
               float *y, void *ws, size_t ws_bytes, cw_stream_t stream);

/* ---- routing ---------------------------------------------------------------------------- */

/* Softmax over E logits per token, the K likeliest experts best first (ties to the lowest
 * index), their probabilities renormalised over the K when norm != 0.
 * ids[T][K] u32, w[T][K] f32. E <= 1024, K <= 32.
 * Replaces experts::route (crates/engine/src/experts.rs:2364-2372) and the fused cw_route
 * (crates/engine/src/fuse_kernel.rs:20-75, 347-352), whose limits were E <= 256, K <= 16. */
int cw_route_topk(const float *logits, int T, int E, int K, int norm, uint32_t *ids, float *w,
                  cw_stream_t stream);

/* logits[t][e] = x[t] . W[e] (+ bias[e], when bias is not NULL) for the router weight W
 * (n_experts x hidden), f32 (CW_F32) or f16 (CW_F16) weights, f32 x and accumulation; x is
 * T rows of hidden, 16-byte aligned, hidden a multiple of 4. Replaces the gate Linear
 * (crates/engine/src/experts.rs:2428, 2577; gpt-oss adds the bias, model_gptoss.rs:168-175) and
 * its f16 decode variant cw_mv_f16 (crates/engine/src/fuse_kernel.rs:160-178, 537-559). The
 * logits then go to cw_route_topk or cw_moe_layer on the same stream. */
int cw_router_logits(int wdtype, const void *w, int n_experts, int hidden, const float *bias,
                     const float *x, int T, float *logits, cw_stream_t stream);

/* ---- expert matvec ---------------------------------------------------------------------- */

/* For each token t < T and pick j < K: out[t][j][0..n) = W[s] . x_row, with s = ids[t][j] a
 * slot index, W[s] the n x k matrix at bank + s * slot_stride bytes, and x_row = x[t]
 * (x_rows_per_expert == 0) or x[t*K + j] (!= 0). Ids >= n_slots are rejected on the device
 * (the output row is set to NaN and the call still completes).
 * Replaces MoeMatvec (crates/engine/src/experts.rs:2183-2309) and its launchers
 * mv_id::matvec_id / matvec_id_new (crates/engine/src/mv_id.rs:17-31, 158-171). */
int cw_matvec_id(int dtype, int64_t n, int64_t k, int64_t n_slots, int64_t slot_stride,
                 const void *bank, const float *x, int x_rows_per_expert, const uint32_t *ids,
                 int K, int T, float *out, cw_stream_t stream);

/* The cw_matvec_id contract for a batch of tokens, as grouped GEMMs on the matrix cores: picks are
 * grouped by slot, and each slot's picks multiply its matrix as one small matrix product (the
 * activations rounded to fp16 with a power-of-two scale per row: rel-L2 about 3e-4 against f64,
 * where cw_matvec_id's f32 path is about 1e-7; MXFP4 matrices above 128 weights per row run on
 * the block-scaled MFMA, FP4 weights as stored against three FP6 terms of each activation with
 * a power-of-two scale per 32 values: rel-L2 about 2e-5). Ids >= n_slots give NaN rows, as in
 * cw_matvec_id. x is 4-byte aligned (any f32 offset), k a multiple of 4. The workspace is sized by
 * cw_matmul_id_grouped_workspace_size (0 when the call is not supported).
 * CW_ENOTSUP (the caller falls back to cw_matvec_id) for a dtype without a grouped kernel, more
 * than 1024 slots, k above 8192, or rows that are not whole 256-weight super-blocks (Q8_0 and
 * MXFP4 need only whole blocks).
 * Replaces mv_id::matmul_id_grouped / matmul_id_piles (crates/engine/src/mv_id.rs:213-227,
 * 282-297), which MoeMatvec takes above 8 tokens (crates/engine/src/experts.rs:2225-2239), and
 * their Ok(false) probe. */
size_t cw_matmul_id_grouped_workspace_size(int dtype, int64_t n, int64_t k, int64_t n_slots,
                                           int64_t slot_stride, int x_rows_per_expert, int K, int T);
int cw_matmul_id_grouped(int dtype, int64_t n, int64_t k, int64_t n_slots, int64_t slot_stride,
                         const void *bank, const float *x, int x_rows_per_expert,
                         const uint32_t *ids, int K, int T, float *out, void *ws, size_t ws_bytes,
                         cw_stream_t stream);

/* CW_MXFP4 matrices into CW_MXFP4_R16, on the device: n_mats matrices of n rows of k weights
 * (src_stride bytes apart) to dst (dst_stride bytes apart, at least cw_rows16_bytes(n, k) each; dst
 * and dst_stride 16-byte aligned; not in place). k above 128, a multiple of 32.
 * No counterpart in the reference, which reads GGUF rows as stored: a device layout of the same
 * blocks, for callers that load expert matrices once and run the MoE layer on them. */
int64_t cw_rows16_bytes(int64_t n, int64_t k);
int cw_repack_rows16(const void *src, int64_t src_stride, void *dst, int64_t dst_stride, int64_t n_mats, int64_t n,
                     int64_t k, cw_stream_t stream);

/* ---- activations and combine ------------------------------------------------------------ */

/* h = silu(g) * u elementwise (cw_silu_mul, crates/engine/src/fuse_kernel.rs:77-85). */
int cw_swiglu(const float *g, const float *u, float *h, int64_t n, cw_stream_t stream);

/* gpt-oss clamped SwiGLU on rows of `width` (ExpertAct::ClampedSwiglu::hidden,
 * crates/engine/src/experts.rs:2384-2404): g += gate_b[ids[r]], u += up_b[ids[r]],
 * g = min(g, limit), u = clamp(u, -limit, limit), h = (u + 1) * g * sigmoid(alpha * g); output
 * rows are max(pad, width) wide with zeros past width. Biases are (E x width) or NULL. */
int cw_clamped_swiglu(const float *g, const float *u, const float *gate_b, const float *up_b,
                      const uint32_t *ids, int64_t rows, int width, int pad, float alpha,
                      float limit, float *h, cw_stream_t stream);

/* out[t][:] = sum_j w[t][j] * (down[t][j][:] + (down_b ? down_b[ids[t][j]][:] : 0)), summed in
 * pick order. Replaces cw_weighted_sum (crates/engine/src/fuse_kernel.rs:277-291, 377-398) and
 * ExpertAct::finish (crates/engine/src/experts.rs:2412-2415); ids may be NULL without down_b. */
int cw_weighted_sum(const float *down, const float *w, const float *down_b, const uint32_t *ids,
                    int T, int K, int H, float *out, cw_stream_t stream);

/* ---- bank slot table -------------------------------------------------------------------- */

/* slots[i] = table[ids[i]]; a CW_NO_SLOT entry resolves to slot 0 and adds 1 to *missing
 * (device u32; the caller zeroes it). Replaces coachwhip_resolve
 * (crates/engine/src/gpu_sync.rs:49-66, op 262-293). */
int cw_slots_resolve(const uint32_t *ids, const uint32_t *table, int n, uint32_t *slots,
                     uint32_t *missing, cw_stream_t stream);

/* ---- the MoE layer ---------------------------------------------------------------------- */

/* One MoE layer's experts. Matrices are slot-major as GGUF stores ffn_{gate,up,down}_exps:
 * gate and up are [slots][inter][hidden], down is [slots][hidden][max(pad, inter)]. */
typedef struct cw_moe_desc {
    int n_experts;           /* E: router width */
    int top_k;               /* K */
    int hidden;              /* h */
    int inter;               /* I: expert FFN width */
    int norm;                /* renormalise the K weights */
    int act;                 /* enum cw_act */
    float alpha, limit;      /* clamped SwiGLU constants (1.702, 7; model_gptoss.rs:16-17) */
    int pad;                 /* width down reads, >= inter; 0 = inter */
    int dtype[3];            /* gate, up, down */
    const void *w[3];        /* device bank of each matrix */
    int64_t slot_stride[3];  /* bytes per slot */
    const float *bias[3];    /* gate_b, up_b (E x inter), down_b (E x hidden), or NULL */
    const uint32_t *slot_table; /* device expert -> slot map (CW_NO_SLOT = absent), or NULL
                                   when slot == expert (all experts resident) */
    int n_slots;             /* slots per bank (= n_experts when slot_table is NULL) */
} cw_moe_desc;

/* out[T][hidden] = the resident MoE layer for T tokens: route the logits, gate and up
 * matvecs over the picked experts' slots, the activation, down, the weighted combine.
 * Replaces StreamedMoe::forward's resident branch (crates/engine/src/experts.rs:2562-2614)
 * and its bank branch with a slot map (3003-3015, with coachwhip_resolve). When slot_table is
 * set, picks whose expert has no slot read slot 0 and are counted in *missing (device u32,
 * may be NULL). ids_out / w_out (T x K, device, may be NULL) receive the routing.
 * The workspace (256-byte aligned) must be zero-filled once before its first use, for example
 * when it is allocated, and then belong to this layer's calls alone (not to a pool that hands the
 * bytes to other work between calls): its first CW_MOE_STATE_BYTES bytes hold the one-token
 * layer's sync state (arrival counters, which every call leaves at zero again, generation words,
 * which every call moves on together, and a marker word), at the same offset for every T (so one
 * workspace serves calls of any size). Zero-filling it again between calls is harmless. A call
 * that finds other bytes there (or a counter past its block count) uses no counter, gives NaN
 * outputs and counts the failure; the region must then be zero-filled again. Calls that overlap
 * in time need distinct workspaces (and one-token calls must not overlap any other work).
 * The u32 at byte CW_MOE_STATUS_OFFSET of the workspace counts, over the workspace's life, the
 * blocks of one-token calls whose barrier gave up or found the state invalid (their outputs are
 * NaN): a caller reads it on its stream (an asynchronous copy after the call), with no device
 * synchronize, and compares it with the value before the call. No counterpart in the reference
 * (its layer is several dispatches). */
#define CW_MOE_STATE_BYTES 8448
#define CW_MOE_STATUS_OFFSET 8320
size_t cw_moe_workspace_size(const cw_moe_desc *desc, int T);
int cw_moe_layer(const cw_moe_desc *desc, const float *x, const float *logits, int T, float *out,
                 uint32_t *ids_out, float *w_out, uint32_t *missing, void *ws, size_t ws_bytes,
                 cw_stream_t stream);

/* cw_moe_layer without a workspace, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation). No counterpart in the
 * reference. Its scratch is one static array per device in the library (CW_MOE_NOALLOC_BYTES,
 * held from the library's load until the process ends); a call whose cw_moe_workspace_size is
 * larger is refused with CW_EINVAL (config 3's shape fits about 90 tokens). The call allocates
 * nothing. Every call on a device shares that device's array: calls that overlap in time on one
 * device (on different streams, or from different threads) race and must not be made. Outputs
 * equal cw_moe_layer's bit for bit (the same kernels). */
#define CW_MOE_NOALLOC_BYTES ((size_t)8 << 20)
int cw_moe_layer_noalloc(const cw_moe_desc *desc, const float *x, const float *logits, int T,
                         float *out, uint32_t *ids_out, float *w_out, uint32_t *missing,
                         cw_stream_t stream);

/* The shared expert of a Qwen3.5/3.6 MoE block: every token uses it, scaled by its own sigmoid
 * gate. Dense quantized matrices as GGUF stores ffn_{gate,up,down}_shexp: gate and up are
 * inter x hidden, down is hidden x inter. */
typedef struct cw_shared_desc {
    int hidden;              /* h */
    int inter;               /* shared FFN width */
    int dtype[3];            /* gate, up, down */
    const void *w[3];        /* device matrices (raw GGUF blocks) */
    const float *gate_inp;   /* ffn_gate_inp_shexp: h floats on the device (16-byte aligned, h a
                                multiple of 4), or NULL (factor 1) */
} cw_shared_desc;

/* out[t] = sigmoid(x[t] . gate_inp) * down(silu(gate x[t]) * (up x[t])), added to out when
 * accumulate != 0 (the block sums routed and shared outputs). Replaces SharedExpert::forward
 * (crates/engine/src/model_next.rs:723-742; the sum at 1430-1437). x is T rows of hidden,
 * 16-byte aligned; ws from cw_shared_expert_workspace_size. */
size_t cw_shared_expert_workspace_size(const cw_shared_desc *desc, int T);
int cw_shared_expert(const cw_shared_desc *desc, const float *x, int T, float *out, int accumulate,
                     void *ws, size_t ws_bytes, cw_stream_t stream);

/* ---- GGUF files (host) -------------------------------------------------------------------- */

/* A GGUF file (versions 1-3): header, metadata and tensor directory read by cw_gguf_open, the
 * tensor data mapped read-only until cw_gguf_close. Follows candle's Content::read
 * (vendor/candle-core/src/quantized/gguf_file.rs:469-567: caps on lengths and nesting, tensor
 * data at the next multiple of general.alignment, default 32) and accepts IQ3_S (21) and IQ2_S
 * (22), which the reference rejects (quantized/mod.rs:314-339). NULL on error (cw_last_error). */
typedef struct cw_gguf cw_gguf;
cw_gguf *cw_gguf_open(const char *path);
void cw_gguf_close(cw_gguf *g);
int cw_gguf_version(const cw_gguf *g);
int64_t cw_gguf_n_tensors(const cw_gguf *g);
/* index of the tensor called name, or -1 */
int64_t cw_gguf_find(const cw_gguf *g, const char *name);
/* tensor i: name, GGUF type id, dims outermost first (as candle reports them; unused entries 0),
 * offset of its bytes from the start of the file, and their count. Pointers may be NULL. */
int cw_gguf_tensor(const cw_gguf *g, int64_t i, const char **name, int *dtype, int *n_dims,
                   int64_t dims[4], int64_t *file_offset, int64_t *bytes);
/* tensor i's bytes in the mapping (host memory), or NULL */
const void *cw_gguf_data(const cw_gguf *g, int64_t i);
/* metadata: an integer (any integer type or bool), a float (f32/f64), a string (NULL when
 * absent or of another type; owned by g) */
int cw_gguf_meta_int(const cw_gguf *g, const char *key, int64_t *v);
int cw_gguf_meta_float(const cw_gguf *g, const char *key, double *v);
const char *cw_gguf_meta_str(const cw_gguf *g, const char *key);
/* The experts of one layer: blk.{layer}.ffn_{gate,up,down}_exps.weight (which = 0, 1, 2) as
 * n_experts matrices of n rows by k, expert e at data + e * expert_bytes, the layout
 * cw_moe_desc takes as a bank once copied to the device (ExpertStore::new,
 * crates/engine/src/experts.rs:697-718). */
int cw_gguf_experts(const cw_gguf *g, int layer, int which, int *dtype, int64_t *n_experts,
                    int64_t *n, int64_t *k, int64_t *expert_bytes, const void **data);

/* Device-side failures on the current device since the library loaded: a one-token layer runs as
 * one persistent launch whose blocks meet at a device-wide barrier; a barrier wait that gives up
 * (a block could not be scheduled; CWMOE_BARRIER_POLLS in the environment sets the polls, 131072
 * by default) or a sync state that is not the layer's makes the call's outputs NaN and is counted
 * here (and in the workspace's status word, CW_MOE_STATUS_OFFSET, which needs no device
 * synchronize). No counterpart in the reference (its layer is several dispatches). Synchronizes
 * the device. */
uint32_t cw_device_errors(void);

/* ---- the shrink to Q2_K ----------------------------------------------------------------- */

/* dst (n_blocks x 84 bytes of Q2_K) = the GPU shrink of n_blocks super-blocks of src (Q3_K,
 * Q4_K or Q5_K): each super-block dequantized, each sub-block of 16 fitted by min/max and two
 * weighted least-squares rounds, scales and mins put on 4 bits against the block's largest,
 * quants rounded to 2 bits. Replaces Requant::run (crates/engine/src/requant.rs:361-380,
 * kernels 228-304) and, with shape != NULL, Requant::run_shaped (385-406): value i of block b
 * is then weighted by sqrt(max(shape[(b % blocks_per_row) * 256 + i], 0)) + 1e-6, shape
 * holding one f32 per column of a row of blocks_per_row super-blocks. Unlike the reference,
 * which waits for the GPU, the call only enqueues. CW_ENOTSUP for another source type. */
int cw_requant_q2k(int src_dtype, const void *src, int64_t n_blocks, const float *shape,
                   int64_t blocks_per_row, void *dst, cw_stream_t stream);

/* ---- host bank bookkeeping (no GPU) ----------------------------------------------------- */

/* The expert bank's slot bookkeeping without its memory: Slots in
 * crates/engine/src/experts.rs:84-286 (new 222-224, assign 227-248, release 251-258,
 * pop 261-269, reserve 273-285). A handle is owned by one thread at a time.
 * `ready` is a host array of n_slots flags (NULL = every slot ready). */
typedef struct cw_slots cw_slots;
cw_slots *cw_slots_new(int n_slots);
void cw_slots_free(cw_slots *s);
/* Returns 1 and fills hit/miss lists ((expert, slot) pairs, host arrays sized n_needed) and
 * *prefetch_hits on success; 0 and no change when too few slots are free (the caller then reads
 * the experts fresh); -1 on a bad argument. */
int cw_slots_assign(cw_slots *s, const uint32_t *needed, int n_needed, const uint8_t *ready,
                    uint32_t *hits, int *n_hits, uint32_t *misses, int *n_misses,
                    uint64_t *prefetch_hits);
void cw_slots_release(cw_slots *s, uint32_t expert);
void cw_slots_pop(cw_slots *s, const uint32_t *used, int n);
/* Reserves slots for predicted experts not yet held; returns how many (expert, slot) pairs
 * were written to out (sized n_predicted). */
int cw_slots_reserve(cw_slots *s, const uint32_t *predicted, int n_predicted,
                     const uint8_t *ready, uint32_t *out);
/* Introspection for tests: holder of a slot (CW_NO_SLOT if empty), slot of an expert
 * (-1 if absent), the LRU order (least recent first, n_slots entries), prefetched flag. */
uint32_t cw_slots_holder(const cw_slots *s, int slot);
int cw_slots_slot_of(const cw_slots *s, uint32_t expert);
void cw_slots_lru(const cw_slots *s, int *order);
int cw_slots_is_prefetched(const cw_slots *s, uint32_t expert);
/* Writes the expert -> slot table for experts [0, n_experts) (CW_NO_SLOT when absent), the
 * host image of Bank::sync_table (crates/engine/src/experts.rs:73-81). */
void cw_slots_table(const cw_slots *s, uint32_t *table, int n_experts);

/* ---- expert banks on the device (host manager) ----------------------------------------- */

/* Where a layer's experts come from: matrix m (gate, up, down) of expert e is expert_bytes[m]
 * bytes at host[m] + e * expert_bytes[m], rows[m] x cols[m] weights of GGUF type dtype[m]
 * (cw_gguf_experts gives these for a GGUF file), and must hold n_experts experts of each.
 * Host memory from hipHostMalloc (which the device can address) is read by the bank's fill
 * kernel over PCIe without blocking the host; other host memory is copied by DMA, each copy
 * returning once HIP has staged its bytes. */
typedef struct cw_bank_source {
    int n_experts;
    int dtype[3];
    int64_t rows[3], cols[3];
    int64_t expert_bytes[3];
    const void *host[3];
    /* nonzero: matrix m (Q3_K, Q4_K or Q5_K in the store) is held in the slots as Q2_K, shrunk on
     * arrival as cw_requant_q2k does (ExpertStore::shrink_into, experts.rs:1245-1273) */
    int shrink[3];
    /* with shrink: cols[m] f32 column weights on the device (run_shaped), or NULL */
    const float *shape[3];
} cw_bank_source;

typedef struct cw_bank_stats {
    uint64_t hits;            /* needed experts already in a slot */
    uint64_t prefetch_hits;   /* ... of which a prefetch brought in */
    uint64_t loads;           /* experts copied in by cw_bank_ensure */
    uint64_t bytes_loaded;    /* their bytes */
    uint64_t prefetch_copies; /* experts copied in by cw_bank_prefetch */
    uint64_t crowded;         /* ensure calls refused for too few free slots */
} cw_bank_stats;

/* One layer's expert bank on the current device: n_slots slots of each matrix (slot-major, one
 * expert's matrix per slot), the device expert -> slot table (CW_NO_SLOT when absent), the LRU
 * bookkeeping of cw_slots, and the host source. Replaces ExpertStore's Bank and make_bank
 * (crates/engine/src/experts.rs:62-82, 1320-1378), GpuBank's table (gpu_sync.rs:70-148) and
 * sync_table (experts.rs:73-81); the bytes cross PCIe from host memory instead of being read
 * from the SSD into shared memory. Device memory comes from the caller: device_mem holds
 * cw_bank_device_bytes(src, n_slots) bytes (256-byte aligned) for the bank's lifetime. The
 * source's host memory must outlive the bank. A handle is used by one thread at a time, and
 * its ensure calls, and the work that reads the bank, go on one stream. NULL on error
 * (cw_last_error). */
typedef struct cw_bank cw_bank;
size_t cw_bank_device_bytes(const cw_bank_source *src, int n_slots);
cw_bank *cw_bank_new(const cw_bank_source *src, int n_slots, void *device_mem, size_t bytes);
/* Waits for the bank's copies, then releases its HIP stream and events. */
void cw_bank_free(cw_bank *b);

/* Places every expert in needed (duplicates ignored) in a slot before any later work on stream:
 * the plain branch of ExpertStore::ensure (experts.rs:1489-1641). Hits stay; misses take the
 * least recently used slots that no needed expert holds and no prefetch is filling, and their
 * bytes are copied in on stream; a hit still being prefetched is waited for on stream (not on
 * the host); the device table is brought up to date on stream. CW_EFULL, and nothing changed,
 * when more experts are needed than the bank has slots or too few slots are free (the
 * reference's Ok(None)). *n_loaded (may be NULL) receives the number of misses copied. Work
 * that reads the bank for these experts goes on stream after this call and reads only experts
 * placed here (a prefetch may since have taken any other slot, and takes its expert out of the
 * table first); the slots placed here are kept from prefetches until the next ensure. */
int cw_bank_ensure(cw_bank *b, const uint32_t *needed, int n_needed, cw_stream_t stream, int *n_loaded);
/* Reserves slots for predicted experts not yet held (Slots::reserve, experts.rs:273-285; the
 * prefetch of experts.rs:1004-1098) and copies them in on the bank's own copy stream, after
 * the work queued on the last ensure's stream up to this call. The experts whose slots are
 * taken leave the device table first, in that stream's order (experts.rs:1052-1058: the slot is
 * marked not ready and the GPU table synced before the copy), so later work there counts them
 * missing instead of reading a slot being overwritten; that stream must still exist. Slots being
 * filled are not taken by ensure and are waited for on the stream when needed. Returns the number
 * of experts reserved (>= 0), or a negative status. */
int cw_bank_prefetch(cw_bank *b, const uint32_t *predicted, int n_predicted);
/* Fills the bank fields of a layer descriptor: dtype (CW_Q2_K for a shrunk matrix), w and
 * slot_stride of the three matrices, slot_table and n_slots (cw_moe_layer then resolves picks
 * through the table). */
int cw_bank_fill_desc(const cw_bank *b, cw_moe_desc *d);
/* The device expert -> slot table (n_experts u32), the slot of an expert in the host
 * bookkeeping (-1 if none), counters. */
const uint32_t *cw_bank_table(const cw_bank *b);
int cw_bank_slot_of(const cw_bank *b, uint32_t expert);
void cw_bank_get_stats(const cw_bank *b, cw_bank_stats *out);

#ifdef __cplusplus
}
#endif
#endif
