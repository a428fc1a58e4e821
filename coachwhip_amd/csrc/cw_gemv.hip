// Dequantize and matrix-vector kernels over raw GGUF blocks (gfx950, wave64).
//
// One kernel template, k_gemv, serves the dense quantized matvec (QMatMul at small M) and the
// expert matvec over a bank of slots (MoeMatvec); the fused MoE-layer kernels live in
// cw_moe_fused.hip:
//
//  - A row of k weights is nsb = k/32 sub-blocks. LPR lanes of a wavefront share one row
//    (LPR = 8, 16, 32 or 64, the smallest power of two >= nsb, capped at 64) and lane l always
//    takes sub-blocks l % LPR + i*LPR, i < NX, so its activation slice stays in registers for
//    every row the wave visits. A wave covers 64/LPR rows per pass; partial dots are summed
//    across the LPR lanes with cross-lane shuffles.
//  - Weights are read once, straight from their blocks (unaligned dword loads); IQ lattice
//    tables sit in LDS.
#include "cw_common.h"
#include "cw_device.h"
#include "cw_gemv.h"
#include "cw_wave.h"

namespace cw {

template <int NX>
__device__ __forceinline__ void load_x(float (&xr)[NX][32], const float *xrow, int sub, int lpr, int nsb) {
#pragma unroll
    for (int i = 0; i < NX; i++) {
        int sb = sub + i * lpr;
        if (sb < nsb) {
            const float4 *p = (const float4 *)(xrow + 32 * sb);
#pragma unroll
            for (int v = 0; v < 8; v++) {
                float4 f = p[v];
                xr[i][4 * v] = f.x; xr[i][4 * v + 1] = f.y; xr[i][4 * v + 2] = f.z; xr[i][4 * v + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int v = 0; v < 32; v++) xr[i][v] = 0.f;
        }
    }
}

template <class Fmt, int LPR, int NX>
__device__ __forceinline__ float row_dot(const uint8_t *row, const void *lds, const float (&xr)[NX][32], int sub, int nsb) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NX; i++) {
        int sb = sub + i * LPR;
        if (sb < nsb) acc += Fmt::dot(Fmt::load(row, sb), lds, xr[i]);
    }
    return acc;
}

// blockIdx.y = pick p (a token of a dense matmul, or a (token, expert pick) of an expert
// matvec); the block's waves stride over the n rows of that pick's matrix.
template <class Fmt, int LPR, int NX>
__global__ __launch_bounds__(256) void k_gemv(const GemvArgs a) {
    __shared__ __align__(16) uint8_t lds[Fmt::LDS_BYTES > 0 ? Fmt::LDS_BYTES : 16];
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int sub = lane % LPR, rsub = lane / LPR;
    const int p = blockIdx.y;
    const uint32_t slot = a.ids ? a.ids[p] : 0u;
    const bool bad = slot >= (uint32_t)a.n_slots;
    float xr[NX][32];
    load_x<NX>(xr, a.x + (int64_t)(a.x_per_pick ? p : p / a.K) * a.k, sub, LPR, a.nsb);
    Fmt::fill_lds(lds, threadIdx.x, blockDim.x);
    if (Fmt::LDS_BYTES > 0) __syncthreads();
    const uint8_t *base = a.w0 + (int64_t)(bad ? 0 : slot) * a.slot_stride0;
    for (int r0 = (blockIdx.x * nwaves + wave) * RPW; r0 < a.n; r0 += gridDim.x * nwaves * RPW) {
        const int r = r0 + rsub;
        float g = 0.f;
        if (r < a.n) g = row_dot<Fmt, LPR, NX>(base + (int64_t)r * a.row_bytes, lds, xr, sub, a.nsb);
        g = group_sum<LPR>(g);
        if (sub == 0 && r < a.n) a.out[(int64_t)p * a.out_width + r] = bad ? __int_as_float(0x7fc00000) : g;
    }
}

template <class Fmt>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t *blocks, int64_t n_sub, float *out) {
    __shared__ __align__(16) uint8_t lds[Fmt::LDS_BYTES > 0 ? Fmt::LDS_BYTES : 16];
    Fmt::fill_lds(lds, threadIdx.x, blockDim.x);
    if (Fmt::LDS_BYTES > 0) __syncthreads();
    for (int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; s < n_sub; s += (int64_t)gridDim.x * blockDim.x) {
        // sub-block s of a flat run of blocks: block s / (BS/32), sub-block s % (BS/32)
        constexpr int SPB = Fmt::BS / 32;
        const uint8_t *blk = blocks + (s / SPB) * Fmt::TS;
        float y[32];
        Fmt::dequant(Fmt::load(blk, (int)(s % SPB)), lds, y);
        float4 *o = (float4 *)(out + 32 * s);
#pragma unroll
        for (int v = 0; v < 8; v++) o[v] = make_float4(y[4 * v], y[4 * v + 1], y[4 * v + 2], y[4 * v + 3]);
    }
}

// ------------------------------------------------------------------------------ dispatch

static int pick_lpr(int nsb) {
    int l = 8;
    while (l < nsb && l < 64) l <<= 1;
    return l;
}

template <class Fmt>
static int launch_lpr(const GemvArgs &a, dim3 grid, int threads, size_t shmem, hipStream_t s) {
    const int lpr = pick_lpr(a.nsb);
    const int nx = (a.nsb + lpr - 1) / lpr;
#define CW_GEMV_CASE(L, X) \
    if (lpr == L && nx == X) { hipLaunchKernelGGL((k_gemv<Fmt, L, X>), grid, dim3(threads), shmem, s, a); return check_launch("k_gemv"); }
    CW_GEMV_CASE(8, 1) CW_GEMV_CASE(16, 1) CW_GEMV_CASE(32, 1) CW_GEMV_CASE(64, 1)
    CW_GEMV_CASE(64, 2) CW_GEMV_CASE(64, 3) CW_GEMV_CASE(64, 4)
#undef CW_GEMV_CASE
    return set_error(CW_ENOTSUP, "gemv: rows of %d weights exceed the %d-weight limit", a.k, 64 * 4 * 32);
}

static int launch_fmt(int dtype, const GemvArgs &a, dim3 grid, int threads, size_t shmem, hipStream_t s) {
    switch (dtype) {
    case CW_Q8_0: return launch_lpr<FQ8_0>(a, grid, threads, shmem, s);
    case CW_Q2_K: return launch_lpr<FQ2_K>(a, grid, threads, shmem, s);
    case CW_Q4_K: return launch_lpr<FQ4_K>(a, grid, threads, shmem, s);
    case CW_MXFP4: return launch_lpr<FMXFP4>(a, grid, threads, shmem, s);
    case CW_IQ2_XXS: return launch_lpr<FIQ2_XXS>(a, grid, threads, shmem, s);
    case CW_IQ2_S: return launch_lpr<FIQ2_S>(a, grid, threads, shmem, s);
    case CW_IQ3_S: return launch_lpr<FIQ3_S>(a, grid, threads, shmem, s);
    default: return set_error(CW_ENOTSUP, "gemv: dtype %d is not supported", dtype);
    }
}

int max_gemv_k() { return 64 * 4 * 32; }

// rows per block for PLAIN / GATEUP: 4 waves, one pass each
static dim3 rows_grid(const GemvArgs &a, int picks) {
    const int lpr = pick_lpr(a.nsb);
    const int rows_per_block = 4 * (64 / lpr);
    return dim3((a.n + rows_per_block - 1) / rows_per_block, picks);
}

int gemv_plain(int dtype, const GemvArgs &a, int picks, hipStream_t s) {
    if (picks == 0 || a.n == 0) return CW_OK;
    return launch_fmt(dtype, a, rows_grid(a, picks), 256, 0, s);
}

int dequantize(int dtype, const void *blocks, int64_t n_elems, float *out, hipStream_t s) {
    const int64_t n_sub = n_elems / 32;
    if (n_sub == 0) return CW_OK;
    int64_t blocks_needed = (n_sub + 255) / 256;
    dim3 grid((unsigned)(blocks_needed < 4096 ? blocks_needed : 4096));
    const uint8_t *b = (const uint8_t *)blocks;
    switch (dtype) {
    case CW_Q8_0: hipLaunchKernelGGL(k_dequant<FQ8_0>, grid, dim3(256), 0, s, b, n_sub, out); break;
    case CW_Q2_K: hipLaunchKernelGGL(k_dequant<FQ2_K>, grid, dim3(256), 0, s, b, n_sub, out); break;
    case CW_Q4_K: hipLaunchKernelGGL(k_dequant<FQ4_K>, grid, dim3(256), 0, s, b, n_sub, out); break;
    case CW_MXFP4: hipLaunchKernelGGL(k_dequant<FMXFP4>, grid, dim3(256), 0, s, b, n_sub, out); break;
    case CW_IQ2_XXS: hipLaunchKernelGGL(k_dequant<FIQ2_XXS>, grid, dim3(256), 0, s, b, n_sub, out); break;
    case CW_IQ2_S: hipLaunchKernelGGL(k_dequant<FIQ2_S>, grid, dim3(256), 0, s, b, n_sub, out); break;
    case CW_IQ3_S: hipLaunchKernelGGL(k_dequant<FIQ3_S>, grid, dim3(256), 0, s, b, n_sub, out); break;
    default: return set_error(CW_ENOTSUP, "dequantize: dtype %d is not supported", dtype);
    }
    return check_launch("k_dequant");
}

}  // namespace cw
