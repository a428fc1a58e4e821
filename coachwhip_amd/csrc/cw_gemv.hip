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

// Dense matvec (one matrix, blockIdx.y = row t of x). Each wave takes P consecutive passes of
// 64/LPR rows and requests all of their weight bytes at once; the block stages x[t] in LDS once
// (every lane needs its slice of x for every row it visits: one copy per block instead of one per
// wave) with the x loads issued behind the weight loads, so a wave waits for its memory once. Every
// load is unconditional, from a clamped address: a load under a branch makes the compiler wait
// for it at the branch's end, which serializes the round trips.
template <class Fmt, int LPR, int NX, int P>
__global__ __launch_bounds__(256) void k_gemv_dense(const GemvArgs a) {
    __shared__ __align__(16) uint8_t lds[Fmt::LDS_BYTES > 0 ? Fmt::LDS_BYTES : 16];
    extern __shared__ __align__(16) float xs[];
    constexpr int RPW = 64 / LPR, XV = (NX * LPR * 8 + 255) / 256;  // float4 pieces of x per thread
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, rsub = lane / LPR;
    const int t = blockIdx.y;
    const int r0 = (blockIdx.x * 4 + wave) * P * RPW + rsub;
    typename Fmt::Raw raw[P][NX];
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int r = min(r0 + p * RPW, a.n - 1);  // rows past the matrix: unused
#pragma unroll
        for (int i = 0; i < NX; i++) {
            const int sb = sub + i * LPR;
            raw[p][i] = Fmt::load(a.w0 + (int64_t)r * a.row_bytes, sb < a.nsb ? sb : a.nsb - 1);
        }
    }
    const float4 *xg = (const float4 *)(a.x + (int64_t)t * a.k);
    const int nx4 = a.k / 4;
    float4 xv[XV];
#pragma unroll
    for (int v = 0; v < XV; v++) {
        const int i = threadIdx.x + 256 * v;
        xv[v] = xg[i < nx4 ? i : nx4 - 1];
    }
    // unconditional stores: xs holds 256 * XV pieces, those past x are never read
#pragma unroll
    for (int v = 0; v < XV; v++) ((float4 *)xs)[threadIdx.x + 256 * v] = xv[v];
    Fmt::fill_lds(lds, threadIdx.x, blockDim.x);
    __syncthreads();
    float xr[NX][32], xsum[NX][2];
#pragma unroll
    for (int i = 0; i < NX; i++) {
        const int sb = sub + i * LPR;
        const float4 *src = (const float4 *)(xs + 32 * (sb < a.nsb ? sb : 0));
#pragma unroll
        for (int v = 0; v < 8; v++) *(float4 *)(xr[i] + 4 * v) = src[v];
        half_sums(xr[i], xsum[i]);
    }
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int r = r0 + p * RPW;
        float g = 0.f;
#pragma unroll
        for (int i = 0; i < NX; i++) {
            const int sb = sub + i * LPR;
            if (r < a.n && sb < a.nsb) g += dot_xs<Fmt>(raw[p][i], lds, xr[i], xsum[i]);
        }
        g = group_sum<LPR>(g);
        if (sub == 0 && r < a.n) a.out[(int64_t)t * a.out_width + r] = g;
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
    case CW_Q5_K: return launch_lpr<FQ5_K>(a, grid, threads, shmem, s);
    case CW_Q6_K: return launch_lpr<FQ6_K>(a, grid, threads, shmem, s);
    case CW_IQ3_XXS: return launch_lpr<FIQ3_XXS>(a, grid, threads, shmem, s);
    case CW_IQ4_XS: return launch_lpr<FIQ4_XS>(a, grid, threads, shmem, s);
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

template <class Fmt, int LPR, int NX>
static int dense_launch(const GemvArgs &a, int m, hipStream_t s) {
    constexpr int RPW = 64 / LPR;
    // about 2048 waves (two 4-wave blocks per CU) of 1, 2 or 4 passes each
    const int64_t passes_all = (a.n + RPW - 1) / RPW;
    const int64_t want = (passes_all + 2047) / 2048;
    const int P = want <= 1 ? 1 : want <= 2 ? 2 : 4;
    const int64_t waves = (passes_all + P - 1) / P;
    const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)m);
    const size_t shmem = (size_t)256 * 16 * ((NX * LPR * 8 + 255) / 256);  // x staging, padded (k_gemv_dense)
    if (P == 1) hipLaunchKernelGGL((k_gemv_dense<Fmt, LPR, NX, 1>), grid, dim3(256), shmem, s, a);
    else if (P == 2) hipLaunchKernelGGL((k_gemv_dense<Fmt, LPR, NX, 2>), grid, dim3(256), shmem, s, a);
    else hipLaunchKernelGGL((k_gemv_dense<Fmt, LPR, NX, 4>), grid, dim3(256), shmem, s, a);
    return check_launch("k_gemv_dense");
}

template <class Fmt>
static int dense_lpr(const GemvArgs &a, int m, hipStream_t s) {
    const int lpr = pick_lpr(a.nsb);
    const int nx = (a.nsb + lpr - 1) / lpr;
#define CW_DENSE_CASE(L, X) \
    if (lpr == L && nx == X) return dense_launch<Fmt, L, X>(a, m, s);
    CW_DENSE_CASE(8, 1) CW_DENSE_CASE(16, 1) CW_DENSE_CASE(32, 1) CW_DENSE_CASE(64, 1)
    CW_DENSE_CASE(64, 2) CW_DENSE_CASE(64, 3) CW_DENSE_CASE(64, 4)
#undef CW_DENSE_CASE
    return set_error(CW_ENOTSUP, "gemv: rows of %d weights exceed the %d-weight limit", a.k, 64 * 4 * 32);
}

int gemv_dense(int dtype, const GemvArgs &a, int m, hipStream_t s) {
    if (m == 0 || a.n == 0) return CW_OK;
    if (a.k % 4) return set_error(CW_ENOTSUP, "gemv: row of %d weights is not whole float4s", a.k);
    switch (dtype) {
    case CW_Q8_0: return dense_lpr<FQ8_0>(a, m, s);
    case CW_Q2_K: return dense_lpr<FQ2_K>(a, m, s);
    case CW_Q4_K: return dense_lpr<FQ4_K>(a, m, s);
    case CW_MXFP4: return dense_lpr<FMXFP4>(a, m, s);
    case CW_IQ2_XXS: return dense_lpr<FIQ2_XXS>(a, m, s);
    case CW_IQ2_S: return dense_lpr<FIQ2_S>(a, m, s);
    case CW_IQ3_S: return dense_lpr<FIQ3_S>(a, m, s);
    case CW_Q5_K: return dense_lpr<FQ5_K>(a, m, s);
    case CW_Q6_K: return dense_lpr<FQ6_K>(a, m, s);
    case CW_IQ3_XXS: return dense_lpr<FIQ3_XXS>(a, m, s);
    case CW_IQ4_XS: return dense_lpr<FIQ4_XS>(a, m, s);
    default: return set_error(CW_ENOTSUP, "gemv: dtype %d is not supported", dtype);
    }
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
    case CW_Q5_K: hipLaunchKernelGGL(k_dequant<FQ5_K>, grid, dim3(256), 0, s, b, n_sub, out); break;
    case CW_Q6_K: hipLaunchKernelGGL(k_dequant<FQ6_K>, grid, dim3(256), 0, s, b, n_sub, out); break;
    case CW_IQ3_XXS: hipLaunchKernelGGL(k_dequant<FIQ3_XXS>, grid, dim3(256), 0, s, b, n_sub, out); break;
    case CW_IQ4_XS: hipLaunchKernelGGL(k_dequant<FIQ4_XS>, grid, dim3(256), 0, s, b, n_sub, out); break;
    default: return set_error(CW_ENOTSUP, "dequantize: dtype %d is not supported", dtype);
    }
    return check_launch("k_dequant");
}

}  // namespace cw
