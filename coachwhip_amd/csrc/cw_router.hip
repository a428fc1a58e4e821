// Router logits: logits[t][e] = x[t] . W[e] (+ bias[e]) for the router weight W (E x h), f32 or
// f16 weights, f32 activations and accumulation.
//
// Replaces the engine's gate Linear (crates/engine/src/experts.rs:2428, 2577; the weight is
// dequantized to f32 at load, model_next.rs:1036; gpt-oss adds a bias, model_gptoss.rs:168-175)
// and its f16 decode variant cw_mv_f16 (crates/engine/src/fuse_kernel.rs:160-178, 537-559).
//
//  - A few tokens (decode): one wave per expert row; lanes stride the row in 4-element pieces,
//    each piece of W read once and used for every token; a DPP wave sum per token.
//  - Many tokens (prefill): a 64-expert x 64-token tile per block, K in chunks of 32 staged in
//    LDS (k-major, so a thread's 4 experts and 4 tokens are one 16-byte read each), 4 x 4
//    outputs per thread.
#include "cw_common.h"
#include "cw_router.h"
#include "cw_wave.h"

namespace cw {

template <class WT>
__device__ __forceinline__ float4 load4(const WT *p);
template <>
__device__ __forceinline__ float4 load4<float>(const float *p) {
    return *(const float4 *)p;
}
template <>
__device__ __forceinline__ float4 load4<_Float16>(const _Float16 *p) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 v = *(const h4 *)p;
    return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}

constexpr int ROUTER_FEW = 8;  // tokens up to which the per-row kernel runs

template <class WT, int TT>
__global__ __launch_bounds__(256) void k_router_rows(const WT *w, const float *bias, const float *x, int E, int h, int T,
                                                     float *logits) {
    const int lane = threadIdx.x & 63, e = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (e >= E) return;  // whole wave
    const WT *wr = w + (int64_t)e * h;
    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) acc[t] = 0.f;
    for (int k = 4 * lane; k < h; k += 256) {
        const float4 a = load4<WT>(wr + k);
#pragma unroll
        for (int t = 0; t < TT; t++) {
            if (t >= T) break;
            const float4 b = *(const float4 *)(x + (int64_t)t * h + k);
            acc[t] = fmaf(a.x, b.x, fmaf(a.y, b.y, fmaf(a.z, b.z, fmaf(a.w, b.w, acc[t]))));
        }
    }
    const float be = bias ? bias[e] : 0.f;
#pragma unroll
    for (int t = 0; t < TT; t++) {
        if (t >= T) break;
        const float s = wave_sum(acc[t]);
        if (lane == 0) logits[(int64_t)t * E + e] = s + be;
    }
}

template <class WT>
__global__ __launch_bounds__(256) void k_router_tiles(const WT *w, const float *bias, const float *x, int E, int h, int T,
                                                      float *logits) {
    constexpr int TE = 64, TTK = 64, KC = 32, PAD = 4;
    __shared__ __align__(16) float Ws[KC][TE + PAD], Xs[KC][TTK + PAD];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int e0 = blockIdx.x * TE, t0 = blockIdx.y * TTK;
    float acc[4][4] = {};
    // loader: thread tid copies 4 consecutive k of row (tid >> 3) and (tid >> 3) + 32, piece tid & 7
    const int lr = tid >> 3, lk = 4 * (tid & 7);
    for (int kc = 0; kc < h; kc += KC) {
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const int r = lr + 32 * half;
            const int e = e0 + r, t = t0 + r, k = kc + lk;
            const float4 a = e < E && k < h ? load4<WT>(w + (int64_t)e * h + k) : make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 b = t < T && k < h ? *(const float4 *)(x + (int64_t)t * h + k) : make_float4(0.f, 0.f, 0.f, 0.f);
            Ws[lk][r] = a.x; Ws[lk + 1][r] = a.y; Ws[lk + 2][r] = a.z; Ws[lk + 3][r] = a.w;
            Xs[lk][r] = b.x; Xs[lk + 1][r] = b.y; Xs[lk + 2][r] = b.z; Xs[lk + 3][r] = b.w;
        }
        __syncthreads();
#pragma unroll 8
        for (int k = 0; k < KC; k++) {
            const float4 a = *(const float4 *)&Ws[k][4 * tx];
            const float4 b = *(const float4 *)&Xs[k][4 * ty];
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int t = t0 + 4 * ty + j;
        if (t >= T) break;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = e0 + 4 * tx + i;
            if (e < E) logits[(int64_t)t * E + e] = acc[i][j] + (bias ? bias[e] : 0.f);
        }
    }
}

template <class WT>
static int launch(const void *w, const float *bias, const float *x, int E, int h, int T, float *logits, hipStream_t s) {
    const WT *wt = (const WT *)w;
    if (T <= ROUTER_FEW) {
        const dim3 grid((E + 3) / 4);
#define CW_ROWS(N) \
    if (T <= N) { hipLaunchKernelGGL((k_router_rows<WT, N>), grid, dim3(256), 0, s, wt, bias, x, E, h, T, logits); return check_launch("k_router_rows"); }
        CW_ROWS(1) CW_ROWS(2) CW_ROWS(4) CW_ROWS(8)
#undef CW_ROWS
    }
    hipLaunchKernelGGL((k_router_tiles<WT>), dim3((E + 63) / 64, (T + 63) / 64), dim3(256), 0, s, wt, bias, x, E, h, T, logits);
    return check_launch("k_router_tiles");
}

int router_logits(int wdtype, const void *w, int E, int h, const float *bias, const float *x, int T, float *logits,
                  hipStream_t s) {
    if (T == 0 || E == 0) return CW_OK;
    if (h % 4) return set_error(CW_ENOTSUP, "router: hidden %d is not a multiple of 4", h);
    switch (wdtype) {
    case CW_F32: return launch<float>(w, bias, x, E, h, T, logits, s);
    case CW_F16: return launch<_Float16>(w, bias, x, E, h, T, logits, s);
    default: return set_error(CW_ENOTSUP, "router: weight dtype %d (f32 or f16 only)", wdtype);
    }
}

}  // namespace cw
