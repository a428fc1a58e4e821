// Wavefront-level helpers (wave64): cross-lane reductions and the router's top-k.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace cw {

// Cross-lane steps without LDS traffic: DPP moves within 16-lane rows, readlane across rows.
// DPP controls (GCN3+ encoding): quad_perm [1,0,3,2] = 0xB1 and [2,3,0,1] = 0x4E swap lanes
// 1 and 2 apart; row_half_mirror (0x141) pairs quads of an 8-lane half-row, row_mirror (0x140)
// pairs the two halves of a row. After the four steps every lane holds its row's reduction.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// sum over groups of G consecutive lanes (G = 8, 16, 32 or 64), the result in every lane
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    if constexpr (G >= 16) v += dpp_f<0x140>(v);
    if constexpr (G == 32) v += __shfl_xor(v, 16);
    if constexpr (G == 64) v = (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// (value, index) order of the router: larger value first, the lower index among equals;
// index ~0u marks an exhausted candidate.
__device__ __forceinline__ bool route_better(float va, uint32_t ia, float vb, uint32_t ib) {
    if (ia == 0xFFFFFFFFu) return false;
    if (ib == 0xFFFFFFFFu) return true;
    return va > vb || (va == vb && ia < ib);
}

template <int CTRL>
__device__ __forceinline__ void argmax_step(float &v, uint32_t &i) {
    const float ov = dpp_f<CTRL>(v);
    const uint32_t oi = dpp_u<CTRL>(i);
    if (route_better(ov, oi, v, i)) { v = ov; i = oi; }
}

// the best (value, index) of the wave, in every lane
__device__ __forceinline__ void wave_argmax(float &v, uint32_t &i) {
    argmax_step<0xB1>(v, i);
    argmax_step<0x4E>(v, i);
    argmax_step<0x141>(v, i);
    argmax_step<0x140>(v, i);
    float bv = readlane_f(v, 0);
    uint32_t bi = (uint32_t)__builtin_amdgcn_readlane((int)i, 0);
#pragma unroll
    for (int row = 16; row < 64; row += 16) {
        const float rv = readlane_f(v, row);
        const uint32_t ri = (uint32_t)__builtin_amdgcn_readlane((int)i, row);
        if (route_better(rv, ri, bv, bi)) { bv = rv; bi = ri; }
    }
    v = bv;
    i = bi;
}

// One wavefront routes one token: softmax over E = 64*PER (or fewer) logits as candle-nn's
// softmax_last_dim computes it (max, exp of the differences, sum, divide), then the K best
// picks, best first, the lowest index winning ties (the stable descending argsort of
// crates/engine/src/experts.rs:2364-2372). Picks are made on the logits themselves: softmax is
// monotone and comparing logits is exact. Lane j < K returns pick j's expert in *id and its
// weight (renormalised over the K when norm) in *w; other lanes return id ~0u.
template <int PER>
__device__ __forceinline__ void wave_route(const float *logits, int E, int K, int norm, uint32_t *id, float *w) {
    const int lane = threadIdx.x & 63;
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int e = lane + 64 * i;
        v[i] = e < E ? logits[e] : -INFINITY;
    }
    float m = v[0];
#pragma unroll
    for (int i = 1; i < PER; i++) m = fmaxf(m, v[i]);
    m = wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < PER; i++) s += (lane + 64 * i < E) ? expf(v[i] - m) : 0.f;
    s = wave_sum(s);
    uint32_t taken = 0;  // bit i: v[i] already picked
    uint32_t my_id = 0xFFFFFFFFu;
    float my_v = 0.f;
    for (int j = 0; j < K; j++) {
        float bv = -INFINITY;
        uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const uint32_t e = (uint32_t)(lane + 64 * i);
            if (e < (uint32_t)E && !((taken >> i) & 1u) && route_better(v[i], e, bv, bi)) { bv = v[i]; bi = e; }
        }
        wave_argmax(bv, bi);
        if ((bi & 63u) == (uint32_t)lane) taken |= 1u << (bi >> 6);
        if (lane == j) { my_id = bi; my_v = bv; }
    }
    float p = lane < K ? expf(my_v - m) / s : 0.f;
    if (norm) p = p / wave_sum(p);
    *id = my_id;
    *w = p;
}

}  // namespace cw
