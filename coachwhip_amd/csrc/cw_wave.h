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

// Router key: the float's bits made order-preserving as an unsigned number, above the bitwise
// complement of the expert index. The unsigned maximum is then the largest logit, the lowest
// index among equal logits (the stable descending argsort's order), and 0 marks a taken or absent
// candidate (every real key is above it).
__device__ __forceinline__ uint64_t route_key(float v, uint32_t e) {
    const uint32_t b = __float_as_uint(v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (uint64_t)(0xFFFFFFFFu - e);
}
__device__ __forceinline__ float key_value(uint64_t k) {
    const uint32_t o = (uint32_t)(k >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}
__device__ __forceinline__ uint32_t key_index(uint64_t k) { return 0xFFFFFFFFu - (uint32_t)k; }

template <int CTRL>
__device__ __forceinline__ uint64_t max_step(uint64_t k) {
    const uint64_t o = ((uint64_t)dpp_u<CTRL>((uint32_t)(k >> 32)) << 32) | dpp_u<CTRL>((uint32_t)k);
    return o > k ? o : k;
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t k, int lane) {
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(k >> 32), lane) << 32) |
           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, lane);
}
// the largest key of the wave, in every lane
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
    k = max_step<0xB1>(k);
    k = max_step<0x4E>(k);
    k = max_step<0x141>(k);
    k = max_step<0x140>(k);
    uint64_t a = readlane_u64(k, 0), b = readlane_u64(k, 16), c = readlane_u64(k, 32), d = readlane_u64(k, 48);
    a = a > b ? a : b;
    c = c > d ? c : d;
    return a > c ? a : c;
}

// One wavefront routes one token: softmax over E = 64*PER (or fewer) logits as candle-nn's
// softmax_last_dim computes it (max, exp of the differences, sum, divide), then the K best
// picks, best first, the lowest index winning ties (the stable descending argsort of
// crates/engine/src/experts.rs:2364-2372). Picks are made on the logits themselves: softmax is
// monotone and comparing logits is exact. Lane j < K returns pick j's expert in *id and its
// weight (renormalised over the K when norm) in *w; other lanes return id ~0u.
template <int PER>
__device__ __forceinline__ void route_load(const float *logits, int E, float (&v)[PER]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int e = lane + 64 * i;
        v[i] = e < E ? logits[e] : -INFINITY;
    }
}
// the routing of logits already loaded by route_load
template <int PER>
__device__ __forceinline__ void wave_route(const float (&v)[PER], int E, int K, int norm, uint32_t *id, float *w) {
    const int lane = threadIdx.x & 63;
    uint64_t key[PER];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int e = lane + 64 * i;
        key[i] = e < E ? route_key(v[i], (uint32_t)e) : 0ull;
        m = fmaxf(m, v[i]);
    }
    m = wave_max(m);
    uint64_t mine = 0;
    for (int j = 0; j < K; j++) {
        uint64_t best = key[0];
#pragma unroll
        for (int i = 1; i < PER; i++) best = key[i] > best ? key[i] : best;
        best = wave_max_key(best);
#pragma unroll
        for (int i = 0; i < PER; i++) key[i] = key[i] == best ? 0ull : key[i];
        mine = lane == j ? best : mine;
    }
    float p = lane < K ? expf(key_value(mine) - m) : 0.f;
    if (norm) {
        p = p / wave_sum(p);
    } else {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < PER; i++) s += lane + 64 * i < E ? expf(v[i] - m) : 0.f;
        p = p / wave_sum(s);
    }
    *id = lane < K ? key_index(mine) : 0xFFFFFFFFu;
    *w = p;
}
template <int PER>
__device__ __forceinline__ void wave_route(const float *logits, int E, int K, int norm, uint32_t *id, float *w) {
    float v[PER];
    route_load<PER>(logits, E, v);
    wave_route<PER>(v, E, K, norm, id, w);
}

}  // namespace cw
