// Wavefront-level helpers (wave64): reductions and the router's top-k, shared by the kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace cw {

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// (value, index) order of the router: larger value first, the lower index among equals;
// index ~0u marks an exhausted candidate.
__device__ __forceinline__ bool route_better(float va, uint32_t ia, float vb, uint32_t ib) {
    if (ia == 0xFFFFFFFFu) return false;
    if (ib == 0xFFFFFFFFu) return true;
    return va > vb || (va == vb && ia < ib);
}

__device__ __forceinline__ void wave_argmax(float &v, uint32_t &i) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        float ov = __shfl_xor(v, off);
        uint32_t oi = __shfl_xor(i, off);
        if (route_better(ov, oi, v, i)) { v = ov; i = oi; }
    }
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
