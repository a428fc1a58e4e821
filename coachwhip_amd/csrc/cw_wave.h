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

// Router key: the float's bits made order-preserving as an unsigned number, so the unsigned
// maximum is the largest logit and equal logits have equal keys (-0 is keyed as +0); 0 marks a
// taken or absent candidate (the one float that maps to 0, a negative NaN, is raised to 1,
// among the other NaNs).
__device__ __forceinline__ uint32_t route_key(float v) {
    uint32_t b = __float_as_uint(v);
    if (b == 0x80000000u) b = 0u;
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return o ? o : 1u;
}
__device__ __forceinline__ float key_value(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

// the largest key of the wave, in every lane: the row maximum (four DPP steps), then
// row_bcast:15 into rows 1 and 3 and row_bcast:31 into rows 2 and 3 (gfx9 DPP), so lane 63
// holds the wave's maximum and one readlane returns it (unsigned max: 0 is the identity for the
// lanes a broadcast does not write)
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_rows_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_max_key(uint32_t k) {
    k = max(k, dpp_u<0xB1>(k));
    k = max(k, dpp_u<0x4E>(k));
    k = max(k, dpp_u<0x141>(k));
    k = max(k, dpp_u<0x140>(k));
    k = max(k, dpp_rows_u<0x142, 0xA>(k));
    k = max(k, dpp_rows_u<0x143, 0xC>(k));
    return (uint32_t)__builtin_amdgcn_readlane((int)k, 63);
}

// lane l loads logits PER*l .. PER*l + PER-1 (-inf past E)
template <int PER>
__device__ __forceinline__ void route_load(const float *logits, int E, float (&v)[PER]) {
    const int lane = threadIdx.x & 63;
    if constexpr (PER >= 8 && PER % 4 == 0) {
        // every lane full and the logits 16-byte aligned: PER / 4 16-byte loads per lane (a
        // dword load per logit makes each instruction touch every cache line of the logits;
        // config 5's decode layer 16.5 -> 16.2 us, while 4 logits per lane measured 0.1 us
        // slower as one 16-byte load)
        if (E == 64 * PER && ((uintptr_t)logits & 15) == 0) {
#pragma unroll
            for (int c = 0; c < PER / 4; c++) {
                const float4 t = ((const float4 *)logits)[lane * (PER / 4) + c];
                v[4 * c] = t.x;
                v[4 * c + 1] = t.y;
                v[4 * c + 2] = t.z;
                v[4 * c + 3] = t.w;
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < PER; i++) {
        // clamped, not branched: loads in branches make the compiler wait for every later load
        // before the first use
        const int e = PER * lane + i;
        const float t = logits[e < E ? e : E - 1];
        v[i] = e < E ? t : -INFINITY;
    }
}

// One wavefront routes one token: softmax over E = 64*PER (or fewer) logits as candle-nn's
// softmax_last_dim computes it (max, exp of the differences, sum, divide), then the K best
// picks, best first, the lowest index winning ties (the stable descending argsort of
// crates/engine/src/experts.rs:2364-2372). Picks are made on the logits themselves: softmax is
// monotone and comparing logits is exact. Lane l holds experts PER*l .. PER*l + PER-1, so the
// lowest index holding a round's maximum is in the lowest lane holding it, at that lane's lowest
// slot holding it: per round one wave maximum of 32-bit keys, one ballot, one find-first-set and
// one readlane. Lane j < K returns pick j's expert in *id and its weight (renormalised over the
// K when norm) in *w; other lanes return id ~0u.
// The routing is in two parts, so a caller can issue other loads once the logits are in:
// route_keys turns the loaded logits into keys and their maximum (waiting for the logits),
// route_pick makes the K picks and their weights.
template <int PER>
struct RouteState {
    uint32_t key[PER];
    float m;
};
template <int PER>
__device__ __forceinline__ void route_keys(const float (&v)[PER], int E, RouteState<PER> &r) {
    const int lane = threadIdx.x & 63;
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        r.key[i] = PER * lane + i < E ? route_key(v[i]) : 0u;
        m = fmaxf(m, v[i]);
    }
    r.m = wave_max(m);
}
// the K picks for PER = 4 or 8: each lane first sorts its keys (by key, then by slot, so equal
// keys keep index order; a bitonic network on 64-bit key|slot values); a round then needs only
// the wave maximum of the lanes' heads, the lowest lane holding it, and a pop of that lane's list
template <int PER>
__device__ __forceinline__ void route_tournament(uint32_t (&key)[PER], int K, uint32_t &mine_k, uint32_t &mine_e) {
    const int lane = threadIdx.x & 63;
    // 64-bit sort keys: key above the slot's complement, so larger is better and ties go to the lower slot
    uint64_t q[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) q[i] = ((uint64_t)key[i] << 8) | (uint64_t)(255 - i);
    // ascending bitonic sort; the list is read from the top
#pragma unroll
    for (int k = 2; k <= PER; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1)
#pragma unroll
            for (int i = 0; i < PER; i++) {
                const int l = i ^ j;
                if (l > i) {
                    const uint64_t x = q[i], y = q[l];
                    const bool swap = (i & k) == 0 ? x > y : x < y;
                    q[i] = swap ? y : x;
                    q[l] = swap ? x : y;
                }
            }
    uint32_t k[PER], sl[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        k[i] = (uint32_t)(q[PER - 1 - i] >> 8);
        sl[i] = 255u - (uint32_t)(q[PER - 1 - i] & 0xFF);
    }
    for (int j = 0; j < K; j++) {
        const uint32_t best = wave_max_key(k[0]);
        const int at = __builtin_ctzll(__ballot(k[0] == best));  // the lowest lane holding it
        const uint32_t slot = __builtin_amdgcn_readlane((int)sl[0], at);
        if (lane == at) {
#pragma unroll
            for (int i = 0; i + 1 < PER; i++) {
                k[i] = k[i + 1];
                sl[i] = sl[i + 1];
            }
            k[PER - 1] = 0u;
        }
        if (lane == j) {
            mine_k = best;
            mine_e = (uint32_t)PER * (uint32_t)at + slot;
        }
    }
}

template <int PER>
__device__ __forceinline__ void route_pick(const float (&v)[PER], RouteState<PER> &r, int E, int K, int norm, uint32_t *id,
                                           float *w) {
    const int lane = threadIdx.x & 63;
    uint32_t mine_k = 0, mine_e = 0xFFFFFFFFu;
    if constexpr (PER <= 8) route_tournament<PER>(r.key, K, mine_k, mine_e);
    else for (int j = 0; j < K; j++) {
        uint32_t best = r.key[0];
#pragma unroll
        for (int i = 1; i < PER; i++) best = max(best, r.key[i]);
        best = wave_max_key(best);
        int c = PER;  // this lane's lowest slot holding best
#pragma unroll
        for (int i = PER - 1; i >= 0; i--) c = r.key[i] == best ? i : c;
        const int at = __builtin_ctzll(__ballot(c < PER));  // the lowest lane holding it
        const int slot = __builtin_amdgcn_readlane(c, at);
#pragma unroll
        for (int i = 0; i < PER; i++)
            if (lane == at && i == slot) r.key[i] = 0u;
        if (lane == j) {
            mine_k = best;
            mine_e = (uint32_t)(PER * at + slot);
        }
    }
    float p = lane < K ? expf(key_value(mine_k) - r.m) : 0.f;
    if (norm) {
        p = p / wave_sum(p);
    } else {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < PER; i++) s += PER * lane + i < E ? expf(v[i] - r.m) : 0.f;
        p = p / wave_sum(s);
    }
    *id = lane < K ? mine_e : 0xFFFFFFFFu;
    *w = p;
}
template <int PER>
__device__ __forceinline__ void wave_route(const float (&v)[PER], int E, int K, int norm, uint32_t *id, float *w) {
    RouteState<PER> r;
    route_keys<PER>(v, E, r);
    route_pick<PER>(v, r, E, K, norm, id, w);
}
template <int PER>
__device__ __forceinline__ void wave_route(const float *logits, int E, int K, int norm, uint32_t *id, float *w) {
    float v[PER];
    route_load<PER>(logits, E, v);
    wave_route<PER>(v, E, K, norm, id, w);
}

}  // namespace cw
