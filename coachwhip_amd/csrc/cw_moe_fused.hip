// The MoE layer in two kernels (gfx950):
//
//  k_moe_gateup: every wavefront routes its token (softmax + top-k, cw_wave.h), looks its pick's
//    slot up (identity, or the bank's slot table), and computes rows of gate and up for that
//    pick with the activation fused: h = silu(g) * u, or gpt-oss's clamped SwiGLU with biases.
//    The first block of each pick also publishes (expert, weight, slot) for the down kernel.
//  k_moe_down: a tile of output rows of one token, every pick; waves split the picks, each
//    pick's dots land in LDS and are combined in pick order (deterministic), with down's bias.
//
// Decode is bound by memory latency rather than bandwidth (a layer reads ~7 MB), so both kernels
// issue all their weight loads before anything that waits: the IQ grid copy into LDS and the
// barrier come after the loads are in flight.
#include "cw_common.h"
#include "cw_device.h"
#include "cw_moe_fused.h"
#include "cw_wave.h"

namespace cw {

template <int NX>
__device__ __forceinline__ void load_xs(float (&xr)[NX][32], const float *xrow, int sub, int lpr, int nsb) {
#pragma unroll
    for (int i = 0; i < NX; i++) {
        const int sb = sub + i * lpr;
        if (sb < nsb) {
            const float4 *p = (const float4 *)(xrow + 32 * sb);
#pragma unroll
            for (int v = 0; v < 8; v++) {
                const float4 f = p[v];
                xr[i][4 * v] = f.x; xr[i][4 * v + 1] = f.y; xr[i][4 * v + 2] = f.z; xr[i][4 * v + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int v = 0; v < 32; v++) xr[i][v] = 0.f;
        }
    }
}

// ------------------------------------------------------------------------------ gate / up

template <class Fmt, int LPR, int NX, int PER, int ROWS>
__global__ __launch_bounds__(256) void k_moe_gateup(const MoeArgs a) {
    __shared__ __align__(16) uint8_t lds[Fmt::LDS_BYTES > 0 ? Fmt::LDS_BYTES : 16];
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int sub = lane % LPR, rsub = lane / LPR;
    const int p = blockIdx.y, t = p / a.K, j = p - t * a.K;

    uint32_t rid;
    float rw;
    wave_route<PER>(a.logits + (int64_t)t * a.E, a.E, a.K, a.norm, &rid, &rw);
    const uint32_t expert = __shfl(rid, j);
    uint32_t slot = a.table ? a.table[expert] : expert;
    const bool absent = slot == CW_NO_SLOT;
    if (absent) slot = 0;
    const bool bad = slot >= (uint32_t)a.n_slots;
    const float wj = __shfl(rw, j);
    if (blockIdx.x == 0 && wave == 0 && lane == 0) {
        a.ids[p] = expert;
        a.w[p] = wj;
        a.slots[p] = bad ? 0xFFFFFFFFu : slot;
        if (absent && a.missing) atomicAdd(a.missing, 1u);
    }

    // weight loads for ROWS passes, in flight before anything waits
    const uint8_t *bg = a.wg + (int64_t)(bad ? 0 : slot) * a.sg;
    const uint8_t *bu = a.wu + (int64_t)(bad ? 0 : slot) * a.su;
    const int nsb = a.H / 32;
    const int r_first = (blockIdx.x * nwaves + wave) * RPW * ROWS + rsub;
    typename Fmt::Raw rg[ROWS][NX], ru[ROWS][NX];
#pragma unroll
    for (int q = 0; q < ROWS; q++) {
        const int r = r_first + q * RPW;
#pragma unroll
        for (int i = 0; i < NX; i++) {
            const int sb = sub + i * LPR;
            if (r < a.I && sb < nsb) {
                rg[q][i] = Fmt::load(bg + (int64_t)r * a.rbg, sb);
                ru[q][i] = Fmt::load(bu + (int64_t)r * a.rbg, sb);
            }
        }
    }
    float xr[NX][32];
    load_xs<NX>(xr, a.x + (int64_t)t * a.H, sub, LPR, nsb);
    Fmt::fill_lds(lds, threadIdx.x, blockDim.x);
    if (Fmt::LDS_BYTES > 0) __syncthreads();

    const int P = a.P;
#pragma unroll
    for (int q = 0; q < ROWS; q++) {
        const int r = r_first + q * RPW;
        float g = 0.f, u = 0.f;
#pragma unroll
        for (int i = 0; i < NX; i++) {
            const int sb = sub + i * LPR;
            if (r < a.I && sb < nsb) {
                g += Fmt::dot(rg[q][i], lds, xr[i]);
                u += Fmt::dot(ru[q][i], lds, xr[i]);
            }
        }
        g = group_sum<LPR>(g);
        u = group_sum<LPR>(u);
        if (sub == 0 && r < a.I) {
            float o;
            if (a.act == CW_ACT_SILU) {
                o = g / (1.0f + expf(-g)) * u;
            } else {
                if (a.bg) g += a.bg[(int64_t)expert * a.I + r];
                if (a.bu) u += a.bu[(int64_t)expert * a.I + r];
                g = fminf(g, a.limit);
                u = fminf(fmaxf(u, -a.limit), a.limit);
                o = (u + 1.0f) * (g * (1.0f / (1.0f + expf(-(g * a.alpha)))));
            }
            a.h[(int64_t)p * P + r] = bad ? __int_as_float(0x7fc00000) : o;
        }
    }
    // zero padding of the hidden row up to the width down reads
    for (int c = a.I + blockIdx.x * blockDim.x + threadIdx.x; c < P; c += gridDim.x * blockDim.x)
        a.h[(int64_t)p * P + c] = 0.f;
}

// ------------------------------------------------------------------------------ down + combine

// tile = 64/LPR rows: one pass of every wave per pick
template <class Fmt, int LPR, int NX, int PPW>
__global__ __launch_bounds__(256) void k_moe_down(const MoeArgs a) {
    __shared__ __align__(16) uint8_t lds[Fmt::LDS_BYTES > 0 ? Fmt::LDS_BYTES : 16];
    __shared__ float part[32 * (64 / LPR)];
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int sub = lane % LPR, rsub = lane / LPR;
    const int t = blockIdx.y;
    const int r = blockIdx.x * RPW + rsub;
    const int nsb = a.P / 32;

    // PPW picks per wave: j = wave + q * nwaves
    typename Fmt::Raw raw[PPW][NX];
    float xr[PPW][NX][32];
    bool bad[PPW];
#pragma unroll
    for (int q = 0; q < PPW; q++) {
        const int j = wave + q * nwaves;
        bad[q] = true;
        if (j < a.K) {
            const uint32_t slot = a.slots[t * a.K + j];
            bad[q] = slot >= (uint32_t)a.n_slots;
            const uint8_t *base = a.wd + (int64_t)(bad[q] ? 0 : slot) * a.sd;
#pragma unroll
            for (int i = 0; i < NX; i++) {
                const int sb = sub + i * LPR;
                if (r < a.H && sb < nsb) raw[q][i] = Fmt::load(base + (int64_t)r * a.rbd, sb);
            }
            load_xs<NX>(xr[q], a.h + (int64_t)(t * a.K + j) * a.P, sub, LPR, nsb);
        }
    }
    Fmt::fill_lds(lds, threadIdx.x, blockDim.x);
    if (Fmt::LDS_BYTES > 0) __syncthreads();
#pragma unroll
    for (int q = 0; q < PPW; q++) {
        const int j = wave + q * nwaves;
        if (j >= a.K) break;  // uniform across the wave
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < NX; i++) {
            const int sb = sub + i * LPR;
            if (r < a.H && sb < nsb) d += Fmt::dot(raw[q][i], lds, xr[q][i]);
        }
        d = group_sum<LPR>(d);
        if (sub == 0) part[j * RPW + rsub] = bad[q] ? __int_as_float(0x7fc00000) : d;
    }
    __syncthreads();
    if (threadIdx.x < RPW) {
        const int rr = blockIdx.x * RPW + threadIdx.x;
        if (rr < a.H) {
            float acc = 0.f;
            for (int j = 0; j < a.K; j++) {
                const int pick = t * a.K + j;
                float d = part[j * RPW + threadIdx.x];
                if (a.bd) d += a.bd[(int64_t)a.ids[pick] * a.H + rr];
                acc += a.w[pick] * d;
            }
            a.out[(int64_t)t * a.H + rr] = acc;
        }
    }
}

// ------------------------------------------------------------------------------ dispatch

static int lpr_for(int nsb) {
    int l = 8;
    while (l < nsb && l < 64) l <<= 1;
    return l;
}

template <class Fmt, int LPR, int NX>
static int gateup_per(const MoeArgs &a, int T, hipStream_t s) {
    constexpr int RPW = 64 / LPR;
    constexpr int ROWS = LPR == 64 ? 2 : 1;
    const int rows_per_block = 4 * RPW * ROWS;
    dim3 grid((a.I + rows_per_block - 1) / rows_per_block, T * a.K);
    if (a.E <= 256) hipLaunchKernelGGL((k_moe_gateup<Fmt, LPR, NX, 4, ROWS>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_moe_gateup<Fmt, LPR, NX, 16, ROWS>), grid, dim3(256), 0, s, a);
    return check_launch("k_moe_gateup");
}

template <class Fmt, int LPR, int NX>
static int down_per(const MoeArgs &a, int T, hipStream_t s) {
    constexpr int RPW = 64 / LPR;
    dim3 grid((a.H + RPW - 1) / RPW, T);
    const int ppw = (a.K + 3) / 4;
    if (ppw == 1) hipLaunchKernelGGL((k_moe_down<Fmt, LPR, NX, 1>), grid, dim3(256), 0, s, a);
    else if (ppw == 2) hipLaunchKernelGGL((k_moe_down<Fmt, LPR, NX, 2>), grid, dim3(256), 0, s, a);
    else if (ppw <= 4) hipLaunchKernelGGL((k_moe_down<Fmt, LPR, NX, 4>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_moe_down<Fmt, LPR, NX, 8>), grid, dim3(256), 0, s, a);
    return check_launch("k_moe_down");
}

template <class Fmt, bool DOWN>
static int by_shape(const MoeArgs &a, int T, hipStream_t s) {
    const int nsb = (DOWN ? a.P : a.H) / 32;
    const int lpr = lpr_for(nsb);
    const int nx = (nsb + lpr - 1) / lpr;
#define CW_CASE(L, X) \
    if (lpr == L && nx == X) return DOWN ? down_per<Fmt, L, X>(a, T, s) : gateup_per<Fmt, L, X>(a, T, s);
    CW_CASE(8, 1) CW_CASE(16, 1) CW_CASE(32, 1) CW_CASE(64, 1) CW_CASE(64, 2) CW_CASE(64, 3) CW_CASE(64, 4)
#undef CW_CASE
    return set_error(CW_ENOTSUP, "moe: rows of %d weights exceed %d", nsb * 32, 64 * 4 * 32);
}

template <bool DOWN>
static int by_fmt(int dtype, const MoeArgs &a, int T, hipStream_t s) {
    switch (dtype) {
    case CW_Q8_0: return by_shape<FQ8_0, DOWN>(a, T, s);
    case CW_Q4_K: return by_shape<FQ4_K, DOWN>(a, T, s);
    case CW_MXFP4: return by_shape<FMXFP4, DOWN>(a, T, s);
    case CW_IQ2_XXS: return by_shape<FIQ2_XXS, DOWN>(a, T, s);
    case CW_IQ2_S: return by_shape<FIQ2_S, DOWN>(a, T, s);
    case CW_IQ3_S: return by_shape<FIQ3_S, DOWN>(a, T, s);
    default: return set_error(CW_ENOTSUP, "moe: dtype %d is not supported", dtype);
    }
}

int moe_gateup(int dtype, const MoeArgs &a, int T, hipStream_t s) { return T ? by_fmt<false>(dtype, a, T, s) : CW_OK; }
int moe_down(int dtype, const MoeArgs &a, int T, hipStream_t s) {
    if (a.K > 32) return set_error(CW_ENOTSUP, "moe: top_k %d above 32", a.K);
    return T ? by_fmt<true>(dtype, a, T, s) : CW_OK;
}

}  // namespace cw
