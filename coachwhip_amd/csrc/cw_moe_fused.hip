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
#include <stddef.h>

#include <mutex>

#include "cw_common.h"
#include "cw_device.h"
#include "cw_moe_fused.h"
#include "cw_wave.h"

namespace cw {

template <int NX>
__device__ __forceinline__ void load_xs(float (&xr)[NX][32], const float *xrow, int sub, int lpr, int nsb) {
#pragma unroll
    for (int i = 0; i < NX; i++) {
        // clamped, not branched, so later waits on other loads stay exact
        const int sb = sub + i * lpr;
        const bool in = sb < nsb;
        const float4 *p = (const float4 *)(xrow + 32 * (in ? sb : nsb - 1));
#pragma unroll
        for (int v = 0; v < 8; v++) {
            const float4 f = p[v];
            xr[i][4 * v] = in ? f.x : 0.f;
            xr[i][4 * v + 1] = in ? f.y : 0.f;
            xr[i][4 * v + 2] = in ? f.z : 0.f;
            xr[i][4 * v + 3] = in ? f.w : 0.f;
        }
    }
}

// ------------------------------------------------------------------------------ gate / up

// MXFP4 matrices with their rows in groups of 16 (CW_MXFP4_R16): the same blocks, block sb of row r
// at rows16_offset(r, sb). The one-launch decode stages their gate/up rows in LDS as row pairs.
struct FMXFP4R16 : FMXFP4 {};
template <class F> struct Rows16 { static constexpr bool on = false; };
template <> struct Rows16<FMXFP4R16> { static constexpr bool on = true; };

// rows16_offset in 32 bits (the decode's matrices are below 2 GiB: its launch checks)
__device__ __forceinline__ uint32_t rows16_off32(int r, int b, int nblk) {
    const int c = b >> 2, cb = 4 * c + 4 <= nblk ? 4 : nblk - 4 * c;
    return (uint32_t)(r >> 4) * (uint32_t)(272 * nblk) + (uint32_t)(c * 1088 + ((r & 15) * cb + (b & 3)) * 17);
}
// block sb of row r of the matrix at mat (rows of rb bytes), in format F's layout
template <class F>
__device__ __forceinline__ typename F::Raw load_rc(const uint8_t *mat, int64_t r, int64_t rb, int sb) {
    if constexpr (Rows16<F>::on) return F::load(mat + rows16_off32((int)r, sb, (int)rb / 17), 0);
    else return F::load(mat + r * rb, sb);
}

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
                rg[q][i] = load_rc<Fmt>(bg, r, a.rbg, sb);
                ru[q][i] = load_rc<Fmt>(bu, r, a.rbg, sb);
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
                if (r < a.H && sb < nsb) raw[q][i] = load_rc<Fmt>(base, r, a.rbd, sb);
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

// ------------------------------------------------------------------------------ one-kernel decode

// Device-wide barrier of the persistent decode kernel. Its state (DecodeBarrier) lives in the
// caller's workspace, which the caller zero-fills once, and every call leaves it at zero again, so
// calls with distinct workspaces are independent. Blocks first arrive on one of 32 counters
// (blockIdx % 32: blocks go to the 8 XCDs round-robin, so each counter's blocks share an XCD); the
// last of each clears it and arrives on a top counter, and the last of those clears it and bumps
// the generation, held in 32 copies 128 bytes apart: block b polls copy b % 32, and the last block
// stores all 32 with one instruction. Splitting the arrivals over 33 counters keeps them from
// serializing on one address (a microbenchmark of 512 blocks: one counter 6.1 us above an empty
// launch, 8 counters 1.4 us, 32 counters 1.0 us); with one generation word, the polls of 768
// blocks on it spread the blocks' release over ~1.3 us. Everything the blocks
// exchange through memory inside the kernel is written and read with agent-scope atomics, which go
// to the coherence point, so the counters need no fences: an agent-scope release / acquire pair
// here (L2 write-back and invalidate in every block) measured 3x slower, and so did polling all 8
// XCD counters from every block. A wait gives up after `polls` polls and counts an error
// (g_decode_errors, and the workspace's status word) instead of hanging; every block still
// arrives exactly once, so the counters are back at zero (and the generation one further) when
// the kernel ends, timed out or not.
// The state must start zero-filled and then belong to the layer's calls alone. The last block to
// arrive stores a marker word; a launch that finds neither zero nor the marker there (other bytes
// written over the region) uses no counter, counts an error and gives NaN outputs, and so does an
// arrival whose counter was already past its block count. Both leave the state as they found it:
// the caller zero-fills it again.
struct DecodeBarrier {
    uint32_t sub[32][32];  // arrival counter x at sub[x][0]; the top counter at sub[0][16]
    uint32_t gen[32][32];  // generation copy x at gen[x][0]
    uint32_t mark;         // 0 (never used) or STATE_MARK (left by a completed call)
    uint32_t pad[31];
    uint32_t status;       // blocks of one-token calls that gave up or found the state invalid
};
constexpr uint32_t STATE_MARK = 0x434d5753u;
static_assert(sizeof(DecodeBarrier) <= DECODE_STATE_BYTES && DECODE_STATE_BYTES == CW_MOE_STATE_BYTES,
              "the decode state does not fit its workspace region");
static_assert(offsetof(DecodeBarrier, status) == CW_MOE_STATUS_OFFSET, "the status word is where cwmoe.h says");
static __device__ uint32_t g_decode_errors;

#define CW_AGENT __HIP_MEMORY_SCOPE_AGENT
// buffer descriptor word 3 for raw byte-addressed buffers on gfx9, and the cache policy bit of
// agent-scope coherent loads (sc1)
#define CW_BUFFER_DWORD3 0x00020000
#define CW_CPOL_SC1 16
typedef float f32x4 __attribute__((ext_vector_type(4)));
// `gen` is generation copy blockIdx % 32 as read by wave 0 at any point of this launch before it
// arrives (the copies move only when every block has arrived, and they are equal between calls),
// so that read is off the barrier's critical path.
// a failed wait or an invalid state: counted on the device and in the workspace's status word
__device__ __forceinline__ void barrier_fail(DecodeBarrier *b) {
    __hip_atomic_fetch_add(&g_decode_errors, 1u, __ATOMIC_RELAXED, CW_AGENT);
    __hip_atomic_fetch_add(&b->status, 1u, __ATOMIC_RELAXED, CW_AGENT);
}
// `mark` is the state's marker word as read by wave 0 at kernel start (before any block can have
// arrived, so every block reads the same value).
// Phase stamps of the one-launch decode (a separate build, libcwmoe_phases.so, compiled with
// CWMOE_PHASES; the library proper has none): thread 0 of every block stores s_memrealtime (a
// 100 MHz clock) at 8 points of the kernel into stamps[block][point], which cw_dbg_phases copies
// out after the call. A store issued at a point does not wait for anything; a later wait on this
// block's stores (the barrier's) includes it, one store per block.
#ifdef CWMOE_PHASES
__device__ unsigned long long g_phase_stamps[4096 * 8];
#define CW_PHASE(i)                                                                                    \
    do {                                                                                               \
        if (threadIdx.x == 0 && blockIdx.x < 4096) g_phase_stamps[blockIdx.x * 8 + (i)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define CW_PHASE(i) \
    do {            \
    } while (0)
#endif

__device__ bool grid_barrier(DecodeBarrier *b, uint32_t nblocks, uint32_t polls, uint32_t gen, uint32_t mark) {
    __builtin_amdgcn_s_waitcnt(0);  // this thread's coherent stores have landed
    __syncthreads();
    CW_PHASE(4);  // arrived: the block's stores have landed
    __shared__ int ok;
    if (mark != 0 && mark != STATE_MARK) {  // foreign bytes: no counter is touched
        if (threadIdx.x == 0) {
            ok = 0;
            if (blockIdx.x == 0) barrier_fail(b);
        }
        __syncthreads();
        return false;
    }
    if (threadIdx.x < 64) {
        const uint32_t x = blockIdx.x & 31;
        int last = 0, sane = 1;
        if (threadIdx.x == 0) {
            const uint32_t nsub = (nblocks - x + 31) / 32, nx = nblocks < 32 ? nblocks : 32;
            const uint32_t c = __hip_atomic_fetch_add(&b->sub[x][0], 1u, __ATOMIC_RELAXED, CW_AGENT);
            if (c == nsub - 1) {
                // the reset only has to land before the next call, which the kernel's end ensures
                __hip_atomic_store(&b->sub[x][0], 0u, __ATOMIC_RELAXED, CW_AGENT);
                const uint32_t t = __hip_atomic_fetch_add(&b->sub[0][16], 1u, __ATOMIC_RELAXED, CW_AGENT);
                last = t == nx - 1;
                if (last) __hip_atomic_store(&b->sub[0][16], 0u, __ATOMIC_RELAXED, CW_AGENT);
                sane = t < nx;
            } else {
                sane = c < nsub;
            }
            if (!sane) barrier_fail(b);  // a counter past its block count: the state was not zero
        }
        last = __builtin_amdgcn_readfirstlane(last);
        sane = __builtin_amdgcn_readfirstlane(sane);
        if (last) {
            if (threadIdx.x < 32) __hip_atomic_store(&b->gen[threadIdx.x][0], gen + 1, __ATOMIC_RELAXED, CW_AGENT);
            if (threadIdx.x == 0) {
                __hip_atomic_store(&b->mark, STATE_MARK, __ATOMIC_RELAXED, CW_AGENT);
                ok = sane;
            }
        } else if (threadIdx.x == 0) {
            int good = sane;
            uint32_t n = 0;
            while (good && __hip_atomic_load(&b->gen[x][0], __ATOMIC_RELAXED, CW_AGENT) == gen) {
                if (n++ >= polls) {
                    good = 0;
                    barrier_fail(b);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            ok = good;
        }
    }
    __syncthreads();
    return ok != 0;
}

__device__ __forceinline__ void store_coherent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Gate/up rows staged through LDS. A row of 17-byte MXFP4 blocks read by each lane as its own
// blocks (a byte and an unaligned 16-byte load per block) streams at ~2.9 TB/s on MI355X in a
// microbenchmark of the config-4 gate/up pattern (4 picks x 2 matrices x 2,880 rows, 1 or 2 items
// in flight per wave); the same rows as aligned 16-byte chunks copied into LDS by the load unit
// (global_load_lds_dwordx4) and read back there stream at 4.1-4.4 TB/s. Each wave owns two item
// buffers: the next item's rows (and its bias values) go out before the current item is read.
template <class F> struct RowDma { static constexpr bool on = false; };
template <> struct RowDma<FMXFP4> { static constexpr bool on = true; };
template <> struct RowDma<FMXFP4R16> { static constexpr bool on = true; };

// K-split items of an MXFP4_R16 gate/up pair in the one-launch decode: an item is one pick's group
// of 16 rows, its steps in parts of up to KS_STEPS (each part one contiguous run of each matrix:
// 1,088 bytes per full step, 272 cb for a last step of cb blocks), two parts in flight in two LDS
// buffers; each wave takes 2 steps of each part for all 16 rows (lane: row l / 4, block l % 4 of
// the step), and the waves' partial sums meet in LDS in wave order. (Staging a row pair per wave
// instead, as GGUF rows are, made the pair 23 short runs: 80 MB fetched per layer against 55.)
// LDS: two buffers of two matrices' parts (9 KB each), then x (whole 16-byte chunks, as copied),
// the waves' partial sums (16 rows x gate, up x 4 waves) and the 32 bias values.
constexpr int KS_STEPS = 8, KS_SPAN = 9 * 1024, KS_BUF = 2 * KS_SPAN, KS_X = 2 * KS_BUF;
__host__ __device__ __forceinline__ int ks_x_bytes(int h) { return (h / 4 + 255) / 256 * 256 * 16; }
__host__ __device__ __forceinline__ int ks_part_off(int h) { return KS_X + ks_x_bytes(h); }
__host__ __device__ __forceinline__ int ks_bias_off(int h) { return ks_part_off(h) + 4 * 16 * 2 * 4; }
__host__ __device__ __forceinline__ int ks_lds(int h) { return ks_bias_off(h) + 32 * 4; }

// One 16-byte chunk per lane from global memory into LDS at lds_base + 16 * lane. Issued as inline
// asm: the compiler's waits then do not cover these loads (the kernel waits for them itself with
// vmcnt), and no LDS read of the kernel is taken to alias them. M0 is saved and restored.
// lds_base is an LDS byte address (lds_addr of the kernel's dynamic LDS plus an offset).
__device__ __forceinline__ void lds_dma16(const void *g, uint32_t lds_base) {
    const uint32_t m = __builtin_amdgcn_readfirstlane(lds_base);
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep) : "v"(g), "s"(m) : "memory");
}
// The same for one dword per lane, at lds_base + 4 * lane.
__device__ __forceinline__ void lds_dma4(const void *g, uint32_t lds_base) {
    const uint32_t m = __builtin_amdgcn_readfirstlane(lds_base);
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep) : "v"(g), "s"(m) : "memory");
}

// s_waitcnt vmcnt(n) for a run-time n in 0..31 (the instruction takes an immediate)
__device__ __forceinline__ void wait_vm(int n) {
#define CW_VM(N) case N: asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory"); break;
#define CW_VM8(B) CW_VM(B) CW_VM(B + 1) CW_VM(B + 2) CW_VM(B + 3) CW_VM(B + 4) CW_VM(B + 5) CW_VM(B + 6) CW_VM(B + 7)
    switch (n < 0 ? 0 : n > 31 ? 31 : n) { CW_VM8(0) CW_VM8(8) CW_VM8(16) CW_VM8(24) }
#undef CW_VM8
#undef CW_VM
}

// An MXFP4 block at byte o of an LDS row window: the scale byte, then 16 code bytes read as five
// aligned dwords and shifted into place.
__device__ __forceinline__ FMXFP4::Raw mx_from_lds(const uint8_t *win, int o) {
    FMXFP4::Raw r;
    r.e = win[o];
    const int a = o + 1;
    const uint32_t *w = (const uint32_t *)(win + (a & ~3));
    const uint32_t d0 = w[0], d1 = w[1], d2 = w[2], d3 = w[3], d4 = w[4], sh = a & 3;
    r.q.x = __builtin_amdgcn_alignbyte(d1, d0, sh);
    r.q.y = __builtin_amdgcn_alignbyte(d2, d1, sh);
    r.q.z = __builtin_amdgcn_alignbyte(d3, d2, sh);
    r.q.w = __builtin_amdgcn_alignbyte(d4, d3, sh);
    return r;
}

// Bytes of a row's window in LDS: its 16-byte chunks from the one holding its first byte, plus the
// 4 bytes that the last block's dword reads may touch past its end.
__host__ __device__ __forceinline__ int row_window(int row_bytes) { return ((row_bytes + 15 + 15 + 4) >> 4) << 4; }

// The whole decode layer (one token) in one launch of a grid that fits on the device at once.
// Loads are issued as early as their addresses are known, since every wait on them counts in
// issue order:
//   1. every wave loads the logits, then the LDS tables and its x slice, and routes the token;
//   2. each wave issues the loads of its first gate/up item (pick, 2 rows) and of its block's
//      first down rows (all its picks), stores the tables to LDS, then computes its gate/up
//      items: dots, activation, hidden rows stored at the coherence point;
//   3. device-wide barrier;
//   4. each block copies all K hidden rows into LDS (one read per block, not per wave), and each
//      of its G groups of 4 waves computes down row groups of 64/LD rows: per-pick dots,
//      combined in pick order.
// At least 3 waves per SIMD (at most 168 VGPRs): the grid is sized from occupancy, and the
// gpt-oss shape's 182-VGPR build ran 2 blocks per CU (39.0 us per layer; 36.4 at 3, with a few
// spilled registers, none since its gate/up rows are staged through LDS: 155 VGPRs); the other
// instances fit already.
// RI: rows (of RPG) per gate/up item.
template <class FG, int LG, int XG, class FD, int LD, int XD, int PER, int PPW, int G, int RI>
__global__ __launch_bounds__(256 * G, G == 1 ? 3 : 1) void k_moe_decode(const MoeArgs a) {
    constexpr int NW = 4 * G, NT = 64 * NW;  // waves and threads of a block: G groups of 4 waves
    __shared__ __align__(16) uint8_t ldsg[FG::LDS_BYTES > 0 ? FG::LDS_BYTES : 16];
    __shared__ __align__(16) uint8_t ldsd[FD::LDS_BYTES > 0 ? FD::LDS_BYTES : 16];
    constexpr int RPG = 64 / LG, RPD = 64 / LD;
    __shared__ float part[G][32 * RPD];
    __shared__ float pick_w[32];
    __shared__ uint32_t pick_e[32], pick_slot[32];
    extern __shared__ __align__(16) float hs[];  // hidden rows, sub-blocks of 32 floats 36 apart
    const uint32_t hs_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float *)hs;  // its LDS address
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = a.K;
    CW_PHASE(0);  // start
    // the logits alone first: every wave of the grid starts at once, and the table and x loads
    // of 2048 waves queued in front of them in L2 (~2.5 us to the first logit). Those loads are
    // issued once the logits are in and complete during the top-k. With 8 logits per lane or
    // more, wave 0 alone routes (the other waves would only repeat it on the same SIMDs: 0.5 us
    // of a 512-expert layer) and hands the picks to the block through LDS behind a barrier; with
    // fewer, every wave routes for itself, which is faster than waiting at the barrier.
    constexpr bool ONE_ROUTER = PER >= 8;
    const bool routes = !ONE_ROUTER || wave == 0;
    float lv[PER];
    RouteState<PER> rst;
    uint32_t gen = 0, mark = 0;  // the barrier's generation and the state's marker, read by wave 0 ahead of the logits
    if (wave == 0) {
        gen = __hip_atomic_load(&((DecodeBarrier *)a.state)->gen[blockIdx.x & 31][0], __ATOMIC_RELAXED, CW_AGENT);
        mark = __hip_atomic_load(&((DecodeBarrier *)a.state)->mark, __ATOMIC_RELAXED, CW_AGENT);
    }
    if (routes) {
        route_load<PER>(a.logits, a.E, lv);
        route_keys<PER>(lv, a.E, rst);
    }
    TableRegs<FG> tg;
    TableRegs<FD> td;
    if (wave < 4) tg.load(threadIdx.x);  // the tables take 256 threads
    const int subg = lane % LG, rsg = lane / LG, nsbg = a.H / 32;
    float xr[XG][32];
    // GDMA: item buffer b of wave w at hs + (b * NW + w) * ibuf; x goes into the buffer-1 region
    const int x_off = Rows16<FG>::on ? KS_X : RowDma<FG>::on ? NW * (2 * RI * row_window(a.H / 32 * FG::TS) + 16) : 0;
    if constexpr (RowDma<FG>::on) {
        // x once per block into the (not yet used) hidden-row region, read into registers below:
        // every wave loading all of x (35 MB across config 4's grid) held up the logits and x
        // loads of the blocks placed third on a CU by ~7 us
        const int nxc = a.H / 4;
        for (int c0 = 0; c0 < nxc; c0 += NT)
            lds_dma16(a.x + 4 * min(c0 + (int)threadIdx.x, nxc - 1), hs_lds + x_off + 16 * (c0 + wave * 64));
    } else {
        load_xs<XG>(xr, a.x, subg, LG, nsbg);
    }

    uint32_t rid = 0xFFFFFFFFu;      // lane j < K: pick j's expert
    uint32_t my_slot = 0xFFFFFFFFu;  // ... and its slot
    if (routes) {
        float rw;
        route_pick<PER>(lv, rst, a.E, K, a.norm, &rid, &rw);
        if (lane < K) {
            my_slot = a.table ? a.table[rid] : rid;
            const bool absent = my_slot == CW_NO_SLOT;
            if (absent) my_slot = 0;
            if (my_slot >= (uint32_t)a.n_slots) my_slot = 0xFFFFFFFFu;
            if (wave == 0) {
                pick_w[lane] = rw;
                pick_e[lane] = rid;
                pick_slot[lane] = my_slot;
                if (blockIdx.x == 0) {
                    a.ids[lane] = rid;
                    a.w[lane] = rw;
                    if (absent && a.missing) atomicAdd(a.missing, 1u);
                }
            }
        }
    }
    if (ONE_ROUTER) {
        __syncthreads();
        rid = lane < K ? pick_e[lane] : 0xFFFFFFFFu;
        my_slot = lane < K ? pick_slot[lane] : 0xFFFFFFFFu;
    }
    CW_PHASE(1);  // routed

    // gate / up items (pick j, RI*RPG rows) spread over every wave of the grid; the first item's
    // weights and the block's first down rows are requested right after routing. With one sub-block
    // per lane the loads are unconditional, from a clamped row and sub-block: a load under a
    // per-lane branch is waited for at the branch's end (config 3 layer 13.15 -> 12.92 us, config 5
    // 17.97 -> 17.08). Rows of more than 64 sub-blocks keep the conditional form: most lanes have no
    // second sub-block, and the unconditional form measured 2.6-4 us slower for config 4.
    const int row_items = (a.I + RI * RPG - 1) / (RI * RPG);
    const int n_items = K * row_items;
    const int gwave = blockIdx.x * NW + wave, total_waves = gridDim.x * NW;
    typename FG::Raw rg[RI][XG], ru[RI][XG];
    auto load_item = [&](int it) {
        const int j = it / row_items, r0 = (it - j * row_items) * RI * RPG + rsg;
        const uint32_t slot = __shfl(my_slot, j);
        const uint32_t sl = slot == 0xFFFFFFFFu ? 0 : slot;
        const uint8_t *bg = a.wg + (int64_t)sl * a.sg;
        const uint8_t *bu = a.wu + (int64_t)sl * a.su;
#pragma unroll
        for (int q = 0; q < RI; q++) {
            if constexpr (XG == 1) {
                const int r = min(r0 + q * RPG, a.I - 1), sb = min(subg, nsbg - 1);
                rg[q][0] = FG::load(bg + (int64_t)r * a.rbg, sb);
                ru[q][0] = FG::load(bu + (int64_t)r * a.rbg, sb);
            } else {
                const int r = r0 + q * RPG;
#pragma unroll
                for (int i = 0; i < XG; i++) {
                    const int sb = subg + i * LG;
                    if (r < a.I && sb < nsbg) {
                        rg[q][i] = FG::load(bg + (int64_t)r * a.rbg, sb);
                        ru[q][i] = FG::load(bu + (int64_t)r * a.rbg, sb);
                    }
                }
            }
        }
    };
    constexpr bool GDMA = RowDma<FG>::on;
    static_assert(!GDMA || (LG == 64 && XG == 2), "the LDS-staged gate/up rows take one row per wave pass");
    // GDMA: this wave's two item buffers in the (not yet used) hidden-row region: per buffer RI
    // gate rows, RI up rows, then the 2*RI bias values
    const int win = row_window(nsbg * FG::TS);
    const int ibuf = 2 * RI * win + 16;
    uint8_t *wbuf = (uint8_t *)hs + wave * ibuf;
    auto issue_item = [&](int it, int b) {
        const int j = it / row_items, r0 = (it - j * row_items) * RI;
        // both shuffles with every lane active: a lane outside a branch gives 0 to a shuffle
        const uint32_t slot = __shfl(my_slot, j), e = __shfl(rid, j);
        const uint32_t sl = slot == 0xFFFFFFFFu ? 0 : slot;
        uint8_t *ib = wbuf + b * NW * ibuf;
        {
#pragma unroll
        for (int q = 0; q < RI; q++) {
            const int r = min(r0 + q, a.I - 1);
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const uint8_t *row = (m ? a.wu + (int64_t)sl * a.su : a.wg + (int64_t)sl * a.sg) + (int64_t)r * a.rbg;
                const uint8_t *al = (const uint8_t *)((uintptr_t)row & ~(uintptr_t)15);
                // chunks past the row's last one re-read that chunk: no load leaves the 16-byte
                // granule of the row's last byte
                const int nch = (int)(((uintptr_t)row & 15) + nsbg * FG::TS + 15) >> 4;
                const uint32_t w = hs_lds + (uint32_t)(ib - (uint8_t *)hs) + (2 * q + m) * win;
                lds_dma16(al + 16 * min(lane, nch - 1), w);
                if (lane < (win >> 4) - 64) lds_dma16(al + 16 * min(64 + lane, nch - 1), w + 1024);
            }
        }
        }
        // bias values (gate rows, then up rows); a layer without biases re-reads x
        if (lane < 2 * RI) {
            const int q = lane % RI;
            const float *bsrc = lane < RI ? a.bg : a.bu;
            const float *src = bsrc ? bsrc + (int64_t)(e < (uint32_t)a.E ? e : 0) * a.I + min(r0 + q, a.I - 1) : a.x;
            lds_dma4(src, hs_lds + (uint32_t)(ib - (uint8_t *)hs) + (ibuf - 16));
        }
    };
    if constexpr (GDMA) {
        // the first item's rows go out at once (into buffer 0); x (copied during the top-k into
        // the buffer-1 region) is read into registers meanwhile, before any buffer 1 is filled
        if (!Rows16<FG>::on && gwave < n_items) {
            issue_item(gwave, 0);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * RI + 1) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < (Rows16<FG>::on ? 0 : XG); i++) {
            const int sb = subg + i * LG;
            const bool in = sb < nsbg;
            const float4 *src = (const float4 *)((const float *)((const uint8_t *)hs + x_off) + 32 * (in ? sb : nsbg - 1));
#pragma unroll
            for (int v = 0; v < 8; v++) {
                const float4 f = src[v];
                xr[i][4 * v] = in ? f.x : 0.f;
                xr[i][4 * v + 1] = in ? f.y : 0.f;
                xr[i][4 * v + 2] = in ? f.z : 0.f;
                xr[i][4 * v + 3] = in ? f.w : 0.f;
            }
        }
        __syncthreads();
    } else {
        if (gwave < n_items) load_item(gwave);
    }

    const int subd = lane % LD, rsd = lane / LD, nsbd = a.P / 32;
    const int grp = wave >> 2, wl = wave & 3;  // the down phase: wave group, and wave within it
    typename FD::Raw draw[PPW][XD];
    uint32_t dslot[PPW];
    {
        const int r = (blockIdx.x * G + grp) * RPD + rsd;
#pragma unroll
        for (int q = 0; q < PPW; q++) {
            const int j = wl + 4 * q;
            dslot[q] = __shfl(my_slot, j < K ? j : 0);
            if constexpr (XD == 1) {  // unconditional (unused past K)
                const uint8_t *mat = a.wd + (int64_t)(dslot[q] == 0xFFFFFFFFu ? 0 : dslot[q]) * a.sd;
                draw[q][0] = load_rc<FD>(mat, min(r, a.H - 1), a.rbd, min(subd, nsbd - 1));
            } else if (j < K && dslot[q] != 0xFFFFFFFFu && r < a.H) {
                const uint8_t *mat = a.wd + (int64_t)dslot[q] * a.sd;
#pragma unroll
                for (int i = 0; i < XD; i++) {
                    const int sb = subd + i * LD;
                    if (sb < nsbd) draw[q][i] = load_rc<FD>(mat, r, a.rbd, sb);
                }
            }
        }
    }
    // down's table is needed only after the barrier: its loads go out behind the weights', and
    // it is stored to LDS once the gate/up items are done
    if (wave < 4) {
        td.load(threadIdx.x);
        tg.store(ldsg, threadIdx.x);
    }
    __syncthreads();

    if constexpr (GDMA) {
        // the previous item's hidden values, stored once the next wait is behind (a store counts
        // in vmcnt, and a wait issued right after it would wait for its round trip)
        float hv[RI];
        int hj = -1, hr0 = 0;
        bool hbad = false;
        auto flush = [&]() {
            if (hj >= 0 && lane == 0) {
#pragma unroll
                for (int q = 0; q < RI; q++)
                    if (hr0 + q < a.I) store_coherent(a.h + (int64_t)hj * a.P + hr0 + q, hbad ? __int_as_float(0x7fc00000) : hv[q]);
            }
        };
        // Items go out in rounds: round r covers the next wr(r) items, one per wave from wave 0.
        // With several blocks per CU, the blocks placed later on a CU start their first items a
        // few microseconds later (their loads queue behind the others'), so each later round
        // leaves out one more of the CU's placement groups (blocks are placed in index order).
        auto wr = [&](int r) { return a.per_cu > 1 ? total_waves * max(a.per_cu - r, 1) / a.per_cu : total_waves; };
        if constexpr (Rows16<FG>::on) {
            const int nst = (nsbg + 3) >> 2, nfull = nsbg >> 2, cbl = nsbg & 3, nparts = (nst + KS_STEPS - 1) / KS_STEPS;
            const int ngi = (a.I + 15) >> 4, n_gi = K * ngi;
            const int row = lane >> 2, blk = lane & 3;
            // part p's bytes per matrix (full steps, then a last step of cbl blocks) and this wave's
            // share of its 2 x ceil(bytes / 1 KB) loads: loads w, w + 4, ...
            auto part_bytes = [&](int p) {
                const int s0 = p * KS_STEPS, s1 = min(s0 + KS_STEPS, nst), full = min(s1, nfull) - s0;
                return full * 1088 + (s1 > nfull ? 272 * cbl : 0);
            };
            auto part_loads = [&](int p) { return (2 * ((part_bytes(p) + 1023) >> 10) - wave + 3) >> 2; };
            const float *xl = (const float *)((const uint8_t *)hs + KS_X);
            float *partial = (float *)((uint8_t *)hs + ks_part_off(a.H));
            const float *bias = (const float *)((const uint8_t *)hs + ks_bias_off(a.H));
            for (int it = blockIdx.x; it < n_gi; it += gridDim.x) {
                const int j = it / ngi, g = it - j * ngi;
                const uint32_t slot = __shfl(my_slot, j), e = __shfl(rid, j);
                const uint32_t sl = slot == 0xFFFFFFFFu ? 0 : slot;
                const uint8_t *mg = a.wg + (int64_t)sl * a.sg, *mu = a.wu + (int64_t)sl * a.su;
                auto issue_part = [&](int p) {
                    const int pieces = part_bytes(p) >> 4, nins = (pieces + 63) >> 6;
                    const uint32_t base = (uint32_t)g * (uint32_t)(272 * nsbg) + (uint32_t)(p * KS_STEPS * 1088);
                    for (int ii = wave; ii < 2 * nins; ii += 4) {
                        const int m = ii >= nins ? 1 : 0, ci = ii - m * nins;
                        lds_dma16((m ? mu : mg) + base + 16u * (uint32_t)min(64 * ci + lane, pieces - 1),
                                  hs_lds + (uint32_t)((p & 1) * KS_BUF + m * KS_SPAN + 1024 * ci));
                    }
                };
                __syncthreads();  // the previous item is done with the buffers and the partial sums
                issue_part(0);
                if (wave == 0) {  // the group's 16 gate and 16 up bias values (a layer without biases re-reads x)
                    const float *bsrc = lane < 16 ? a.bg : a.bu;
                    const float *src = bsrc ? bsrc + (int64_t)(e < (uint32_t)a.E ? e : 0) * a.I + min(16 * g + (lane & 15), a.I - 1) : a.x;
                    if (lane < 32) lds_dma4(src, hs_lds + (uint32_t)ks_bias_off(a.H));
                }
                if (nparts > 1) issue_part(1);
                float accg = 0.f, accu = 0.f;
                for (int p = 0; p < nparts; p++) {
                    wait_vm(p + 1 < nparts ? part_loads(p + 1) : 0);  // this wave's loads of part p are in
                    __syncthreads();                                  // everyone's
                    const uint8_t *bgl = (const uint8_t *)hs + (p & 1) * KS_BUF;
#pragma unroll
                    for (int t = 0; t < 2; t++) {
                        const int s = p * KS_STEPS + 2 * wave + t;  // this wave's step
                        if (s < min(p * KS_STEPS + KS_STEPS, nst)) {
                            const int cb = s < nfull ? 4 : cbl;
                            if (blk < cb) {
                                const int o = (s - p * KS_STEPS) * 1088 + (row * cb + blk) * 17;
                                const typename FG::Raw wg = mx_from_lds(bgl, o);
                                const typename FG::Raw wu = mx_from_lds(bgl + KS_SPAN, o);
                                float xv[32];
                                const float4 *xs4 = (const float4 *)(xl + 32 * (4 * s + blk));
#pragma unroll
                                for (int v = 0; v < 8; v++) {
                                    const float4 f = xs4[v];
                                    xv[4 * v] = f.x;
                                    xv[4 * v + 1] = f.y;
                                    xv[4 * v + 2] = f.z;
                                    xv[4 * v + 3] = f.w;
                                }
                                accg += FG::dot(wg, ldsg, xv);
                                accu += FG::dot(wu, ldsg, xv);
                            }
                        }
                    }
                    if (p + 2 < nparts) {
                        __syncthreads();  // everyone is done with buffer p & 1
                        issue_part(p + 2);
                    }
                }
                // the row's 4 lanes, then the 4 waves in order
                accg += dpp_f<0xB1>(accg);
                accg += dpp_f<0x4E>(accg);
                accu += dpp_f<0xB1>(accu);
                accu += dpp_f<0x4E>(accu);
                if (blk == 0) {
                    partial[(wave * 16 + row) * 2] = accg;
                    partial[(wave * 16 + row) * 2 + 1] = accu;
                }
                __syncthreads();
                if (wave == 0 && lane < 16 && 16 * g + lane < a.I) {
                    float gs = partial[lane * 2], us = partial[lane * 2 + 1];
#pragma unroll
                    for (int w = 1; w < 4; w++) {
                        gs += partial[(w * 16 + lane) * 2];
                        us += partial[(w * 16 + lane) * 2 + 1];
                    }
                    float o;
                    if (a.act == CW_ACT_SILU) {
                        o = gs / (1.0f + expf(-gs)) * us;
                    } else {
                        if (a.bg) gs += bias[lane];
                        if (a.bu) us += bias[16 + lane];
                        gs = fminf(gs, a.limit);
                        us = fminf(fmaxf(us, -a.limit), a.limit);
                        o = (us + 1.0f) * (gs * (1.0f / (1.0f + expf(-(gs * a.alpha)))));
                    }
                    store_coherent(a.h + (int64_t)j * a.P + 16 * g + lane, slot == 0xFFFFFFFFu ? __int_as_float(0x7fc00000) : o);
                }
            }
        } else
        for (int it = gwave, b = 0, r = 0; it < n_items; it = gwave < wr(r + 1) ? it + wr(r) : n_items, r++, b ^= 1) {
            // per item: 2*RI rows of two chunk loads each, and the bias load
            const int nx = gwave < wr(r + 1) ? it + wr(r) : n_items;
            if (nx < n_items) {
                issue_item(nx, b ^ 1);
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * RI + 1) : "memory");
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            flush();
            const int j = it / row_items, r0 = (it - j * row_items) * RI;
            const uint32_t slot = __shfl(my_slot, j);
            const uint32_t sl = slot == 0xFFFFFFFFu ? 0 : slot;
            const uint8_t *ib = wbuf + b * NW * ibuf;
#pragma unroll
            for (int q = 0; q < RI; q++) {
                const int r = min(r0 + q, a.I - 1);
                float g = 0.f, u = 0.f;
#pragma unroll
                for (int i = 0; i < XG; i++) {
                    const int sb = subg + i * LG, sbc = min(sb, nsbg - 1);
                    const int og = (int)((uintptr_t)(a.wg + (int64_t)sl * a.sg + (int64_t)r * a.rbg) & 15);
                    const int ou = (int)((uintptr_t)(a.wu + (int64_t)sl * a.su + (int64_t)r * a.rbg) & 15);
                    const typename FG::Raw wg = mx_from_lds(ib + (2 * q) * win, og + FG::TS * sbc);
                    const typename FG::Raw wu = mx_from_lds(ib + (2 * q + 1) * win, ou + FG::TS * sbc);
                    if (sb < nsbg) {
                        g += FG::dot(wg, ldsg, xr[i]);
                        u += FG::dot(wu, ldsg, xr[i]);
                    }
                }
                g = group_sum<LG>(g);
                u = group_sum<LG>(u);
                float o;
                if (a.act == CW_ACT_SILU) {
                    o = g / (1.0f + expf(-g)) * u;
                } else {
                    const float *bias = (const float *)(ib + (ibuf - 16));
                    if (a.bg) g += bias[q];
                    if (a.bu) u += bias[RI + q];
                    g = fminf(g, a.limit);
                    u = fminf(fmaxf(u, -a.limit), a.limit);
                    o = (u + 1.0f) * (g * (1.0f / (1.0f + expf(-(g * a.alpha)))));
                }
                hv[q] = o;
            }
            hj = j;
            hr0 = r0;
            hbad = slot == 0xFFFFFFFFu;
        }
        flush();
    } else
    for (int it = gwave; it < n_items; it += total_waves) {
        if (it != gwave) load_item(it);
        const int j = it / row_items, r0 = (it - j * row_items) * RI * RPG + rsg;
        const uint32_t slot = __shfl(my_slot, j);
        const uint32_t expert = __shfl(rid, j);
        const bool bad = slot == 0xFFFFFFFFu;
#pragma unroll
        for (int q = 0; q < RI; q++) {
            const int r = r0 + q * RPG;
            float g = 0.f, u = 0.f;
#pragma unroll
            for (int i = 0; i < XG; i++) {
                const int sb = subg + i * LG;
                if (r < a.I && sb < nsbg) {
                    g += FG::dot(rg[q][i], ldsg, xr[i]);
                    u += FG::dot(ru[q][i], ldsg, xr[i]);
                }
            }
            g = group_sum<LG>(g);
            u = group_sum<LG>(u);
            if (subg == 0 && r < a.I) {
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
                store_coherent(a.h + (int64_t)j * a.P + r, bad ? __int_as_float(0x7fc00000) : o);
            }
        }
    }
    CW_PHASE(2);  // this wave 0's gate/up items done
    // zero padding of hidden rows up to the width down reads
    for (int c = gwave * 64 + lane; c < K * (a.P - a.I); c += total_waves * 64) {
        const int j = c / (a.P - a.I);
        store_coherent(a.h + (int64_t)j * a.P + a.I + (c - j * (a.P - a.I)), 0.f);
    }

    // the second down pass's rows, requested before the barrier (x's registers are free by now),
    // so they are in by the time the hidden rows are staged (config 4, whose rows take two passes:
    // 29.7-30.0 -> 29.1-29.4 us per layer; the other instances keep their code: 12.50 against
    // 12.59 us for config 3, which has one pass)
    constexpr bool PF2 = RowDma<FG>::on;
    typename FD::Raw draw2[PPW][XD];
    const int bp2 = blockIdx.x + gridDim.x;
    if (PF2 && bp2 * G * RPD < a.H) {
        const int r2 = (bp2 * G + grp) * RPD + rsd;
#pragma unroll
        for (int q = 0; q < PPW; q++) {
            const int j = wl + 4 * q;
            if (j >= K) break;
            if (dslot[q] == 0xFFFFFFFFu || r2 >= a.H) continue;
#pragma unroll
            for (int i = 0; i < XD; i++) {
                const int sb = subd + i * LD;
                if (sb < nsbd) draw2[q][i] = load_rc<FD>(a.wd + (int64_t)dslot[q] * a.sd, r2, a.rbd, sb);
            }
        }
    }
    // the combine's down-bias values of this thread's row in both passes, also before the barrier
    // (a load in the combine is a memory round trip after each pass's dots)
    constexpr bool PFB = PF2 && PPW == 1;  // (more picks per wave would spill)
    float bq[2][4 * PPW];
    if constexpr (PFB) {
        const int tg4 = threadIdx.x & 255;
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const int rr = ((blockIdx.x + p * gridDim.x) * G + grp) * RPD + tg4;
#pragma unroll
            for (int j = 0; j < 4 * PPW; j++)
                bq[p][j] = a.bd && tg4 < RPD && rr < a.H && j < K ? a.bd[(int64_t)pick_e[j] * a.H + rr] : 0.f;
        }
    }
    if (wave < 4) td.store(ldsd, threadIdx.x);
    CW_PHASE(3);  // at the barrier
    const bool ok = grid_barrier((DecodeBarrier *)a.state, gridDim.x, a.polls, gen, mark);
    CW_PHASE(5);  // barrier open

    // every hidden row into LDS once per block, read at the coherence point (16-byte buffer
    // loads with the sc1 policy, the form of an agent-scope atomic load, 8 in flight per thread),
    // and stored with the padding (36 floats per sub-block of 32) that keeps the 16 sub-block
    // readers of a row on distinct LDS banks
    {
        const int nbytes = K * a.P * 4, hp = a.P / 4;
        const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc((void *)a.h, (short)0, nbytes, CW_BUFFER_DWORD3);
        for (int v0 = 0; v0 < nbytes / 16; v0 += NT * 8) {
            f32x4 t[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int v = v0 + NT * u + threadIdx.x;
                t[u] = __builtin_amdgcn_raw_buffer_load_b128(hr, 16 * v, 0, CW_CPOL_SC1);  // past the end: 0, unused
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int v = v0 + NT * u + threadIdx.x;
                if (v < nbytes / 16) {
                    const int j = v / hp, c = 4 * (v - j * hp);
                    *(f32x4 *)(hs + (j * nsbd + (c >> 5)) * 36 + (c & 31)) = t[u];
                }
            }
        }
    }
    __syncthreads();
    CW_PHASE(6);  // hidden rows staged

    // down + combine: each wave group takes RPD rows per block pass (the loop's bound is the
    // block's, so every thread meets the same barriers)
    for (int bp = blockIdx.x, first = 1; bp * G * RPD < a.H; bp += gridDim.x, first = 0) {
        const int grp_i = bp * G + grp;
        const int r = grp_i * RPD + rsd;
        if (PF2 && !first && bp == bp2) {
#pragma unroll
            for (int q = 0; q < PPW; q++)
#pragma unroll
                for (int i = 0; i < XD; i++) draw[q][i] = draw2[q][i];
        } else if (!first) {
#pragma unroll
            for (int q = 0; q < PPW; q++) {
                const int j = wl + 4 * q;
                if (j >= K) break;  // uniform across the wave
                if (dslot[q] == 0xFFFFFFFFu || r >= a.H) continue;
#pragma unroll
                for (int i = 0; i < XD; i++) {
                    const int sb = subd + i * LD;
                    if (sb < nsbd) draw[q][i] = load_rc<FD>(a.wd + (int64_t)dslot[q] * a.sd, r, a.rbd, sb);
                }
            }
        }
#pragma unroll
        for (int q = 0; q < PPW; q++) {
            const int j = wl + 4 * q;
            if (j >= K) break;
            const bool live = dslot[q] != 0xFFFFFFFFu && r < a.H;
            float d = 0.f;
#pragma unroll
            for (int i = 0; i < XD; i++) {
                const int sb = subd + i * LD;
                if (live && sb < nsbd) {
                    float hx[32];
                    const float4 *src = (const float4 *)(hs + (j * nsbd + sb) * 36);
#pragma unroll
                    for (int c = 0; c < 8; c++) *(float4 *)(hx + 4 * c) = src[c];
                    d += FD::dot(draw[q][i], ldsd, hx);
                }
            }
            d = group_sum<LD>(d);
            if (subd == 0) part[grp][j * RPD + rsd] = (dslot[q] == 0xFFFFFFFFu || !ok) ? __int_as_float(0x7fc00000) : d;
        }
        __syncthreads();
        const int tg4 = threadIdx.x & 255;
        if (tg4 < RPD) {
            const int rr = grp_i * RPD + tg4;
            if (rr < a.H) {
                float acc = 0.f;
                if (PFB && (first || bp == bp2)) {
#pragma unroll
                    for (int j = 0; j < 4 * PPW; j++)
                        if (j < K) acc += pick_w[j] * (part[grp][j * RPD + tg4] + bq[first ? 0 : 1][j]);
                } else {
                    for (int j = 0; j < K; j++) {
                        float d = part[grp][j * RPD + tg4];
                        if (a.bd) d += a.bd[(int64_t)pick_e[j] * a.H + rr];
                        acc += pick_w[j] * d;
                    }
                }
                a.out[rr] = acc;
            }
        }
        __syncthreads();
    }
    CW_PHASE(7);  // end
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
    else if (a.E <= 512) hipLaunchKernelGGL((k_moe_gateup<Fmt, LPR, NX, 8, ROWS>), grid, dim3(256), 0, s, a);
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
    case CW_Q2_K: return by_shape<FQ2_K, DOWN>(a, T, s);
    case CW_Q4_K: return by_shape<FQ4_K, DOWN>(a, T, s);
    case CW_MXFP4: return by_shape<FMXFP4, DOWN>(a, T, s);
    case CW_MXFP4_R16: return by_shape<FMXFP4R16, DOWN>(a, T, s);
    case CW_IQ2_XXS: return by_shape<FIQ2_XXS, DOWN>(a, T, s);
    case CW_IQ2_S: return by_shape<FIQ2_S, DOWN>(a, T, s);
    case CW_IQ3_S: return by_shape<FIQ3_S, DOWN>(a, T, s);
    case CW_Q5_K: return by_shape<FQ5_K, DOWN>(a, T, s);
    case CW_Q6_K: return by_shape<FQ6_K, DOWN>(a, T, s);
    case CW_IQ3_XXS: return by_shape<FIQ3_XXS, DOWN>(a, T, s);
    case CW_IQ4_XS: return by_shape<FIQ4_XS, DOWN>(a, T, s);
    default: return set_error(CW_ENOTSUP, "moe: dtype %d is not supported", dtype);
    }
}

// LDS for the staged hidden rows of one decode call: K rows of P floats, 36 per 32
static size_t decode_hidden_lds(const MoeArgs &a) { return (size_t)a.K * (a.P / 32) * 36 * sizeof(float); }
// the dynamic LDS of an instance: the hidden rows, or for LDS-staged gate/up rows (RI = 2) the
// waves' two item buffers or x if those are larger (they are used before the hidden rows)
template <class FG, int G, int RI>
static size_t decode_lds(const MoeArgs &a) {
    size_t n = decode_hidden_lds(a);
    if (RowDma<FG>::on) {
        const size_t items = Rows16<FG>::on ? (size_t)ks_lds(a.H) : 4 * G * 2 * (size_t)(2 * RI * row_window(a.H / 32 * FG::TS) + 16);
        const size_t xs = (size_t)(a.H / 4 + 256 * G - 1) / (256 * G) * (256 * G) * 16;  // x, copied in rounds of one chunk per thread
        if (items > n) n = items;
        if (xs > n) n = xs;
    }
    return n;
}
static constexpr size_t DECODE_MAX_HIDDEN_LDS = 64 * 1024;

// Grid of the persistent decode kernel: every block must be resident at once for the barrier, so
// the grid is sized from the occupancy of this kernel at this call's LDS size on the current
// device (a few entries remembered, under a lock, so concurrent callers never size a grid from
// another call's entry). 0 on failure.
template <class Kern>
static int decode_grid(Kern kern, int which, const MoeArgs &a, size_t lds, int threads, int want, int *per_cu) {
    struct Occ {
        int dev = -1, which = -1;
        size_t lds = 0;
        int per_cu = 0, cus = 0;
    };
    static std::mutex mu;
    static Occ cache[8];
    static int next = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    Occ o;
    {
        std::lock_guard<std::mutex> lock(mu);
        for (const Occ &c : cache)
            if (c.dev == dev && c.which == which && c.lds == lds) o = c;
    }
    if (!o.per_cu) {
        o.dev = dev;
        o.which = which;
        o.lds = lds;
        if (hipDeviceGetAttribute(&o.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&o.per_cu, kern, threads, lds) != hipSuccess || o.per_cu < 1)
            return 0;
        std::lock_guard<std::mutex> lock(mu);
        cache[next++ & 7] = o;
    }
    const int grid = o.per_cu * o.cus < want ? o.per_cu * o.cus : want;
    *per_cu = (grid + o.cus - 1) / o.cus;
    return grid;
}

template <class FG, int LG, int XG, class FD, int LD, int XD, int PER, int PPW, int G, int RI>
static int decode_launch_per(const MoeArgs &a, int which, hipStream_t s) {
    // LDS-staged gate/up rows: two chunk loads per row, so that every load instruction the
    // kernel's waits count has active lanes
    if (RowDma<FG>::on) {
        const int w = row_window(a.H / 32 * FG::TS);
        if (w <= 1024 || w > 2048) return CW_ENOTSUP;
        if ((uintptr_t)a.x & 15) return CW_ENOTSUP;  // x is copied in 16-byte chunks
    }
    if (Rows16<FG>::on) {  // K-split items: matrices 16-byte aligned, at most 16 loads per wave per part
        if (((uintptr_t)a.wg | (uintptr_t)a.wu | (uintptr_t)a.sg | (uintptr_t)a.su) & 15) return CW_ENOTSUP;
        if ((int64_t)(a.I + 15) * a.rbg >= ((int64_t)1 << 31)) return CW_ENOTSUP;  // 32-bit offsets
    }
    if (Rows16<FD>::on && (int64_t)(a.H + 15) * a.rbd >= ((int64_t)1 << 31)) return CW_ENOTSUP;  // 32-bit offsets in down
    const size_t lds = decode_lds<FG, G, RI>(a);
    const int RPD = 64 / LD;
    auto kern = k_moe_decode<FG, LG, XG, FD, LD, XD, PER, PPW, G, RI>;
    MoeArgs b = a;
    const int grid = decode_grid(kern, 4 * which + G, a, lds, 256 * G, (a.H + RPD * G - 1) / (RPD * G), &b.per_cu);
    if (!grid) return set_error(CW_EHIP, "moe decode: occupancy query failed");
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256 * G), lds, s, b);
    return check_launch("k_moe_decode");
}

template <class FG, int LG, int XG, class FD, int LD, int XD, int PPW, int G, int RI>
static int decode_launch(const MoeArgs &a, hipStream_t s) {
    // lanes hold 4, 8 or 16 router logits each (E up to 256, 512, 1024)
    if (a.E <= 256) return decode_launch_per<FG, LG, XG, FD, LD, XD, 4, PPW, G, RI>(a, 0, s);
    if (a.E <= 512) return decode_launch_per<FG, LG, XG, FD, LD, XD, 8, PPW, G, RI>(a, 1, s);
    return decode_launch_per<FG, LG, XG, FD, LD, XD, 16, PPW, G, RI>(a, 2, s);
}

template <class FG, int LG, int XG, class FD, int LD, int XD, int G = 1, int RI = 2>
static int decode_ppw(const MoeArgs &a, hipStream_t s) {
    const int ppw = (a.K + 3) / 4;
    if (ppw == 1) return decode_launch<FG, LG, XG, FD, LD, XD, 1, G, RI>(a, s);
    if (ppw == 2) return decode_launch<FG, LG, XG, FD, LD, XD, 2, G, RI>(a, s);
    if (ppw == 3) return decode_launch<FG, LG, XG, FD, LD, XD, 3, G, RI>(a, s);
    return CW_ENOTSUP;
}

// the format / shape pairs of the benchmark configurations; others take the two-kernel path
int moe_decode(int dtg, int dtd, const MoeArgs &a, hipStream_t s) {
    if (a.K > 12 || a.E > 1024 || decode_hidden_lds(a) > DECODE_MAX_HIDDEN_LDS) return CW_ENOTSUP;
    const int nsg = a.H / 32, nsd = a.P / 32;
    // config 3 in blocks of 8 waves, one per CU: each hidden row is staged once per CU, and half
    // as many blocks meet at the barrier (12.58 -> 12.50 us per layer; config 5 measured slower
    // so, 16.9 -> 18.9, and config 4 in blocks of 12 waves 30.1 -> 32.0)
    if (dtg == CW_IQ2_XXS && dtd == CW_IQ2_S && nsg == 64 && nsd == 16) return decode_ppw<FIQ2_XXS, 64, 1, FIQ2_S, 16, 1, 2>(a, s);
    if (dtg == CW_IQ2_XXS && dtd == CW_IQ2_XXS && nsg == 64 && nsd == 16) return decode_ppw<FIQ2_XXS, 64, 1, FIQ2_XXS, 16, 1>(a, s);
    if (dtg == CW_IQ2_S && dtd == CW_IQ2_S && nsg == 64 && nsd == 16) return decode_ppw<FIQ2_S, 64, 1, FIQ2_S, 16, 1>(a, s);
    if (dtg == CW_IQ3_S && dtd == CW_Q4_K && nsg == 64 && nsd == 16) return decode_ppw<FIQ3_S, 64, 1, FQ4_K, 16, 1>(a, s);
    // gpt-oss rows (2,880 weights): down at 32 lanes per row, two rows per block pass (half the
    // passes, reductions and block barriers of 64 lanes per row: 44.9 -> 39.2 us per layer)
    if (dtg == CW_MXFP4 && dtd == CW_MXFP4 && nsg == 90 && nsd == 90) return decode_ppw<FMXFP4, 64, 2, FMXFP4, 32, 3>(a, s);
    if (dtg == CW_MXFP4_R16 && dtd == CW_MXFP4_R16 && nsg == 90 && nsd == 90)
        return decode_ppw<FMXFP4R16, 64, 2, FMXFP4R16, 32, 3>(a, s);
    // gate/up as GGUF rows, down in row groups of 16: the decode's down phase reads both as fast
    if (dtg == CW_MXFP4 && dtd == CW_MXFP4_R16 && nsg == 90 && nsd == 90) return decode_ppw<FMXFP4, 64, 2, FMXFP4R16, 32, 3>(a, s);
    return CW_ENOTSUP;
}

#ifdef CWMOE_PHASES
extern "C" int cw_dbg_phases(unsigned long long *out, int blocks) {
    if (blocks < 0 || blocks > 4096) return -1;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_phase_stamps), (size_t)blocks * 8 * sizeof(unsigned long long), 0,
                               hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
#endif

uint32_t decode_barrier_errors() {
    uint32_t n = 0;
    if (hipMemcpyFromSymbol(&n, HIP_SYMBOL(g_decode_errors), sizeof n) != hipSuccess) return 0xFFFFFFFFu;
    return n;
}

int moe_gateup(int dtype, const MoeArgs &a, int T, hipStream_t s) { return T ? by_fmt<false>(dtype, a, T, s) : CW_OK; }
int moe_down(int dtype, const MoeArgs &a, int T, hipStream_t s) {
    if (a.K > 32) return set_error(CW_ENOTSUP, "moe: top_k %d above 32", a.K);
    return T ? by_fmt<true>(dtype, a, T, s) : CW_OK;
}

}  // namespace cw
