// Router top-k, activations, weighted combine, slot resolve and the MoE layer (gfx950).
#include <math.h>
#include <stdlib.h>
#include <algorithm>
#include <mutex>

#include "cw_common.h"
#include "cw_gemv.h"
#include "cw_mfma.h"
#include "cw_router.h"
#include "cw_moe_fused.h"
#include "cw_wave.h"

namespace cw {

// ------------------------------------------------------------------------------ router

// One wavefront per token (cw_wave.h: softmax, top-k on the logits, ties to the lower index).
template <int PER>
__global__ __launch_bounds__(64) void k_route(const float *logits, int E, int K, int norm, uint32_t *ids, float *w) {
    const int t = blockIdx.x, lane = threadIdx.x;
    uint32_t id;
    float wt;
    wave_route<PER>(logits + (int64_t)t * E, E, K, norm, &id, &wt);
    if (lane < K) {
        ids[(int64_t)t * K + lane] = id;
        w[(int64_t)t * K + lane] = wt;
    }
}

__global__ void k_swiglu(const float *g, const float *u, float *h, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float v = g[i];
        h[i] = v / (1.0f + expf(-v)) * u[i];
    }
}

// silu != 0: plain h = silu(g) * u with zero padding (the fallback of mixed gate/up formats)
__global__ void k_clamped_swiglu(const float *g, const float *u, const float *gb, const float *ub, const uint32_t *ids,
                                 int64_t rows, int width, int out_w, float alpha, float limit, float *h, int silu) {
    const int64_t n = rows * out_w;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / out_w;
        const int c = (int)(i % out_w);
        if (c >= width) { h[i] = 0.f; continue; }
        if (silu) {
            const float v = g[r * width + c];
            h[i] = v / (1.0f + expf(-v)) * u[r * width + c];
            continue;
        }
        const uint32_t e = ids[r];
        float gv = g[r * width + c] + (gb ? gb[(int64_t)e * width + c] : 0.f);
        float uv = u[r * width + c] + (ub ? ub[(int64_t)e * width + c] : 0.f);
        gv = fminf(gv, limit);
        uv = fminf(fmaxf(uv, -limit), limit);
        h[i] = (uv + 1.0f) * (gv * (1.0f / (1.0f + expf(-(gv * alpha)))));
    }
}

__global__ void k_weighted_sum(const float *down, const float *w, const float *bd, const uint32_t *ids, int T, int K, int H,
                               float *out) {
    const int64_t n = (int64_t)T * H;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = i / H;
        const int j = (int)(i % H);
        float acc = 0.f;
        for (int e = 0; e < K; e++) {
            float d = down[(t * K + e) * H + j];
            if (bd) d += bd[(int64_t)ids[t * K + e] * H + j];
            acc += d * w[t * K + e];
        }
        out[i] = acc;
    }
}

__global__ void k_resolve(const uint32_t *ids, const uint32_t *table, int n, uint32_t *slots, uint32_t *missing) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        uint32_t s = table[ids[i]];
        if (s == CW_NO_SLOT) {
            if (missing) atomicAdd(missing, 1u);
            s = 0;
        }
        slots[i] = s;
    }
}

static dim3 flat_grid(int64_t n) {
    int64_t b = (n + 255) / 256;
    return dim3((unsigned)(b < 8192 ? (b > 0 ? b : 1) : 8192));
}

static int route(const float *logits, int T, int E, int K, int norm, uint32_t *ids, float *w, hipStream_t s) {
    if (T == 0) return CW_OK;
    if (E <= 256) hipLaunchKernelGGL(k_route<4>, dim3(T), dim3(64), 0, s, logits, E, K, norm, ids, w);
    else if (E <= 512) hipLaunchKernelGGL(k_route<8>, dim3(T), dim3(64), 0, s, logits, E, K, norm, ids, w);
    else hipLaunchKernelGGL(k_route<16>, dim3(T), dim3(64), 0, s, logits, E, K, norm, ids, w);
    return check_launch("k_route");
}

// ------------------------------------------------------------------------------ MoE layer

struct MoeLayout {
    size_t state, ids, w, slots, g, u, h, total;
    // grouped (MFMA) path
    bool grouped;
    size_t pile_pick, pile_tok, tiles, n_tiles, x16, xscale, h16, hscale, dn;
};

// Token count from which the layer runs as grouped MFMA GEMMs instead of per-pick matvecs
// (CWMOE_PREFILL_MIN_TOKENS overrides; the reference switches to grouped kernels above 8 tokens,
// crates/engine/src/experts.rs:2225).
static int prefill_min_tokens() {
    const char *e = getenv("CWMOE_PREFILL_MIN_TOKENS");
    return e ? atoi(e) : 16;
}

// One-token layers run as one persistent launch unless CWMOE_DECODE_KERNELS=2 asks for the
// two-kernel form (gate/up, then down).
static bool decode_single_launch() {
    const char *e = getenv("CWMOE_DECODE_KERNELS");
    return !(e && atoi(e) == 2);
}

// Polls of the one-launch decode's device-wide barrier before a block gives up (outputs NaN, the
// error counted): CWMOE_BARRIER_POLLS overrides, for tests of the give-up path.
static uint32_t decode_polls() {
    const char *e = getenv("CWMOE_BARRIER_POLLS");
    return e ? (uint32_t)strtoul(e, nullptr, 10) : (1u << 17);
}

static bool grouped_path(const cw_moe_desc *d, int T) {
    return T >= prefill_min_tokens() && d->dtype[0] == d->dtype[1] && mfma_supported(d->dtype[0]) &&
           mfma_supported(d->dtype[2]) && (d->slot_table ? d->n_slots : d->n_experts) <= 1024;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static int check_desc(const cw_moe_desc *d, int T) {
    CW_REQUIRE(d != nullptr, "moe: null descriptor");
    CW_REQUIRE(T >= 0, "moe: negative token count %d", T);
    CW_REQUIRE(d->n_experts > 0 && d->n_experts <= 1024, "moe: %d experts (1..1024 supported)", d->n_experts);
    CW_REQUIRE(d->top_k > 0 && d->top_k <= 32 && d->top_k <= d->n_experts, "moe: top_k %d for %d experts", d->top_k, d->n_experts);
    CW_REQUIRE(d->hidden > 0 && d->inter > 0, "moe: hidden %d, inter %d", d->hidden, d->inter);
    CW_REQUIRE(d->act == CW_ACT_SILU || d->act == CW_ACT_CLAMPED_SWIGLU, "moe: unknown activation %d", d->act);
    CW_REQUIRE(d->pad == 0 || d->pad >= d->inter, "moe: pad %d below inter %d", d->pad, d->inter);
    const int P = d->pad > d->inter ? d->pad : d->inter;
    const int ks[3] = {d->hidden, d->hidden, P};
    const int ns[3] = {d->inter, d->inter, d->hidden};
    const int n_slots = d->slot_table ? d->n_slots : d->n_experts;
    CW_REQUIRE(n_slots > 0, "moe: %d slots", n_slots);
    for (int m = 0; m < 3; m++) {
        if (!is_expert_type(d->dtype[m])) return set_error(CW_ENOTSUP, "moe: matrix %d has unsupported dtype %d", m, d->dtype[m]);
        const int bs = cw_block_size(d->dtype[m]);
        CW_REQUIRE(ks[m] % bs == 0, "moe: matrix %d rows of %d weights are not whole %d-weight blocks", m, ks[m], bs);
        if (ks[m] > max_gemv_k()) return set_error(CW_ENOTSUP, "moe: rows of %d weights exceed %d", ks[m], max_gemv_k());
        const int64_t need = matrix_bytes(d->dtype[m], ns[m], (int64_t)(ks[m] / bs) * cw_type_size(d->dtype[m]));
        CW_REQUIRE(d->slot_stride[m] >= need, "moe: matrix %d slot stride %lld below its %lld bytes", m,
                   (long long)d->slot_stride[m], (long long)need);
        CW_REQUIRE(d->w[m] != nullptr, "moe: matrix %d is null", m);
    }
    CW_REQUIRE(d->act == CW_ACT_CLAMPED_SWIGLU || (!d->bias[0] && !d->bias[1] && !d->bias[2]),
               "moe: biases need the clamped SwiGLU activation");
    if ((d->dtype[0] == CW_MXFP4_R16 || d->dtype[1] == CW_MXFP4_R16) && d->dtype[0] != d->dtype[1])
        return set_error(CW_ENOTSUP, "moe: gate and up in row groups of 16 need the same format");
    for (int m = 0; m < 3; m++)
        if (d->dtype[m] == CW_MXFP4_R16 && !mxfp4_scaled_for(CW_MXFP4_R16, ks[m]))
            return set_error(CW_ENOTSUP, "moe: matrix %d in row groups of 16 has rows of %d weights (over 128 needed)", m, ks[m]);
    return CW_OK;
}

static MoeLayout layout(const cw_moe_desc *d, int T) {
    const size_t TK = (size_t)T * d->top_k;
    const int P = d->pad > d->inter ? d->pad : d->inter;
    MoeLayout L;
    size_t off = 0;
    // the decode's sync state first, at the same offset for every token count, so that a workspace
    // reused across calls of any size keeps it (zero between calls)
    L.state = off; off = align256(off + DECODE_STATE_BYTES);
    L.ids = off; off = align256(off + TK * 4);
    L.w = off; off = align256(off + TK * 4);
    L.slots = off; off = align256(off + TK * 4);
    const bool split = d->dtype[0] != d->dtype[1];
    L.g = off; off = align256(off + (split ? TK * d->inter * 4 : 0));
    L.u = off; off = align256(off + (split ? TK * d->inter * 4 : 0));
    L.h = off; off = align256(off + TK * (size_t)P * 4);
    L.grouped = grouped_path(d, T);
    if (L.grouped) {
        const int n_slots = d->slot_table ? d->n_slots : d->n_experts;
        L.pile_pick = off; off = align256(off + TK * 4);
        L.pile_tok = off; off = align256(off + TK * 4);
        L.tiles = off; off = align256(off + (size_t)max_tiles((int)TK, n_slots) * sizeof(MfTile));
        L.n_tiles = off; off = align256(off + 4);
        // fp16 rows, or for MXFP4 on the scaled MFMA the rows packed as FP6 terms
        const bool gx = mxfp4_scaled_for(d->dtype[0], d->hidden), dx = mxfp4_scaled_for(d->dtype[2], P);
        L.x16 = off; off = align256(off + (gx ? fp6_rows_bytes(T, d->hidden) : (size_t)T * d->hidden * 2));
        L.xscale = off; off = align256(off + (size_t)T * 4);
        L.h16 = off; off = align256(off + (dx ? fp6_rows_bytes((int64_t)TK, P) : TK * (size_t)P * 2));
        L.hscale = off; off = align256(off + TK * 4);
        L.dn = off; off = align256(off + TK * (size_t)d->hidden * 4);
    }
    L.total = off;
    return L;
}

// Prefill: route, group the picks by slot, gate/up and down as grouped MFMA GEMMs.
static int moe_grouped(const cw_moe_desc *d, const MoeArgs &a, const MoeLayout &L, uint8_t *base, int T, hipStream_t s) {
    int rc;
    const int K = a.K, TK = T * K, P = a.P;
    if ((rc = route(a.logits, T, a.E, K, d->norm, a.ids, a.w, s))) return rc;
    const uint32_t *slots = a.ids;
    if (d->slot_table) {
        hipLaunchKernelGGL(k_resolve, flat_grid(TK), dim3(256), 0, s, a.ids, d->slot_table, TK, a.slots, a.missing);
        if ((rc = check_launch("k_resolve"))) return rc;
        slots = a.slots;
    }
    int *pile_pick = (int *)(base + L.pile_pick), *pile_tok = (int *)(base + L.pile_tok), *n_tiles = (int *)(base + L.n_tiles);
    MfTile *tiles = (MfTile *)(base + L.tiles);
    if ((rc = mfma_piles(slots, a.ids, TK, K, a.n_slots, pile_pick, pile_tok, tiles, n_tiles, s))) return rc;
    uint16_t *x16 = (uint16_t *)(base + L.x16), *h16 = (uint16_t *)(base + L.h16);
    float *xscale = (float *)(base + L.xscale), *hscale = (float *)(base + L.hscale);
    // MXFP4 matrices run on the block-scaled MFMA (activations as FP6 terms), the others on fp16 MFMA
    const bool gx = mxfp4_scaled_for(d->dtype[0], a.H), dx = mxfp4_scaled_for(d->dtype[2], P);
    if (gx) rc = pack_rows_fp6(a.x, T, a.H, a.H, (uint8_t *)x16, s);
    else rc = pack_rows_f16(a.x, T, a.H, a.H, x16, xscale, s, nullptr, mfma_k_permuted(d->dtype[0]));
    if (rc) return rc;
    // gate/up and down both on the scaled MFMA: gate/up packs the hidden rows itself
    const bool fuse_h = gx && dx;
    if (!fuse_h && P > a.I && (rc = fill_zero(a.h, (int64_t)TK * P, s))) return rc;
    const int tmax = max_tiles(TK, a.n_slots);

    MfArgs g = {};
    g.w0 = a.wg;
    g.w1 = a.wu;
    g.s0 = a.sg;
    g.s1 = a.su;
    g.row_bytes = a.rbg;
    g.n = a.I;
    g.k = a.H;
    g.a16 = x16;
    g.ascale = xscale;
    g.lda = a.H;
    g.rows = pile_tok;
    g.tiles = tiles;
    g.n_tiles = n_tiles;
    g.pile_pick = pile_pick;
    g.K = K;
    g.act = a.act;
    g.alpha = a.alpha;
    g.limit = a.limit;
    g.bias0 = a.bg;
    g.bias1 = a.bu;
    g.ids = a.ids;
    g.h = a.h;
    g.ldh = P;
    g.layout = d->dtype[0] == CW_MXFP4_R16;
    if (gx) {
        g.ap = (const uint8_t *)x16;
        g.ap_row = (int64_t)fp6_rows_bytes(1, a.H);
        g.ap_rows = T;
        if (fuse_h) {
            g.hp = (uint8_t *)h16;
            g.hp_row = (int64_t)fp6_rows_bytes(1, P);
            g.hp_blocks = (int)(g.hp_row / 304 * 4);
        }
        rc = mxfp4_gateup(g, tmax, s);
    } else {
        rc = mfma_gateup(d->dtype[0], g, tmax, s);
    }
    if (rc) return rc;
    if (fuse_h) rc = CW_OK;
    else if (dx) rc = pack_rows_fp6(a.h, TK, P, P, (uint8_t *)h16, s);
    else rc = pack_rows_f16(a.h, TK, P, P, h16, hscale, s, nullptr, mfma_k_permuted(d->dtype[2]));
    if (rc) return rc;

    MfArgs dn = {};
    dn.w0 = a.wd;
    dn.s0 = a.sd;
    dn.row_bytes = a.rbd;
    dn.n = a.H;
    dn.k = P;
    dn.a16 = h16;
    dn.ascale = hscale;
    dn.lda = P;
    dn.rows = nullptr;
    dn.tiles = tiles;
    dn.n_tiles = n_tiles;
    dn.pile_pick = pile_pick;
    dn.K = K;
    dn.dn = (float *)(base + L.dn);
    dn.layout = d->dtype[2] == CW_MXFP4_R16;
    if (dx) {
        dn.ap = (const uint8_t *)h16;
        dn.ap_row = (int64_t)fp6_rows_bytes(1, P);
        dn.ap_rows = TK;
        rc = mxfp4_down(dn, tmax, s);
    } else {
        rc = mfma_down(d->dtype[2], dn, tmax, s);
    }
    if (rc) return rc;
    return combine_picks(dn.dn, a.w, a.bd, a.ids, slots, a.n_slots, T, K, a.H, a.out, s);
}

static int moe_layer(const cw_moe_desc *d, const float *x, const float *logits, int T, float *out, uint32_t *ids_out,
                     float *w_out, uint32_t *missing, void *ws, size_t ws_bytes, hipStream_t s) {
    int rc = check_desc(d, T);
    if (rc) return rc;
    if (T == 0) return CW_OK;
    CW_REQUIRE(x && logits && out, "moe: null x, logits or out");
    const MoeLayout L = layout(d, T);
    CW_REQUIRE(ws && ws_bytes >= L.total, "moe: workspace of %zu bytes, %zu needed", ws_bytes, L.total);
    uint8_t *base = (uint8_t *)ws;
    const int K = d->top_k, P = d->pad > d->inter ? d->pad : d->inter;

    MoeArgs a = {};
    a.wg = (const uint8_t *)d->w[0];
    a.wu = (const uint8_t *)d->w[1];
    a.wd = (const uint8_t *)d->w[2];
    a.sg = d->slot_stride[0];
    a.su = d->slot_stride[1];
    a.sd = d->slot_stride[2];
    a.rbg = (int64_t)(d->hidden / cw_block_size(d->dtype[0])) * cw_type_size(d->dtype[0]);
    a.rbd = (int64_t)(P / cw_block_size(d->dtype[2])) * cw_type_size(d->dtype[2]);
    a.E = d->n_experts;
    a.K = K;
    a.H = d->hidden;
    a.I = d->inter;
    a.P = P;
    a.n_slots = d->slot_table ? d->n_slots : d->n_experts;
    a.norm = d->norm;
    a.act = d->act;
    a.alpha = d->alpha;
    a.limit = d->limit;
    a.bg = d->bias[0];
    a.bu = d->bias[1];
    a.bd = d->bias[2];
    a.table = d->slot_table;
    a.missing = missing;
    a.x = x;
    a.logits = logits;
    a.ids = ids_out ? ids_out : (uint32_t *)(base + L.ids);
    a.w = w_out ? w_out : (float *)(base + L.w);
    a.slots = (uint32_t *)(base + L.slots);
    a.h = (float *)(base + L.h);
    a.out = out;
    a.state = base + L.state;
    a.polls = decode_polls();

    if (L.grouped) return moe_grouped(d, a, L, base, T, s);
    if (T == 1 && d->dtype[0] == d->dtype[1] && decode_single_launch()) {
        rc = moe_decode(d->dtype[0], d->dtype[2], a, s);
        if (rc != CW_ENOTSUP) return rc;
    }
    if (d->dtype[0] == d->dtype[1]) {
        if ((rc = moe_gateup(d->dtype[0], a, T, s))) return rc;
    } else {
        // gate and up in different formats: route, resolve, two matvecs, the activation
        if ((rc = route(logits, T, a.E, K, d->norm, a.ids, a.w, s))) return rc;
        if (d->slot_table) {
            hipLaunchKernelGGL(k_resolve, flat_grid((int64_t)T * K), dim3(256), 0, s, a.ids, d->slot_table, T * K, a.slots,
                               missing);
            if ((rc = check_launch("k_resolve"))) return rc;
        } else {
            a.slots = a.ids;
        }
        float *g = (float *)(base + L.g), *u = (float *)(base + L.u);
        for (int m = 0; m < 2; m++) {
            GemvArgs b = {};
            b.w0 = (const uint8_t *)d->w[m];
            b.slot_stride0 = d->slot_stride[m];
            b.row_bytes = (int64_t)(d->hidden / cw_block_size(d->dtype[m])) * cw_type_size(d->dtype[m]);
            b.n = d->inter;
            b.k = d->hidden;
            b.nsb = d->hidden / 32;
            b.n_slots = a.n_slots;
            b.x = x;
            b.x_per_pick = 0;
            b.ids = a.slots;
            b.K = K;
            b.out = m == 0 ? g : u;
            b.out_width = d->inter;
            if ((rc = gemv_plain(d->dtype[m], b, T * K, s))) return rc;
        }
        const int64_t rows = (int64_t)T * K;
        const bool silu = d->act == CW_ACT_SILU;
        hipLaunchKernelGGL(k_clamped_swiglu, flat_grid(rows * P), dim3(256), 0, s, g, u, silu ? nullptr : d->bias[0],
                           silu ? nullptr : d->bias[1], a.ids, rows, d->inter, P, silu ? 1.0f : d->alpha,
                           silu ? INFINITY : d->limit, a.h, silu ? 1 : 0);
        if ((rc = check_launch("k_clamped_swiglu"))) return rc;
    }
    return moe_down(d->dtype[2], a, T, s);
}

// ------------------------------------------------------------------------------ grouped expert matmul

// rows of picks whose slot is past the bank: NaN (they are in no pile, so the GEMM writes nothing)
__global__ void k_nan_rows(const uint32_t *ids, int n_picks, uint32_t n_slots, int n, float *out) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n_picks; i += gridDim.x * blockDim.x)
        if (ids[i] >= n_slots)
            for (int r = 0; r < n; r++) out[(int64_t)i * n + r] = __int_as_float(0x7fc00000);
}

struct GroupedLayout {
    size_t pile_pick, pile_tok, tiles, n_tiles, x16, xscale, total;
};
static GroupedLayout grouped_layout(int dtype, int64_t k, int64_t n_slots, int x_per_pick, int K, int T) {
    const size_t TK = (size_t)T * K, rows = x_per_pick ? TK : (size_t)T;
    GroupedLayout L;
    size_t off = 0;
    L.pile_pick = off; off = align256(off + TK * 4);
    L.pile_tok = off; off = align256(off + TK * 4);
    L.tiles = off; off = align256(off + (size_t)max_tiles((int)TK, (int)n_slots) * sizeof(MfTile));
    L.n_tiles = off; off = align256(off + 4);
    const bool gx = mxfp4_scaled_for(dtype, k);  // rows packed as FP6 terms for the scaled MFMA
    L.x16 = off; off = align256(off + (gx ? fp6_rows_bytes((int64_t)rows, k) : rows * (size_t)k * 2));
    L.xscale = off; off = align256(off + rows * 4);
    L.total = off;
    return L;
}

// CW_OK when the grouped GEMM takes this call, else the status to return (CW_ENOTSUP: use cw_matvec_id)
static int grouped_check(int dtype, int64_t n, int64_t k, int64_t n_slots, int64_t slot_stride, int K, int T) {
    if (!is_expert_type(dtype)) return set_error(CW_ENOTSUP, "matmul_id_grouped: dtype %d is not supported", dtype);
    if (!mfma_supported(dtype)) return set_error(CW_ENOTSUP, "matmul_id_grouped: dtype %d has no grouped kernel", dtype);
    const int bs = cw_block_size(dtype);
    CW_REQUIRE(n > 0 && k > 0 && n < (1ll << 31), "matmul_id_grouped: n %lld, k %lld", (long long)n, (long long)k);
    CW_REQUIRE(k % bs == 0, "matmul_id_grouped: k %lld is not whole %d-weight blocks", (long long)k, bs);
    CW_REQUIRE(K > 0 && K <= 32 && T >= 0, "matmul_id_grouped: K %d, T %d", K, T);
    CW_REQUIRE(n_slots > 0, "matmul_id_grouped: %lld slots", (long long)n_slots);
    CW_REQUIRE((int64_t)T * K < (1ll << 30), "matmul_id_grouped: %lld picks", (long long)T * K);
    const int64_t row_bytes = k / bs * cw_type_size(dtype);
    CW_REQUIRE(slot_stride >= matrix_bytes(dtype, n, row_bytes), "matmul_id_grouped: slot stride %lld below the %lld-byte matrix",
               (long long)slot_stride, (long long)matrix_bytes(dtype, n, row_bytes));
    if (n_slots > 1024) return set_error(CW_ENOTSUP, "matmul_id_grouped: %lld slots (1024 max)", (long long)n_slots);
    if (dtype == CW_MXFP4_R16 && !mxfp4_scaled_for(dtype, k))
        return set_error(CW_ENOTSUP, "matmul_id_grouped: rows in groups of 16 of %lld weights (over 128 needed)", (long long)k);
    if (k % 256 && dtype != CW_Q8_0 && dtype != CW_MXFP4 && dtype != CW_MXFP4_R16)
        return set_error(CW_ENOTSUP, "matmul_id_grouped: k %lld is not whole super-blocks", (long long)k);
    if (k > 8192) return set_error(CW_ENOTSUP, "matmul_id_grouped: k %lld above 8192", (long long)k);
    return CW_OK;
}

// ------------------------------------------------------------------------------ the layer without a workspace

// Scratch of cw_moe_layer_noalloc, for callers that cannot allocate: one array per device, loaded
// with the library (zero-filled, as the decode's sync state at its start must be) and kept until the
// process ends. Every call on a device shares it: the layer's regions are rewritten by each call
// before they are read, and the sync state is back at zero when each call's kernels end, so a call
// needs nothing cleared; calls that overlap in time on one device race on it.
constexpr size_t NOALLOC_SCRATCH_BYTES = CW_MOE_NOALLOC_BYTES;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

// The device address of this device's copy of `scratch`, looked up once per device (host code
// must not use the array's name as an address: that is a host-side stand-in).
static int noalloc_scratch(void **out) {
    constexpr int MAX_DEV = 64;
    static std::mutex mu;
    static void *ptr[MAX_DEV];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV)
        return set_error(CW_EHIP, "moe noalloc: no current device (or device %d past %d)", dev, MAX_DEV);
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return set_error(CW_EHIP, "moe noalloc: scratch address: %s", hipGetErrorString(e));
        ptr[dev] = p;
    }
    *out = ptr[dev];
    return CW_OK;
}

// out[t][i] = (accumulate ? out[t][i] : 0) + y[t][i] * sigmoid(glog[t]) (glog NULL: factor 1)
__global__ void k_gate_scale_add(const float *y, const float *glog, int T, int H, int accumulate, float *out) {
    const int64_t n = (int64_t)T * H;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float g = glog ? 1.0f / (1.0f + expf(-glog[i / H])) : 1.0f;
        out[i] = (accumulate ? out[i] : 0.0f) + y[i] * g;
    }
}

static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

// workspace of the shared expert: gate and up rows (the hidden rows overwrite gate), down rows,
// gate logits, and one region the three matmuls take in turn
struct SharedLayout {
    size_t g, u, y, glog, mm, total;
};
static SharedLayout shared_layout(const cw_shared_desc *d, int T) {
    SharedLayout L;
    const size_t ti = (size_t)T * d->inter * 4, th = (size_t)T * d->hidden * 4;
    size_t mm = cw_qmatmul_workspace_size(d->dtype[0], d->inter, d->hidden, T);
    mm = std::max(mm, cw_qmatmul_workspace_size(d->dtype[1], d->inter, d->hidden, T));
    mm = std::max(mm, cw_qmatmul_workspace_size(d->dtype[2], d->hidden, d->inter, T));
    L.g = 0;
    L.u = L.g + al256(ti);
    L.y = L.u + al256(ti);
    L.glog = L.y + al256(th);
    L.mm = L.glog + al256((size_t)T * 4);
    L.total = L.mm + al256(mm);
    return L;
}

}  // namespace cw

using namespace cw;

extern "C" {

size_t cw_shared_expert_workspace_size(const cw_shared_desc *d, int T) {
    if (!d || T <= 0 || d->hidden <= 0 || d->inter <= 0) return 0;
    return shared_layout(d, T).total;
}

int cw_shared_expert(const cw_shared_desc *d, const float *x, int T, float *out, int accumulate, void *ws,
                     size_t ws_bytes, cw_stream_t stream) {
    CW_REQUIRE(d && d->hidden > 0 && d->inter > 0 && T >= 0, "shared expert: bad descriptor or T %d", T);
    if (T == 0) return CW_OK;
    CW_REQUIRE(x && out && d->w[0] && d->w[1] && d->w[2], "shared expert: null pointer");
    const SharedLayout L = shared_layout(d, T);
    CW_REQUIRE(ws && ws_bytes >= L.total, "shared expert: workspace of %zu bytes, %zu needed", ws_bytes, L.total);
    hipStream_t s = (hipStream_t)stream;
    uint8_t *base = (uint8_t *)ws;
    float *g = (float *)(base + L.g), *u = (float *)(base + L.u), *y = (float *)(base + L.y);
    float *glog = d->gate_inp ? (float *)(base + L.glog) : nullptr;
    void *mm = base + L.mm;
    const size_t mm_bytes = L.total - L.mm;
    int rc;
    if ((rc = cw_qmatmul(d->dtype[0], d->w[0], d->inter, d->hidden, x, T, g, mm, mm_bytes, stream))) return rc;
    if ((rc = cw_qmatmul(d->dtype[1], d->w[1], d->inter, d->hidden, x, T, u, mm, mm_bytes, stream))) return rc;
    if ((rc = cw_swiglu(g, u, g, (int64_t)T * d->inter, stream))) return rc;
    if ((rc = cw_qmatmul(d->dtype[2], d->w[2], d->hidden, d->inter, g, T, y, mm, mm_bytes, stream))) return rc;
    if (glog && (rc = router_logits(CW_F32, d->gate_inp, 1, d->hidden, nullptr, x, T, glog, s))) return rc;
    hipLaunchKernelGGL(k_gate_scale_add, flat_grid((int64_t)T * d->hidden), dim3(256), 0, s, y, glog, T, d->hidden, accumulate,
                       out);
    return check_launch("k_gate_scale_add");
}

size_t cw_matmul_id_grouped_workspace_size(int dtype, int64_t n, int64_t k, int64_t n_slots, int64_t slot_stride,
                                           int x_rows_per_expert, int K, int T) {
    if (grouped_check(dtype, n, k, n_slots, slot_stride, K, T) != CW_OK) return 0;
    return grouped_layout(dtype, k, n_slots, x_rows_per_expert ? 1 : 0, K, T).total;
}

int cw_matmul_id_grouped(int dtype, int64_t n, int64_t k, int64_t n_slots, int64_t slot_stride, const void *bank,
                         const float *x, int x_rows_per_expert, const uint32_t *ids, int K, int T, float *out, void *ws,
                         size_t ws_bytes, cw_stream_t stream) {
    int rc = grouped_check(dtype, n, k, n_slots, slot_stride, K, T);
    if (rc) return rc;
    if (T == 0) return CW_OK;
    CW_REQUIRE(bank && x && ids && out, "matmul_id_grouped: null pointer");
    // the activation packs read 16 bytes at a time from any 4-byte aligned row start (gfx950 runs
    // with unaligned memory access enabled), as the reference takes any offset of x
    CW_REQUIRE(((uintptr_t)x & 3u) == 0, "matmul_id_grouped: x is not 4-byte aligned");
    if (k % 4 != 0) return set_error(CW_ENOTSUP, "matmul_id_grouped: rows of %lld are not whole float4s", (long long)k);
    const int xpp = x_rows_per_expert ? 1 : 0;
    const GroupedLayout L = grouped_layout(dtype, k, n_slots, xpp, K, T);
    CW_REQUIRE(ws && ws_bytes >= L.total, "matmul_id_grouped: workspace of %zu bytes, %zu needed", ws_bytes, L.total);
    hipStream_t s = (hipStream_t)stream;
    uint8_t *base = (uint8_t *)ws;
    const int TK = T * K;
    int *pile_pick = (int *)(base + L.pile_pick), *pile_tok = (int *)(base + L.pile_tok), *n_tiles = (int *)(base + L.n_tiles);
    MfTile *tiles = (MfTile *)(base + L.tiles);
    uint16_t *x16 = (uint16_t *)(base + L.x16);
    float *xscale = (float *)(base + L.xscale);
    if ((rc = mfma_piles(ids, nullptr, TK, K, (int)n_slots, pile_pick, pile_tok, tiles, n_tiles, s))) return rc;
    const bool gx = mxfp4_scaled_for(dtype, k);
    if (gx) rc = pack_rows_fp6(x, xpp ? TK : T, (int)k, (int)k, (uint8_t *)x16, s);
    else rc = pack_rows_f16(x, xpp ? TK : T, (int)k, (int)k, x16, xscale, s, nullptr, mfma_k_permuted(dtype));
    if (rc) return rc;
    MfArgs a = {};
    a.w0 = (const uint8_t *)bank;
    a.s0 = slot_stride;
    a.row_bytes = k / cw_block_size(dtype) * cw_type_size(dtype);
    a.n = (int)n;
    a.k = (int)k;
    a.a16 = x16;
    a.ascale = xscale;
    a.lda = (int)k;
    a.rows = xpp ? pile_pick : pile_tok;  // the activation row of each pile position
    a.tiles = tiles;
    a.n_tiles = n_tiles;
    a.pile_pick = pile_pick;
    a.K = K;
    a.dn = out;
    a.layout = dtype == CW_MXFP4_R16;
    if (gx) {
        a.ap = (const uint8_t *)x16;
        a.ap_row = (int64_t)fp6_rows_bytes(1, k);
        a.ap_rows = xpp ? TK : T;
        rc = mxfp4_down(a, max_tiles(TK, (int)n_slots), s);
    } else {
        rc = mfma_down(dtype, a, max_tiles(TK, (int)n_slots), s);
    }
    if (rc) return rc;
    hipLaunchKernelGGL(k_nan_rows, flat_grid(TK), dim3(256), 0, s, ids, TK, (uint32_t)n_slots, (int)n, out);
    return check_launch("k_nan_rows");
}

int64_t cw_rows16_bytes(int64_t n, int64_t k) {
    return n > 0 && k > 0 && k % 32 == 0 ? matrix_bytes(CW_MXFP4_R16, n, k / 32 * 17) : 0;
}

int cw_repack_rows16(const void *src, int64_t src_stride, void *dst, int64_t dst_stride, int64_t n_mats, int64_t n,
                     int64_t k, cw_stream_t stream) {
    CW_REQUIRE(n > 0 && n < (1ll << 31) && n_mats >= 0, "repack_rows16: n %lld, %lld matrices", (long long)n, (long long)n_mats);
    CW_REQUIRE(k > 128 && k % 32 == 0 && k <= 8192, "repack_rows16: k %lld (a multiple of 32, 160..8192)", (long long)k);
    const int64_t rb = k / 32 * 17;
    CW_REQUIRE(src_stride >= n * rb && dst_stride >= cw_rows16_bytes(n, k), "repack_rows16: strides %lld, %lld too small",
               (long long)src_stride, (long long)dst_stride);
    CW_REQUIRE(n_mats == 0 || (src && dst), "repack_rows16: null pointer");
    CW_REQUIRE((((uintptr_t)dst | (uintptr_t)dst_stride) & 15) == 0, "repack_rows16: dst and its stride must be 16-byte aligned");
    const uint8_t *s8 = (const uint8_t *)src;
    uint8_t *d8 = (uint8_t *)dst;
    CW_REQUIRE(n_mats == 0 || s8 + (n_mats - 1) * src_stride + n * rb <= d8 || d8 + (n_mats - 1) * dst_stride + cw_rows16_bytes(n, k) <= s8,
               "repack_rows16: source and destination overlap");
    return rows16_repack(s8, src_stride, d8, dst_stride, n_mats, (int)n, (int)k, (hipStream_t)stream);
}

int cw_route_topk(const float *logits, int T, int E, int K, int norm, uint32_t *ids, float *w, cw_stream_t stream) {
    CW_REQUIRE(T >= 0, "route: negative token count %d", T);
    CW_REQUIRE(E > 0 && E <= 1024, "route: %d experts (1..1024 supported)", E);
    CW_REQUIRE(K > 0 && K <= 32 && K <= E, "route: top-%d of %d experts", K, E);
    CW_REQUIRE(T == 0 || (logits && ids && w), "route: null pointer");
    return route(logits, T, E, K, norm, ids, w, (hipStream_t)stream);
}

int cw_router_logits(int wdtype, const void *w, int n_experts, int hidden, const float *bias, const float *x, int T,
                     float *logits, cw_stream_t stream) {
    CW_REQUIRE(T >= 0 && n_experts >= 0 && hidden > 0, "router: T %d, %d experts, hidden %d", T, n_experts, hidden);
    CW_REQUIRE(T == 0 || n_experts == 0 || (w && x && logits), "router: null pointer");
    CW_REQUIRE(((uintptr_t)x & 15u) == 0 && ((uintptr_t)w & 7u) == 0, "router: x must be 16-byte and w 8-byte aligned");
    CW_REQUIRE(wdtype != CW_F32 || ((uintptr_t)w & 15u) == 0, "router: f32 weights must be 16-byte aligned");
    return router_logits(wdtype, w, n_experts, hidden, bias, x, T, logits, (hipStream_t)stream);
}

int cw_swiglu(const float *g, const float *u, float *h, int64_t n, cw_stream_t stream) {
    CW_REQUIRE(n >= 0, "swiglu: negative size");
    if (n == 0) return CW_OK;
    CW_REQUIRE(g && u && h, "swiglu: null pointer");
    hipLaunchKernelGGL(k_swiglu, flat_grid(n), dim3(256), 0, (hipStream_t)stream, g, u, h, n);
    return check_launch("k_swiglu");
}

int cw_clamped_swiglu(const float *g, const float *u, const float *gate_b, const float *up_b, const uint32_t *ids,
                      int64_t rows, int width, int pad, float alpha, float limit, float *h, cw_stream_t stream) {
    CW_REQUIRE(rows >= 0 && width > 0, "clamped_swiglu: %lld rows of %d", (long long)rows, width);
    CW_REQUIRE(pad == 0 || pad >= width, "clamped_swiglu: pad %d below width %d", pad, width);
    if (rows == 0) return CW_OK;
    CW_REQUIRE(g && u && h, "clamped_swiglu: null pointer");
    CW_REQUIRE(ids || (!gate_b && !up_b), "clamped_swiglu: biases need ids");
    const int out_w = pad > width ? pad : width;
    hipLaunchKernelGGL(k_clamped_swiglu, flat_grid(rows * out_w), dim3(256), 0, (hipStream_t)stream, g, u, gate_b, up_b, ids,
                       rows, width, out_w, alpha, limit, h, 0);
    return check_launch("k_clamped_swiglu");
}

int cw_weighted_sum(const float *down, const float *w, const float *down_b, const uint32_t *ids, int T, int K, int H,
                    float *out, cw_stream_t stream) {
    CW_REQUIRE(T >= 0 && K > 0 && H > 0, "weighted_sum: T %d, K %d, H %d", T, K, H);
    CW_REQUIRE(!down_b || ids, "weighted_sum: a down bias needs ids");
    if (T == 0) return CW_OK;
    CW_REQUIRE(down && w && out, "weighted_sum: null pointer");
    hipLaunchKernelGGL(k_weighted_sum, flat_grid((int64_t)T * H), dim3(256), 0, (hipStream_t)stream, down, w, down_b, ids, T,
                       K, H, out);
    return check_launch("k_weighted_sum");
}

int cw_slots_resolve(const uint32_t *ids, const uint32_t *table, int n, uint32_t *slots, uint32_t *missing,
                     cw_stream_t stream) {
    CW_REQUIRE(n >= 0, "resolve: negative count");
    if (n == 0) return CW_OK;
    CW_REQUIRE(ids && table && slots, "resolve: null pointer");
    hipLaunchKernelGGL(k_resolve, flat_grid(n), dim3(256), 0, (hipStream_t)stream, ids, table, n, slots, missing);
    return check_launch("k_resolve");
}

uint32_t cw_device_errors(void) {
    (void)hipDeviceSynchronize();
    return decode_barrier_errors();
}

int cw_moe_layer_noalloc(const cw_moe_desc *desc, const float *x, const float *logits, int T, float *out, uint32_t *ids_out,
                         float *w_out, uint32_t *missing, cw_stream_t stream) {
    int rc = check_desc(desc, T);
    if (rc) return rc;
    if (T == 0) return CW_OK;
    const size_t need = layout(desc, T).total;
    if (need > NOALLOC_SCRATCH_BYTES)
        return set_error(CW_EINVAL, "moe noalloc: %d tokens need %zu bytes of scratch, above the %zu the library holds", T, need,
                         NOALLOC_SCRATCH_BYTES);
    void *ws = nullptr;
    if ((rc = noalloc_scratch(&ws))) return rc;
    return moe_layer(desc, x, logits, T, out, ids_out, w_out, missing, ws, NOALLOC_SCRATCH_BYTES, (hipStream_t)stream);
}

size_t cw_moe_workspace_size(const cw_moe_desc *desc, int T) {
    if (check_desc(desc, T)) return 0;
    return layout(desc, T).total;
}

int cw_moe_layer(const cw_moe_desc *desc, const float *x, const float *logits, int T, float *out, uint32_t *ids_out,
                 float *w_out, uint32_t *missing, void *ws, size_t ws_bytes, cw_stream_t stream) {
    return moe_layer(desc, x, logits, T, out, ids_out, w_out, missing, ws, ws_bytes, (hipStream_t)stream);
}

}  // extern "C"
