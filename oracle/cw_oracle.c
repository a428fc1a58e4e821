/* TEST INFRASTRUCTURE ONLY: the CPU oracle (see cw_oracle.h). Plain C11, no SIMD, so the
 * arithmetic order is the one written here. Reference citations are file:line relative to the
 * reference checkout root. */
#include "cw_oracle.h"
#include "../coachwhip_amd/csrc/cw_grids.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK_K 256

int or_block_size(int dtype) {
    switch (dtype) {
    case OR_F32: case OR_F16: return 1;
    case OR_Q8_0: case OR_MXFP4: return 32;
    case OR_Q2_K: case OR_Q3_K: case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: case OR_Q8_K: case OR_IQ2_XXS:
    case OR_IQ2_S: case OR_IQ3_XXS: case OR_IQ3_S: case OR_IQ4_XS: return QK_K;
    default: return 0;
    }
}

int or_type_size(int dtype) {
    /* struct sizes: k_quants.rs:125-130 (Q8_0 34), 142-148 (Q2_K 84), 152-158 (Q3_K 110),
     * 163-170 (Q4_K 144), 173-181 (Q5_K 176), 185-191 (Q6_K 210), 195-200 (Q8_K 292), 631-635
     * (MXFP4 17), 2959-2968 (IQ2_XXS 66, IQ3_XXS 98, IQ4_XS 136); quantized.metal:217-257 (IQ2_S 82,
     * IQ3_S 110). */
    switch (dtype) {
    case OR_Q2_K: return 84;
    case OR_Q3_K: return 110;
    case OR_Q5_K: return 176;
    case OR_Q6_K: return 210;
    case OR_IQ3_XXS: return 98;
    case OR_IQ4_XS: return 136;
    case OR_F32: return 4;
    case OR_F16: return 2;
    case OR_Q8_0: return 34;
    case OR_Q4_K: return 144;
    case OR_Q8_K: return 292;
    case OR_IQ2_XXS: return 66;
    case OR_IQ2_S: return 82;
    case OR_IQ3_S: return 110;
    case OR_MXFP4: return 17;
    default: return 0;
    }
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in f32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return u2f(f2u(v) | sign);
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112) << 23) | (m << 13));
}

uint16_t or_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t e = (x >> 23) & 0xff, m = x & 0x7fffff;
    if (e == 0xff) return (uint16_t)(sign | 0x7c00u | (m ? (0x200u | (m >> 13)) : 0));
    int32_t he = (int32_t)e - 112;
    if (he >= 31) return (uint16_t)(sign | 0x7c00u);
    if (he <= 0) {
        if (e == 0) return sign; /* f32 zero / subnormal is far below f16's range */
        uint32_t M = m | 0x800000u;
        int shift = 14 - he;
        if (shift > 24) return sign;
        uint32_t hm = M >> shift, rem = M & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = m >> 13, rem = m & 0x1fff;
    uint32_t r = ((uint32_t)he << 10) + hm;
    if (rem > 0x1000 || (rem == 0x1000 && (hm & 1))) r++;
    return (uint16_t)(sign | r);
}

float or_e8m0_half(uint8_t e) {
    /* k_quants.rs:642-649: 2^(e-128), e < 2 are f32 subnormals */
    uint32_t bits = e < 2 ? (0x00200000u << e) : ((uint32_t)(e - 1) << 23);
    return u2f(bits);
}

/* doubled E2M1 values, k_quants.rs:639 */
static const int8_t KV_MXFP4[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

/* ksigns_iq2xs[i] (quantized.metal:305): the 7 sign bits i plus an 8th bit that makes the
 * number of set bits even. */
static uint8_t ksign(uint32_t i) {
    uint32_t p = i ^ (i >> 4); p ^= p >> 2; p ^= p >> 1;
    return (uint8_t)(i | ((p & 1) << 7));
}

/* vendor/candle-core/src/quantized/utils.rs:50-60 */
static void scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* k_quants.rs:766-782 */
static void deq_q8_0(const uint8_t *b, float *y) {
    float d = or_f16_to_f32(rd16(b));
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)b[2 + j] * d;
}

/* k_quants.rs:1821-1849 */
static void deq_q4_k(const uint8_t *b, float *y) {
    float d = or_f16_to_f32(rd16(b)), mn = or_f16_to_f32(rd16(b + 2));
    const uint8_t *sc = b + 4, *q = b + 16;
    int is = 0;
    for (int j = 0; j < QK_K; j += 64) {
        uint8_t s, m;
        scale_min_k4(is, sc, &s, &m);
        float d1 = d * (float)s, m1 = mn * (float)m;
        scale_min_k4(is + 1, sc, &s, &m);
        float d2 = d * (float)s, m2 = mn * (float)m;
        const uint8_t *qq = q + j / 2;
        for (int l = 0; l < 32; l++) y[j + l] = d1 * (float)(qq[l] & 0xF) - m1;
        for (int l = 0; l < 32; l++) y[j + 32 + l] = d2 * (float)(qq[l] >> 4) - m2;
        is += 2;
    }
}

/* Q2_K {scales[16], qs[64], d, dmin}: k_quants.rs:1152-1190 */
static void deq_q2_k(const uint8_t *b, float *y) {
    const uint8_t *sc = b, *qs = b + 16;
    float d = or_f16_to_f32(rd16(b + 80)), mn = or_f16_to_f32(rd16(b + 82));
    int is = 0;
    for (int half = 0; half < 2; half++) {
        const uint8_t *q = qs + 32 * half;
        float *yb = y + 128 * half;
        int yi = 0;
        for (int shift = 0; shift < 8; shift += 2) {
            for (int part = 0; part < 2; part++) {
                uint8_t s = sc[is++];
                float dl = d * (float)(s & 0xF), ml = mn * (float)(s >> 4);
                for (int i = 0; i < 16; i++) yb[yi++] = dl * (float)((q[16 * part + i] >> shift) & 3) - ml;
            }
        }
    }
}

/* Q3_K {hmask[32], qs[64], scales[12], d}: k_quants.rs:1514-1571 */
static void deq_q3_k(const uint8_t *b, float *y) {
    const uint8_t *hm = b, *qs = b + 32, *sr = b + 96;
    float d_all = or_f16_to_f32(rd16(b + 108));
    uint32_t aux[4];
    memcpy(aux, sr, 12);
    uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & 0x0f0f0f0fu) | (((tmp >> 4) & 0x03030303u) << 4);
    aux[3] = ((aux[1] >> 4) & 0x0f0f0f0fu) | (((tmp >> 6) & 0x03030303u) << 4);
    aux[0] = (aux[0] & 0x0f0f0f0fu) | ((tmp & 0x03030303u) << 4);
    aux[1] = (aux[1] & 0x0f0f0f0fu) | (((tmp >> 2) & 0x03030303u) << 4);
    int8_t scales[16];
    memcpy(scales, aux, 16);
    int is = 0;
    uint8_t m = 1;
    for (int half = 0; half < 2; half++) {
        const uint8_t *q = qs + 32 * half;
        for (int shift = 0; shift < 8; shift += 2) {
            for (int part = 0; part < 2; part++) {
                float dl = d_all * ((float)scales[is] - 32.0f);
                for (int i = 0; i < 16; i++) {
                    int v = (int)((q[i + 16 * part] >> shift) & 3) - ((hm[i + 16 * part] & m) ? 0 : 4);
                    *y++ = dl * (float)v;
                }
                is++;
            }
            m <<= 1;
        }
    }
}

/* Q5_K {d, dmin, scales[12], qh[32], qs[128]}: k_quants.rs:2120-2152 */
static void deq_q5_k(const uint8_t *b, float *y) {
    float d = or_f16_to_f32(rd16(b)), mn = or_f16_to_f32(rd16(b + 2));
    const uint8_t *sc = b + 4, *qh = b + 16, *ql = b + 48;
    int is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0; j < QK_K; j += 64) {
        uint8_t s, m;
        scale_min_k4(is, sc, &s, &m);
        float d1 = d * (float)s, m1 = mn * (float)m;
        scale_min_k4(is + 1, sc, &s, &m);
        float d2 = d * (float)s, m2 = mn * (float)m;
        const uint8_t *q = ql + j / 2;
        for (int l = 0; l < 32; l++) y[j + l] = d1 * ((float)(q[l] & 0xF) + ((qh[l] & u1) ? 16.0f : 0.0f)) - m1;
        for (int l = 0; l < 32; l++) y[j + 32 + l] = d2 * ((float)(q[l] >> 4) + ((qh[l] & u2) ? 16.0f : 0.0f)) - m2;
        is += 2;
        u1 <<= 2;
        u2 <<= 2;
    }
}

/* k_quants.rs:673-691 */
static void deq_mxfp4(const uint8_t *b, float *y) {
    float d = or_e8m0_half(b[0]);
    for (int j = 0; j < 16; j++) {
        y[j] = (float)KV_MXFP4[b[1 + j] & 0xF] * d;
        y[j + 16] = (float)KV_MXFP4[b[1 + j] >> 4] * d;
    }
}

/* dequantize_iq2_xxs, quantized.metal:6820-6843 (the reference has no CPU path). */
static void deq_iq2_xxs(const uint8_t *b, float *y) {
    float d = or_f16_to_f32(rd16(b));
    for (int ib = 0; ib < 8; ib++) {
        const uint8_t *q = b + 2 + 8 * ib;
        uint32_t g = (uint32_t)rd16(q) | ((uint32_t)rd16(q + 2) << 16);
        uint32_t s = (uint32_t)rd16(q + 4) | ((uint32_t)rd16(q + 6) << 16);
        float dl = d * (0.5f + (float)(s >> 28)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            uint64_t grid = cw_iq2xxs_grid[(g >> (8 * l)) & 0xFF];
            uint8_t signs = ksign((s >> (7 * l)) & 127);
            for (int i = 0; i < 8; i++) {
                float gv = (float)((grid >> (8 * i)) & 0xFF);
                y[32 * ib + 8 * l + i] = dl * gv * ((signs >> i) & 1 ? -1.f : 1.f);
            }
        }
    }
}

/* dequantize_iq2_s, quantized.metal:6918-6935 (GGUF type 22; not a reference dtype). */
static void deq_iq2_s(const uint8_t *b, float *y) {
    float d = or_f16_to_f32(rd16(b));
    const uint8_t *qs = b + 2, *signs = b + 2 + 32, *qh = b + 66, *scales = b + 74;
    for (int ib = 0; ib < 8; ib++) {
        for (int t = 0; t < 4; t++) {
            int il = t / 2;
            float dl = d * (0.5f + (float)((scales[ib] >> (4 * il)) & 0xF)) * 0.25f;
            uint32_t idx = qs[4 * ib + t] | ((((uint32_t)qh[ib] >> (2 * t)) & 3) << 8);
            uint64_t grid = cw_iq2s_grid[idx];
            uint8_t sg = signs[4 * ib + t];
            for (int i = 0; i < 8; i++) {
                float gv = (float)((grid >> (8 * i)) & 0xFF);
                y[32 * ib + 8 * t + i] = dl * gv * ((sg >> i) & 1 ? -1.f : 1.f);
            }
        }
    }
}

/* dequantize_iq3_s, quantized.metal:6893-6916 (GGUF type 21; not a reference dtype). */
static void deq_iq3_s(const uint8_t *b, float *y) {
    float d = or_f16_to_f32(rd16(b));
    const uint8_t *qs = b + 2, *qh = b + 66, *signs = b + 74, *scales = b + 106;
    for (int ib = 0; ib < 8; ib++) {
        float dl = d * (float)(1 + 2 * ((scales[ib / 2] >> (4 * (ib % 2))) & 0xF));
        for (int g = 0; g < 8; g++) {
            uint32_t idx = qs[8 * ib + g] | ((((uint32_t)qh[ib] >> g) & 1) << 8);
            uint32_t grid = cw_iq3s_grid[idx];
            for (int i = 0; i < 4; i++) {
                int v = 4 * g + i;
                float gv = (float)((grid >> (8 * i)) & 0xFF);
                int neg = (signs[4 * ib + v / 8] >> (v % 8)) & 1;
                y[32 * ib + v] = dl * gv * (neg ? -1.f : 1.f);
            }
        }
    }
}

/* Q6_K {ql[128], qh[64], scales[16] (i8), d}: k_quants.rs:2420-2451, y = (d * sc) * (q - 32) */
static void deq_q6_k(const uint8_t *b, float *y) {
    float d = or_f16_to_f32(rd16(b + 208));
    for (int h = 0; h < 2; h++) {
        const uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h;
        const int8_t *sc = (const int8_t *)(b + 192 + 8 * h);
        float *yy = y + 128 * h;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            yy[l] = d * (float)sc[is] * (float)q1;
            yy[l + 32] = d * (float)sc[is + 2] * (float)q2;
            yy[l + 64] = d * (float)sc[is + 4] * (float)q3;
            yy[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
    }
}

/* dequantize_iq3_xxs, quantized.metal:6866-6891 (GGUF type 18; the reference has no CPU path).
 * Sub-block ib: 8 grid indices qs[8ib..8ib+8) of 4 values each, and the little-endian word at
 * qs[64 + 4ib]: four 7-bit sign indices and the 4-bit scale s on top; dl = d * (s + 0.5) * 0.5.
 * Weights 8h'..8h'+7 (h' = 0..3) take sign index h' and grid indices 2h', 2h'+1. */
static void deq_iq3_xxs(const uint8_t *b, float *y) {
    float d = or_f16_to_f32(rd16(b));
    for (int ib = 0; ib < 8; ib++) {
        const uint8_t *q3 = b + 2 + 8 * ib, *gs = b + 2 + 64 + 4 * ib;
        uint32_t aux = (uint32_t)gs[0] | ((uint32_t)gs[1] << 8) | ((uint32_t)gs[2] << 16) | ((uint32_t)gs[3] << 24);
        float dl = d * (0.5f + (float)(aux >> 28)) * 0.5f;
        for (int h = 0; h < 4; h++) {
            uint8_t signs = ksign((aux >> (7 * h)) & 127);
            for (int t = 0; t < 2; t++) {
                uint32_t grid = cw_iq3xxs_grid[q3[2 * h + t]];
                for (int i = 0; i < 4; i++) {
                    float gv = (float)((grid >> (8 * i)) & 0xFF);
                    y[32 * ib + 8 * h + 4 * t + i] = dl * gv * ((signs >> (4 * t + i)) & 1 ? -1.f : 1.f);
                }
            }
        }
    }
}

/* kvalues_iq4nl_f, quantized.metal:4561-4563: the 16 non-linear IQ4 levels (format data) */
static const float KV_IQ4NL[16] = {-127.f, -104.f, -83.f, -65.f, -49.f, -35.f, -22.f, -10.f,
                                   1.f, 13.f, 25.f, 38.f, 53.f, 69.f, 89.f, 113.f};

/* dequantize_iq4_xs, quantized.metal:7000-7016 (GGUF type 23): {d, scales_h (u16), scales_l[4],
 * qs[128]}; sub-block ib has the 6-bit scale ls = scales_l nibble | 2 bits of scales_h << 4,
 * d_ib = d * (ls - 32), and its 32 weights are the low then the high nibbles of qs[16ib..16ib+16). */
static void deq_iq4_xs(const uint8_t *b, float *y) {
    float d0 = or_f16_to_f32(rd16(b));
    uint32_t sh = rd16(b + 2);
    const uint8_t *sl = b + 4, *qs = b + 8;
    for (int ib = 0; ib < 8; ib++) {
        int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 0xF) | (int)(((sh >> (2 * ib)) & 3) << 4);
        float d = d0 * (float)(ls - 32);
        for (int j = 0; j < 16; j++) {
            y[32 * ib + j] = d * KV_IQ4NL[qs[16 * ib + j] & 0xF];
            y[32 * ib + 16 + j] = d * KV_IQ4NL[qs[16 * ib + j] >> 4];
        }
    }
}

int or_dequantize(int dtype, const void *blocks, int64_t n, float *out) {
    int bs = or_block_size(dtype), ts = or_type_size(dtype);
    if (bs == 0 || n < 0 || n % bs) return -1;
    const uint8_t *p = (const uint8_t *)blocks;
    for (int64_t i = 0; i < n / bs; i++) {
        const uint8_t *b = p + i * ts;
        float *y = out + i * bs;
        switch (dtype) {
        case OR_F32: memcpy(y, b, 4); break;
        case OR_F16: *y = or_f16_to_f32(rd16(b)); break;
        case OR_Q8_0: deq_q8_0(b, y); break;
        case OR_Q2_K: deq_q2_k(b, y); break;
        case OR_Q3_K: deq_q3_k(b, y); break;
        case OR_Q4_K: deq_q4_k(b, y); break;
        case OR_Q5_K: deq_q5_k(b, y); break;
        case OR_Q6_K: deq_q6_k(b, y); break;
        case OR_IQ3_XXS: deq_iq3_xxs(b, y); break;
        case OR_IQ4_XS: deq_iq4_xs(b, y); break;
        case OR_MXFP4: deq_mxfp4(b, y); break;
        case OR_IQ2_XXS: deq_iq2_xxs(b, y); break;
        case OR_IQ2_S: deq_iq2_s(b, y); break;
        case OR_IQ3_S: deq_iq3_s(b, y); break;
        default: return -1;
        }
    }
    return 0;
}

/* ---- the GPU shrink to Q2_K, crates/engine/src/requant.rs:113-304 ---- */

static float min_sel(float a, float b) { return b < a ? b : a; }
static float max_sel(float a, float b) { return b > a ? b : a; }
/* clamp((int)v, 0, 3) and min(15, (int)v) with the shader's saturating float -> int conversion
 * (the same as the C cast wherever that is defined; NaN gives 0) */
static int level3(float v) { return v >= 3.f ? 3 : v >= 2.f ? 2 : v >= 1.f ? 1 : 0; }
static int level15(float v) { return v >= 15.f ? 15 : v >= 1.f ? (int)v : 0; }

/* fit16, requant.rs:119-138 */
static void fit16(const float *x, const float *w, float *scale, float *mn) {
    for (int round = 0; round < 2; ++round) {
        float sw = 0.f, swl = 0.f, swll = 0.f, swx = 0.f, swlx = 0.f;
        for (int i = 0; i < 16; ++i) {
            int l = 0;
            if (*scale > 0.f) l = level3((x[i] + *mn) / *scale + 0.5f);
            const float wi = w[i], fl = (float)l;
            sw += wi;
            swl += wi * fl;
            swll += wi * fl * fl;
            swx += wi * x[i];
            swlx += wi * fl * x[i];
        }
        const float det = sw * swll - swl * swl;
        if (det > 1e-12f) {
            const float a = (sw * swlx - swl * swx) / det;
            const float b = (swl * swlx - swll * swx) / det;
            if (a > 0.f && b >= 0.f) {
                *scale = a;
                *mn = b;
            }
        }
    }
}

/* q2k_encode / q2k_encode_w, requant.rs:141-232 (w == NULL: every weight 1) */
static void q2k_encode(const float *x, const float *w, uint8_t *y) {
    float scales[16], mins[16], max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 16; ++j) {
        float lo = x[16 * j], hi = x[16 * j];
        for (int i = 1; i < 16; ++i) {
            lo = min_sel(lo, x[16 * j + i]);
            hi = max_sel(hi, x[16 * j + i]);
        }
        if (lo > 0.f) lo = 0.f;
        float sc = (hi - lo) / 3.f, mn = -lo, wl[16];
        for (int i = 0; i < 16; ++i) wl[i] = w ? sqrtf(max_sel(w[16 * j + i], 0.f)) + 1e-6f : 1.f;
        fit16(x + 16 * j, wl, &sc, &mn);
        scales[j] = sc;
        mins[j] = mn;
        max_scale = max_sel(max_scale, sc);
        max_min = max_sel(max_min, mn);
    }
    const float inv_scale = max_scale > 0.f ? 15.f / max_scale : 0.f;
    const float inv_min = max_min > 0.f ? 15.f / max_min : 0.f;
    uint8_t ls[16], lm[16];
    for (int j = 0; j < 16; ++j) {
        ls[j] = (uint8_t)level15(scales[j] * inv_scale + 0.5f);
        lm[j] = (uint8_t)level15(mins[j] * inv_min + 0.5f);
        y[j] = (uint8_t)(ls[j] | (lm[j] << 4));
    }
    const uint16_t dh = or_f32_to_f16(max_scale / 15.f), mh = or_f32_to_f16(max_min / 15.f);
    y[80] = (uint8_t)dh; y[81] = (uint8_t)(dh >> 8);
    y[82] = (uint8_t)mh; y[83] = (uint8_t)(mh >> 8);
    const float d = or_f16_to_f32(dh), dmin = or_f16_to_f32(mh);
    uint8_t L[256];
    for (int j = 0; j < 16; ++j) {
        const float dj = d * (float)ls[j], mj = dmin * (float)lm[j];
        for (int i = 0; i < 16; ++i) {
            int l = 0;
            if (dj > 0.f) l = level3((x[16 * j + i] + mj) / dj + 0.5f);
            L[16 * j + i] = (uint8_t)l;
        }
    }
    for (int j = 0; j < QK_K; j += 128)
        for (int l = 0; l < 32; ++l)
            y[16 + j / 4 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
}

int or_requant_q2k(int src_dtype, const void *src, int64_t n_blocks, const float *shape,
                   int64_t blocks_per_row, void *dst) {
    if (src_dtype != OR_Q3_K && src_dtype != OR_Q4_K && src_dtype != OR_Q5_K) return -1;
    if (n_blocks < 0 || (shape && blocks_per_row <= 0)) return -1;
    const int ts = or_type_size(src_dtype);
    #pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < n_blocks; t++) {
        float x[QK_K];
        or_dequantize(src_dtype, (const uint8_t *)src + t * ts, QK_K, x);
        q2k_encode(x, shape ? shape + (t % blocks_per_row) * QK_K : NULL, (uint8_t *)dst + t * 84);
    }
    return 0;
}

static int64_t row_bytes(int dtype, int64_t k) {
    int bs = or_block_size(dtype);
    return bs ? k / bs * or_type_size(dtype) : 0;
}

int or_qmatmul_f64(int dtype, const void *w, int64_t n, int64_t k, const float *x, int64_t m,
                   double *y) {
    int bs = or_block_size(dtype);
    if (bs == 0 || k % bs) return -1;
    int64_t rb = row_bytes(dtype, k);
    int bad = 0;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; r++) {
        float *row = (float *)malloc(sizeof(float) * (size_t)k);
        if (!row || or_dequantize(dtype, (const uint8_t *)w + r * rb, k, row)) { bad = 1; free(row); continue; }
        for (int64_t t = 0; t < m; t++) {
            double acc = 0.0;
            const float *xr = x + t * k;
            for (int64_t c = 0; c < k; c++) acc += (double)row[c] * (double)xr[c];
            y[t * n + r] = acc;
        }
        free(row);
    }
    return bad ? -1 : 0;
}

void or_softmax(const float *logits, int T, int E, float *probs) {
    /* candle-nn softmax_last_dim CPU: running max (cpu/kernels.rs:62-67), exp of the
     * differences, sum (sequential here; candle's AVX vec_sum splits it into 8 lanes, so the
     * weights agree to about 1e-7 relative), divide. */
    for (int t = 0; t < T; t++) {
        const float *x = logits + (int64_t)t * E;
        float *p = probs + (int64_t)t * E;
        float mx = x[0];
        for (int e = 1; e < E; e++) mx = fmaxf(mx, x[e]);
        float s = 0.f;
        for (int e = 0; e < E; e++) { p[e] = expf(x[e] - mx); }
        for (int e = 0; e < E; e++) s += p[e];
        for (int e = 0; e < E; e++) p[e] /= s;
    }
}

void or_route(const float *logits, int T, int E, int K, int norm, uint32_t *ids, float *w) {
    float *p = (float *)malloc(sizeof(float) * (size_t)E);
    uint8_t *taken = (uint8_t *)malloc((size_t)E);
    for (int t = 0; t < T; t++) {
        or_softmax(logits + (int64_t)t * E, 1, E, p);
        memset(taken, 0, (size_t)E);
        /* stable descending sort (sort.rs:40-53) truncated to K: the k-th pick is the largest
         * probability not yet taken, lowest index first among equals. */
        for (int j = 0; j < K; j++) {
            int best = -1;
            for (int e = 0; e < E; e++) {
                if (taken[e]) continue;
                if (best < 0 || p[e] > p[best]) best = e;
            }
            taken[best] = 1;
            ids[(int64_t)t * K + j] = (uint32_t)best;
            w[(int64_t)t * K + j] = p[best];
        }
        if (norm) {
            /* broadcast_div by sum_keepdim (experts.rs:2369): sequential sum of the K picks */
            float s = 0.f;
            for (int j = 0; j < K; j++) s += w[(int64_t)t * K + j];
            for (int j = 0; j < K; j++) w[(int64_t)t * K + j] /= s;
        }
    }
    free(p);
    free(taken);
}

void or_rank(const float *scores, int n, uint32_t *ids) {
    /* experts.rs:676-680: stable sort by score descending, incomparable (NaN) as equal, then id */
    for (int i = 0; i < n; i++) ids[i] = (uint32_t)i;
    for (int i = 1; i < n; i++) {
        uint32_t v = ids[i];
        int j = i - 1;
        while (j >= 0) {
            float a = scores[ids[j]], b = scores[v];
            int before = (b > a) || (!(b < a) && !(b > a) && v < ids[j]);
            if (!before) break;
            ids[j + 1] = ids[j];
            j--;
        }
        ids[j + 1] = v;
    }
}

void or_silu_mul(const float *g, const float *u, float *h, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float v = g[i];
        h[i] = v / (1.0f + expf(-v)) * u[i];
    }
}

void or_clamped_swiglu(const float *g, const float *u, const float *gate_b, const float *up_b,
                       const uint32_t *ids, int64_t rows, int width, int pad, float alpha,
                       float limit, float *h) {
    int out_w = pad > width ? pad : width;
    for (int64_t r = 0; r < rows; r++) {
        uint32_t e = ids[r];
        for (int c = 0; c < width; c++) {
            float gv = g[r * width + c] + (gate_b ? gate_b[(int64_t)e * width + c] : 0.f);
            float uv = u[r * width + c] + (up_b ? up_b[(int64_t)e * width + c] : 0.f);
            gv = fminf(gv, limit);
            uv = fminf(fmaxf(uv, -limit), limit);
            float glu = gv * (1.0f / (1.0f + expf(-(gv * alpha))));
            h[r * out_w + c] = (uv + 1.0f) * glu;
        }
        for (int c = width; c < out_w; c++) h[r * out_w + c] = 0.f;
    }
}

void or_weighted_sum(const float *down, const float *w, int T, int K, int H, float *out) {
    for (int t = 0; t < T; t++)
        for (int j = 0; j < H; j++) {
            float acc = 0.f;
            for (int e = 0; e < K; e++) acc += down[((int64_t)t * K + e) * H + j] * w[(int64_t)t * K + e];
            out[(int64_t)t * H + j] = acc;
        }
}

void or_resolve(const uint32_t *ids, const uint32_t *table, int n, uint32_t *slots,
                uint32_t *missing) {
    for (int i = 0; i < n; i++) {
        uint32_t s = table[ids[i]];
        if (s == 0xFFFFFFFFu) { (*missing)++; s = 0; }
        slots[i] = s;
    }
}

int or_matvec_id(int dtype, int64_t n, int64_t k, int64_t n_slots, int64_t slot_stride,
                 const void *bank, const float *x, int rows_per_expert, const uint32_t *ids,
                 int K, int T, double *out) {
    int bs = or_block_size(dtype);
    if (bs == 0 || k % bs) return -1;
    int64_t rb = row_bytes(dtype, k);
    if (n * rb > slot_stride) return -1;
    for (int64_t i = 0; i < (int64_t)T * K; i++)
        if (ids[i] >= (uint64_t)n_slots) return -1;
    int bad = 0;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t i = 0; i < (int64_t)T * K; i++) {
        int64_t t = i / K;
        const float *xr = x + (rows_per_expert ? i : t) * k;
        const uint8_t *wm = (const uint8_t *)bank + (int64_t)ids[i] * slot_stride;
        float *row = (float *)malloc(sizeof(float) * (size_t)k);
        if (!row) { bad = 1; continue; }
        for (int64_t r = 0; r < n; r++) {
            or_dequantize(dtype, wm + r * rb, k, row);
            double acc = 0.0;
            for (int64_t c = 0; c < k; c++) acc += (double)row[c] * (double)xr[c];
            out[i * n + r] = acc;
        }
        free(row);
    }
    return bad ? -1 : 0;
}

static double sigmoid_d(double v) { return 1.0 / (1.0 + exp(-v)); }

int or_moe_layer(const or_moe_desc *d, const float *x, const float *logits, int T, double *out,
                 uint32_t *ids, float *w) {
    int E = d->n_experts, K = d->top_k, H = d->hidden, I = d->inter;
    int P = d->pad > I ? d->pad : I;
    if (E <= 0 || K <= 0 || K > E || H <= 0 || I <= 0 || T < 0) return -1;
    int n_slots = d->slot_table ? d->n_slots : E;
    for (int m = 0; m < 3; m++) {
        int bs = or_block_size(d->dtype[m]);
        int64_t kk = m == 2 ? P : H;
        if (bs == 0 || kk % bs) return -1;
    }
    or_route(logits, T, E, K, d->norm, ids, w);
    int missing = 0;
    int64_t TK = (int64_t)T * K;
    int32_t *slot = (int32_t *)malloc(sizeof(int32_t) * (size_t)(TK ? TK : 1));
    for (int64_t i = 0; i < TK; i++) {
        uint32_t s = d->slot_table ? d->slot_table[ids[i]] : ids[i];
        if (s == 0xFFFFFFFFu) { missing++; s = 0; }
        slot[i] = (int32_t)s;
    }
    for (int64_t i = 0; i < (int64_t)T * H; i++) out[i] = 0.0;
    /* group picks by slot, dequantize each used slot's three matrices once (experts.rs:2500-2537
     * groups tokens per expert the same way) */
    double *down = (double *)calloc((size_t)(TK ? TK : 1) * (size_t)H, sizeof(double));
    int bad = 0;
#pragma omp parallel for schedule(dynamic, 1)
    for (int s = 0; s < n_slots; s++) {
        int used = 0;
        for (int64_t i = 0; i < TK; i++) used |= slot[i] == s;
        if (!used) continue;
        float *wg = (float *)malloc(sizeof(float) * (size_t)I * H);
        float *wu = (float *)malloc(sizeof(float) * (size_t)I * H);
        float *wd = (float *)malloc(sizeof(float) * (size_t)H * P);
        double *hbuf = (double *)malloc(sizeof(double) * (size_t)P);
        if (!wg || !wu || !wd || !hbuf) { bad = 1; free(wg); free(wu); free(wd); free(hbuf); continue; }
        or_dequantize(d->dtype[0], (const uint8_t *)d->w[0] + (int64_t)s * d->slot_stride[0], (int64_t)I * H, wg);
        or_dequantize(d->dtype[1], (const uint8_t *)d->w[1] + (int64_t)s * d->slot_stride[1], (int64_t)I * H, wu);
        or_dequantize(d->dtype[2], (const uint8_t *)d->w[2] + (int64_t)s * d->slot_stride[2], (int64_t)H * P, wd);
        for (int64_t i = 0; i < TK; i++) {
            if (slot[i] != s) continue;
            int64_t t = i / K;
            uint32_t e = ids[i];
            const float *xr = x + t * H;
            for (int r = 0; r < I; r++) {
                double g = 0.0, u = 0.0;
                const float *gr = wg + (int64_t)r * H, *ur = wu + (int64_t)r * H;
                for (int c = 0; c < H; c++) { g += (double)gr[c] * xr[c]; u += (double)ur[c] * xr[c]; }
                if (d->act == 0) {
                    hbuf[r] = g * sigmoid_d(g) * u;
                } else {
                    if (d->bias[0]) g += d->bias[0][(int64_t)e * I + r];
                    if (d->bias[1]) u += d->bias[1][(int64_t)e * I + r];
                    if (g > d->limit) g = d->limit;
                    if (u > d->limit) u = d->limit;
                    if (u < -d->limit) u = -d->limit;
                    hbuf[r] = (u + 1.0) * g * sigmoid_d((double)d->alpha * g);
                }
            }
            for (int r = I; r < P; r++) hbuf[r] = 0.0;
            for (int r = 0; r < H; r++) {
                double acc = 0.0;
                const float *dr = wd + (int64_t)r * P;
                for (int c = 0; c < P; c++) acc += (double)dr[c] * hbuf[c];
                if (d->act == 1 && d->bias[2]) acc += d->bias[2][(int64_t)e * H + r];
                down[i * H + r] = acc;
            }
        }
        free(wg); free(wu); free(wd); free(hbuf);
    }
    /* weighted combine in pick order (fuse_kernel.rs:277-291) */
    for (int64_t t = 0; t < T; t++)
        for (int j = 0; j < K; j++) {
            double wj = (double)w[t * K + j];
            for (int r = 0; r < H; r++) out[t * H + r] += wj * down[(t * K + j) * H + r];
        }
    free(down);
    free(slot);
    return bad ? -1 : missing;
}

/* ---- threads ---- */

/* the OpenMP thread count of the parallel loops below (the CPU baseline sets it to the host's
 * physical cores, candle's default: vendor/candle-core/src/utils.rs:382-421) */
void or_set_threads(int n) { if (n > 0) omp_set_num_threads(n); }
int or_get_threads(void) { return omp_get_max_threads(); }

/* ---- candle's CPU quantized path (baseline numerics) ---- */

void or_quantize_q8_0(const float *x, int64_t n, void *blocks) {
    uint8_t *out = (uint8_t *)blocks;
    for (int64_t i = 0; i < n / 32; i++) {
        const float *xs = x + i * 32;
        uint8_t *b = out + i * 34;
        float amax = 0.f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xs[j]));
        float dd = amax / 127.f;
        float id = dd != 0.f ? 1.f / dd : 0.f;
        uint16_t h = or_f32_to_f16(dd);
        b[0] = (uint8_t)h; b[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; j++) b[2 + j] = (uint8_t)(int8_t)roundf(xs[j] * id);
    }
}

void or_quantize_q8_k(const float *x, int64_t n, void *blocks) {
    uint8_t *out = (uint8_t *)blocks;
    for (int64_t i = 0; i < n / QK_K; i++) {
        const float *xs = x + i * QK_K;
        uint8_t *b = out + i * 292;
        float mx = 0.f, amax = 0.f;
        for (int j = 0; j < QK_K; j++)
            if (amax < fabsf(xs[j])) { amax = fabsf(xs[j]); mx = xs[j]; }
        int8_t *qs = (int8_t *)(b + 4);
        int16_t bsums[16];
        float dd;
        if (amax == 0.f) {
            dd = 0.f;
            memset(qs, 0, QK_K);
            memset(bsums, 0, sizeof bsums);
        } else {
            float iscale = -127.f / mx;
            for (int j = 0; j < QK_K; j++) {
                float v = roundf(iscale * xs[j]);
                v = v < -128.f ? -128.f : (v > 127.f ? 127.f : v);
                qs[j] = (int8_t)v;
            }
            for (int j = 0; j < 16; j++) {
                int s = 0;
                for (int ii = 0; ii < 16; ii++) s += qs[j * 16 + ii];
                bsums[j] = (int16_t)s;
            }
            dd = 1.f / iscale;
        }
        memcpy(b, &dd, 4);
        memcpy(b + 260, bsums, sizeof bsums);
    }
}

static float dot_q8_0(int64_t k, const uint8_t *w, const uint8_t *q) {
    float sumf = 0.f;
    for (int64_t i = 0; i < k / 32; i++) {
        const uint8_t *a = w + i * 34, *b = q + i * 34;
        int32_t s = 0;
        for (int j = 0; j < 32; j++) s += (int32_t)(int8_t)a[2 + j] * (int32_t)(int8_t)b[2 + j];
        sumf += (float)s * or_f16_to_f32(rd16(a)) * or_f16_to_f32(rd16(b));
    }
    return sumf;
}

static float dot_mxfp4(int64_t k, const uint8_t *w, const uint8_t *q) {
    float sumf = 0.f;
    for (int64_t i = 0; i < k / 32; i++) {
        const uint8_t *a = w + i * 17, *b = q + i * 34;
        float dd = or_f16_to_f32(rd16(b)) * or_e8m0_half(a[0]);
        int32_t s1 = 0, s2 = 0;
        for (int j = 0; j < 16; j++) {
            s1 += (int32_t)(int8_t)b[2 + j] * KV_MXFP4[a[1 + j] & 0xF];
            s2 += (int32_t)(int8_t)b[2 + j + 16] * KV_MXFP4[a[1 + j] >> 4];
        }
        sumf += dd * (float)(s1 + s2);
    }
    return sumf;
}

static float dot_q4_k(int64_t k, const uint8_t *w, const uint8_t *q) {
    /* k_quants.rs:1612-1692 (vec_dot_unopt) */
    float sums[8] = {0};
    float sumf = 0.f;
    for (int64_t i = 0; i < k / QK_K; i++) {
        const uint8_t *x = w + i * 144, *y = q + i * 292;
        float yd;
        memcpy(&yd, y, 4);
        const int8_t *q8 = (const int8_t *)(y + 4);
        int16_t bsums[16];
        memcpy(bsums, y + 260, sizeof bsums);
        int8_t aux8[QK_K];
        const uint8_t *q4 = x + 16;
        for (int j = 0; j < QK_K / 64; j++) {
            for (int l = 0; l < 32; l++) aux8[64 * j + l] = (int8_t)(q4[32 * j + l] & 0xF);
            for (int l = 0; l < 32; l++) aux8[64 * j + 32 + l] = (int8_t)(q4[32 * j + l] >> 4);
        }
        uint8_t scales[8], mins[8];
        for (int j = 0; j < 8; j++) scale_min_k4(j, x + 4, &scales[j], &mins[j]);
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) sumi += bsums[j] * mins[j / 2];
        int32_t aux32[8] = {0};
        int idx = 0;
        for (int s = 0; s < 8; s++) {
            int32_t scale = scales[s];
            for (int r = 0; r < 4; r++) {
                for (int l = 0; l < 8; l++) aux32[l] += scale * (int32_t)((int16_t)q8[idx + l] * (int16_t)aux8[idx + l]);
                idx += 8;
            }
        }
        float dd = or_f16_to_f32(rd16(x)) * yd;
        for (int l = 0; l < 8; l++) sums[l] += dd * (float)aux32[l];
        float dmin = or_f16_to_f32(rd16(x + 2)) * yd;
        sumf -= dmin * (float)sumi;
    }
    float tot = 0.f;
    for (int l = 0; l < 8; l++) tot += sums[l];
    return sumf + tot;
}

float or_vec_dot(int dtype, int64_t k, const void *wrow, const void *xq) {
    switch (dtype) {
    case OR_Q8_0: return dot_q8_0(k, (const uint8_t *)wrow, (const uint8_t *)xq);
    case OR_MXFP4: return dot_mxfp4(k, (const uint8_t *)wrow, (const uint8_t *)xq);
    case OR_Q4_K: return dot_q4_k(k, (const uint8_t *)wrow, (const uint8_t *)xq);
    default: return NAN;
    }
}

int or_candle_matmul(int dtype, const void *w, int64_t n, int64_t k, const float *x, int64_t m,
                     float *y, int threads) {
    int vdt = dtype == OR_Q4_K ? OR_Q8_K : OR_Q8_0;
    if (dtype != OR_Q8_0 && dtype != OR_Q4_K && dtype != OR_MXFP4) return -1;
    int bs = or_block_size(dtype), vbs = or_block_size(vdt);
    if (k % bs || k % vbs) return -1;
    int64_t rb = row_bytes(dtype, k), qb = row_bytes(vdt, k);
    uint8_t *xq = (uint8_t *)malloc((size_t)(qb * m));
    if (!xq) return -1;
    for (int64_t t = 0; t < m; t++) {
        if (vdt == OR_Q8_K) or_quantize_q8_k(x + t * k, k, xq + t * qb);
        else or_quantize_q8_0(x + t * k, k, xq + t * qb);
    }
#ifdef _OPENMP
    int nt = threads > 0 ? threads : 0;
#pragma omp parallel for schedule(static) num_threads(nt > 0 ? nt : omp_get_max_threads())
#endif
    for (int64_t r = 0; r < n; r++)
        for (int64_t t = 0; t < m; t++)
            y[t * n + r] = or_vec_dot(dtype, k, (const uint8_t *)w + r * rb, xq + t * qb);
    free(xq);
    (void)threads;
    return 0;
}
