/* TEST INFRASTRUCTURE ONLY (the timed CPU baseline of the dense QMatMul configs).
 *
 * candle's x86 repacked quantized matmul, restated: vendor/candle-core/src/quantized/repack.rs:
 * 219-283 (try_matmul_f32, x86_64 arm) and repack_x86.rs. The weights of a Q4_K, Q6_K or Q8_0
 * matrix are repacked once into tiles of 16 output rows (candle caches them in a OnceLock); each
 * call quantizes the activation rows to Q8_K (quantize_lhs, repack_x86.rs:487-507) and runs
 * units of (16 output rows x up to 4 activation rows) over the threads. Inside a unit, one
 * 512-bit vpdpbusd multiplies 4 consecutive k-values of 16 rows (unsigned weight codes) by 4
 * broadcast activation codes (signed) into 16 exact i32 sums; per sub-block the sums are turned
 * into f32 and folded into the accumulators with the sub-block scale, and the Q4_K mins, the
 * Q6_K offset 32 and the Q8_0 offset 128 are taken out through the Q8_K bsums.
 *
 * Two implementations of the same unit arithmetic: AVX-512 VNNI intrinsics (what candle selects
 * on a host with avx512f + avx512vnni, repack_x86.rs:905-928) and plain C. The integer sums are
 * exact in both and the f32 operations are the same, in the same order, with the fused
 * multiply-adds written as fmaf, so both give the same bits. The 256-bit AVX-VNNI / AVX2 tiers
 * and the AMX tile path for Q4_K at M >= 32 (repack.rs:262-268) are not restated: on a host
 * without AVX-512 VNNI this file runs the plain-C unit, and on a host with AMX candle would be
 * faster than this restatement for Q4_K at M >= 32.
 *
 * The tile layout has to be the one vpdpbusd consumes (4 k-values of a row in one 32-bit lane,
 * the 16 rows of a tile side by side), so it matches repack_x86.rs:13-34 field for field.
 */
#include "cw_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#define QK_K 256
#define TN 16      /* output rows per tile (TILE_N) */
#define MAX_MT 4   /* activation rows per unit */
#define Q8K_BYTES 292

/* One super-block (256 k-values) of 16 rows. qs: [k8-group (32)][row (16)][4 bytes], byte j of
 * a group holds q[8g+j] in its low nibble and q[8g+j+4] in its high nibble. */
typedef struct {
    float sc[8][TN];
    float mn[8][TN];
    uint8_t qs[32 * TN * 4];
} tile_q4k;

/* One super-block of 16 rows, the 6-bit codes (0..63, value = code - 32) as bytes:
 * qs [k4-group (64)][row (16)][4 bytes]. */
typedef struct {
    float sc[16][TN];
    uint8_t qs[64 * TN * 4];
} tile_q6k;

/* One 32-value block of 16 rows, codes offset by +128: qs [k4-group (8)][row (16)][4 bytes]. */
typedef struct {
    uint16_t d[TN];
    uint8_t qs[8 * TN * 4];
} tile_q8_0;

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ggml's 6-bit scale/min unpack, repack_x86.rs:76-86 */
static void scale_min(int j, const uint8_t *s, uint8_t *sc, uint8_t *mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *mn = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

int or_x86_level(void) {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512vnni")) return 2;
    if (__builtin_cpu_supports("avxvnni") && __builtin_cpu_supports("avx2")) return 1;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return 0;
    return -1;
}

/* repack_x86.rs:43-60 */
int or_x86_select(int dtype, int64_t m, int64_t n, int64_t k) {
    int lv = or_x86_level();
    if (lv < 0 || k <= 0 || n % TN || k % QK_K) return 0;
    switch (dtype) {
    case OR_Q4_K: return 1;
    case OR_Q6_K: return m > 1;
    case OR_Q8_0: return lv != 0;
    default: return 0;
    }
}

int64_t or_x86_packed_bytes(int dtype, int64_t n, int64_t k) {
    if (n % TN || k % QK_K) return 0;
    int64_t tiles = (n / TN) * (k / QK_K);
    switch (dtype) {
    case OR_Q4_K: return tiles * (int64_t)sizeof(tile_q4k);
    case OR_Q6_K: return tiles * (int64_t)sizeof(tile_q6k);
    case OR_Q8_0: return tiles * 8 * (int64_t)sizeof(tile_q8_0);
    default: return 0;
    }
}

/* repack_x86.rs:88-208 (pack_q4k, pack_q6k, pack_q8_0) */
int or_x86_pack(int dtype, const void *w, int64_t n, int64_t k, void *packed) {
    if (!or_x86_packed_bytes(dtype, n, k)) return -1;
    const uint8_t *src = (const uint8_t *)w;
    int64_t kb = k / QK_K, nt = n / TN;
    for (int64_t t = 0; t < nt; t++) {
        for (int64_t b = 0; b < kb; b++) {
            for (int r = 0; r < TN; r++) {
                int64_t row = t * TN + r;
                if (dtype == OR_Q4_K) {
                    tile_q4k *tl = (tile_q4k *)packed + t * kb + b;
                    const uint8_t *blk = src + (row * kb + b) * 144;
                    float d = or_f16_to_f32(rd16(blk)), dmin = or_f16_to_f32(rd16(blk + 2));
                    for (int s = 0; s < 8; s++) {
                        uint8_t sc, mn;
                        scale_min(s, blk + 4, &sc, &mn);
                        tl->sc[s][r] = d * (float)sc;
                        tl->mn[s][r] = dmin * (float)mn;
                    }
                    uint8_t v[QK_K];
                    for (int c = 0; c < 4; c++)
                        for (int j = 0; j < 32; j++) {
                            uint8_t q = blk[16 + c * 32 + j];
                            v[c * 64 + j] = q & 0x0F;
                            v[c * 64 + 32 + j] = q >> 4;
                        }
                    for (int g = 0; g < 32; g++)
                        for (int j = 0; j < 4; j++)
                            tl->qs[(g * TN + r) * 4 + j] = (uint8_t)(v[g * 8 + j] | (v[g * 8 + j + 4] << 4));
                } else if (dtype == OR_Q6_K) {
                    tile_q6k *tl = (tile_q6k *)packed + t * kb + b;
                    const uint8_t *blk = src + (row * kb + b) * 210;
                    const uint8_t *ql = blk, *qh = blk + 128;
                    const int8_t *scales = (const int8_t *)(blk + 192);
                    float d = or_f16_to_f32(rd16(blk + 208));
                    for (int s = 0; s < 16; s++) tl->sc[s][r] = d * (float)scales[s];
                    uint8_t v[QK_K];
                    for (int h = 0; h < 2; h++) {
                        const uint8_t *l = ql + h * 64, *hh = qh + h * 32;
                        for (int j = 0; j < 32; j++) {
                            v[h * 128 + j] = (uint8_t)((l[j] & 0x0F) | ((hh[j] & 3) << 4));
                            v[h * 128 + j + 32] = (uint8_t)((l[j + 32] & 0x0F) | (((hh[j] >> 2) & 3) << 4));
                            v[h * 128 + j + 64] = (uint8_t)((l[j] >> 4) | (((hh[j] >> 4) & 3) << 4));
                            v[h * 128 + j + 96] = (uint8_t)((l[j + 32] >> 4) | (((hh[j] >> 6) & 3) << 4));
                        }
                    }
                    for (int g = 0; g < 64; g++)
                        for (int j = 0; j < 4; j++) tl->qs[(g * TN + r) * 4 + j] = v[g * 4 + j];
                } else {
                    for (int s = 0; s < 8; s++) {
                        tile_q8_0 *tl = (tile_q8_0 *)packed + (t * kb + b) * 8 + s;
                        const uint8_t *blk = src + (row * kb * 8 + b * 8 + s) * 34;
                        tl->d[r] = rd16(blk);
                        for (int g = 0; g < 8; g++)
                            for (int j = 0; j < 4; j++)
                                tl->qs[(g * TN + r) * 4 + j] = (uint8_t)((int)(int8_t)blk[2 + g * 4 + j] + 128);
                    }
                }
            }
        }
    }
    return 0;
}

/* --- one unit: 16 output rows (tile column nt) x mt activation rows, over all k --- */

static float q8k_d(const uint8_t *a) { float d; memcpy(&d, a, 4); return d; }
static const int8_t *q8k_qs(const uint8_t *a) { return (const int8_t *)(a + 4); }
static int16_t q8k_bsum(const uint8_t *a, int i) { int16_t v; memcpy(&v, a + 260 + 2 * i, 2); return v; }

/* 4 weight codes of row r in group g times 4 activation codes */
static int32_t dot4(const uint8_t *qs, int g, int r, const int8_t *a) {
    const uint8_t *w = qs + (g * TN + r) * 4;
    return w[0] * a[0] + w[1] * a[1] + w[2] * a[2] + w[3] * a[3];
}

static void unit_plain(int dtype, const void *packed, int64_t kb, int64_t nt, const uint8_t *lhs,
                       int mt, float *acc /* [MAX_MT][TN] */) {
    for (int i = 0; i < mt * TN; i++) acc[i] = 0.f;
    for (int64_t b = 0; b < kb; b++) {
        if (dtype == OR_Q4_K) {
            /* q4k_tile, repack_x86.rs:221-259 */
            const tile_q4k *tl = (const tile_q4k *)packed + nt * kb + b;
            for (int s = 0; s < 8; s++) {
                for (int m = 0; m < mt; m++) {
                    const uint8_t *a = lhs + (m * kb + b) * Q8K_BYTES;
                    const int8_t *q = q8k_qs(a);
                    float dall = q8k_d(a);
                    float bsum = (float)((int32_t)q8k_bsum(a, 2 * s) + (int32_t)q8k_bsum(a, 2 * s + 1));
                    for (int r = 0; r < TN; r++) {
                        int32_t isum = 0;
                        for (int g4 = 0; g4 < 4; g4++) {
                            int g = s * 4 + g4;
                            const uint8_t *w = tl->qs + (g * TN + r) * 4;
                            const int8_t *lo = q + s * 32 + g4 * 8, *hi = lo + 4;
                            for (int j = 0; j < 4; j++) isum += (w[j] & 0x0F) * lo[j] + (w[j] >> 4) * hi[j];
                        }
                        float *o = acc + m * TN + r;
                        *o = fmaf((float)isum, tl->sc[s][r] * dall, *o);
                        *o = fmaf(-tl->mn[s][r], dall * bsum, *o);
                    }
                }
            }
        } else if (dtype == OR_Q6_K) {
            /* q6k_tile, repack_x86.rs:262-285 */
            const tile_q6k *tl = (const tile_q6k *)packed + nt * kb + b;
            for (int s = 0; s < 16; s++) {
                for (int m = 0; m < mt; m++) {
                    const uint8_t *a = lhs + (m * kb + b) * Q8K_BYTES;
                    const int8_t *q = q8k_qs(a);
                    float dall = q8k_d(a);
                    float bsum = (float)q8k_bsum(a, s);
                    for (int r = 0; r < TN; r++) {
                        int32_t isum = 0;
                        for (int g4 = 0; g4 < 4; g4++) isum += dot4(tl->qs, s * 4 + g4, r, q + s * 16 + g4 * 4);
                        float f = (float)isum - 32.f * bsum;
                        float *o = acc + m * TN + r;
                        *o = fmaf(f, tl->sc[s][r] * dall, *o);
                    }
                }
            }
        } else {
            /* q8_0_tile2, repack_x86.rs:289-321: 8 tiles of 32 values per Q8_K super-block */
            for (int s = 0; s < 8; s++) {
                const tile_q8_0 *tl = (const tile_q8_0 *)packed + (nt * kb + b) * 8 + s;
                for (int m = 0; m < mt; m++) {
                    const uint8_t *a = lhs + (m * kb + b) * Q8K_BYTES;
                    const int8_t *q = q8k_qs(a);
                    float ad = q8k_d(a);
                    float bsum = (float)((int32_t)q8k_bsum(a, 2 * s) + (int32_t)q8k_bsum(a, 2 * s + 1));
                    for (int r = 0; r < TN; r++) {
                        int32_t isum = 0;
                        for (int g4 = 0; g4 < 8; g4++) isum += dot4(tl->qs, g4, r, q + s * 32 + g4 * 4);
                        float f = (float)isum - 128.f * bsum;
                        float *o = acc + m * TN + r;
                        *o = fmaf(f, or_f16_to_f32(tl->d[r]) * ad, *o);
                    }
                }
            }
        }
    }
}

#define AVX512 __attribute__((target("avx512f,avx512vnni,avx512bw")))

AVX512 static inline __m512i bcast4(const int8_t *p) {
    int32_t v;
    memcpy(&v, p, 4);
    return _mm512_set1_epi32(v);
}

AVX512 static void unit_512(int dtype, const void *packed, int64_t kb, int64_t nt, const uint8_t *lhs,
                            int mt, float *out) {
    __m512 acc[MAX_MT];
    for (int m = 0; m < MAX_MT; m++) acc[m] = _mm512_setzero_ps();
    const __m512i nib = _mm512_set1_epi8(0x0F);
    for (int64_t b = 0; b < kb; b++) {
        const uint8_t *a[MAX_MT];
        for (int m = 0; m < mt; m++) a[m] = lhs + (m * kb + b) * Q8K_BYTES;
        if (dtype == OR_Q4_K) {
            const tile_q4k *tl = (const tile_q4k *)packed + nt * kb + b;
            for (int p = 0; p < 4; p++) {
                /* sub-blocks in pairs, each with its own integer accumulators */
                int sa = 2 * p, sb = sa + 1;
                __m512i ia[MAX_MT], ib[MAX_MT];
                for (int m = 0; m < MAX_MT; m++) ia[m] = ib[m] = _mm512_setzero_si512();
                for (int g4 = 0; g4 < 4; g4++) {
                    __m512i wa = _mm512_loadu_si512(tl->qs + (sa * 4 + g4) * TN * 4);
                    __m512i wb = _mm512_loadu_si512(tl->qs + (sb * 4 + g4) * TN * 4);
                    __m512i la = _mm512_and_si512(wa, nib), ha = _mm512_and_si512(_mm512_srli_epi16(wa, 4), nib);
                    __m512i lb = _mm512_and_si512(wb, nib), hb = _mm512_and_si512(_mm512_srli_epi16(wb, 4), nib);
                    for (int m = 0; m < mt; m++) {
                        const int8_t *q = q8k_qs(a[m]);
                        ia[m] = _mm512_dpbusd_epi32(ia[m], la, bcast4(q + sa * 32 + g4 * 8));
                        ia[m] = _mm512_dpbusd_epi32(ia[m], ha, bcast4(q + sa * 32 + g4 * 8 + 4));
                        ib[m] = _mm512_dpbusd_epi32(ib[m], lb, bcast4(q + sb * 32 + g4 * 8));
                        ib[m] = _mm512_dpbusd_epi32(ib[m], hb, bcast4(q + sb * 32 + g4 * 8 + 4));
                    }
                }
                for (int h = 0; h < 2; h++) {
                    int s = h ? sb : sa;
                    __m512 sc = _mm512_loadu_ps(tl->sc[s]), mn = _mm512_loadu_ps(tl->mn[s]);
                    for (int m = 0; m < mt; m++) {
                        float dall = q8k_d(a[m]);
                        float bsum = (float)((int32_t)q8k_bsum(a[m], 2 * s) + (int32_t)q8k_bsum(a[m], 2 * s + 1));
                        __m512 f = _mm512_cvtepi32_ps(h ? ib[m] : ia[m]);
                        acc[m] = _mm512_fmadd_ps(f, _mm512_mul_ps(sc, _mm512_set1_ps(dall)), acc[m]);
                        acc[m] = _mm512_fnmadd_ps(mn, _mm512_set1_ps(dall * bsum), acc[m]);
                    }
                }
            }
        } else if (dtype == OR_Q6_K) {
            const tile_q6k *tl = (const tile_q6k *)packed + nt * kb + b;
            for (int s = 0; s < 16; s++) {
                __m512i is[MAX_MT];
                for (int m = 0; m < MAX_MT; m++) is[m] = _mm512_setzero_si512();
                for (int g4 = 0; g4 < 4; g4++) {
                    __m512i w = _mm512_loadu_si512(tl->qs + (s * 4 + g4) * TN * 4);
                    for (int m = 0; m < mt; m++)
                        is[m] = _mm512_dpbusd_epi32(is[m], w, bcast4(q8k_qs(a[m]) + s * 16 + g4 * 4));
                }
                __m512 sc = _mm512_loadu_ps(tl->sc[s]);
                for (int m = 0; m < mt; m++) {
                    float dall = q8k_d(a[m]);
                    float bsum = (float)q8k_bsum(a[m], s);
                    __m512 f = _mm512_sub_ps(_mm512_cvtepi32_ps(is[m]), _mm512_set1_ps(32.f * bsum));
                    acc[m] = _mm512_fmadd_ps(f, _mm512_mul_ps(sc, _mm512_set1_ps(dall)), acc[m]);
                }
            }
        } else {
            for (int s = 0; s < 8; s += 2) {
                const tile_q8_0 *t0 = (const tile_q8_0 *)packed + (nt * kb + b) * 8 + s, *t1 = t0 + 1;
                __m512i ia[MAX_MT], ib[MAX_MT];
                for (int m = 0; m < MAX_MT; m++) ia[m] = ib[m] = _mm512_setzero_si512();
                for (int g4 = 0; g4 < 8; g4++) {
                    __m512i wa = _mm512_loadu_si512(t0->qs + g4 * TN * 4);
                    __m512i wb = _mm512_loadu_si512(t1->qs + g4 * TN * 4);
                    for (int m = 0; m < mt; m++) {
                        const int8_t *q = q8k_qs(a[m]);
                        ia[m] = _mm512_dpbusd_epi32(ia[m], wa, bcast4(q + s * 32 + g4 * 4));
                        ib[m] = _mm512_dpbusd_epi32(ib[m], wb, bcast4(q + (s + 1) * 32 + g4 * 4));
                    }
                }
                for (int h = 0; h < 2; h++) {
                    int blk = s + h;
                    const tile_q8_0 *tl = h ? t1 : t0;
                    __m512 dw = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i *)tl->d));
                    for (int m = 0; m < mt; m++) {
                        float bsum = (float)((int32_t)q8k_bsum(a[m], 2 * blk) + (int32_t)q8k_bsum(a[m], 2 * blk + 1));
                        __m512 f = _mm512_sub_ps(_mm512_cvtepi32_ps(h ? ib[m] : ia[m]), _mm512_set1_ps(128.f * bsum));
                        acc[m] = _mm512_fmadd_ps(f, _mm512_mul_ps(dw, _mm512_set1_ps(q8k_d(a[m]))), acc[m]);
                    }
                }
            }
        }
    }
    for (int m = 0; m < mt; m++) _mm512_storeu_ps(out + m * TN, acc[m]);
}

/* matmul_tiles, repack_x86.rs:425-475: y[m][n] = x[m] . W[n] over the packed tiles.
 * simd: 1 = the AVX-512 VNNI unit (when the host has it), 0 = the plain-C unit. */
int or_x86_matmul(int dtype, const void *packed, int64_t n, int64_t k, const float *x, int64_t m,
                  float *y, int simd, int threads) {
    if (!or_x86_packed_bytes(dtype, n, k) || m <= 0) return -1;
    int use512 = simd && or_x86_level() == 2;
    int64_t kb = k / QK_K, n_tiles = n / TN, m_units = (m + MAX_MT - 1) / MAX_MT;
    uint8_t *lhs = (uint8_t *)malloc((size_t)(m * kb * Q8K_BYTES));
    if (!lhs) return -1;
    int nth = threads > 0 ? threads : omp_get_max_threads();
    /* quantize_lhs: one row without threads, several rows over the threads */
    if (m == 1) {
        or_quantize_q8_k(x, k, lhs);
    } else {
#pragma omp parallel for schedule(static) num_threads(nth)
        for (int64_t r = 0; r < m; r++) or_quantize_q8_k(x + r * k, k, lhs + r * kb * Q8K_BYTES);
    }
#pragma omp parallel for schedule(static) num_threads(nth)
    for (int64_t u = 0; u < n_tiles * m_units; u++) {
        int64_t nt = u / m_units, m0 = (u % m_units) * MAX_MT;
        int mt = (int)(m - m0 < MAX_MT ? m - m0 : MAX_MT);
        float acc[MAX_MT * TN];
        const uint8_t *a = lhs + m0 * kb * Q8K_BYTES;
        if (use512) unit_512(dtype, packed, kb, nt, a, mt, acc);
        else unit_plain(dtype, packed, kb, nt, a, mt, acc);
        for (int i = 0; i < mt; i++) memcpy(y + (m0 + i) * n + nt * TN, acc + i * TN, TN * sizeof(float));
    }
    free(lhs);
    return 0;
}
