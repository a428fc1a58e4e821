"""Pins the CPU oracle's dequantizers (TEST INFRASTRUCTURE) against what fixes them independently
of its own code: hand-decoded blocks, the reference's second formulation of each layout
(candle's vec_dot for Q8_0/Q4_K/MXFP4, the Metal matvec kernels for the IQ formats, the Metal
MXFP4 table), IEEE f16 conversion, and the table contents in the reference's shader text."""
import numpy as np
import pytest

from coachwhip_amd import formats as F
from coachwhip_amd import synth
from oracle import oracle as O
from tests import grids as G


def f16(v):
    return int(np.float16(v).view(np.uint16))


def le16(v):
    return [v & 0xFF, v >> 8]


# ---------------------------------------------------------------- f16 conversions (half 2.7.1)

def test_f16_widening_is_ieee_for_every_bit_pattern():
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([O.lib().or_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))


def test_f16_narrowing_rounds_to_nearest_even():
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.uniform(-70000, 70000, 3000), rng.uniform(-1e-4, 1e-4, 3000),
                           rng.uniform(-1e-7, 1e-7, 1000),
                           [0.0, -0.0, 65504.0, 65520.0, 65519.99, 2.0 ** -24, 2.0 ** -25,
                            3 * 2.0 ** -26, 2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]]).astype(np.float32)
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([O.lib().or_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- hand-decoded blocks

def test_q8_0_hand_block():
    qs = [1, -2, 127, -127] + [0] * 28
    blk = np.array(le16(0x3800) + [q & 0xFF for q in qs], dtype=np.uint8)  # d = 0.5
    y = O.dequantize(F.Q8_0, blk, 32)
    assert list(y[:4]) == [0.5, -1.0, 63.5, -63.5] and not y[4:].any()


def test_q4_k_hand_block_covers_both_scale_branches():
    # (scale, min) per sub-block, encoded by hand into the 12 packed bytes: sub-blocks 0-3 keep
    # their 6 bits in bytes 0-7; sub-blocks 4-7 split 4 low bits into bytes 8-11 and 2 high
    # bits into the top of bytes 0-7.
    sc = [1, 2, 3, 4, 17, 33, 49, 63]
    mn = [0, 1, 2, 3, 16, 32, 48, 5]
    scales = [65, 130, 195, 196, 64, 129, 194, 3, 1, 1, 1, 95]
    qs = [(l % 16) | ((15 - l % 16) << 4) for l in range(128)]
    blk = np.array(le16(0x3C00) + le16(0x3800) + scales + qs, dtype=np.uint8)  # d 1.0, dmin 0.5
    y = O.dequantize(F.Q4_K, blk, 256)
    for s in range(8):
        for l in range(32):
            q = (l % 16) if s % 2 == 0 else 15 - (l % 16)
            assert y[32 * s + l] == sc[s] * q - 0.5 * mn[s], (s, l)


def test_mxfp4_hand_block_including_subnormal_scales():
    # e = 127 -> 2^-1, so a doubled E2M1 code k dequantizes to k/2 = the E2M1 value itself
    qs = [(j & 0xF) | (((15 - j) & 0xF) << 4) for j in range(16)]
    y = O.dequantize(F.MXFP4, np.array([127] + qs, dtype=np.uint8), 32)
    e2m1 = [0, 0.5, 1, 1.5, 2, 3, 4, 6, 0, -0.5, -1, -1.5, -2, -3, -4, -6]
    assert list(y[:16]) == e2m1 and list(y[16:]) == e2m1[::-1]
    # e = 0 and e = 1 give f32 subnormal scales 2^-128 and 2^-127
    y0 = O.dequantize(F.MXFP4, np.array([0] + [0x71] * 16, dtype=np.uint8), 32)
    assert y0[0] == np.float32(2.0 ** -128) and y0[16] == np.float32(12 * 2.0 ** -128)
    y1 = O.dequantize(F.MXFP4, np.array([1] + [0x01] * 16, dtype=np.uint8), 32)
    assert y1[0] == np.float32(2.0 ** -127)
    y254 = O.dequantize(F.MXFP4, np.array([254] + [0xA1] * 16, dtype=np.uint8), 32)
    assert float(y254[0]) == 2.0 ** 126 and float(y254[16]) == -2.0 ** 127


def test_iq2_xxs_hand_block():
    g = G.grid_bytes("iq2xxs_grid")
    # sub-block 0: grid bytes (0, 1, 2, 255), sign indices (0, 1, 127, 64), scale nibble 3
    aux_g = 0 | (1 << 8) | (2 << 16) | (255 << 24)
    aux_s = 0 | (1 << 7) | (127 << 14) | (64 << 21) | (3 << 28)
    qs = [aux_g & 0xFFFF, aux_g >> 16, aux_s & 0xFFFF, aux_s >> 16] + [0] * 28
    blk = np.array(le16(0x3C00) + sum((le16(q) for q in qs), []), dtype=np.uint8)
    y = O.dequantize(F.IQ2_XXS, blk, 256)
    dl = 0.875  # 1.0 * (0.5 + 3) * 0.25
    assert list(g[0]) == [8] * 8 and list(g[1]) == [43] + [8] * 7 and list(g[2]) == [25, 25] + [8] * 6
    assert list(y[0:8]) == [7.0] * 8
    assert list(y[8:16]) == [-37.625] + [7.0] * 6 + [-7.0]          # ksigns[1] = 0b10000001
    assert list(y[16:24]) == [-21.875, -21.875] + [-7.0] * 6        # ksigns[127] = all negative
    want = [dl * float(g[255][i]) * (-1 if i >= 6 else 1) for i in range(8)]  # ksigns[64] = 0b11000000
    assert list(y[24:32]) == want
    assert list(y[32:]) == [1.0] * 224  # zero bytes: grid 0 (all 8) times 0.125


def test_iq2_s_hand_block():
    g = G.grid_bytes("iq2s_grid")
    qs = [1, 2, 0, 3] + [0] * 28
    signs = [0x01, 0x80, 0xFF, 0x00] + [0] * 28
    qh = [0b11100100] + [0] * 7
    scales = [0x52] + [0] * 7
    blk = np.array(le16(0x3C00) + qs + signs + qh + scales, dtype=np.uint8)
    y = O.dequantize(F.IQ2_S, blk, 256)
    # group t takes grid index qs[t] | (2 qh bits << 8): 1, 2 | 256, 0 | 512, 3 | 768
    idx = [1, 258, 512, 771]
    dls = [0.625, 0.625, 1.375, 1.375]   # (0.5 + 2) / 4 and (0.5 + 5) / 4
    sgn = [[-1] + [1] * 7, [1] * 7 + [-1], [-1] * 8, [1] * 8]
    for t in range(4):
        assert list(y[8 * t:8 * t + 8]) == [dls[t] * float(g[idx[t]][i]) * sgn[t][i] for i in range(8)], t
    assert list(y[32:]) == [0.125 * float(g[0][i % 8]) for i in range(224)]


def test_iq3_s_hand_block():
    g = G.grid_bytes("iq3s_grid")
    qs = [0] * 8 + list(range(8)) + [0] * 48
    qh = [0, 0b10000001] + [0] * 6
    signs = [0] * 4 + [0x0F, 0xF0, 0x00, 0xAA] + [0] * 24
    scales = [0x70, 0, 0, 0]
    blk = np.array(le16(0x3C00) + qs + qh + signs + scales, dtype=np.uint8)
    y = O.dequantize(F.IQ3_S, blk, 256)
    assert list(y[:32]) == [float(g[0][i % 4]) for i in range(32)]  # sub-block 0: dl = 1
    # sub-block 1: dl = 1 + 2 * 7 = 15; group v takes grid index v | (qh bit v << 8)
    sbytes = [0x0F, 0xF0, 0x00, 0xAA]
    for v in range(32):
        gi = v // 4
        idx = gi | (256 if gi in (0, 7) else 0)
        neg = (sbytes[v // 8] >> (v % 8)) & 1
        assert y[32 + v] == 15.0 * float(g[idx][v % 4]) * (-1 if neg else 1), v


def test_q6_k_hand_block():
    # k_quants.rs:2420-2451: value l of half h is ql/qh bits, minus 32, times d * scales[8h + l//16 + 2r]
    ql = [0] * 128
    qh = [0] * 64
    ql[0] = 0x21          # l = 0: low nibble 1 (r = 0), high nibble 2 (r = 2)
    ql[32] = 0x43         # l = 0: low nibble 3 (r = 1), high nibble 4 (r = 3)
    qh[0] = 0b11100100    # l = 0: 2-bit highs 0, 1, 2, 3 for r = 0..3
    ql[64 + 17] = 0xFF    # half 1, l = 17: codes 15 | 16 * qh bits
    qh[32 + 17] = 0xFF
    scales = [2, -3, 4, -5, 6, -7, 8, -9] + [1, 10, 1, 1, 1, 1, 1, 1]
    blk = np.array(ql + qh + [v & 0xFF for v in scales] + le16(0x3800), dtype=np.uint8)  # d = 0.5
    y = O.dequantize(F.Q6_K, blk, 256)
    assert y[0] == 0.5 * 2 * (1 - 32)                # r = 0 uses scale 0
    assert y[32] == 0.5 * 4 * (3 + 16 - 32)          # r = 1: scale 2, qh bits 2-3 = 1
    assert y[64] == 0.5 * 6 * (2 + 32 - 32)          # r = 2: scale 4, qh bits 4-5 = 2
    assert y[96] == 0.5 * 8 * (4 + 48 - 32)          # r = 3: scale 6, qh bits 6-7 = 3
    assert y[1] == 0.5 * 2 * -32 and y[16] == 0.5 * -3 * -32   # l >= 16 takes the next scale
    assert y[128 + 17] == 0.5 * 10 * (63 - 32)       # half 1, l = 17: scale 8 + 1
    assert y[128 + 17 + 64] == 0.5 * 1 * (63 - 32)   # high nibble, qh bits 4-5: scale 8 + 1 + 4


def test_iq3_xxs_hand_block():
    g = G.grid_bytes("iq3xxs_grid")
    # sub-block 1: grid indices 0..7, sign indices (1, 0, 127, 2) and scale nibble 5 in its word
    qs = [0] * 8 + list(range(8)) + [0] * 48
    aux = 1 | (0 << 7) | (127 << 14) | (2 << 21) | (5 << 28)
    gas = [0, 0, 0, 0] + [(aux >> (8 * i)) & 0xFF for i in range(4)] + [0] * 24
    blk = np.array(le16(0x3C00) + qs + gas, dtype=np.uint8)
    y = O.dequantize(F.IQ3_XXS, blk, 256)
    assert list(y[:32]) == [0.25 * float(g[0][i % 4]) for i in range(32)]  # dl = (0 + 0.5) * 0.5
    dl = (5 + 0.5) * 0.5
    ks = {1: 0b10000001, 0: 0, 127: 0xFF, 2: 0b10000010}   # 7 sign bits + even parity
    for h, si in enumerate((1, 0, 127, 2)):
        for t in range(2):
            for i in range(4):
                v = 8 * h + 4 * t + i
                neg = (ks[si] >> (4 * t + i)) & 1
                assert y[32 + v] == dl * float(g[2 * h + t][i]) * (-1 if neg else 1), v


def test_iq4_xs_hand_block():
    kv = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    # sub-block scales ls_ib = (scales_l nibble) | (2 bits of scales_h) << 4
    ls = [32, 33, 0, 63, 31, 40, 17, 48]
    sl = [(ls[2 * i] & 0xF) | ((ls[2 * i + 1] & 0xF) << 4) for i in range(4)]
    sh = sum(((v >> 4) & 3) << (2 * i) for i, v in enumerate(ls))
    qs = [(j % 16) | ((15 - j % 16) << 4) for j in range(128)]
    blk = np.array(le16(0x3800) + le16(sh) + sl + qs, dtype=np.uint8)  # d = 0.5
    y = O.dequantize(F.IQ4_XS, blk, 256)
    for ib in range(8):
        d = 0.5 * (ls[ib] - 32)
        for j in range(16):
            assert y[32 * ib + j] == d * kv[j % 16] and y[32 * ib + 16 + j] == d * kv[15 - j % 16], (ib, j)


# ---------------------------------------------------------------- second formulations

def _utmp_scales(sc12):
    """Q4_K scale/min unpacking as candle's vec_dot_unopt writes it (k_quants.rs:1645-1655):
    three little-endian u32 words and the KMASK constants."""
    u = [int.from_bytes(bytes(sc12[4 * i:4 * i + 4]), "little") for i in range(3)] + [0]
    k1, k2, k3 = 0x3F3F3F3F, 0x0F0F0F0F, 0x03030303
    u[3] = ((u[2] >> 4) & k2) | (((u[1] >> 6) & k3) << 4)
    uaux = u[1] & k1
    u[1] = (u[2] & k2) | (((u[0] >> 6) & k3) << 4)
    u[2] = uaux
    u[0] &= k1
    b = b"".join(x.to_bytes(4, "little") for x in u)
    return list(b[0:8]), list(b[8:16])


def _metal_just2(j, k, q):
    """get_scale_min_k4_just2 (quantized.metal:6748-6751)."""
    if j < 4:
        return q[j + k] & 63, q[j + 4 + k] & 63
    return (q[j + 4 + k] & 0xF) | ((q[j - 4 + k] & 0xC0) >> 2), (q[j + 4 + k] >> 4) | ((q[j + k] & 0xC0) >> 2)


def test_q4_k_scale_unpacking_matches_both_reference_formulations():
    rng = np.random.default_rng(7)
    for _ in range(200):
        sc12 = list(rng.integers(0, 256, 12))
        scales, mins = _utmp_scales(sc12)
        # oracle: d = 1, dmin = 0, all nibbles 1 -> each sub-block dequantizes to its scale
        blk = np.array(le16(0x3C00) + le16(0) + sc12 + [0x11] * 128, dtype=np.uint8)
        y = O.dequantize(F.Q4_K, blk, 256).reshape(8, 32)
        assert list(y[:, 0]) == [float(s) for s in scales]
        # d = 0, dmin = 1 -> each sub-block dequantizes to minus its min
        blk = np.array(le16(0) + le16(0x3C00) + sc12 + [0x11] * 128, dtype=np.uint8)
        y = O.dequantize(F.Q4_K, blk, 256).reshape(8, 32)
        assert list(-y[:, 0]) == [float(m) for m in mins]
        for s in range(8):
            # Metal reads sub-block pairs (is = 2*(il/4), k = il/2 of the pair)
            assert _metal_just2(s - s % 2, s % 2, sc12) == (scales[s], mins[s])


@pytest.mark.parametrize("dtype", [F.Q8_0, F.Q4_K, F.MXFP4])
def test_candle_vec_dot_agrees_with_dequantize_then_dot(dtype):
    # vec_dot (k_quants.rs:738-759, 855-874, 1612-1692) reads the blocks with its own index
    # arithmetic; on exactly representable activations it must give the dequantize-then-dot sum.
    rng = np.random.default_rng(11)
    k = 512
    for _ in range(20):
        w = synth.random_blocks(dtype, k, rng)
        x = rng.standard_normal(k).astype(np.float32)
        xq = O.quantize_q8_k(x) if dtype == F.Q4_K else O.quantize_q8_0(x)
        if dtype == F.Q4_K:
            nb = k // 256
            blocks = xq.reshape(nb, 292)
            xd = np.concatenate([blocks[i, 4:260].view(np.int8).astype(np.float64) *
                                 float(blocks[i, 0:4].view(np.float32)[0]) for i in range(nb)])
        else:
            nb = k // 32
            blocks = xq.reshape(nb, 34)
            xd = np.concatenate([blocks[i, 2:34].view(np.int8).astype(np.float64) *
                                 float(blocks[i, 0:2].view(np.float16)[0]) for i in range(nb)])
        want = float(np.dot(O.dequantize(dtype, w, k).astype(np.float64), xd))
        got = O.vec_dot(dtype, k, w, xq)
        assert abs(got - want) <= 1e-5 * max(1.0, abs(want)), (got, want)


def _q8k_rows(x):
    """x quantized to Q8_K: (codes, d, bsums) per super-block."""
    qb = O.quantize_q8_k(x).reshape(-1, 292)
    d = qb[:, 0:4].copy().view(np.float32)[:, 0].astype(np.float64)
    return qb[:, 4:260].view(np.int8).astype(np.int64), d, qb[:, 260:292].copy().view(np.int16).astype(np.int64)


def _vd_q6_k(blk, q8, yd):
    """candle's Q6_K x Q8_K vec_dot_unopt (k_quants.rs:2208-2262) for one row, in f64."""
    tot = 0.0
    for ibl in range(len(blk) // 210):
        b = blk[210 * ibl:210 * ibl + 210].astype(np.int64)
        ql, qh = b[0:128], b[128:192]
        sc = blk[210 * ibl + 192:210 * ibl + 208].view(np.int8).astype(np.int64)
        d = float(blk[210 * ibl + 208:210 * ibl + 210].view(np.float16)[0])
        aux8 = np.zeros(256, dtype=np.int64)
        for j in range(0, 256, 128):
            q4, h = ql[j // 2:], qh[j // 4:]
            for l in range(32):
                aux8[j + l] = ((q4[l] & 0xF) | ((h[l] & 3) << 4)) - 32
                aux8[j + l + 32] = ((q4[l + 32] & 0xF) | (((h[l] >> 2) & 3) << 4)) - 32
                aux8[j + l + 64] = ((q4[l] >> 4) | (((h[l] >> 4) & 3) << 4)) - 32
                aux8[j + l + 96] = ((q4[l + 32] >> 4) | (((h[l] >> 6) & 3) << 4)) - 32
        isum = sum(float(sc[j]) * float(np.dot(q8[ibl, 16 * j:16 * j + 16], aux8[16 * j:16 * j + 16])) for j in range(16))
        tot += d * yd[ibl] * isum
    return tot


def _vd_q5_k(blk, q8, yd, bsums):
    """candle's Q5_K x Q8_K vec_dot_unopt (k_quants.rs:1870-1956) for one row, in f64, with the
    scales and mins unpacked through the utmp word shuffle."""
    tot = 0.0
    for ibl in range(len(blk) // 176):
        b = blk[176 * ibl:176 * ibl + 176].astype(np.int64)
        d = float(blk[176 * ibl:176 * ibl + 2].view(np.float16)[0])
        dmin = float(blk[176 * ibl + 2:176 * ibl + 4].view(np.float16)[0])
        scales, mins = _utmp_scales(blk[176 * ibl + 4:176 * ibl + 16])
        hm, q5 = b[16:48], b[48:176]
        aux8 = np.zeros(256, dtype=np.int64)
        m, pos = 1, 0
        for c in range(4):
            for half in range(2):
                for l in range(32):
                    v = (q5[32 * c + l] & 0xF) if half == 0 else (q5[32 * c + l] >> 4)
                    aux8[pos + l] = v + (16 if hm[l] & m else 0)
                pos += 32
                m <<= 1
        isum = sum(scales[j] * float(np.dot(q8[ibl, 32 * j:32 * j + 32], aux8[32 * j:32 * j + 32])) for j in range(8))
        sumi = sum(int(bsums[ibl, j]) * mins[j // 2] for j in range(16))
        tot += d * yd[ibl] * isum - dmin * yd[ibl] * sumi
    return tot


@pytest.mark.parametrize("dtype", [F.Q5_K, F.Q6_K])
def test_k_quant_dequantize_agrees_with_candle_vec_dot_layout(dtype):
    """The oracle's Q5_K / Q6_K dequantizers against candle's vec_dot_unopt arithmetic (a second
    reading of the same bytes): both in f64 against the same Q8_K activation codes, equal up to the
    f32 rounding of the dequantized weights (a misplaced bit or scale is off by far more)."""
    rng = np.random.default_rng(40 + dtype)
    k, rows = 512, 5
    w = synth.random_blocks(dtype, rows * k, rng).reshape(rows, -1)
    x = rng.standard_normal(k).astype(np.float32)
    q8, yd, bsums = _q8k_rows(x)
    xd = (q8 * yd[:, None]).reshape(-1)
    got = O.qmatmul_f64(dtype, w, rows, k, xd.astype(np.float32))[0]
    if dtype == F.Q6_K:
        want = np.array([_vd_q6_k(w[r], q8, yd) for r in range(rows)])
    else:
        want = np.array([_vd_q5_k(w[r], q8, yd, bsums) for r in range(rows)])
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)


def test_mxfp4_matches_the_metal_table_for_every_exponent_and_code():
    # Metal formulation (quantized.metal:2563-2571): halved E2M1 table times e8m0_to_fp32,
    # which maps e = 0 to 2^-127 and e > 0 to 2^(e-127)
    halved = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], dtype=np.float32)
    codes = np.arange(16, dtype=np.uint8)
    qs = list(codes[::2] | (codes[1::2] << 4))
    # e = 255 is left out: the two formulations part there (Metal's scale is inf, candle's 2^127)
    for e in range(255):
        blk = np.array([e] + qs + qs, dtype=np.uint8)
        y = O.dequantize(F.MXFP4, blk, 32)
        bits = 0x00400000 if e == 0 else (e << 23)
        scale = np.array([bits], dtype=np.uint32).view(np.float32)[0]
        lo = [codes[2 * (j % 8)] for j in range(16)]
        hi = [codes[2 * (j % 8) + 1] for j in range(16)]
        want = np.array([halved[c] * scale for c in lo] + [halved[c] * scale for c in hi], dtype=np.float32)
        assert np.array_equal(y, want), e


def _mv_iq2_xxs(blk, x):
    """kernel_mul_mv_iq2_xxs_f32_impl (quantized.metal:5421-5519) for one row, in f64."""
    g, ks = G.grid_bytes("iq2xxs_grid"), G.ksigns_closed_form()
    tot = 0.0
    for ibl in range(len(blk) // 66):
        b = blk[66 * ibl:66 * ibl + 66]
        db = float(b[0:2].view(np.float16)[0])
        q2 = b[2:66].view(np.uint16)
        for ib in range(8):
            yl = x[256 * ibl + 32 * ib:256 * ibl + 32 * ib + 32]
            aux8 = q2[4 * ib:4 * ib + 2].view(np.uint8)
            aux32 = int(q2[4 * ib + 2]) | (int(q2[4 * ib + 3]) << 16)
            d = db * (0.5 + (aux32 >> 28))
            s = 0.0
            for l in range(4):
                signs = ks[(aux32 >> 7 * l) & 127]
                for j in range(8):
                    s += yl[8 * l + j] * float(g[aux8[l]][j]) * (-1.0 if signs & (1 << j) else 1.0)
            tot += d * s
    return tot * 0.25


def _mv_iq2_s(blk, x):
    """kernel_mul_mv_iq2_s_f32_impl (quantized.metal:5953-6056) for one row, in f64."""
    g = G.grid_bytes("iq2s_grid")
    tot = 0.0
    for ibl in range(len(blk) // 82):
        b = blk[82 * ibl:82 * ibl + 82].astype(np.int64)
        db = float(blk[82 * ibl:82 * ibl + 2].view(np.float16)[0])
        for ib in range(8):
            yl = x[256 * ibl + 32 * ib:256 * ibl + 32 * ib + 32]
            qs = b[2 + 4 * ib:]
            signs = b[2 + 32 + 4 * ib:]
            qh, sc = int(b[66 + ib]), int(b[74 + ib])
            d1, d2 = db * (0.5 + (sc & 0xF)), db * (0.5 + (sc >> 4))
            s0 = s1 = 0.0
            for l in range(2):
                g1 = g[int(qs[l]) | ((qh << (8 - 2 * l)) & 0x300)]
                g2 = g[int(qs[l + 2]) | ((qh << (4 - 2 * l)) & 0x300)]
                for j in range(8):
                    s0 += yl[8 * l + j] * float(g1[j]) * (-1.0 if signs[l] & (1 << j) else 1.0)
                    s1 += yl[8 * l + j + 16] * float(g2[j]) * (-1.0 if signs[l + 2] & (1 << j) else 1.0)
            tot += d1 * s0 + d2 * s1
    return tot * 0.25


def _mv_iq3_s(blk, x):
    """kernel_mul_mv_iq3_s_f32_impl (quantized.metal:5821-5923) for one row, in f64."""
    g = G.grid_bytes("iq3s_grid")
    tot = 0.0
    for ibl in range(len(blk) // 110):
        b = blk[110 * ibl:110 * ibl + 110].astype(np.int64)
        db = float(blk[110 * ibl:110 * ibl + 2].view(np.float16)[0])
        for ib in range(8):
            yl = x[256 * ibl + 32 * ib:256 * ibl + 32 * ib + 32]
            qs = b[2 + 8 * ib:]
            qh = int(b[66 + ib])
            signs = b[74 + 4 * ib:]
            sc = int(b[106 + ib // 2])
            d = db * (1 + 2 * ((sc >> 4 * (ib % 2)) & 0xF))
            s0 = s1 = 0.0
            for l in range(4):
                t1 = 256 if qh & (1 << (2 * l)) else 0
                t2 = 256 if qh & (1 << (2 * l + 1)) else 0
                g1, g2 = g[t1 + int(qs[2 * l])], g[t2 + int(qs[2 * l + 1])]
                for j in range(4):
                    s0 += yl[8 * l + j] * float(g1[j]) * (-1.0 if signs[l] & (1 << j) else 1.0)
                    s1 += yl[8 * l + j + 4] * float(g2[j]) * (-1.0 if signs[l] & (1 << (j + 4)) else 1.0)
            tot += d * (s0 + s1)
    return tot


def _mv_iq3_xxs(blk, x):
    """kernel_mul_mv_iq3_xxs_f32_impl (quantized.metal:5700-5786) for one row, in f64."""
    g, ks = G.grid_bytes("iq3xxs_grid"), G.ksigns_closed_form()
    tot = 0.0
    for ibl in range(len(blk) // 98):
        b = blk[98 * ibl:98 * ibl + 98].astype(np.int64)
        db = float(blk[98 * ibl:98 * ibl + 2].view(np.float16)[0])
        for ib in range(8):
            yl = x[256 * ibl + 32 * ib:256 * ibl + 32 * ib + 32]
            q3 = b[2 + 8 * ib:]
            gas = b[2 + 64 + 4 * ib:]
            aux32 = int(gas[0]) | (int(gas[1]) << 8) | (int(gas[2]) << 16) | (int(gas[3]) << 24)
            d = db * (0.5 + (aux32 >> 28))
            s0 = s1 = 0.0
            for l in range(4):
                g1, g2 = g[int(q3[2 * l])], g[int(q3[2 * l + 1])]
                signs = ks[(aux32 >> 7 * l) & 127]
                for j in range(4):
                    s0 += yl[8 * l + j] * float(g1[j]) * (-1.0 if signs & (1 << j) else 1.0)
                    s1 += yl[8 * l + j + 4] * float(g2[j]) * (-1.0 if signs & (1 << (j + 4)) else 1.0)
            tot += d * (s0 + s1)
    return tot * 0.5


def _mv_iq4_xs(blk, x):
    """kernel_mul_mv_iq4_xs_f32_impl (quantized.metal:6384-6460) for one row, in f64: lane
    (ib, il) pairs the low nibbles of bytes 8il..8il+8 of the sub-block with x[32ib + 8il ..) and
    the high nibbles with x[32ib + 16 + 8il ..)."""
    kv = G.reference_kvalues_iq4nl() or [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    tot = 0.0
    for ibl in range(len(blk) // 136):
        b = blk[136 * ibl:136 * ibl + 136].astype(np.int64)
        db = float(blk[136 * ibl:136 * ibl + 2].view(np.float16)[0])
        sh = int(b[2]) | (int(b[3]) << 8)
        for ib in range(8):
            ls = (((int(b[4 + ib // 2]) >> 4 * (ib % 2)) & 0xF) | (((sh >> 2 * ib) & 3) << 4)) - 32
            acc = 0.0
            for il in range(2):
                yb = x[256 * ibl + 32 * ib + 8 * il:]
                q4 = b[8 + 16 * ib + 8 * il:]
                for j in range(8):
                    acc += yb[j] * kv[int(q4[j]) & 0xF] + yb[16 + j] * kv[int(q4[j]) >> 4]
            tot += db * ls * acc
    return tot


@pytest.mark.parametrize("dtype,mv", [(F.IQ2_XXS, _mv_iq2_xxs), (F.IQ2_S, _mv_iq2_s), (F.IQ3_S, _mv_iq3_s),
                                      (F.IQ3_XXS, _mv_iq3_xxs), (F.IQ4_XS, _mv_iq4_xs)])
def test_iq_dequantize_agrees_with_the_metal_matvec_formulation(dtype, mv):
    rng = np.random.default_rng(dtype)
    k, rows = 512, 6
    w = synth.random_blocks(dtype, rows * k, rng).reshape(rows, -1)
    x = rng.standard_normal(k).astype(np.float32)
    want = np.array([mv(w[r], x.astype(np.float64)) for r in range(rows)])
    got = O.qmatmul_f64(dtype, w, rows, k, x)[0]
    assert np.allclose(got, want, rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("dtype", F.WEIGHT_TYPES)
def test_dequantized_values_are_exact_products(dtype):
    # every in-scope dequantization is (f16 or power-of-two scale) x (small integer); exact in
    # f32, so f64 recomputation of the same product from the raw fields reproduces the bits.
    rng = np.random.default_rng(100 + dtype)
    w = synth.random_blocks(dtype, 4096, rng)
    y = O.dequantize(dtype, w, 4096)
    assert np.all(np.isfinite(y))
    if dtype in (F.IQ2_XXS, F.IQ2_S):
        nb = 4096 // 256
        d = w.reshape(nb, -1)[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(nb, 1)
        units = y.reshape(nb, 256).astype(np.float64) / (d / 8)   # (2s+1) * grid * sign
        assert np.all(units == np.round(units)) and np.all(np.abs(units) <= 31 * 43)
    if dtype == F.IQ3_S:
        nb = 4096 // 256
        d = w.reshape(nb, -1)[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(nb, 1)
        units = y.reshape(nb, 256).astype(np.float64) / d          # (2s+1) * grid * sign
        assert np.all(units == np.round(units)) and np.all(np.abs(units) <= 31 * 15)


# ---------------------------------------------------------------- tables

def test_grid_table_invariants():
    assert G.GRIDS["iq2xxs_grid"].size == 256 and G.GRIDS["iq2s_grid"].size == 1024
    assert G.GRIDS["iq3s_grid"].size == 512 and G.GRIDS["iq3xxs_grid"].size == 256
    assert set(np.unique(G.grid_bytes("iq2xxs_grid"))) == {8, 25, 43}
    assert set(np.unique(G.grid_bytes("iq2s_grid"))) == {8, 25, 43}
    assert set(np.unique(G.grid_bytes("iq3s_grid"))) == set(range(1, 16, 2))
    assert set(np.unique(G.grid_bytes("iq3xxs_grid"))) == {4, 12, 20, 28, 36, 44, 52, 62}
    # lattice points are distinct within each table
    for name in ("iq2xxs_grid", "iq2s_grid", "iq3s_grid", "iq3xxs_grid"):
        assert len(np.unique(G.GRIDS[name])) == G.GRIDS[name].size


@pytest.mark.skipif(G.reference_table("iq2xxs_grid") is None, reason="reference checkout absent")
def test_tables_equal_the_reference_shader_text():
    for name in ("iq2xxs_grid", "iq2s_grid", "iq3s_grid", "iq3xxs_grid"):
        assert [int(v) for v in G.GRIDS[name]] == G.reference_table(name), name
    # the oracle's IQ4 levels: one code per sub-block position with d = 1 and scale 33 (d_ib = 1)
    blk = np.zeros(136, dtype=np.uint8)
    blk[0:2] = np.array([np.float16(1.0)]).view(np.uint8)
    blk[2:4] = [0xAA, 0xAA]                              # scales_h: bits 10 per sub-block -> 32
    blk[4:8] = 0x11                                      # scales_l nibbles 1 -> ls = 1 + 32 = 33
    blk[8:24] = np.arange(16, dtype=np.uint8)            # sub-block 0: codes 0..15 (low nibbles)
    y = O.dequantize(F.IQ4_XS, blk, 256)
    assert list(y[:16]) == G.reference_kvalues_iq4nl()
    assert list(G.ksigns_closed_form()) == G.reference_table("ksigns_iq2xs")
    assert G.reference_table("kmask_iq2xs") == [1 << i for i in range(8)]


@pytest.mark.parametrize("n,nblk", [(40, 90), (16, 5), (33, 8), (17, 7)])
def test_rows16_offsets_are_a_block_permutation_with_contiguous_steps(n, nblk):
    """MXFP4_R16 (rows in groups of 16): every block of the padded matrix lands on its own 17-byte
    slot of the same bytes, each group keeps the bytes its 16 GGUF rows take, and a group's blocks
    of one 4-block step are one run, row after row (what the kernels load per step)."""
    rows = (n + 15) // 16 * 16
    offs = {(r, b): F.rows16_offset(r, b, nblk) for r in range(rows) for b in range(nblk)}
    assert sorted(offs.values()) == list(range(0, rows * nblk * 17, 17))
    rb = nblk * 17
    for (r, b), o in offs.items():
        assert (r // 16) * 16 * rb <= o < (r // 16 + 1) * 16 * rb
    for g in range(rows // 16):
        for c in range((nblk + 3) // 4):
            cb = min(4, nblk - 4 * c)
            run = [offs[(16 * g + i, 4 * c + k)] for i in range(16) for k in range(cb)]
            assert run == list(range(run[0], run[0] + 17 * 16 * cb, 17))
    assert F.matrix_bytes(F.MXFP4_R16, n, 32 * nblk) == rows * rb
