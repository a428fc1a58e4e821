"""Pins of the oracle's restatement of candle's CPU quantized path: the activation quantizers
(Q8_0 and Q8_K from_float) byte for byte against numpy closed forms of
vendor/candle-core/src/quantized/k_quants.rs:784-821 and 2495-2534, the generic matmul driver
(k_quants.rs:2551-2670) against its pieces, and the x86 repacked tile path (repack_x86.rs)
against the f64 product it computes and against its own plain-C unit.

The closed forms are written from the Rust text, not from the C: f32 arithmetic throughout,
Rust's f32::round (half away from zero, which numpy's round is not), the saturating `as i8`, the
first index of the largest |x| for Q8_K's signed max, f16 storage of Q8_0's d by round to
nearest even. Cases that tell a plausible slip apart: exact .5 products (half to even would
differ), an all-zero block (d = 0, and id = 0 rather than inf), equal |x| of opposite signs
(the first one sets Q8_K's sign), blocks where id from the f16-rounded d would round some
quants differently, and values that saturate at -128 in Q8_K."""
import numpy as np
import pytest

from coachwhip_amd import formats as F
from coachwhip_amd import synth
from oracle import oracle as O


def round_half_away(v):
    """Rust f32::round on f32 values, exactly (|v| + 0.5 is exact in f64 for any f32 |v| < 2^52)."""
    v = np.asarray(v, dtype=np.float32).astype(np.float64)
    return (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.float32)


def q8_0_closed_form(x):
    x = np.asarray(x, dtype=np.float32).reshape(-1, 32)
    out = np.zeros((x.shape[0], 34), dtype=np.uint8)
    for i, xs in enumerate(x):
        amax = np.float32(np.max(np.abs(xs)))
        d = np.float32(amax / np.float32(127.0))
        idd = np.float32(np.float32(1.0) / d) if d != 0 else np.float32(0.0)
        q = np.clip(round_half_away(xs * idd), -128, 127).astype(np.int8)
        out[i, 0:2] = np.array([d], dtype=np.float32).astype(np.float16).view(np.uint8)
        out[i, 2:34] = q.view(np.uint8)
    return out.reshape(-1)


def q8_k_closed_form(x):
    x = np.asarray(x, dtype=np.float32).reshape(-1, 256)
    out = np.zeros((x.shape[0], 292), dtype=np.uint8)
    for i, xs in enumerate(x):
        a = np.abs(xs)
        if a.max() == 0:
            continue                                    # d = 0, quants and bsums 0
        mx = xs[int(np.argmax(a))]                      # the first largest |x|, with its sign
        iscale = np.float32(np.float32(-127.0) / mx)
        q = np.clip(round_half_away(iscale * xs), -128, 127).astype(np.int8)
        bs = q.astype(np.int32).reshape(16, 16).sum(axis=1).astype(np.int16)
        out[i, 0:4] = np.array([np.float32(1.0) / iscale], dtype=np.float32).view(np.uint8)
        out[i, 4:260] = q.view(np.uint8)
        out[i, 260:292] = bs.view(np.uint8)
    return out.reshape(-1)


def _edge_blocks(rng, bs):
    blocks = [np.zeros(bs, np.float32)]                                     # all zero
    t = rng.standard_normal(bs).astype(np.float32)
    t[3], t[9] = 10.0, -10.0                                                # first largest is +
    blocks.append(t)
    t = rng.standard_normal(bs).astype(np.float32)
    t[3], t[9] = -10.0, 10.0                                                # first largest is -
    blocks.append(t)
    # exact .5 products: amax 127 gives d = 1 (and Q8_K's iscale = -1), so x * id = x
    t = (np.arange(bs, dtype=np.float32) % 9 - 4) + 0.5
    t[0] = 127.0
    blocks.append(t.astype(np.float32))
    blocks.append(-t.astype(np.float32))
    t = rng.standard_normal(bs).astype(np.float32) * 1e-30                 # tiny values
    blocks.append(t)
    return np.concatenate(blocks)


def test_q8_0_quantizer_bytes():
    rng = np.random.default_rng(31)
    x = np.concatenate([_edge_blocks(rng, 32), rng.standard_normal(32 * 400).astype(np.float32) * 3])
    got = O.quantize_q8_0(x)
    want = q8_0_closed_form(x)
    assert np.array_equal(got, want)
    # the .5 block rounds half away from zero: 0.5 -> 1, -3.5 -> -4
    q = got.reshape(-1, 34)[3, 2:].view(np.int8)
    assert q[1] == -3 and q[4] == 1 and q[0] == 127
    # a slip (id from the f16-rounded d) changes some quants of random blocks
    xs = x.reshape(-1, 32)[6:]
    d16 = np.abs(xs).max(axis=1).astype(np.float32) / np.float32(127)
    id16 = (np.float32(1) / d16.astype(np.float16).astype(np.float32))[:, None]
    slip = np.clip(round_half_away(xs * id16), -128, 127).astype(np.int8)
    assert not np.array_equal(slip, got.reshape(-1, 34)[6:, 2:].view(np.int8))


def test_q8_k_quantizer_bytes():
    rng = np.random.default_rng(32)
    x = np.concatenate([_edge_blocks(rng, 256), rng.standard_normal(256 * 60).astype(np.float32) * 3])
    got = O.quantize_q8_k(x)
    want = q8_k_closed_form(x)
    assert np.array_equal(got, want)
    b = got.reshape(-1, 292)
    assert np.frombuffer(b[0, 0:4].tobytes(), np.float32)[0] == 0 and not b[0, 4:].any()
    d1 = np.frombuffer(b[1, 0:4].tobytes(), np.float32)[0]
    d2 = np.frombuffer(b[2, 0:4].tobytes(), np.float32)[0]
    assert d1 < 0 < d2                                  # the first largest |x| sets the sign of d
    assert b[1, 4 + 3].view(np.int8) == -127 and b[1, 4 + 9].view(np.int8) == 127
    # .5 ties: with iscale = -1 the codes are -(x) rounded half away, e.g. 4.5 -> -5 (not -4)
    q = b[3, 4:260].view(np.int8)
    assert q[0] == -127 and q[8] == -5 and q[4] == -1
    # quants saturate at -128 (a value just past the max's magnitude cannot occur, but the clamp is
    # the reference's): the dequantized block is within half a step of x
    xs = x.reshape(-1, 256)[6:]
    d = np.frombuffer(b[6:, 0:4].copy().tobytes(), np.float32)[:, None]
    assert np.all(np.abs(b[6:, 4:260].view(np.int8) * d - xs) <= 0.5 * np.abs(d) * (1 + 1e-6))
    # bsums are the sums of 16 quants
    assert np.array_equal(b[6:, 260:292].copy().view(np.int16),
                          b[6:, 4:260].view(np.int8).astype(np.int32).reshape(-1, 16, 16).sum(axis=2))


@pytest.mark.parametrize("dtype", [F.Q8_0, F.Q4_K, F.MXFP4])
def test_candle_matmul_is_quantize_then_vec_dot(dtype):
    """The generic driver (k_quants.rs:2551-2670): x rows quantized to the weight type's vec-dot type
    (Q8_K for Q4_K, Q8_0 otherwise), one vec_dot per (row, token), bit for bit; and the result is
    the f64 product of the dequantized weights and the dequantized activation blocks up to f32
    rounding of the block sums (1e-6), far inside the ~1e-2 the activation quantization costs."""
    rng = np.random.default_rng(33 + dtype)
    n, k, m = 24, 512, 3
    w = synth.random_blocks(dtype, n * k, rng)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = O.candle_matmul(dtype, w, n, k, x)
    rb = F.matrix_bytes(dtype, 1, k)
    quant = O.quantize_q8_k if dtype == F.Q4_K else O.quantize_q8_0
    for t in range(m):
        xq = quant(x[t])
        for r in range(n):
            assert y[t, r] == O.vec_dot(dtype, k, w[r * rb:(r + 1) * rb], xq)
    wd = O.dequantize(dtype, w, n * k).reshape(n, k).astype(np.float64)
    if dtype == F.Q4_K:
        qb = np.stack([O.quantize_q8_k(x[t]).reshape(-1, 292) for t in range(m)])
        d = qb[:, :, 0:4].copy().view(np.float32)[..., 0].astype(np.float64)
        xd = (qb[:, :, 4:260].view(np.int8).astype(np.float64) * d[..., None]).reshape(m, k)
    else:
        qb = np.stack([O.quantize_q8_0(x[t]).reshape(-1, 34) for t in range(m)])
        d = qb[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
        xd = (qb[:, :, 2:34].view(np.int8).astype(np.float64) * d[..., None]).reshape(m, k)
    assert O.rel_l2(y, xd @ wd.T) < 1e-6
    assert O.rel_l2(y, x.astype(np.float64) @ wd.T) > 1e-4


# ---------------------------------------------------------------- candle's x86 repacked path

def _q8k_dequantized(x):
    qb = np.stack([O.quantize_q8_k(r).reshape(-1, 292) for r in x])
    d = qb[:, :, 0:4].copy().view(np.float32)[..., 0].astype(np.float64)
    return (qb[:, :, 4:260].view(np.int8).astype(np.float64) * d[..., None]).reshape(x.shape[0], -1)


@pytest.mark.parametrize("dtype", [F.Q4_K, F.Q6_K, F.Q8_0])
def test_x86_tiles_compute_the_q8k_product(dtype):
    """repack_x86.rs: the tile units give W . Q8_K(x) (weights dequantized, activations quantized
    to Q8_K as quantize_lhs does) up to f32 accumulation; the +128 (Q8_0) and +32 (Q6_K) code
    offsets and the Q4_K mins, taken out through the bsums, would leave errors of order 1 if
    wrong. The AVX-512 VNNI unit and the plain-C unit give the same bits, for row counts on and
    off the 4-row unit."""
    rng = np.random.default_rng(50 + dtype)
    n, k = 48, 512
    w = synth.random_blocks(dtype, n * k, rng)
    packed = O.x86_pack(dtype, w, n, k)
    wd = O.dequantize(dtype, w, n * k).reshape(n, k).astype(np.float64)
    for m in (1, 3, 4, 5, 9):
        x = rng.standard_normal((m, k)).astype(np.float32) * 2
        y = O.x86_matmul(dtype, packed, n, k, x, simd=False)
        want = _q8k_dequantized(x) @ wd.T
        assert O.rel_l2(y, want) < 2e-6, (m, O.rel_l2(y, want))
        if O.x86_level() == 2:
            assert np.array_equal(O.x86_matmul(dtype, packed, n, k, x, simd=True), y), m


def test_x86_q4k_agrees_with_the_generic_driver():
    """Both quantize x to Q8_K; the tiles and k_quants' vec_dot differ only in f32 summation order."""
    rng = np.random.default_rng(60)
    n, k, m = 32, 1024, 6
    w = synth.random_blocks(F.Q4_K, n * k, rng)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = O.x86_matmul(F.Q4_K, O.x86_pack(F.Q4_K, w, n, k), n, k, x)
    assert O.rel_l2(y, O.candle_matmul(F.Q4_K, w, n, k, x)) < 1e-6


def test_x86_path_selection():
    """repack_x86.rs:43-60: n a multiple of 16 and k of 256; Q6_K only for m > 1; Q8_0 not on the
    AVX2-only tier."""
    lv = O.x86_level()
    if lv < 0:
        assert not O.x86_select(F.Q4_K, 1, 64, 256)
        return
    assert O.x86_select(F.Q4_K, 1, 64, 256) and not O.x86_select(F.Q4_K, 1, 72, 256)
    assert not O.x86_select(F.Q4_K, 1, 64, 288) and not O.x86_select(F.Q4_K, 1, 64, 0)
    assert not O.x86_select(F.Q6_K, 1, 64, 256) and O.x86_select(F.Q6_K, 2, 64, 256)
    assert O.x86_select(F.Q8_0, 1, 64, 256) == (lv != 0)
    assert not O.x86_select(F.MXFP4, 1, 64, 256)
