"""HIP path vs the CPU oracle on the same seeded inputs, through the C ABI.

Gates (tolerances stated per test): dequantized weights bit-exact; routing ids identical and
weights within 1e-5; matmul / matvec / MoE outputs within 1e-3 relative L2 of the f64 oracle
(the f32 kernels land near 1e-6, which the tighter f32 checks below also hold them to)."""
import zlib

import numpy as np
import pytest
import torch

import coachwhip_amd as cw
from coachwhip_amd import formats as F
from coachwhip_amd import ops, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu

REL_L2_GATE = 1e-3      # north-star tolerance for matmul / MoE outputs
REL_L2_F32 = 2e-5       # what an f32-activation path must reach
MFMA_TYPES = (F.IQ2_XXS, F.IQ2_S, F.IQ3_S, F.MXFP4, F.Q4_K, F.Q8_0, F.Q2_K, F.IQ3_XXS, F.IQ4_XS)  # formats of the grouped / dense GEMM


def dev(a):
    return ops.to_device(a)


def dev_u8(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to("cuda")


def host(t):
    return t.detach().cpu().numpy()


def say(*a):
    print(*a, flush=True)


# ------------------------------------------------------------------------------ dequantize

@pytest.mark.parametrize("dtype", F.WEIGHT_TYPES)
def test_dequantize_is_bit_exact(dtype):
    say("dequantize", F.NAMES[dtype])
    rng = np.random.default_rng(1000 + dtype)
    n = 256 * 1024
    raw = synth.random_blocks(dtype, n, rng)
    # scale edge cases: negative and subnormal f16 scales, every e8m0 exponent
    if dtype == F.MXFP4:
        nb = n // 32
        raw.reshape(nb, 17)[:256, 0] = np.arange(256, dtype=np.uint8)
    else:
        ts = F.type_size(dtype)
        nb = n // F.block_size(dtype)
        edge = np.array([0x8001, 0x0001, 0x03FF, 0xBC00, 0x7BFF, 0x0000], dtype=np.uint16).view(np.uint8).reshape(-1, 2)
        o = F.D_OFFSET[dtype]
        raw.reshape(nb, ts)[:len(edge), o:o + 2] = edge
    got = host(ops.dequantize(dtype, dev(raw), n))
    want = O.dequantize(dtype, raw, n)
    if dtype == F.MXFP4:
        # e = 255 overflows to inf in both; compare the bit patterns of everything
        pass
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------------------ dense matvec

QMM_CASES = [
    (F.Q8_0, 2048, 2048, 1),      # config 1
    (F.Q4_K, 4096, 4096, 1),      # config 2, M = 1
    (F.Q4_K, 4096, 4096, 16),     # config 2, M = 16
    (F.MXFP4, 512, 2880, 2),      # gpt-oss rows (90 blocks: two sub-blocks on some lanes)
    (F.IQ2_XXS, 512, 2048, 3),
    (F.IQ2_S, 2048, 512, 3),
    (F.IQ3_S, 512, 2048, 2),
    (F.Q8_0, 96, 64, 5),          # short rows: 2 blocks, 8 lanes per row
    (F.Q4_K, 33, 256, 1),         # one super-block per row, ragged row count
    (F.Q5_K, 512, 2048, 1),
    (F.Q6_K, 1024, 1024, 3),
    (F.Q6_K, 77, 256, 1),
    (F.IQ3_XXS, 512, 2048, 2),
    (F.IQ4_XS, 300, 1024, 4),
]


# the MFMA GEMM path (from CWMOE_MM_MIN_ROWS rows) rounds activations to fp16 once and is held to
# the 1e-3 gate; the matvec path keeps f32 activations and is held to the f32 bar as well
MM_PATHS = {"matvec": "1000000", "mfma": "1"}
MM_CASES = [
    (F.Q4_K, 200, 768, 5),        # Q4_K at 2..16 rows (one launch after the pack): ragged row tile, 3 super-blocks, one wave
    (F.Q4_K, 1000, 8192, 16),     # 32 super-blocks over 8 waves
    (F.Q4_K, 64, 2560, 2),        # 10 super-blocks over 4 waves, 2 or 3 each
    (F.Q4_K, 4096, 4096, 128),    # config 2, M = 128
    (F.Q4_K, 4096, 4096, 512),    # config 2, M = 512
    (F.Q8_0, 2048, 2048, 77),     # config 1 rows, a ragged last tile
    (F.Q4_K, 200, 512, 70),       # N-blocks past the last row, two super-blocks per row
    (F.Q8_0, 96, 1056, 33),       # 33 blocks per row: a partial last stage
    (F.MXFP4, 512, 2880, 40),
    (F.IQ2_XXS, 512, 2048, 20),
    (F.IQ3_S, 300, 1024, 65),
    (F.Q2_K, 512, 2048, 1),
    (F.Q2_K, 2048, 512, 9),
    (F.Q2_K, 200, 768, 70),       # three super-blocks per row, N-blocks past the last row
    (F.IQ3_XXS, 512, 2048, 24),
    (F.IQ4_XS, 300, 1024, 65),
    (F.IQ4_XS, 2048, 512, 9),
]


@pytest.mark.parametrize("path", sorted(MM_PATHS))
@pytest.mark.parametrize("dtype,n,k,m", QMM_CASES + MM_CASES)
def test_qmatmul_matches_the_oracle(dtype, n, k, m, path, monkeypatch):
    monkeypatch.setenv("CWMOE_MM_MIN_ROWS", MM_PATHS[path])
    say("qmatmul", F.NAMES[dtype], n, k, m, path)
    rng = np.random.default_rng(n * 7 + k + m)
    raw = synth.random_blocks(dtype, n * k, rng)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = host(ops.QMatMul(ops.QTensor.from_blocks(raw, dtype, (n, k))).forward(dev(x)))
    want = O.qmatmul_f64(dtype, raw, n, k, x)
    err = O.rel_l2(y, want)
    say("  rel_l2", err)
    assert err <= REL_L2_GATE
    if path == "matvec":
        assert err <= REL_L2_F32


@pytest.mark.parametrize("m", [32, 512])
def test_qmatmul_split_sum_is_deterministic(m, monkeypatch):
    """Split over K, the dense GEMM's last split of each work item to finish adds the partial rows
    in split order, whichever split that is: two calls give the same bits, and the result is the
    oracle's at the fp16-activation bar."""
    monkeypatch.setenv("CWMOE_MM_MIN_ROWS", "1")
    say("qmatmul split sum", m)
    rng = np.random.default_rng(70 + m)
    n, k = 4096, 4096
    raw = synth.random_blocks(F.Q4_K, n * k, rng)
    x = rng.standard_normal((m, k)).astype(np.float32)
    qm = ops.QMatMul(ops.QTensor.from_blocks(raw, F.Q4_K, (n, k)))
    y1 = host(qm.forward(dev(x)))
    y2 = host(qm.forward(dev(x)))
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    assert O.rel_l2(y1, O.qmatmul_f64(F.Q4_K, raw, n, k, x)) <= REL_L2_GATE


@pytest.mark.parametrize("path", sorted(MM_PATHS))
def test_qmatmul_edge_scales(path, monkeypatch):
    # zero and subnormal f16 scales (and a zero dmin) take the kernels' zero-scale branches
    monkeypatch.setenv("CWMOE_MM_MIN_ROWS", MM_PATHS[path])
    rng = np.random.default_rng(77)
    for dtype, n, k, d_at in ((F.Q4_K, 64, 1024, 0), (F.Q8_0, 64, 512, 0), (F.Q2_K, 64, 1024, 80),
                              (F.IQ2_XXS, 64, 1024, 0), (F.IQ2_S, 64, 1024, 0), (F.IQ3_S, 64, 1024, 0)):
        raw = synth.random_blocks(dtype, n * k, rng).reshape(-1, F.type_size(dtype)).copy()
        raw[::3, d_at:d_at + 2] = 0                  # d = 0
        raw[1::5, d_at:d_at + 2] = [0x01, 0x00]      # smallest subnormal d
        if dtype in (F.Q4_K, F.Q2_K):
            raw[2::7, d_at + 2:d_at + 4] = 0         # dmin = 0
        raw = raw.reshape(-1)
        x = rng.standard_normal((48, k)).astype(np.float32)
        y = host(ops.QMatMul(ops.QTensor.from_blocks(raw, dtype, (n, k))).forward(dev(x)))
        want = O.qmatmul_f64(dtype, raw, n, k, x)
        err = O.rel_l2(y, want)
        say("edge scales", F.NAMES[dtype], path, err)
        assert err <= REL_L2_GATE


@pytest.mark.parametrize("path", sorted(MM_PATHS))
def test_qmatmul_mxfp4_exponents(path, monkeypatch):
    # e8m0 block scales from subnormal (e = 0, 1: 2^-128, 2^-127) to 2^23, mixed within rows: the
    # matvec path's scaled FP4 conversion and the MFMA path's exponents against the stage's largest
    # (a block 2^150 below it contributes nothing); the f64 oracle decodes with k_quants.rs:638-691
    monkeypatch.setenv("CWMOE_MM_MIN_ROWS", MM_PATHS[path])
    rng = np.random.default_rng(78)
    n, k = 64, 2880
    raw = synth.random_blocks(F.MXFP4, n * k, rng).reshape(-1, F.type_size(F.MXFP4)).copy()
    exps = np.array([0, 1, 2, 90, 120, 127, 140, 150], np.uint8)
    raw[:, 0] = exps[rng.integers(0, len(exps), raw.shape[0])]
    raw[::11, 1:] = 0x88                             # codes 8 (the i8 table's +0) in both nibbles
    raw = raw.reshape(-1)
    for m in (1, 40):
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = host(ops.QMatMul(ops.QTensor.from_blocks(raw, F.MXFP4, (n, k))).forward(dev(x)))
        want = O.qmatmul_f64(F.MXFP4, raw, n, k, x)
        err = O.rel_l2(y, want)
        say("mxfp4 exponents", path, m, err)
        assert np.all(np.isfinite(y))
        assert err <= REL_L2_GATE
        if path == "matvec":
            assert err <= REL_L2_F32


def test_grouped_gemm_mxfp4_exponents_across_stages():
    """The grouped MFMA GEMM runs a whole row of 90 MXFP4 blocks (12 stages) in one work item: its
    accumulators follow the largest block exponent seen so far, and rows whose e8m0 scales swing
    from 2^23 down to 2^-128 between stages stay finite (moving the accumulators up onto a smaller
    stage base overflowed f32). One expert, 40 picks, against the f64 oracle at the fp16 bar."""
    rng = np.random.default_rng(79)
    n, k, T = 64, 2880, 40
    raw = synth.random_blocks(F.MXFP4, n * k, rng).reshape(n, k // 32, F.type_size(F.MXFP4)).copy()
    raw[:, :, 0] = np.array([0, 1, 90, 150], np.uint8)[rng.integers(0, 4, raw.shape[:2])]
    raw[:, :8, 0] = 150                               # the first stage holds the row's largest scale
    raw = raw.reshape(-1)
    bank = ops.ExpertBank.from_blocks(raw, F.MXFP4, n, k, 1)
    mv = ops.MoeMatvec(bank, 1, False)
    assert T > mv.grouped_above
    x = rng.standard_normal((T, k)).astype(np.float32)
    out = host(mv.forward(dev(x), dev(np.zeros((T, 1), np.uint32))))[:, 0]
    want = O.qmatmul_f64(F.MXFP4, raw, n, k, x)
    assert np.all(np.isfinite(out))
    assert O.rel_l2(out, want) <= REL_L2_GATE


@pytest.mark.parametrize("k,T", [(2880, 40), (256, 24), (160, 17), (1056, 90)])
def test_mxfp4_grouped_scaled_and_fp16_paths(k, T, monkeypatch):
    """MXFP4 above 8 tokens runs on the block-scaled MFMA (FP4 weights as stored x three FP6
    activation terms); CWMOE_MXFP4_F16=1 selects the fp16 MFMA path. Both against the f64 oracle
    at the 1e-3 gate, on row lengths with a half step at the end (2880, 1056: K not a multiple of
    128), exactly two steps (256) and one step and a quarter (160), 1-6 token blocks per tile, an
    id past the bank giving a NaN row; the two paths' outputs differ (different arithmetic)."""
    rng = np.random.default_rng(k + T)
    n, slots, K = 96, 5, 4
    raw = synth.random_blocks(F.MXFP4, slots * n * k, rng)
    bank = ops.ExpertBank.from_blocks(raw, F.MXFP4, n, k, slots)
    ids = rng.integers(0, slots, size=(T, K), dtype=np.uint32)
    ids[1, 3] = slots + 2
    x = rng.standard_normal((T, k)).astype(np.float32)
    want = O.matvec_id(F.MXFP4, n, k, raw, bank.slot_stride, x, np.minimum(ids, slots - 1), False)
    outs = {}
    for path, env in (("scaled", "0"), ("fp16", "1")):
        monkeypatch.setenv("CWMOE_MXFP4_F16", env)
        out = host(ops.MoeMatvec(bank, K, False).forward(dev(x), dev(ids)))
        assert np.all(np.isnan(out[1, 3]))
        keep = np.ones((T, K), bool)
        keep[1, 3] = False
        err = O.rel_l2(out[keep], want[keep])
        say("  k", k, "T", T, path, "rel_l2", err)
        assert err <= REL_L2_GATE
        outs[path] = out[keep]
    assert not np.array_equal(outs["scaled"], outs["fp16"])


@pytest.mark.parametrize("off", [0, 4])
def test_qmatmul_q4k_few_rows_any_alignment(off, monkeypatch):
    """Q4_K at 2..16 rows of x on the MFMA path: a 16-byte aligned matrix takes the one-launch
    skinny GEMM (rows copied as 16-byte chunks), a matrix 4 bytes off alignment (a view into a
    larger buffer) the persistent GEMM; both against the oracle at the fp16-activation bar."""
    monkeypatch.setenv("CWMOE_MM_MIN_ROWS", "1")
    rng = np.random.default_rng(90 + off)
    n, k = 130, 1536
    raw = synth.random_blocks(F.Q4_K, n * k, rng)
    buf = torch.zeros(raw.size + 16, dtype=torch.uint8, device="cuda")
    buf[off:off + raw.size] = dev_u8(raw)
    w = buf[off:off + raw.size]
    assert w.data_ptr() % 16 == off
    for m in (2, 11, 16):
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = host(ops.QMatMul(ops.QTensor(w, F.Q4_K, (n, k))).forward(dev(x)))
        assert O.rel_l2(y, O.qmatmul_f64(F.Q4_K, raw, n, k, x)) <= REL_L2_GATE


def test_qmatmul_rejects_bad_shapes():
    qt = ops.QTensor.from_blocks(np.zeros(34 * 2, np.uint8), F.Q8_0, (1, 64))
    with pytest.raises(cw.CwError):
        ops.QMatMul(qt).forward(torch.zeros((2, 32), device="cuda"))


# ------------------------------------------------------------------------------ expert matvec

@pytest.mark.parametrize("dtype,n,k", [(F.IQ2_XXS, 512, 2048), (F.IQ2_S, 2048, 512), (F.Q4_K, 512, 2048),
                                       (F.IQ3_S, 512, 2048), (F.MXFP4, 256, 2880), (F.Q8_0, 128, 1024),
                                       (F.Q2_K, 2048, 512), (F.Q5_K, 512, 2048), (F.Q6_K, 2048, 512),
                                       (F.IQ3_XXS, 512, 2048), (F.IQ4_XS, 2048, 512)])
@pytest.mark.parametrize("rows_per_expert", [False, True])
def test_matvec_id_matches_the_oracle(dtype, n, k, rows_per_expert):
    say("matvec_id", F.NAMES[dtype], n, k, rows_per_expert)
    rng = np.random.default_rng(dtype * 31 + n)
    slots, T, K = 12, 3, 4
    raw = synth.random_blocks(dtype, slots * n * k, rng)
    bank = ops.ExpertBank.from_blocks(raw, dtype, n, k, slots)
    ids = rng.integers(0, slots, size=(T, K), dtype=np.uint32)
    x = rng.standard_normal((T * K if rows_per_expert else T, k)).astype(np.float32)
    out = host(ops.MoeMatvec(bank, K, rows_per_expert).forward(dev(x), dev(ids)))
    want = O.matvec_id(dtype, n, k, raw, bank.slot_stride, x, ids, rows_per_expert)
    err = O.rel_l2(out, want)
    say("  rel_l2", err)
    assert err <= REL_L2_F32


@pytest.mark.parametrize("dtype,n,k", [(F.IQ2_XXS, 512, 2048), (F.IQ2_S, 2048, 512), (F.Q4_K, 512, 2048),
                                       (F.IQ3_S, 512, 2048), (F.MXFP4, 256, 2880), (F.Q8_0, 128, 1056),
                                       (F.Q2_K, 2048, 512), (F.IQ3_XXS, 512, 2048), (F.IQ4_XS, 2048, 512)])
@pytest.mark.parametrize("rows_per_expert", [False, True])
def test_matmul_id_grouped_matches_the_oracle(dtype, n, k, rows_per_expert):
    """cw_matmul_id_grouped (the reference's matmul_id_piles, which MoeMatvec takes above 8 tokens):
    160 picks over 24 slots (one unused, one with a single pick, ragged piles), shared or per-pick
    activation rows, against the oracle's matvec_id at the fp16-activation bar; an id past the bank
    gives a NaN row and leaves the others alone."""
    say("matmul_id_grouped", F.NAMES[dtype], n, k, rows_per_expert)
    rng = np.random.default_rng(dtype * 37 + n)
    slots, T, K = 24, 40, 4
    raw = synth.random_blocks(dtype, slots * n * k, rng)
    bank = ops.ExpertBank.from_blocks(raw, dtype, n, k, slots)
    ids = rng.integers(0, slots - 2, size=(T, K), dtype=np.uint32)
    ids[7, 2] = slots - 1                                   # a pile of one
    x = rng.standard_normal((T * K if rows_per_expert else T, k)).astype(np.float32)
    mv = ops.MoeMatvec(bank, K, rows_per_expert)
    assert mv.grouped_above == 8
    out = host(mv.forward(dev(x), dev(ids)))
    want = O.matvec_id(dtype, n, k, raw, bank.slot_stride, x, ids, rows_per_expert)
    err = O.rel_l2(out, want)
    say("  rel_l2", err)
    assert err <= REL_L2_GATE
    assert err > REL_L2_F32 / 100          # the fp16-activation GEMM ran, not the f32 matvec
    bad = ids.copy()
    bad[3, 1] = slots + 5
    out2 = host(mv.forward(dev(x), dev(bad)))
    assert np.all(np.isnan(out2[3, 1]))
    keep = np.ones((T, K), bool)
    keep[3, 1] = False
    assert np.array_equal(out2[keep].view(np.uint32), out[keep].view(np.uint32))


def test_moe_matvec_grouped_takes_an_x_off_16_byte_alignment():
    """Above 8 tokens MoeMatvec takes the grouped GEMM, as the reference's matmul_id_piles takes
    any offset of x: an x view 4 bytes off 16-byte alignment (its packs read 16 bytes at a time,
    unaligned) against the oracle at the 1e-3 gate, equal to the same x at an aligned address."""
    rng = np.random.default_rng(41)
    n, k, slots, T, K = 64, 512, 6, 20, 4
    raw = synth.random_blocks(F.Q4_K, slots * n * k, rng)
    bank = ops.ExpertBank.from_blocks(raw, F.Q4_K, n, k, slots)
    ids = rng.integers(0, slots, size=(T, K), dtype=np.uint32)
    x = rng.standard_normal((T, k)).astype(np.float32)
    buf = torch.zeros(T * k + 4, dtype=torch.float32, device="cuda")
    buf[1:1 + T * k] = dev(x).reshape(-1)
    xv = buf[1:1 + T * k].view(T, k)
    assert xv.data_ptr() % 16 == 4
    mv = ops.MoeMatvec(bank, K, False)
    assert T > mv.grouped_above
    out = host(mv.forward(xv, dev(ids)))
    want = O.matvec_id(F.Q4_K, n, k, raw, bank.slot_stride, x, ids, False)
    assert O.rel_l2(out, want) <= REL_L2_GATE
    assert np.array_equal(out.view(np.uint32), host(mv.forward(dev(x), dev(ids))).view(np.uint32))


def test_matvec_id_marks_out_of_range_slots():
    rng = np.random.default_rng(2)
    raw = synth.random_blocks(F.Q8_0, 2 * 8 * 64, rng)
    bank = ops.ExpertBank.from_blocks(raw, F.Q8_0, 8, 64, 2)
    ids = np.array([[0, 5]], dtype=np.uint32)
    out = host(ops.MoeMatvec(bank, 2, False).forward(dev(rng.standard_normal((1, 64)).astype(np.float32)), dev(ids)))
    assert np.all(np.isfinite(out[0, 0])) and np.all(np.isnan(out[0, 1]))


# ------------------------------------------------------------------------------ routing

def test_route_reference_known_answers():
    # crates/engine/tests/router.rs:20-30, 56-60
    ids, _ = ops.route(dev(np.array([[0.1, 3.0, 2.0, -1.0, 1.0]], np.float32)), 3, True)
    assert host(ids).tolist() == [[1, 2, 4]]
    ids, _ = ops.route(dev(np.array([[5.0, 0.0, 1.0, 2.0], [0.0, 1.0, 9.0, 3.0]], np.float32)), 2, True)
    assert host(ids).tolist() == [[0, 3], [2, 3]]
    _, w = ops.route(dev(np.array([[0.0, 4.0, 1.0, 2.0, 3.0]], np.float32)), 4, True)
    w = host(w)[0]
    assert all(a >= b for a, b in zip(w, w[1:]))
    ids, _ = ops.route(dev(np.array([[1.0, 2.0, 2.0, 0.0, 2.0]], np.float32)), 3, False)
    assert host(ids).tolist() == [[1, 2, 4]]


def test_route_ties_across_signed_zero_and_slots():
    # -0 and +0 are equal logits: the stable argsort keeps index order among them; equal logits
    # in different 64-wide slots (index 3 and 131) and in the same lane (3 and 67) tie too
    lg = np.full((1, 256), -1.0, np.float32)
    lg[0, [3, 5, 10]] = [0.0, -0.0, 0.0]
    lg[0, [67, 131, 200]] = 2.5
    ids, w = ops.route(dev(lg), 5, True)
    wids, ww = O.route(lg, 5, True)
    assert wids.tolist() == [[67, 131, 200, 3, 5]]
    assert np.array_equal(host(ids).view(np.uint32), wids)
    assert np.max(np.abs(host(w) - ww)) < 1e-6
    # ties in every round: 9 equal maxima, K = 8 takes the 8 lowest indices
    lg = np.zeros((2, 512), np.float32)
    lg[:, ::57] = 1.0
    ids, _ = ops.route(dev(lg), 8, False)
    assert host(ids).tolist() == [list(range(0, 57 * 8, 57))] * 2
    # eight logits per lane (E in 257..512, last lanes partly empty): equal maxima inside one
    # lane's sorted list (9, 13, 15) and across lanes (300), and -0 / +0 in one lane (16, 17)
    lg = np.full((1, 400), -2.0, np.float32)
    lg[0, [15, 13, 9, 300, 301]] = 3.0
    lg[0, [17, 16]] = [-0.0, 0.0]
    ids, w = ops.route(dev(lg), 7, True)
    wids, ww = O.route(lg, 7, True)
    assert wids.tolist() == [[9, 13, 15, 300, 301, 16, 17]]
    assert np.array_equal(host(ids).view(np.uint32), wids)
    assert np.max(np.abs(host(w) - ww)) < 1e-6


@pytest.mark.parametrize("E,K,norm", [(256, 8, True), (128, 4, True), (512, 10, True), (1024, 32, False), (20, 20, True)])
def test_route_matches_the_oracle(E, K, norm):
    rng = np.random.default_rng(E + K)
    T = 200
    logits = rng.standard_normal((T, E)).astype(np.float32)
    assert not synth.near_ties_within_top_k(logits, K)
    ids, w = ops.route(dev(logits), K, norm)
    wids, ww = O.route(logits, K, norm)
    assert np.array_equal(host(ids).view(np.uint32), wids)
    assert np.max(np.abs(host(w) - ww)) < 1e-5


# ------------------------------------------------------------------------------ router logits

@pytest.mark.parametrize("wdt", ["f32", "f16"])
@pytest.mark.parametrize("E,h,T", [(256, 2048, 1), (128, 2880, 3), (512, 2048, 8), (256, 2048, 9), (130, 68, 70),
                                   (256, 2048, 1500)])
def test_router_logits_match_f64(wdt, E, h, T):
    say("router logits", wdt, E, h, T)
    rng = np.random.default_rng(E * 7 + T)
    w = (rng.standard_normal((E, h)) * 0.05).astype(np.float32 if wdt == "f32" else np.float16)
    x = rng.standard_normal((T, h)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if T % 2 else None
    got = host(ops.router_logits(dev(w), dev(x), None if bias is None else dev(bias)))
    want = x.astype(np.float64) @ w.astype(np.float64).T + (0.0 if bias is None else bias.astype(np.float64))
    # f32 accumulation of up to 2,880 products: rel-L2 near 1e-7
    assert np.linalg.norm(got - want) <= 2e-6 * np.linalg.norm(want)


@pytest.mark.parametrize("T", [2, 100])
def test_router_logits_exact_on_small_integers(T):
    # integers in [-8, 8]: every product and partial sum is an integer below 2^24, exact in f32
    # whatever the summation order, so both kernels must return the exact dot products
    rng = np.random.default_rng(T)
    E, h = 96, 2048
    w = rng.integers(-8, 9, (E, h)).astype(np.float16)
    x = rng.integers(-8, 9, (T, h)).astype(np.float32)
    bias = rng.integers(-4, 5, E).astype(np.float32)
    got = host(ops.router_logits(dev(w), dev(x), dev(bias)))
    want = (x.astype(np.int64) @ w.astype(np.int64).T + bias.astype(np.int64)).astype(np.float32)
    assert np.array_equal(got, want)


def test_router_logits_reject_bad_inputs():
    x = torch.zeros((2, 64), device="cuda")
    with pytest.raises(cw.CwError):
        ops.router_logits(torch.zeros((8, 60), device="cuda"), x)                     # width mismatch
    with pytest.raises(cw.CwError):
        ops.router_logits(torch.zeros((8, 64), dtype=torch.bfloat16, device="cuda"), x)  # dtype
    with pytest.raises(cw.CwError):
        ops.router_logits(torch.zeros((8, 66), device="cuda"), torch.zeros((2, 66), device="cuda"))  # hidden % 4


# ------------------------------------------------------------------------------ shared expert

@pytest.mark.parametrize("fmt,T,gated,acc", [((F.Q4_K, F.Q4_K, F.Q8_0), 1, True, False),
                                             ((F.IQ3_S, F.IQ3_S, F.Q4_K), 3, True, True),
                                             ((F.Q8_0, F.Q8_0, F.MXFP4), 40, False, True),
                                             ((F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), 24, True, False)])
def test_shared_expert_matches_the_oracle(fmt, T, gated, acc):
    # out = sigmoid(x . gate_inp) * down(silu(gate x) * up x) (+ out), model_next.rs:733-741
    say("shared expert", [F.NAMES[f] for f in fmt], T, gated, acc)
    rng = np.random.default_rng(T * 31 + fmt[0])
    h, inter = 2048, 512
    shapes = ((inter, h), (inter, h), (h, inter))
    raw = [synth.random_blocks(f, n * k, rng) for f, (n, k) in zip(fmt, shapes)]
    qs = [ops.QTensor.from_blocks(r, f, shp) for r, f, shp in zip(raw, fmt, shapes)]
    gi = (rng.standard_normal(h) * 0.02).astype(np.float32) if gated else None
    x = rng.standard_normal((T, h)).astype(np.float32)
    base = rng.standard_normal((T, h)).astype(np.float32)
    se = ops.SharedExpert(*qs, None if gi is None else dev(gi))
    out = dev(base) if acc else None
    got = host(se.forward(dev(x), out))
    W = [O.dequantize(f, r, n * k).reshape(n, k).astype(np.float64) for f, r, (n, k) in zip(fmt, raw, shapes)]
    x64 = x.astype(np.float64)
    g, u = x64 @ W[0].T, x64 @ W[1].T
    y = (g / (1.0 + np.exp(-g)) * u) @ W[2].T
    if gated:
        y *= (1.0 / (1.0 + np.exp(-(x64 @ gi.astype(np.float64)))))[:, None]
    if acc:
        y += base
    # the dense matmuls run on fp16 activations from 2 rows (Q4_K) or 8 rows: the 1e-3 gate;
    # one f32 token must also meet the f32 bar
    tol = REL_L2_F32 if T == 1 else REL_L2_GATE
    assert np.linalg.norm(got - y) <= tol * np.linalg.norm(y)


# ------------------------------------------------------------------------------ elementwise

def test_activations_combine_and_resolve_match_the_oracle():
    rng = np.random.default_rng(8)
    g = (rng.standard_normal((64, 96)) * 6).astype(np.float32)
    u = (rng.standard_normal((64, 96)) * 6).astype(np.float32)
    h = host(ops.swiglu(dev(g), dev(u)))
    assert np.allclose(h, O.silu_mul(g, u), rtol=2e-6, atol=1e-6)
    ids = rng.integers(0, 5, size=64, dtype=np.uint32)
    gb = rng.normal(0, 0.5, (5, 96)).astype(np.float32)
    ub = rng.normal(0, 0.5, (5, 96)).astype(np.float32)
    hc = host(ops.clamped_swiglu(dev(g), dev(u), dev(gb), dev(ub), dev(ids), pad=128))
    assert np.allclose(hc, O.clamped_swiglu(g, u, gb, ub, ids, pad=128), rtol=2e-6, atol=1e-6)
    down = rng.standard_normal((6, 4, 80)).astype(np.float32)
    wts = rng.random((6, 4)).astype(np.float32)
    assert np.allclose(host(ops.weighted_sum(dev(down), dev(wts))), O.weighted_sum(down, wts), rtol=1e-6, atol=1e-6)
    table = np.array([3, 0xFFFFFFFF, 1, 0xFFFFFFFF, 2], dtype=np.uint32)
    pick = np.array([[0, 1], [2, 3], [4, 0]], dtype=np.uint32)
    slots, missing = ops.slots_resolve(dev(pick), dev(table))
    ws, wm = O.resolve(pick, table)
    assert host(slots).view(np.uint32).reshape(-1).tolist() == ws.tolist() and int(host(missing)[0]) == wm


# ------------------------------------------------------------------------------ MoE layer

def upload_layer(layer, slot_table=None):
    banks = []
    shapes = [(layer.inter, layer.hidden), (layer.inter, layer.hidden), (layer.hidden, max(layer.pad, layer.inter))]
    for m in range(3):
        n, k = shapes[m]
        banks.append(ops.ExpertBank.from_blocks(layer.host[m], layer.dtypes[m], n, k, layer.n_slots))
    act = ops.ExpertAct.silu()
    if layer.act == 1:
        act = ops.ExpertAct.clamped_swiglu(layer.alpha, layer.limit, *[dev(b) for b in layer.bias], pad=layer.pad)
    table = None if slot_table is None else dev(slot_table)
    return ops.MoeLayer(*banks, n_experts=layer.n_experts, top_k=layer.top_k, norm_topk_prob=layer.norm, act=act,
                        slot_table=table)


MOE_CASES = [
    # name, E, K, h, I, dtypes, act, pad, T
    ("c3_decode", 256, 8, 2048, 512, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), 0, 0, 1),
    ("c3_tokens", 256, 8, 2048, 512, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), 0, 0, 24),
    ("c3_prefill_piece", 256, 8, 2048, 512, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), 0, 0, 160),
    ("c3_mixed_gate_up", 64, 8, 2048, 512, (F.IQ2_XXS, F.IQ2_S, F.IQ2_S), 0, 0, 3),
    ("iq2_xxs_decode", 64, 8, 2048, 512, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_XXS), 0, 0, 1),  # its own decode instance
    ("iq2_s_decode_e512", 512, 8, 2048, 512, (F.IQ2_S, F.IQ2_S, F.IQ2_S), 0, 0, 1),  # 8 logits per lane, one router wave
    ("c4_decode_shape", 16, 4, 2880, 2880, (F.MXFP4, F.MXFP4, F.MXFP4), 1, 0, 1),
    ("c4_decode_e128", 128, 4, 2880, 2880, (F.MXFP4, F.MXFP4, F.MXFP4), 1, 0, 1),  # config 4's routing width
    ("c4_decode_top5", 32, 5, 2880, 2880, (F.MXFP4, F.MXFP4, F.MXFP4), 1, 0, 1),  # 3-4 gate/up items per wave
    ("c4_decode_odd_rows", 16, 4, 2880, 2877, (F.MXFP4, F.MXFP4, F.MXFP4), 1, 2880, 1),  # a last item of one row, padded hidden
    ("c4_prefill_shape", 16, 4, 2880, 2880, (F.MXFP4, F.MXFP4, F.MXFP4), 1, 0, 40),
    ("c4_padded", 16, 4, 1024, 720, (F.MXFP4, F.MXFP4, F.Q4_K), 1, 768, 5),
    ("iq3_s_grouped", 32, 6, 1024, 512, (F.IQ3_S, F.IQ3_S, F.IQ3_S), 0, 0, 48),
    ("iq2_s_grouped_padded", 16, 4, 512, 200, (F.IQ2_S, F.IQ2_S, F.IQ2_XXS), 1, 256, 20),
    ("c5_shrunk_q2_k", 64, 10, 2048, 512, (F.Q2_K, F.Q2_K, F.Q2_K), 0, 0, 1),
    ("q2_k_gate_up_tokens", 32, 4, 1024, 512, (F.Q2_K, F.Q2_K, F.Q4_K), 0, 0, 24),
    ("q2_k_grouped", 32, 4, 1024, 512, (F.Q2_K, F.Q2_K, F.Q2_K), 0, 0, 56),
    ("q2_k_top10_tokens", 64, 10, 1024, 512, (F.Q2_K, F.Q2_K, F.Q2_K), 0, 0, 24),  # the combine's picks in chunks 4, 4, 2
    ("iq2_s_top6_biases", 32, 6, 1024, 512, (F.IQ2_S, F.IQ2_S, F.IQ2_S), 1, 0, 24),  # down biases over a partial chunk
    ("iq3_xxs_iq4_xs", 32, 6, 1024, 512, (F.IQ3_XXS, F.IQ3_XXS, F.IQ4_XS), 0, 0, 3),
    ("iq3_xxs_iq4_xs_tokens", 32, 6, 1024, 512, (F.IQ3_XXS, F.IQ3_XXS, F.IQ4_XS), 0, 0, 40),
    ("q5_k_q6_k", 16, 4, 1024, 512, (F.Q5_K, F.Q5_K, F.Q6_K), 0, 0, 2),
    ("q6_k_q5_k_tokens", 16, 4, 1024, 512, (F.Q6_K, F.Q6_K, F.Q5_K), 0, 0, 24),
]

# the grouped MFMA path rounds activations to fp16 once (2^-11 relative): its outputs are held
# to the 1e-3 gate; the matvec path keeps f32 activations and is held to the f32 bar as well
PATHS = {"gemv": "100000", "grouped": "1"}


@pytest.mark.parametrize("path", sorted(PATHS))
@pytest.mark.parametrize("name,E,K,h,I,dts,act,pad,T", MOE_CASES, ids=[c[0] for c in MOE_CASES])
def test_moe_layer_matches_the_oracle(name, E, K, h, I, dts, act, pad, T, path, monkeypatch):
    monkeypatch.setenv("CWMOE_PREFILL_MIN_TOKENS", PATHS[path])
    say("moe", name, path)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    layer = synth.moe_weights(E, K, h, I, dts, rng, act=act, pad=pad)
    x = rng.standard_normal((T, h)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    assert not synth.near_ties_within_top_k(logits, K)
    moe = upload_layer(layer)
    out, ids, w = moe.forward(dev(x), dev(logits))
    want, wids, ww, _ = O.moe_layer(layer, x, logits)
    assert np.array_equal(host(ids).view(np.uint32), wids)
    assert np.max(np.abs(host(w) - ww)) < 1e-5
    err = O.rel_l2(host(out), want)
    say("  rel_l2", err)
    assert err <= REL_L2_GATE
    grouped = path == "grouped" and dts[0] == dts[1] and all(d in MFMA_TYPES for d in (dts[0], dts[2]))
    if not grouped:
        assert err <= REL_L2_F32


def test_moe_layer_through_a_slot_table():
    # config 5's shape on one layer: 512 experts, top-10, 56 resident slots, IQ3_S / Q4_K mix
    say("moe bank")
    rng = np.random.default_rng(55)
    E, K, slots = 512, 10, 56
    layer = synth.moe_weights(E, K, 2048, 512, (F.IQ3_S, F.IQ3_S, F.Q4_K), rng, n_slots=slots)
    table = np.full(E, 0xFFFFFFFF, dtype=np.uint32)
    resident = rng.choice(E, size=slots, replace=False)
    table[resident] = rng.permutation(slots).astype(np.uint32)
    mask = np.full(E, -1e30, dtype=np.float32)
    mask[resident] = 0.0
    x = rng.standard_normal((2, 2048)).astype(np.float32)
    logits = rng.standard_normal((2, E)).astype(np.float32) + mask
    moe = upload_layer(layer, slot_table=table)
    missing = torch.zeros(1, dtype=torch.int32, device="cuda")
    out, ids, w = moe.forward(dev(x), dev(logits), missing=missing)
    want, wids, ww, wmiss = O.moe_layer(layer, x, logits, slot_table=table, n_slots=slots)
    assert wmiss == 0 and int(host(missing)[0]) == 0
    assert np.array_equal(host(ids).view(np.uint32), wids)
    assert O.rel_l2(host(out), want) <= REL_L2_F32
    # unmasked logits pick absent experts: they read slot 0 and are counted, as the oracle does
    logits2 = rng.standard_normal((2, E)).astype(np.float32)
    missing.zero_()
    out2, _, _ = moe.forward(dev(x), dev(logits2), missing=missing)
    want2, _, _, wmiss2 = O.moe_layer(layer, x, logits2, slot_table=table, n_slots=slots)
    assert int(host(missing)[0]) == wmiss2 > 0
    assert O.rel_l2(host(out2), want2) <= REL_L2_F32


@pytest.mark.parametrize("path", sorted(PATHS))
@pytest.mark.parametrize("dts,x_scale", [((F.MXFP4,) * 3, 1.0), ((F.Q4_K, F.Q4_K, F.IQ4_XS), 2.0 ** -8)],
                         ids=["mxfp4", "q4_k"])
def test_moe_biases_follow_the_expert_through_a_slot_table(dts, x_scale, path, monkeypatch):
    # clamped SwiGLU's biases are per expert while the weights are per slot: a permuted table
    # catches a bias read by slot (or by tile) instead of by the picked expert. The synthetic
    # Q4_K rows are large; unscaled x puts the gate/up sums in the thousands, where rounding x to
    # fp16 alone moves the clamped SwiGLU by ~1e-3, so x is scaled down (and kept fp16-exact)
    monkeypatch.setenv("CWMOE_PREFILL_MIN_TOKENS", PATHS[path])
    say("moe bias slots", dts[0], path)
    rng = np.random.default_rng(91)
    E, K, slots, h, I, T = 48, 4, 20, 1024, 512, 40
    layer = synth.moe_weights(E, K, h, I, dts, rng, n_slots=slots, act=1)
    layer.bias = [b * 50.0 for b in layer.bias]  # large enough that a wrong row moves the output
    table = np.full(E, 0xFFFFFFFF, dtype=np.uint32)
    resident = rng.choice(E, size=slots, replace=False)
    table[resident] = rng.permutation(slots).astype(np.uint32)
    mask = np.full(E, -1e30, dtype=np.float32)
    mask[resident] = 0.0
    x = (rng.standard_normal((T, h)) * x_scale).astype(np.float16).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32) + mask
    assert not synth.near_ties_within_top_k(logits, K)
    moe = upload_layer(layer, slot_table=table)
    out, ids, _ = moe.forward(dev(x), dev(logits))
    want, wids, _, wmiss = O.moe_layer(layer, x, logits, slot_table=table, n_slots=slots)
    assert wmiss == 0
    assert np.array_equal(host(ids).view(np.uint32), wids)
    err = O.rel_l2(host(out), want)
    say("  rel_l2", err)
    assert err <= REL_L2_GATE
    # the same layer with the biases of two resident experts swapped must not match
    swapped = list(layer.bias)
    a, b = resident[:2]
    for m in range(3):
        s = swapped[m].copy()
        s[[a, b]] = s[[b, a]]
        swapped[m] = s
    layer.bias = swapped
    other, _, _, _ = O.moe_layer(layer, x, logits, slot_table=table, n_slots=slots)
    assert O.rel_l2(host(out), other) > 10 * REL_L2_GATE


# ------------------------------------------------------------------------------ MXFP4 in row groups of 16

@pytest.mark.parametrize("n,k", [(41, 2880), (96, 1056), (15, 160)])
def test_rows16_repack_is_the_block_permutation(n, k):
    # cw_repack_rows16 against the permutation on the host: block b of row r at rows16_offset(r, b),
    # rows past n to the group's end zero blocks; three slots with a source stride above the matrix
    say("rows16 repack", n, k)
    rng = np.random.default_rng(n + k)
    nb, slots = k // 32, 3
    src_stride = F.matrix_bytes(F.MXFP4, n, k) + 48
    raw = np.full((slots, src_stride), 0xA5, np.uint8)
    raw[:, :n * nb * 17] = synth.random_blocks(F.MXFP4, slots * n * k, rng).reshape(slots, -1)
    raw = raw.reshape(-1)
    bank = ops.ExpertBank(dev(raw), F.MXFP4, n, k, slots, src_stride)
    got = host(bank.rows16().data)
    stride = F.matrix_bytes(F.MXFP4_R16, n, k)
    assert got.size == slots * stride
    want = np.zeros(slots * stride, np.uint8)
    for s in range(slots):
        blocks = raw[s * src_stride:s * src_stride + n * nb * 17].reshape(n, nb, 17)
        for r in range(n):
            for b in range(nb):
                o = s * stride + F.rows16_offset(r, b, nb)
                want[o:o + 17] = blocks[r, b]
    assert np.array_equal(got, want)


R16_CASES = [
    # name, E, K, h, I, pad, T: one token takes the one-launch decode (the gpt-oss row length), a few
    # the per-pick matvecs, more the grouped GEMMs
    ("c4_decode", 16, 4, 2880, 2880, 0, 1),
    ("c4_decode_e128", 128, 4, 2880, 2880, 0, 1),
    ("c4_decode_odd_rows", 16, 4, 2880, 2877, 2880, 1),
    ("c4_decode_top5", 32, 5, 2880, 2880, 0, 1),       # 900 block items: more than one round of the grid
    ("c4_decode_silu", 16, 4, 2880, 2880, 0, 1),       # SiLU, no biases
    ("c4_few_tokens", 16, 4, 2880, 2880, 0, 5),
    ("c4_tokens", 16, 4, 2880, 2880, 0, 40),
    ("c4_odd_rows_tokens", 16, 4, 2880, 2877, 2880, 24),
    ("short_rows_one_token", 16, 4, 1024, 512, 0, 1),   # no decode instance: the matvecs
    ("short_rows", 32, 6, 1024, 720, 768, 33),
]


@pytest.mark.parametrize("which", ["all", "down"])
@pytest.mark.parametrize("name,E,K,h,I,pad,T", R16_CASES, ids=[c[0] for c in R16_CASES])
def test_moe_layer_rows16_matches_gguf_rows(name, E, K, h, I, pad, T, which):
    # the same layer from GGUF rows and with its matrices (all three, or down alone) in row groups
    # of 16, against the oracle at the gate: the same blocks in the same order give the same bits,
    # except in the one-launch decode with gate/up in row groups (K-split, its own f32 order: held
    # to the f32 bar)
    say("moe rows16", name, which)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    layer = synth.moe_weights(E, K, h, I, (F.MXFP4,) * 3, rng, act=0 if "silu" in name else 1, pad=pad)
    x = rng.standard_normal((T, h)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    assert not synth.near_ties_within_top_k(logits, K)
    rows = upload_layer(layer)
    banks = [b.rows16() if which == "all" or m == 2 else b for m, b in enumerate(rows.banks)]
    rp = ops.MoeLayer(*banks, n_experts=E, top_k=K, norm_topk_prob=layer.norm, act=rows.act)
    want, wids, _, _ = O.moe_layer(layer, x, logits)
    op, idsp, _ = rp.forward(dev(x), dev(logits))
    assert np.array_equal(host(idsp).view(np.uint32), wids)
    err = O.rel_l2(host(op), want)
    say("  rel_l2", err)
    assert err <= REL_L2_GATE
    o, _, _ = rows.forward(dev(x), dev(logits))
    if T == 1 and h == 2880 and which == "all":
        assert err <= REL_L2_F32
    else:
        assert np.array_equal(host(o).view(np.uint32), host(op).view(np.uint32))


@pytest.mark.parametrize("T", [1, 24])
def test_moe_layer_rows16_through_a_slot_table(T):
    # row groups of 16 in a bank of fewer slots than experts (slot-major, permuted table, biases
    # per expert): the decode (T = 1) and the grouped GEMMs against the oracle and the GGUF rows
    say("moe rows16 slots", T)
    rng = np.random.default_rng(95 + T)
    E, K, slots, h, I = 48, 4, 20, 2880, 2880
    layer = synth.moe_weights(E, K, h, I, (F.MXFP4,) * 3, rng, n_slots=slots, act=1)
    table = np.full(E, 0xFFFFFFFF, dtype=np.uint32)
    resident = rng.choice(E, size=slots, replace=False)
    table[resident] = rng.permutation(slots).astype(np.uint32)
    mask = np.full(E, -1e30, dtype=np.float32)
    mask[resident] = 0.0
    x = rng.standard_normal((T, h)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32) + mask
    assert not synth.near_ties_within_top_k(logits, K)
    rows = upload_layer(layer, slot_table=table)
    r16 = ops.MoeLayer(*[b.rows16() for b in rows.banks], n_experts=E, top_k=K, norm_topk_prob=layer.norm,
                       act=rows.act, slot_table=dev(table))
    want, wids, _, wmiss = O.moe_layer(layer, x, logits, slot_table=table, n_slots=slots)
    out, ids, _ = r16.forward(dev(x), dev(logits))
    assert wmiss == 0 and np.array_equal(host(ids).view(np.uint32), wids)
    err = O.rel_l2(host(out), want)
    assert err <= REL_L2_GATE
    if T == 1:  # the K-split decode: its own f32 order
        assert err <= REL_L2_F32
    else:
        o, _, _ = rows.forward(dev(x), dev(logits))
        assert np.array_equal(host(o).view(np.uint32), host(out).view(np.uint32))


@pytest.mark.parametrize("T", [40, 5])
def test_matmul_id_grouped_rows16_matches_gguf_rows(T):
    # cw_matmul_id_grouped on an MXFP4_R16 bank (every token count: it has no matvec): the same bits
    # as the GGUF bank on the grouped path, an id past the bank giving a NaN row
    rng = np.random.default_rng(400 + T)
    n, k, slots, K = 200, 2880, 6, 4
    raw = synth.random_blocks(F.MXFP4, slots * n * k, rng)
    bank = ops.ExpertBank.from_blocks(raw, F.MXFP4, n, k, slots)
    ids = rng.integers(0, slots, size=(T, K), dtype=np.uint32)
    ids[1, 2] = slots + 1
    x = rng.standard_normal((T, k)).astype(np.float32)
    outp = host(ops.MoeMatvec(bank.rows16(), K, False).forward(dev(x), dev(ids)))
    out = host(ops.MoeMatvec(bank, K, False, grouped_above=0).forward(dev(x), dev(ids)))
    assert np.all(np.isnan(outp[1, 2]))
    assert np.array_equal(outp.view(np.uint32), out.view(np.uint32))
    keep = np.ones((T, K), bool)
    keep[1, 2] = False
    want = O.matvec_id(F.MXFP4, n, k, raw, bank.slot_stride, x, np.minimum(ids, slots - 1), False)
    assert O.rel_l2(outp[keep], want[keep]) <= REL_L2_GATE


@pytest.mark.parametrize("E", [512, 400])
def test_moe_decode_through_a_slot_table(E):
    """Config 5's one-token layer: the persistent decode kernel with 8 router logits per lane, where
    one wave per block routes and hands the picks to the block (E = 512; E = 400 leaves the top
    lanes partly filled). Top-10, 56 resident slots, IQ3_S gate/up and Q4_K down. Masked logits:
    ids, weights and output equal the oracle's, nothing missing; unmasked logits: absent experts
    read slot 0 and are counted, as the oracle does."""
    say("moe decode bank", E)
    rng = np.random.default_rng(500 + E)
    K, slots = 10, 56
    layer = synth.moe_weights(E, K, 2048, 512, (F.IQ3_S, F.IQ3_S, F.Q4_K), rng, n_slots=slots)
    table = np.full(E, 0xFFFFFFFF, dtype=np.uint32)
    resident = rng.choice(E, size=slots, replace=False)
    table[resident] = rng.permutation(slots).astype(np.uint32)
    mask = np.full(E, -1e30, dtype=np.float32)
    mask[resident] = 0.0
    moe = upload_layer(layer, slot_table=table)
    missing = torch.zeros(1, dtype=torch.int32, device="cuda")
    for trial in range(3):
        x = rng.standard_normal((1, 2048)).astype(np.float32)
        logits = rng.standard_normal((1, E)).astype(np.float32) + mask
        assert not synth.near_ties_within_top_k(logits, K)
        missing.zero_()
        out, ids, w = moe.forward(dev(x), dev(logits), missing=missing)
        want, wids, ww, wmiss = O.moe_layer(layer, x, logits, slot_table=table, n_slots=slots)
        assert wmiss == 0 and int(host(missing)[0]) == 0
        assert np.array_equal(host(ids).view(np.uint32), wids)
        assert np.max(np.abs(host(w) - ww)) < 1e-5
        err = O.rel_l2(host(out), want)
        say("  masked", trial, err)
        assert err <= REL_L2_F32
    x = rng.standard_normal((1, 2048)).astype(np.float32)
    logits = rng.standard_normal((1, E)).astype(np.float32)
    assert not synth.near_ties_within_top_k(logits, K)
    missing.zero_()
    out, ids, w = moe.forward(dev(x), dev(logits), missing=missing)
    want, wids, ww, wmiss = O.moe_layer(layer, x, logits, slot_table=table, n_slots=slots)
    assert int(host(missing)[0]) == wmiss > 0
    assert np.array_equal(host(ids).view(np.uint32), wids)
    err = O.rel_l2(host(out), want)
    say("  unmasked, missing", wmiss, err)
    assert err <= REL_L2_F32


def test_moe_decode_barrier_gives_up_without_hanging(monkeypatch):
    """The one-token layer's device-wide barrier waits a bounded number of polls. With the bound
    forced to 0 from the host, every block that does not arrive last gives up at once: the call
    completes, its outputs are NaN where a block gave up, and the device error count grows. Every
    block still arrives, so the sync state in the workspace is back at zero: the next call on the
    same workspace, with the default bound, matches the oracle."""
    say("moe decode barrier give-up")
    rng = np.random.default_rng(91)
    E, K = 256, 8
    layer = synth.moe_weights(E, K, 2048, 512, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), rng)
    moe = upload_layer(layer)
    x = rng.standard_normal((1, 2048)).astype(np.float32)
    logits = rng.standard_normal((1, E)).astype(np.float32)
    want, _, _, _ = O.moe_layer(layer, x, logits)
    out, _, _ = moe.forward(dev(x), dev(logits))
    assert O.rel_l2(host(out), want) <= REL_L2_F32
    before, st_before = cw.lib().cw_device_errors(), moe.status()
    monkeypatch.setenv("CWMOE_BARRIER_POLLS", "0")
    out, _, _ = moe.forward(dev(x), dev(logits))
    got = host(out)
    st_after = moe.status()  # the workspace's status word, no device synchronize needed
    after = cw.lib().cw_device_errors()
    monkeypatch.delenv("CWMOE_BARRIER_POLLS")
    say("  errors", before, "->", after, "status", st_before, "->", st_after, "NaN outputs", int(np.isnan(got).sum()))
    assert after > before
    assert st_after - st_before == after - before
    assert np.isnan(got).any()
    out, _, _ = moe.forward(dev(x), dev(logits))
    assert O.rel_l2(host(out), want) <= REL_L2_F32
    assert cw.lib().cw_device_errors() == after and moe.status() == st_after


@pytest.mark.parametrize("how", ["foreign_bytes", "counter_past_its_blocks"])
def test_moe_decode_refuses_a_sync_state_that_is_not_its_own(how):
    """The one-token layer's sync state must start zero-filled and then belong to the layer's
    calls. Foreign bytes over the state region (as a pooled buffer would leave) are refused at
    launch: no counter is used, the outputs are NaN, and the status word and the device error
    count grow. A counter already past its block count (state not zeroed) is caught at arrival,
    with NaN outputs. Zero-filling the region again restores the layer."""
    say("moe decode state", how)
    rng = np.random.default_rng(93)
    E, K = 256, 8
    layer = synth.moe_weights(E, K, 2048, 512, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), rng)
    moe = upload_layer(layer)
    x = rng.standard_normal((1, 2048)).astype(np.float32)
    logits = rng.standard_normal((1, E)).astype(np.float32)
    want, _, _, _ = O.moe_layer(layer, x, logits)
    out, _, _ = moe.forward(dev(x), dev(logits))
    assert O.rel_l2(host(out), want) <= REL_L2_F32
    state = moe._ws[:cw.CW_MOE_STATE_BYTES]
    if how == "foreign_bytes":
        state[:cw.CW_MOE_STATUS_OFFSET] = 0x5A       # the status word itself left as it is
    else:
        state[:4] = torch.tensor([1000], dtype=torch.int32).view(torch.uint8).cuda()  # arrival counter 0
    torch.cuda.synchronize()
    before, st_before = cw.lib().cw_device_errors(), moe.status()
    out, _, _ = moe.forward(dev(x), dev(logits))
    got = host(out)
    after, st_after = cw.lib().cw_device_errors(), moe.status()
    say("  errors", before, "->", after, "status", st_before, "->", st_after, "NaN", int(np.isnan(got).sum()))
    assert np.isnan(got).any() and after > before and st_after > st_before
    state[:cw.CW_MOE_STATUS_OFFSET] = 0
    out, _, _ = moe.forward(dev(x), dev(logits))
    assert O.rel_l2(host(out), want) <= REL_L2_F32
    assert cw.lib().cw_device_errors() == after


@pytest.mark.parametrize("path,T,shape", [("gemv", 1, "iq2"), ("gemv", 40, "iq2"), ("grouped", 40, "iq2"),
                                          ("gemv", 1, "mxfp4"), ("grouped", 40, "mxfp4")])
def test_moe_layer_marks_out_of_range_slots(path, T, shape, monkeypatch):
    """A slot table entry past the bank (a corrupt table) is rejected on the device on every path:
    the tokens that pick that expert get NaN outputs (the one-token decode, the two-kernel matvec
    path, and the grouped path, where such a pick is in no pile), the other tokens match the
    oracle run on the intact table. The MXFP4 shape takes the decode instance whose gate/up rows
    go through LDS."""
    monkeypatch.setenv("CWMOE_PREFILL_MIN_TOKENS", PATHS[path])
    say("moe out-of-range slot", path, T, shape)
    rng = np.random.default_rng(93 + T)
    if shape == "iq2":
        E, K, h, I, dts, act = 64, 4, 2048, 512, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), 0
    else:
        E, K, h, I, dts, act = 16, 4, 2880, 2880, (F.MXFP4,) * 3, 1
    layer = synth.moe_weights(E, K, h, I, dts, rng, act=act)
    table = np.arange(E, dtype=np.uint32)
    x = rng.standard_normal((T, h)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    want, wids, _, _ = O.moe_layer(layer, x, logits, slot_table=table, n_slots=E)
    table[wids[0, 1]] = E + 3
    moe = upload_layer(layer, slot_table=table)
    got = host(moe.forward(dev(x), dev(logits))[0])
    hit = np.any(wids == wids[0, 1], axis=1)
    assert hit[0] and np.all(np.isnan(got[hit]))
    assert np.all(np.isfinite(got[~hit]))
    if (~hit).any():
        assert O.rel_l2(got[~hit], want[~hit]) <= REL_L2_GATE


def test_moe_decode_with_x_off_16_byte_alignment():
    """The MXFP4 one-token layer copies x in 16-byte chunks; an x that starts 4 bytes past such a
    boundary takes the two-kernel path, with the same result."""
    say("moe decode, x at a 4-byte offset")
    rng = np.random.default_rng(77)
    E, K = 16, 4
    layer = synth.moe_weights(E, K, 2880, 2880, (F.MXFP4,) * 3, rng, act=1)
    x = rng.standard_normal((1, 2880)).astype(np.float32)
    logits = rng.standard_normal((1, E)).astype(np.float32)
    want, wids, _, _ = O.moe_layer(layer, x, logits)
    moe = upload_layer(layer)
    xs = torch.zeros(2881, dtype=torch.float32, device="cuda")
    xs[1:] = dev(x).reshape(-1)
    xo = xs[1:].reshape(1, 2880)
    assert xo.data_ptr() % 16 == 4
    out, ids, _ = moe.forward(xo, dev(logits))
    aligned, _, _ = moe.forward(dev(x), dev(logits))
    assert np.array_equal(host(ids).view(np.uint32), wids)
    assert O.rel_l2(host(out), want) <= REL_L2_F32
    assert O.rel_l2(host(aligned), want) <= REL_L2_F32


def test_moe_layer_output_is_deterministic():
    rng = np.random.default_rng(77)
    layer = synth.moe_weights(64, 8, 2048, 512, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), rng)
    moe = upload_layer(layer)
    x = dev(rng.standard_normal((4, 2048)).astype(np.float32))
    lg = dev(rng.standard_normal((4, 64)).astype(np.float32))
    a = host(moe.forward(x, lg)[0])
    b = host(moe.forward(x, lg)[0])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_grouped_path_output_is_deterministic(monkeypatch):
    # the grouped path writes one down row per pick and sums each token's rows in pick order
    # (k_combine), so two runs agree bit for bit
    monkeypatch.setenv("CWMOE_PREFILL_MIN_TOKENS", "1")
    rng = np.random.default_rng(78)
    layer = synth.moe_weights(64, 8, 2048, 512, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), rng)
    moe = upload_layer(layer)
    x = dev(rng.standard_normal((40, 2048)).astype(np.float32))
    lg = dev(rng.standard_normal((40, 64)).astype(np.float32))
    a = host(moe.forward(x, lg)[0])
    b = host(moe.forward(x, lg)[0])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ------------------------------------------------------------------------------ the shrink to Q2_K

@pytest.mark.parametrize("weighted", [False, True], ids=["plain", "weighted"])
@pytest.mark.parametrize("dtype", F.SHRINK_SOURCES, ids=[F.NAMES[d] for d in F.SHRINK_SOURCES])
def test_requant_q2k_is_bit_exact(dtype, weighted):
    """cw_requant_q2k against the oracle's restatement of requant.rs: every output byte equal.
    Blocks include negative, subnormal and zero scales and all-zero blocks; the count is not a
    multiple of the 16 blocks a workgroup takes; weights include zeros and negatives."""
    say("requant", F.NAMES[dtype], "weighted" if weighted else "plain")
    rng = np.random.default_rng(dtype * 2 + weighted)
    n, bpr = 4099, 8
    raw = synth.random_blocks(dtype, 256 * n, rng).reshape(n, -1)
    dpos = {F.Q3_K: 108, F.Q4_K: 0, F.Q5_K: 0}[dtype]
    raw[:40, dpos + 1] |= 0x80                      # negative d
    raw[40:80, dpos + 1] &= 0x03                    # subnormal / tiny d
    raw[80:90, dpos:dpos + 2] = 0                   # d = 0
    raw[90:100] = 0                                 # all-zero blocks
    if dtype != F.Q3_K:
        raw[100:140, 3] |= 0x80                     # negative dmin
    raw = raw.reshape(-1)
    shape = None
    if weighted:
        shape = (rng.standard_normal(bpr * 256) ** 2).astype(np.float32)
        shape[:64] = 0.0
        shape[64:96] = -1.0
    got = ops.requant_q2k(dtype, dev(raw), n, None if shape is None else dev(shape), bpr if weighted else 0)
    want = O.requant_q2k(dtype, raw, n, shape, bpr if weighted else 0)
    g = host(got).reshape(n, 84)
    w = want.reshape(n, 84)
    bad = np.nonzero(np.any(g != w, axis=1))[0]
    assert bad.size == 0, "blocks %s differ (first: got %s want %s)" % (bad[:8], g[bad[0]], w[bad[0]])


def test_requant_q2k_full_expert_matrix_round_trip():
    """A full config-5-sized Q4_K matrix (2048 x 512): the shrink equals the oracle's bytes, and
    its Q2_K decodes within the bound the oracle pins (sub-block range + half grid steps)."""
    say("requant: one 2048 x 512 Q4_K matrix")
    rng = np.random.default_rng(77)
    n = 2048 * 512 // 256
    raw = synth.random_blocks(F.Q4_K, 2048 * 512, rng)
    got = host(ops.requant_q2k(F.Q4_K, dev(raw), n))
    assert np.array_equal(got, O.requant_q2k(F.Q4_K, raw, n))
    x = O.dequantize(F.Q4_K, raw, 256 * n).reshape(n, 16, 16)
    back = O.dequantize(F.Q2_K, got, 256 * n).reshape(n, 16, 16)
    yb = got.reshape(n, 84)
    d = np.frombuffer(yb[:, 80:82].copy().tobytes(), np.float16).astype(np.float32)[:, None]
    dm = np.frombuffer(yb[:, 82:84].copy().tobytes(), np.float16).astype(np.float32)[:, None]
    lo = np.minimum(x.min(axis=2), 0)
    assert np.all(np.abs(back - x).max(axis=2) <= (x.max(axis=2) - lo) + 0.5 * d + 0.5 * dm + 1e-6)


def test_requant_q2k_rejects_bad_calls():
    raw = dev(np.zeros(144, np.uint8))
    with pytest.raises(cw.CwNotSupported):
        ops.requant_q2k(F.Q8_0, raw, 1)
    with pytest.raises(cw.CwError):
        ops.requant_q2k(F.Q4_K, raw, 1, dev(np.ones(256, np.float32)), 0)   # weights without a row length
    assert ops.requant_q2k(F.Q4_K, raw, 0).numel() == 0
