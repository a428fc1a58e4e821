"""The GGUF reader (cw_gguf_* through coachwhip_amd.gguf) on files written by tests/gguf_write.py.

Host code only: these run without a GPU. What they pin (candle's Content::read,
vendor/candle-core/src/quantized/gguf_file.rs:469-567, and ExpertStore::new's slicing,
crates/engine/src/experts.rs:697-718): dims reported outermost first; tensor data at the first
multiple of general.alignment (default 32) after the directory; 32-bit lengths in version 1;
every metadata type; arrays skipped; the per-expert slices of a [E][n][k] tensor; and the
rejections of malformed files."""
import numpy as np
import pytest

from coachwhip_amd import CwError, formats as F
from coachwhip_amd.gguf import GGUFFile
from tests import gguf_write as G


def _tensors(rng):
    f32 = rng.standard_normal((3, 5)).astype(np.float32)
    q8 = rng.integers(0, 256, F.matrix_bytes(F.Q8_0, 4, 64), dtype=np.uint8)
    iq2s = rng.integers(0, 256, F.matrix_bytes(F.IQ2_S, 2, 256), dtype=np.uint8)
    iq3s = rng.integers(0, 256, F.matrix_bytes(F.IQ3_S, 1, 512), dtype=np.uint8)
    return [("tok.f32", 0, (3, 5), f32.view(np.uint8).ravel()),
            ("blk.0.q8", F.Q8_0, (4, 64), q8),
            ("blk.0.iq2s", F.IQ2_S, (2, 256), iq2s),
            ("blk.1.iq3s", F.IQ3_S, (1, 512), iq3s)]


META = [("general.architecture", G.STRING, "qwen3moe"),
        ("a.u8", G.U8, 200), ("a.i8", G.I8, -5), ("a.u16", G.U16, 60000), ("a.i16", G.I16, -30000),
        ("a.u32", G.U32, 4000000000), ("a.i32", G.I32, -2000000000), ("a.u64", G.U64, 1 << 40),
        ("a.i64", G.I64, -(1 << 40)), ("a.f32", G.F32, 0.5), ("a.f64", G.F64, -1.25), ("a.bool", G.BOOL, 1),
        ("a.arr", G.ARRAY, (G.STRING, ["x", "yz"])), ("a.nested", G.ARRAY, (G.ARRAY, [(G.U8, [1, 2]), (G.U8, [3])])),
        ("qwen3moe.expert_count", G.U32, 8)]


@pytest.mark.parametrize("version", [1, 2, 3])
def test_directory_metadata_and_data(tmp_path, version):
    rng = np.random.default_rng(version)
    tensors = _tensors(rng)
    path = tmp_path / "m.gguf"
    data_off, offs = G.write_gguf(path, META, tensors, version=version)
    with GGUFFile(path) as g:
        assert g.version == version and len(g) == len(tensors)
        for i, (name, gt, dims, raw) in enumerate(tensors):
            assert g.find(name) == i
            tname, dtype, tdims, foff, nbytes = g.tensor(i)
            assert (tname, dtype, tdims, foff, nbytes) == (name, gt, dims, data_off + offs[i], len(raw))
            assert np.array_equal(g.data(i), raw)
        assert g.find("absent") == -1
        for key, vt, v in META:
            if vt in (G.F32, G.F64):
                assert g.meta_float(key) == v
            elif vt == G.STRING:
                assert g.meta_str(key) == v
            elif vt != G.ARRAY:
                assert g.meta_int(key) == v
        with pytest.raises(CwError):
            g.meta_int("a.f32")                 # a float is not an integer
        assert g.meta_str("a.u8") is None


@pytest.mark.parametrize("key_type,alignment", [(G.U32, 64), (G.I32, 128), (G.U8, 16)])
def test_general_alignment(tmp_path, key_type, alignment):
    rng = np.random.default_rng(alignment)
    tensors = _tensors(rng)
    path = tmp_path / "a.gguf"
    data_off, offs = G.write_gguf(path, [("general.alignment", key_type, alignment)], tensors, alignment=alignment)
    assert data_off % alignment == 0
    with GGUFFile(path) as g:
        for i, (_, _, _, raw) in enumerate(tensors):
            assert g.tensor(i)[3] == data_off + offs[i]
            assert np.array_equal(g.data(i), raw)


def test_negative_alignment_falls_back_to_32(tmp_path):
    # a negative general.alignment is ignored (the reference's match arms only take v >= 0)
    rng = np.random.default_rng(7)
    tensors = _tensors(rng)
    path = tmp_path / "n.gguf"
    data_off, offs = G.write_gguf(path, [("general.alignment", G.I32, -64)], tensors, alignment=32)
    with GGUFFile(path) as g:
        assert g.tensor(0)[3] == data_off + offs[0]


def test_expert_slices(tmp_path):
    rng = np.random.default_rng(11)
    E, n, k = 6, 256, 512
    mats = [rng.integers(0, 256, F.matrix_bytes(dt, n if m < 2 else k, k if m < 2 else n) * E, dtype=np.uint8)
            for m, dt in enumerate((F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S))]
    tensors = [("blk.3.ffn_gate_exps.weight", F.IQ2_XXS, (E, n, k), mats[0]),
               ("blk.3.ffn_up_exps.weight", F.IQ2_XXS, (E, n, k), mats[1]),
               ("blk.3.ffn_down_exps.weight", F.IQ2_S, (E, k, n), mats[2])]
    path = tmp_path / "e.gguf"
    G.write_gguf(path, [], tensors)
    with GGUFFile(path) as g:
        for which, (_, gt, dims, raw) in enumerate(tensors):
            dtype, ne, rows, cols, eb, data = g.experts(3, which)
            assert (dtype, ne, rows, cols) == (gt, E, dims[1], dims[2])
            assert eb == F.matrix_bytes(gt, rows, cols)
            for e in range(E):  # expert e at e * expert_bytes, as the bank layout needs
                assert np.array_equal(data[e * eb:(e + 1) * eb], raw[e * eb:(e + 1) * eb])
        with pytest.raises(CwError):
            g.experts(4, 0)                     # no such layer


def _bad(tmp_path, data, why):
    path = tmp_path / "bad.gguf"
    path.write_bytes(data)
    with pytest.raises(CwError, match=why):
        GGUFFile(path)


def _header(n_tensors, n_kv):
    return b"GGUF" + (3).to_bytes(4, "little") + n_tensors.to_bytes(8, "little") + n_kv.to_bytes(8, "little")


def test_rejects_malformed_files(tmp_path):
    rng = np.random.default_rng(3)
    good, data_off, _ = G.gguf_bytes(META, _tensors(rng))
    _bad(tmp_path, b"GGUX" + good[4:], "unknown magic")
    _bad(tmp_path, good[:4] + (4).to_bytes(4, "little") + good[8:], "unsupported version 4")
    _bad(tmp_path, good[:40], "declared counts do not fit")
    _bad(tmp_path, good[:data_off - 60], "truncated file")                   # inside the directory
    _bad(tmp_path, good[:data_off + 8], "extends past the end")
    five = [("t", 0, (1, 1, 1, 1, 2), np.zeros(8, np.uint8))]
    _bad(tmp_path, G.gguf_bytes([], five)[0], "more than 4 dimensions")
    unknown = [("t", 99, (32,), np.zeros(32, np.uint8))]
    _bad(tmp_path, G.gguf_bytes([], unknown)[0], "unknown type 99")
    ragged = [("t", F.Q8_0, (1, 48), np.zeros(34, np.uint8))]
    _bad(tmp_path, G.gguf_bytes([], ragged)[0], "not whole blocks")
    # 2^62 f32 elements: 2^64 bytes, which a 64-bit product would wrap to 0 and pass the end check
    huge = [("t", F.F32, (1 << 31, 1 << 31), np.zeros(4, np.uint8))]
    _bad(tmp_path, G.gguf_bytes([], huge)[0], "larger than the file")
    _bad(tmp_path, _header(0, 1) + (1 << 40).to_bytes(8, "little") + b"k" * 64, "string length exceeds")
    arr = _header(0, 1) + (1).to_bytes(8, "little") + b"k" + (G.ARRAY).to_bytes(4, "little") + \
        (G.U32).to_bytes(4, "little") + (1 << 35).to_bytes(8, "little") + bytes(64)
    _bad(tmp_path, arr, "array length exceeds")
    with pytest.raises(CwError):
        GGUFFile(tmp_path / "missing.gguf")


# ------------------------------------------------------------------------------ a layer onto the GPU

GGUF_LAYERS = [
    # name, E, K, h, I, dtypes, act, pad, router type, router width, T
    ("qwen3moe_decode", 64, 8, 2048, 512, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), 0, 0, F.F32, 2048, 3),
    ("qwen3moe_prefill", 64, 8, 2048, 512, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), 0, 0, F.F32, 2048, 96),
    ("gptoss_squeezed", 16, 4, 1024, 720, (F.MXFP4, F.MXFP4, F.Q4_K), 1, 768, F.F16, 960, 5),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,E,K,h,I,dts,act,pad,rtype,rw,T", GGUF_LAYERS, ids=[c[0] for c in GGUF_LAYERS])
def test_layer_from_gguf_matches_the_oracle(tmp_path, name, E, K, h, I, dts, act, pad, rtype, rw, T):
    """A layer written to a GGUF file, loaded through GGUFFile.moe_layer, routed by its own router
    (cw_router_logits) and run: ids identical, outputs within 1e-3 relative L2 of the oracle on the
    same logits. The squeezed case pads the router to the experts' input width, whose extra
    input columns are zero (crates/engine/src/model_gptoss.rs:141-175)."""
    import torch
    import zlib
    from coachwhip_amd import ops, synth
    from oracle import oracle as O
    print("gguf layer", name, flush=True)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    layer = synth.moe_weights(E, K, h, I, dts, rng, act=act, pad=pad)
    width = max(pad, I)
    router = (rng.standard_normal((E, rw)) * 0.05).astype(np.float32 if rtype == F.F32 else np.float16)
    tensors = [("blk.2.ffn_gate_exps.weight", dts[0], (E, I, h), layer.host[0]),
               ("blk.2.ffn_up_exps.weight", dts[1], (E, I, h), layer.host[1]),
               ("blk.2.ffn_down_exps.weight", dts[2], (E, h, width), layer.host[2]),
               ("blk.2.ffn_gate_inp.weight", rtype, (E, rw), router.view(np.uint8).ravel())]
    rbias = None
    if act == 1:
        rbias = (rng.standard_normal(E) * 0.1).astype(np.float32)
        for m, b in zip(("gate", "up", "down"), layer.bias):
            tensors.append(("blk.2.ffn_%s_exps.bias" % m, F.F32, b.shape, b.view(np.uint8).ravel()))
        tensors.append(("blk.2.ffn_gate_inp.bias", F.F32, (E,), rbias.view(np.uint8).ravel()))
    path = tmp_path / (name + ".gguf")
    G.write_gguf(path, [("general.architecture", G.STRING, "gpt-oss" if act else "qwen3moe")], tensors)
    x = rng.standard_normal((T, h)).astype(np.float32)
    x[:, rw:] = 0.0
    with GGUFFile(path) as g:
        moe, w, b = g.moe_layer(2, K)
    assert tuple(w.shape) == (E, h) and (b is None) == (rbias is None)
    logits = ops.router_logits(w, ops.to_device(x), b)
    torch.cuda.synchronize()
    got_logits = logits.cpu().numpy()
    want_logits = x[:, :rw].astype(np.float64) @ router.astype(np.float64).T + (0 if rbias is None else rbias)
    assert O.rel_l2(got_logits, want_logits) < 1e-5
    assert not synth.near_ties_within_top_k(got_logits, K)
    out, ids, ww = moe.forward(ops.to_device(x), logits)
    want, wids, wantw, _ = O.moe_layer(layer, x, got_logits)
    assert np.array_equal(ids.cpu().numpy().view(np.uint32), wids)
    assert np.max(np.abs(ww.cpu().numpy() - wantw)) < 1e-5
    err = O.rel_l2(out.cpu().numpy(), want)
    print("  rel_l2", err, flush=True)
    assert err <= 1e-3
