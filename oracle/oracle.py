"""TEST INFRASTRUCTURE ONLY: ctypes front end of the CPU oracle (``liboracle.so``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg import this
module, as the checker. The product (``coachwhip_amd``) never does.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q8_0, Q4_K, Q8_K, IQ2_XXS, IQ3_S, IQ2_S, MXFP4 = 0, 1, 8, 12, 15, 16, 21, 22, 39
Q2_K, Q3_K, Q5_K = 10, 11, 13

_lib = None


def build(force=False):
    """Compile liboracle.so with the committed Makefile (gcc; no reference sources involved)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "liboracle.so"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64


def _declare(L):
    L.or_block_size.argtypes = [_I]
    L.or_type_size.argtypes = [_I]
    L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.or_f16_to_f32.restype = ctypes.c_float
    L.or_f32_to_f16.argtypes = [ctypes.c_float]
    L.or_f32_to_f16.restype = ctypes.c_uint16
    L.or_e8m0_half.argtypes = [ctypes.c_uint8]
    L.or_e8m0_half.restype = ctypes.c_float
    L.or_dequantize.argtypes = [_I, _P, _L, _P]
    L.or_qmatmul_f64.argtypes = [_I, _P, _L, _L, _P, _L, _P]
    L.or_route.argtypes = [_P, _I, _I, _I, _I, _P, _P]
    L.or_route.restype = None
    L.or_softmax.argtypes = [_P, _I, _I, _P]
    L.or_softmax.restype = None
    L.or_rank.argtypes = [_P, _I, _P]
    L.or_rank.restype = None
    L.or_silu_mul.argtypes = [_P, _P, _P, _L]
    L.or_silu_mul.restype = None
    L.or_clamped_swiglu.argtypes = [_P, _P, _P, _P, _P, _L, _I, _I, ctypes.c_float, ctypes.c_float, _P]
    L.or_clamped_swiglu.restype = None
    L.or_weighted_sum.argtypes = [_P, _P, _I, _I, _I, _P]
    L.or_weighted_sum.restype = None
    L.or_resolve.argtypes = [_P, _P, _I, _P, _P]
    L.or_resolve.restype = None
    L.or_matvec_id.argtypes = [_I, _L, _L, _L, _L, _P, _P, _I, _P, _I, _I, _P]
    L.or_moe_layer.argtypes = [ctypes.POINTER(MoeDesc), _P, _P, _I, _P, _P, _P]
    L.or_quantize_q8_0.argtypes = [_P, _L, _P]
    L.or_quantize_q8_0.restype = None
    L.or_quantize_q8_k.argtypes = [_P, _L, _P]
    L.or_quantize_q8_k.restype = None
    L.or_set_threads.argtypes = [_I]
    L.or_set_threads.restype = None
    L.or_get_threads.argtypes = []
    L.or_get_threads.restype = _I
    L.or_vec_dot.argtypes = [_I, _L, _P, _P]
    L.or_vec_dot.restype = ctypes.c_float
    L.or_candle_matmul.argtypes = [_I, _P, _L, _L, _P, _L, _P, _I]
    L.or_x86_level.argtypes = []
    L.or_x86_level.restype = _I
    L.or_x86_select.argtypes = [_I, _L, _L, _L]
    L.or_x86_select.restype = _I
    L.or_x86_packed_bytes.argtypes = [_I, _L, _L]
    L.or_x86_packed_bytes.restype = _L
    L.or_x86_pack.argtypes = [_I, _P, _L, _L, _P]
    L.or_x86_matmul.argtypes = [_I, _P, _L, _L, _P, _L, _P, _I, _I]
    L.or_requant_q2k.argtypes = [_I, _P, _L, _P, _L, _P]


class MoeDesc(ctypes.Structure):
    _fields_ = [("n_experts", _I), ("top_k", _I), ("hidden", _I), ("inter", _I),
                ("norm", _I), ("act", _I), ("alpha", ctypes.c_float), ("limit", ctypes.c_float),
                ("pad", _I), ("dtype", _I * 3), ("w", _P * 3), ("slot_stride", _L * 3),
                ("bias", _P * 3), ("slot_table", _P), ("n_slots", _I)]


def _ptr(a):
    return a.ctypes.data_as(_P) if a is not None else None


def block_size(dtype):
    return lib().or_block_size(dtype)


def type_size(dtype):
    return lib().or_type_size(dtype)


def dequantize(dtype, blocks, n):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    assert lib().or_dequantize(dtype, _ptr(blocks), n, _ptr(out)) == 0
    return out


def qmatmul_f64(dtype, w, n, k, x):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    y = np.empty((x.shape[0], n), dtype=np.float64)
    assert lib().or_qmatmul_f64(dtype, _ptr(w), n, k, _ptr(x), x.shape[0], _ptr(y)) == 0
    return y


def route(logits, k, norm):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    t, e = logits.shape
    ids = np.empty((t, k), dtype=np.uint32)
    w = np.empty((t, k), dtype=np.float32)
    lib().or_route(_ptr(logits), t, e, k, int(norm), _ptr(ids), _ptr(w))
    return ids, w


def softmax(logits):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    t, e = logits.shape
    p = np.empty_like(logits)
    lib().or_softmax(_ptr(logits), t, e, _ptr(p))
    return p


def rank(scores):
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    ids = np.empty(len(scores), dtype=np.uint32)
    lib().or_rank(_ptr(scores), len(scores), _ptr(ids))
    return ids


def silu_mul(g, u):
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    h = np.empty_like(g)
    lib().or_silu_mul(_ptr(g), _ptr(u), _ptr(h), g.size)
    return h


def clamped_swiglu(g, u, gate_b, up_b, ids, pad=0, alpha=1.702, limit=7.0):
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    rows, width = g.shape
    ids = np.ascontiguousarray(ids, dtype=np.uint32).reshape(-1)
    gb = None if gate_b is None else np.ascontiguousarray(gate_b, dtype=np.float32)
    ub = None if up_b is None else np.ascontiguousarray(up_b, dtype=np.float32)
    out_w = max(pad, width)
    h = np.empty((rows, out_w), dtype=np.float32)
    lib().or_clamped_swiglu(_ptr(g), _ptr(u), _ptr(gb), _ptr(ub), _ptr(ids), rows, width, pad,
                            alpha, limit, _ptr(h))
    return h


def weighted_sum(down, w):
    down = np.ascontiguousarray(down, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    t, k, h = down.shape
    out = np.empty((t, h), dtype=np.float32)
    lib().or_weighted_sum(_ptr(down), _ptr(w), t, k, h, _ptr(out))
    return out


def resolve(ids, table):
    ids = np.ascontiguousarray(ids, dtype=np.uint32).reshape(-1)
    table = np.ascontiguousarray(table, dtype=np.uint32)
    slots = np.empty_like(ids)
    missing = np.zeros(1, dtype=np.uint32)
    lib().or_resolve(_ptr(ids), _ptr(table), len(ids), _ptr(slots), _ptr(missing))
    return slots, int(missing[0])


def matvec_id(dtype, n, k, bank, slot_stride, x, ids, rows_per_expert):
    bank = np.ascontiguousarray(bank, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    t, kk = ids.shape
    x = np.ascontiguousarray(x, dtype=np.float32)
    n_slots = bank.size // slot_stride
    out = np.empty((t, kk, n), dtype=np.float64)
    assert lib().or_matvec_id(dtype, n, k, n_slots, slot_stride, _ptr(bank), _ptr(x),
                              int(rows_per_expert), _ptr(ids), kk, t, _ptr(out)) == 0
    return out


def moe_layer(layer, x, logits, slot_table=None, n_slots=None):
    """layer: coachwhip_amd.synth.MoeWeights (host arrays). Returns (out f64, ids, w, missing)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    t = x.shape[0]
    d = MoeDesc()
    d.n_experts, d.top_k, d.hidden, d.inter = layer.n_experts, layer.top_k, layer.hidden, layer.inter
    d.norm, d.act = int(layer.norm), int(layer.act)
    d.alpha, d.limit, d.pad = layer.alpha, layer.limit, layer.pad
    keep = []
    for m in range(3):
        d.dtype[m] = layer.dtypes[m]
        buf = np.ascontiguousarray(layer.host[m], dtype=np.uint8)
        keep.append(buf)
        d.w[m] = buf.ctypes.data
        d.slot_stride[m] = layer.slot_stride[m]
        b = layer.bias[m] if layer.bias is not None else None
        if b is not None:
            b = np.ascontiguousarray(b, dtype=np.float32)
            keep.append(b)
            d.bias[m] = b.ctypes.data
        else:
            d.bias[m] = None
    if slot_table is not None:
        tab = np.ascontiguousarray(slot_table, dtype=np.uint32)
        keep.append(tab)
        d.slot_table = tab.ctypes.data
        d.n_slots = n_slots
    else:
        d.slot_table = None
        d.n_slots = layer.n_experts
    out = np.empty((t, layer.hidden), dtype=np.float64)
    ids = np.empty((t, layer.top_k), dtype=np.uint32)
    w = np.empty((t, layer.top_k), dtype=np.float32)
    missing = lib().or_moe_layer(ctypes.byref(d), _ptr(x), _ptr(logits), t, _ptr(out), _ptr(ids), _ptr(w))
    assert missing >= 0
    return out, ids, w, missing


def quantize_q8_0(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 32 * 34, dtype=np.uint8)
    lib().or_quantize_q8_0(_ptr(x), x.size, _ptr(out))
    return out


def quantize_q8_k(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 256 * 292, dtype=np.uint8)
    lib().or_quantize_q8_k(_ptr(x), x.size, _ptr(out))
    return out


def set_threads(n):
    """OpenMP threads of the oracle's parallel loops."""
    lib().or_set_threads(int(n))


def get_threads():
    return lib().or_get_threads()


def vec_dot(dtype, k, wrow, xq):
    wrow = np.ascontiguousarray(wrow, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    return lib().or_vec_dot(dtype, k, _ptr(wrow), _ptr(xq))


def candle_matmul(dtype, w, n, k, x, threads=0):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    y = np.empty((x.shape[0], n), dtype=np.float32)
    assert lib().or_candle_matmul(dtype, _ptr(w), n, k, _ptr(x), x.shape[0], _ptr(y), threads) == 0
    return y


def candle_moe_layer(layer, x, logits, threads=0):
    """candle's own CPU path for one MoE layer (crates/engine/src/experts.rs:2500-2537): route,
    then per picked expert in expert-id order (the BTreeMap of experts.rs:2503-2510) the gate and up
    QMatMuls (candle_matmul: x quantized to the weight's vec-dot type, Q8_0 for MXFP4,
    k_quants.rs:738-759, 2551-2670), the activation with its biases, the down QMatMul and its bias,
    scaled by the routing weight and index-added into the output in expert order. f32 throughout,
    as candle computes it. Returns (out f32, ids, w)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    t = x.shape[0]
    ids, w = route(logits, layer.top_k, layer.norm)
    H, I = layer.hidden, layer.inter
    width = max(layer.pad, I)
    per_expert = {}
    for tok in range(t):
        for j in range(layer.top_k):
            per_expert.setdefault(int(ids[tok, j]), []).append((tok, float(w[tok, j])))
    out = np.zeros((t, H), dtype=np.float32)
    for e in sorted(per_expert):
        toks = np.array([p[0] for p in per_expert[e]], dtype=np.int64)
        we = np.array([p[1] for p in per_expert[e]], dtype=np.float32)
        xe = x[toks]
        mats = [layer.host[m][e * layer.slot_stride[m]:(e + 1) * layer.slot_stride[m]] for m in range(3)]
        g = candle_matmul(layer.dtypes[0], mats[0], I, H, xe, threads)
        u = candle_matmul(layer.dtypes[1], mats[1], I, H, xe, threads)
        picked = np.full(len(toks), e, dtype=np.uint32)
        if layer.act == 1:
            b = layer.bias
            h = clamped_swiglu(g, u, b[0] if b else None, b[1] if b else None, picked, layer.pad,
                               layer.alpha, layer.limit)
        else:
            h = silu_mul(g, u)
            if width > I:
                h = np.pad(h, ((0, 0), (0, width - I)))
        y = candle_matmul(layer.dtypes[2], mats[2], H, width, h, threads)
        if layer.act == 1 and layer.bias is not None:
            y = y + layer.bias[2][e][None, :]
        np.add.at(out, toks, y * we[:, None])
    return out, ids, w


def x86_level():
    """candle's x86 tier on this host: 2 AVX-512 VNNI, 1 AVX-VNNI, 0 AVX2, -1 none."""
    return lib().or_x86_level()


def x86_select(dtype, m, n, k):
    """Whether candle's repacked x86 path takes (dtype, m, n, k) on this host."""
    return bool(lib().or_x86_select(dtype, m, n, k))


def x86_pack(dtype, w, n, k):
    """The weight tiles of candle's x86 path (packed once per matrix, as candle caches them)."""
    nb = lib().or_x86_packed_bytes(dtype, n, k)
    assert nb > 0
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.empty(nb, dtype=np.uint8)
    assert lib().or_x86_pack(dtype, _ptr(w), n, k, _ptr(out)) == 0
    return out


def x86_matmul(dtype, packed, n, k, x, simd=True, threads=0):
    """candle's x86 QMatMul over packed tiles: x rows to Q8_K, then the tile units."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    y = np.empty((x.shape[0], n), dtype=np.float32)
    assert lib().or_x86_matmul(dtype, _ptr(packed), n, k, _ptr(x), x.shape[0], _ptr(y), int(simd), threads) == 0
    return y


def requant_q2k(src_dtype, blocks, n_blocks, shape=None, blocks_per_row=0):
    """The GPU shrink's Q2_K bytes (n_blocks x 84) for n_blocks source super-blocks."""
    src = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(n_blocks * 84, dtype=np.uint8)
    sh = None if shape is None else np.ascontiguousarray(shape, dtype=np.float32)
    rc = lib().or_requant_q2k(src_dtype, _ptr(src), n_blocks, _ptr(sh), blocks_per_row, _ptr(out))
    assert rc == 0
    return out


def rel_l2(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (den if den > 0 else 1.0))
