"""Seeded synthetic inputs for the quantized expert path: raw GGUF blocks and activations.

Every byte pattern is a valid encoding of these formats, so quant bytes are uniform random and
only the scale fields follow a stated distribution (the benchmark configurations' own, or a
suggested one where they give none):

- Q8_0: d = f16(U[0.001, 0.02]), quants U{-127..127}.
- Q4_K: d, dmin = f16(U[0.001, 0.02]); the 12 scale bytes and 128 quant bytes uniform.
- Q2_K / Q3_K / Q5_K (the shrink's formats): d (and dmin) = f16(U[0.001, 0.02]); the rest uniform.
- IQ2_XXS / IQ2_S / IQ3_S: d = f16(U[0.001, 0.02]); all other bytes uniform.
- MXFP4: e8m0 exponent U{119..123}; nibbles uniform.

Block layouts follow vendor/candle-core/src/quantized/k_quants.rs:125-200, 631-635 and
vendor/candle-metal-kernels/src/metal_src/quantized.metal:217-257 (see ``formats``).
"""
from dataclasses import dataclass, field

import numpy as np

from . import formats as F


def _f16_bits(vals):
    return np.asarray(vals, dtype=np.float32).astype(np.float16).view(np.uint16)


def random_blocks(dtype, n_weights, rng):
    """n_weights weights of `dtype` as a flat uint8 array of raw GGUF blocks."""
    bs, ts = F.block_size(dtype), F.type_size(dtype)
    assert n_weights % bs == 0, (dtype, n_weights)
    nb = n_weights // bs
    raw = rng.integers(0, 256, size=(nb, ts), dtype=np.uint8)
    if dtype == F.Q8_0:
        d = _f16_bits(rng.uniform(0.001, 0.02, nb))
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        raw[:, 2:34] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    elif dtype in (F.Q4_K, F.Q5_K):
        raw[:, 0:2] = _f16_bits(rng.uniform(0.001, 0.02, nb)).view(np.uint8).reshape(nb, 2)
        raw[:, 2:4] = _f16_bits(rng.uniform(0.001, 0.02, nb)).view(np.uint8).reshape(nb, 2)
    elif dtype == F.Q2_K:
        raw[:, 80:82] = _f16_bits(rng.uniform(0.001, 0.02, nb)).view(np.uint8).reshape(nb, 2)
        raw[:, 82:84] = _f16_bits(rng.uniform(0.001, 0.02, nb)).view(np.uint8).reshape(nb, 2)
    elif dtype == F.Q3_K:
        raw[:, 108:110] = _f16_bits(rng.uniform(0.001, 0.02, nb)).view(np.uint8).reshape(nb, 2)
    elif dtype == F.Q6_K:
        raw[:, 208:210] = _f16_bits(rng.uniform(0.001, 0.02, nb)).view(np.uint8).reshape(nb, 2)
    elif dtype in (F.IQ2_XXS, F.IQ2_S, F.IQ3_S, F.IQ3_XXS, F.IQ4_XS):
        raw[:, 0:2] = _f16_bits(rng.uniform(0.001, 0.02, nb)).view(np.uint8).reshape(nb, 2)
    elif dtype == F.MXFP4:
        raw[:, 0] = rng.integers(119, 124, size=nb, dtype=np.uint8)
    else:
        raise ValueError("no generator for dtype %d" % dtype)
    return raw.reshape(-1)


@dataclass
class MoeWeights:
    """One MoE layer's expert matrices as raw blocks, slot-major (GGUF `ffn_*_exps` order:
    gate/up [slots][inter][hidden], down [slots][hidden][pad]), crates/engine/src/experts.rs:697-718."""
    n_experts: int
    top_k: int
    hidden: int
    inter: int
    dtypes: tuple
    host: list
    slot_stride: list
    n_slots: int
    norm: bool = True
    act: int = 0              # 0 silu(gate)*up, 1 clamped SwiGLU with biases
    alpha: float = 1.702
    limit: float = 7.0
    pad: int = 0
    bias: list = None         # [gate_b (E, I), up_b (E, I), down_b (E, H)] for act 1
    experts_of_slot: np.ndarray = field(default=None)


def moe_weights(n_experts, top_k, hidden, inter, dtypes, rng, n_slots=None, act=0, pad=0,
                norm=True):
    n_slots = n_experts if n_slots is None else n_slots
    width = max(pad, inter)
    shapes = [(inter, hidden), (inter, hidden), (hidden, width)]
    host, strides = [], []
    for m in range(3):
        rows, k = shapes[m]
        stride = rows * F.row_bytes(dtypes[m], k)
        host.append(random_blocks(dtypes[m], n_slots * rows * k, rng))
        strides.append(stride)
    bias = None
    if act == 1:
        bias = [rng.normal(0, 0.02, size=(n_experts, inter)).astype(np.float32),
                rng.normal(0, 0.02, size=(n_experts, inter)).astype(np.float32),
                rng.normal(0, 0.02, size=(n_experts, hidden)).astype(np.float32)]
    return MoeWeights(n_experts, top_k, hidden, inter, tuple(dtypes), host, strides, n_slots,
                      norm=norm, act=act, pad=pad, bias=bias)


def activations(shape, rng, dtype=np.float32):
    return rng.standard_normal(size=shape).astype(dtype)


def top_k_margin(logits, k):
    """Smallest gap between the k-th and (k+1)-th largest logit of any row: the routing is only
    comparable bit-for-bit across two softmax implementations when this is well above f32
    rounding."""
    s = -np.sort(-np.asarray(logits, dtype=np.float64), axis=1)
    if s.shape[1] <= k:
        return np.inf
    return float(np.min(s[:, k - 1] - s[:, k]))


def near_ties_within_top_k(logits, k, eps=1e-6):
    """True when two distinct logits among a row's top k+1 are within eps of each other.

    The CPU route ranks f32 softmax probabilities (ties to the lower index) and the GPU ranks
    the logits themselves; the orders can only differ when two distinct logits give the same f32
    probability, which needs a gap of about one ulp of exp (~1e-7). Exact ties are ranked by
    index on both sides and do not count."""
    s = -np.sort(-np.asarray(logits, dtype=np.float64), axis=1)[:, :k + 1]
    gaps = s[:, :-1] - s[:, 1:]
    return bool(np.any((gaps > 0) & (gaps <= eps * np.maximum(1.0, np.abs(s[:, :-1])))))


def device_blocks(dtype, n_weights, gen, device="cuda"):
    """random_blocks' distribution generated on the device with a seeded torch.Generator (for
    benchmark banks of several GB that would be slow to build on the host)."""
    import torch
    bs, ts = F.block_size(dtype), F.type_size(dtype)
    assert n_weights % bs == 0
    nb = n_weights // bs
    raw = torch.randint(0, 256, (nb, ts), dtype=torch.uint8, device=device, generator=gen)

    def f16_scales():
        v = torch.rand(nb, device=device, generator=gen) * (0.02 - 0.001) + 0.001
        return v.to(torch.float16).view(torch.uint8).view(nb, 2)

    if dtype == F.Q8_0:
        raw[:, 0:2] = f16_scales()
        raw[:, 2:34] = torch.randint(-127, 128, (nb, 32), dtype=torch.int8, device=device, generator=gen).view(torch.uint8)
    elif dtype in (F.Q4_K, F.Q5_K):
        raw[:, 0:2] = f16_scales()
        raw[:, 2:4] = f16_scales()
    elif dtype == F.Q2_K:
        raw[:, 80:82] = f16_scales()
        raw[:, 82:84] = f16_scales()
    elif dtype == F.Q3_K:
        raw[:, 108:110] = f16_scales()
    elif dtype == F.Q6_K:
        raw[:, 208:210] = f16_scales()
    elif dtype in (F.IQ2_XXS, F.IQ2_S, F.IQ3_S, F.IQ3_XXS, F.IQ4_XS):
        raw[:, 0:2] = f16_scales()
    elif dtype == F.MXFP4:
        raw[:, 0] = torch.randint(119, 124, (nb,), dtype=torch.uint8, device=device, generator=gen)
    else:
        raise ValueError("no generator for dtype %d" % dtype)
    return raw.view(-1)
