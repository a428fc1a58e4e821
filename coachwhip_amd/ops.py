"""Python mirror of the reference engine's quantized-expert interfaces, running on the HIP C ABI.

Names and argument meanings follow the reference so tests read like its own:

- ``QTensor`` / ``QMatMul``: vendor/candle-core/src/quantized/mod.rs:846-1345 (weights as raw
  GGUF blocks, ``forward`` maps ``[..., k]`` to ``[..., n]``).
- ``route``: crates/engine/src/experts.rs:2364-2372 (softmax, top-k best first, renormalised
  weights when ``norm``).
- ``ExpertAct``: experts.rs:2376-2423 (``Silu`` and ``ClampedSwiglu``).
- ``MoeMatvec``: experts.rs:2183-2309 (``forward(x, ids)`` -> ``(tokens, nei0, n)``).
- ``MoeLayer``: the resident branch of ``StreamedMoe::forward`` (experts.rs:2562-2614), and with
  a slot table the bank branch (3003-3015).

Torch provides device memory and the current stream only; all arithmetic runs in libcwmoe.so.
Shape and dtype errors raise ``CwError`` (the reference bails with the same conditions).
"""
import ctypes
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import formats as F
from ._lib import CwError, MoeDesc, SharedDesc, check, lib, CW_EINVAL, CW_ENOTSUP, CW_MOE_STATE_BYTES, CW_MOE_STATUS_OFFSET


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _need(t, dtype, what):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise CwError(CW_EINVAL, "%s must be a device tensor" % what)
    if t.dtype != dtype:
        raise CwError(CW_EINVAL, "%s must be %s, got %s" % (what, dtype, t.dtype))
    if not t.is_contiguous():
        raise CwError(CW_EINVAL, "%s must be contiguous" % what)


def to_device(a, device="cuda"):
    """A host numpy array as a device tensor (u32 arrays travel as int32 bits)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).to(device)


class QTensor:
    """Raw GGUF blocks of an (n, k) matrix on the device."""

    def __init__(self, data: torch.Tensor, dtype: int, shape):
        n, k = shape
        _need(data, torch.uint8, "QTensor data")
        if data.numel() != F.matrix_bytes(dtype, n, k):
            raise CwError(CW_EINVAL, "QTensor: %d bytes for a %dx%d %s matrix" % (data.numel(), n, k, F.NAMES[dtype]))
        self.data, self.dtype, self.shape = data, dtype, (n, k)

    @classmethod
    def from_blocks(cls, raw, dtype, shape, device="cuda"):
        return cls(to_device(np.asarray(raw, dtype=np.uint8), device), dtype, shape)

    def dequantize(self) -> torch.Tensor:
        n, k = self.shape
        out = torch.empty((n, k), dtype=torch.float32, device=self.data.device)
        check(lib().cw_dequantize(self.dtype, _p(self.data), n * k, _p(out), _stream()))
        return out


def dequantize(dtype, blocks: torch.Tensor, n_elems) -> torch.Tensor:
    """Flat dequantization of n_elems weights of raw blocks."""
    _need(blocks, torch.uint8, "blocks")
    out = torch.empty(n_elems, dtype=torch.float32, device=blocks.device)
    check(lib().cw_dequantize(dtype, _p(blocks), n_elems, _p(out), _stream()))
    return out


class QMatMul:
    def __init__(self, qtensor: QTensor):
        self.w = qtensor

    @classmethod
    def from_qtensor(cls, qtensor):
        return cls(qtensor)

    def forward(self, xs: torch.Tensor) -> torch.Tensor:
        n, k = self.w.shape
        _need(xs, torch.float32, "xs")
        if xs.dim() < 2:
            raise CwError(CW_EINVAL, "input tensor has only one dimension")
        if xs.shape[-1] != k:
            raise CwError(CW_EINVAL, "input tensor %s incompatible with (%d, %d)" % (tuple(xs.shape), n, k))
        m = xs.numel() // k
        y = torch.empty(xs.shape[:-1] + (n,), dtype=torch.float32, device=xs.device)
        ws_bytes = lib().cw_qmatmul_workspace_size(self.w.dtype, n, k, m)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=xs.device) if ws_bytes else None
        check(lib().cw_qmatmul(self.w.dtype, _p(self.w.data), n, k, _p(xs), m, _p(y), _p(ws), ws_bytes, _stream()))
        return y

    __call__ = forward


def router_logits(w: torch.Tensor, x: torch.Tensor, bias: torch.Tensor = None) -> torch.Tensor:
    """x (T, h) f32 times the router weight w (E, h), f32 or f16, plus bias (E,): (T, E) f32 logits.

    The gate Linear of crates/engine/src/experts.rs:2428, 2577 (bias: model_gptoss.rs:168-175),
    and its f16 decode variant cw_mv_f16 (fuse_kernel.rs:160-178)."""
    _need(x, torch.float32, "x")
    if not w.is_cuda or w.dtype not in (torch.float32, torch.float16) or not w.is_contiguous() or w.dim() != 2:
        raise CwError(CW_EINVAL, "router weight must be a contiguous (E, h) f32 or f16 tensor")
    e, h = w.shape
    if x.shape[-1] != h:
        raise CwError(CW_EINVAL, "x %s incompatible with a (%d, %d) router" % (tuple(x.shape), e, h))
    if bias is not None:
        _need(bias, torch.float32, "bias")
    t = x.numel() // h
    logits = torch.empty((t, e), dtype=torch.float32, device=x.device)
    wdtype = 0 if w.dtype == torch.float32 else 1
    check(lib().cw_router_logits(wdtype, _p(w), e, h, _p(bias), _p(x), t, _p(logits), _stream()))
    return logits


def requant_q2k(src_dtype: int, src: torch.Tensor, n_blocks: int, shape: torch.Tensor = None, blocks_per_row: int = 0,
                out: torch.Tensor = None) -> torch.Tensor:
    """The shrink of n_blocks Q3_K / Q4_K / Q5_K super-blocks (device uint8) to Q2_K bytes (n_blocks * 84),
    weighted by shape (f32, blocks_per_row * 256 per row) when given (crates/engine/src/requant.rs:361-406)."""
    if not isinstance(src, torch.Tensor) or not src.is_cuda or src.dtype != torch.uint8:
        raise CwError(CW_EINVAL, "requant: src must be a device uint8 tensor")
    if src_dtype in F.SHRINK_SOURCES and src.numel() < n_blocks * F.type_size(src_dtype):
        raise CwError(CW_EINVAL, "requant: src holds %d bytes, %d blocks need more" % (src.numel(), n_blocks))
    if shape is not None:
        _need(shape, torch.float32, "shape")
        if shape.numel() < blocks_per_row * 256:
            raise CwError(CW_EINVAL, "requant: %d weights for rows of %d blocks" % (shape.numel(), blocks_per_row))
    if out is None:
        out = torch.empty(n_blocks * 84, dtype=torch.uint8, device=src.device)
    elif out.numel() < n_blocks * 84:
        raise CwError(CW_EINVAL, "requant: out holds %d bytes" % out.numel())
    check(lib().cw_requant_q2k(src_dtype, _p(src), n_blocks, _p(shape), blocks_per_row, _p(out), _stream()))
    return out


def route(logits: torch.Tensor, top_k: int, norm: bool):
    """(ids (T, K) u32 as int32 bits, weights (T, K) f32)."""
    _need(logits, torch.float32, "logits")
    t, e = logits.shape
    ids = torch.empty((t, top_k), dtype=torch.int32, device=logits.device)
    w = torch.empty((t, top_k), dtype=torch.float32, device=logits.device)
    check(lib().cw_route_topk(_p(logits), t, e, top_k, int(norm), _p(ids), _p(w), _stream()))
    return ids, w


def swiglu(g, u):
    _need(g, torch.float32, "gate")
    _need(u, torch.float32, "up")
    h = torch.empty_like(g)
    check(lib().cw_swiglu(_p(g), _p(u), _p(h), g.numel(), _stream()))
    return h


def clamped_swiglu(g, u, gate_b, up_b, ids, pad=0, alpha=1.702, limit=7.0):
    _need(g, torch.float32, "gate")
    rows, width = g.shape
    out_w = max(pad, width)
    h = torch.empty((rows, out_w), dtype=torch.float32, device=g.device)
    check(lib().cw_clamped_swiglu(_p(g), _p(u), _p(gate_b), _p(up_b), _p(ids), rows, width, pad, alpha, limit, _p(h),
                                  _stream()))
    return h


def weighted_sum(down, w, down_b=None, ids=None):
    _need(down, torch.float32, "down")
    t, k, h = down.shape
    out = torch.empty((t, h), dtype=torch.float32, device=down.device)
    check(lib().cw_weighted_sum(_p(down), _p(w), _p(down_b), _p(ids), t, k, h, _p(out), _stream()))
    return out


def slots_resolve(ids, table):
    """(slots, missing) with slots the same shape as ids."""
    _need(ids, torch.int32, "ids")
    slots = torch.empty_like(ids)
    missing = torch.zeros(1, dtype=torch.int32, device=ids.device)
    check(lib().cw_slots_resolve(_p(ids), _p(table), ids.numel(), _p(slots), _p(missing), _stream()))
    return slots, missing


class SharedExpert:
    """The expert every token uses, scaled by its own sigmoid gate (SharedExpert,
    crates/engine/src/model_next.rs:723-742): sigmoid(x . gate_inp) * down(silu(gate x) * up x).

    gate, up, down are QTensors ((inter, h), (inter, h), (h, inter)); gate_inp an (h,) f32 device
    tensor or None."""

    def __init__(self, gate: "QTensor", up: "QTensor", down: "QTensor", gate_inp: Optional[torch.Tensor] = None):
        inter, h = gate.shape
        if up.shape != (inter, h) or down.shape != (h, inter):
            raise CwError(CW_EINVAL, "shared expert: gate %s, up %s, down %s" % (gate.shape, up.shape, down.shape))
        if gate_inp is not None:
            _need(gate_inp, torch.float32, "gate_inp")
            if gate_inp.numel() != h:
                raise CwError(CW_EINVAL, "shared expert: gate_inp of %d, hidden %d" % (gate_inp.numel(), h))
        self.gate, self.up, self.down, self.gate_inp = gate, up, down, gate_inp
        d = SharedDesc()
        d.hidden, d.inter = h, inter
        for i, q in enumerate((gate, up, down)):
            d.dtype[i] = q.dtype
            d.w[i] = q.data.data_ptr()
        d.gate_inp = None if gate_inp is None else gate_inp.data_ptr()
        self.desc = d

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The shared expert's output for each row of x; added into ``out`` when it is given."""
        _need(x, torch.float32, "x")
        h = self.desc.hidden
        if x.shape[-1] != h:
            raise CwError(CW_EINVAL, "x %s incompatible with hidden %d" % (tuple(x.shape), h))
        t = x.numel() // h
        acc = out is not None
        if acc:
            _need(out, torch.float32, "out")
            if out.numel() != t * h:
                raise CwError(CW_EINVAL, "out %s for %d rows of %d" % (tuple(out.shape), t, h))
        else:
            out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
        ws_bytes = lib().cw_shared_expert_workspace_size(ctypes.byref(self.desc), t)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        check(lib().cw_shared_expert(ctypes.byref(self.desc), _p(x), t, _p(out), int(acc), _p(ws), ws_bytes, _stream()))
        return out

    __call__ = forward


@dataclass
class ExpertBank:
    """One matrix of a layer's bank: ``n_slots`` (n, k) matrices ``slot_stride`` bytes apart."""
    data: torch.Tensor
    dtype: int
    n: int
    k: int
    n_slots: int
    slot_stride: int

    @classmethod
    def from_blocks(cls, raw, dtype, n, k, n_slots, device="cuda"):
        stride = F.matrix_bytes(dtype, n, k)
        raw = np.asarray(raw, dtype=np.uint8)
        if raw.size != stride * n_slots:
            raise CwError(CW_EINVAL, "bank: %d bytes for %d slots of %d" % (raw.size, n_slots, stride))
        return cls(to_device(raw, device), dtype, n, k, n_slots, stride)

    def rows16(self):
        """This MXFP4 bank with each matrix's rows in groups of 16 (MXFP4_R16), repacked on the device
        into a new bank: the same blocks, whose steps the kernels load as one run per group."""
        if self.dtype != F.MXFP4:
            raise CwError(CW_EINVAL, "rows16: a %s bank (MXFP4 only)" % F.NAMES[self.dtype])
        stride = lib().cw_rows16_bytes(self.n, self.k)
        data = torch.empty(stride * self.n_slots, dtype=torch.uint8, device=self.data.device)
        check(lib().cw_repack_rows16(_p(self.data), self.slot_stride, _p(data), stride, self.n_slots, self.n, self.k,
                                     _stream()))
        return ExpertBank(data, F.MXFP4_R16, self.n, self.k, self.n_slots, stride)


class MoeMatvec:
    """out[t][j] = W[ids[t][j]] . x_row, x_row = x[t] or x[t*nei0 + j] (rows_per_expert).

    Above ``grouped_above`` tokens (8, the reference's switch, crates/engine/src/experts.rs:2225)
    the call runs as grouped GEMMs on the matrix cores (cw_matmul_id_grouped), and falls back to
    the per-pick matvec (cw_matvec_id) when that reports the shape unsupported; ``grouped_above``
    None keeps every call on the matvec."""

    def __init__(self, bank: ExpertBank, nei0: int, rows_per_expert: bool, grouped_above: Optional[int] = 8):
        self.bank, self.nei0, self.rows_per_expert = bank, nei0, rows_per_expert
        self.grouped_above = grouped_above
        self._ws = None

    def _grouped(self, x, ids, out, tokens):
        b = self.bank
        need = lib().cw_matmul_id_grouped_workspace_size(b.dtype, b.n, b.k, b.n_slots, b.slot_stride,
                                                         int(self.rows_per_expert), self.nei0, tokens)
        if need == 0:
            return False
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=x.device)
        rc = lib().cw_matmul_id_grouped(b.dtype, b.n, b.k, b.n_slots, b.slot_stride, _p(b.data), _p(x),
                                        int(self.rows_per_expert), _p(ids), self.nei0, tokens, _p(out), _p(self._ws),
                                        need, _stream())
        if rc == CW_ENOTSUP:
            return False
        check(rc)
        return True

    def forward(self, x: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
        _need(x, torch.float32, "x")
        _need(ids, torch.int32, "ids")
        tokens, nei0 = ids.shape
        if nei0 != self.nei0:
            raise CwError(CW_EINVAL, "%d ids per token, expected %d" % (nei0, self.nei0))
        rows, k = x.shape
        want = tokens * nei0 if self.rows_per_expert else tokens
        if k != self.bank.k or rows != want:
            raise CwError(CW_EINVAL, "x is %dx%d, expected k=%d for %d tokens" % (rows, k, self.bank.k, tokens))
        b = self.bank
        out = torch.empty((tokens, nei0, b.n), dtype=torch.float32, device=x.device)
        if b.dtype == F.MXFP4_R16:  # rows in groups of 16 have the grouped GEMM only
            if tokens and not self._grouped(x, ids, out, tokens):
                raise CwError(CW_ENOTSUP, "a %dx%d MXFP4_R16 bank has no grouped kernel" % (b.n, b.k))
            return out
        if self.grouped_above is not None and tokens > self.grouped_above and self._grouped(x, ids, out, tokens):
            return out
        check(lib().cw_matvec_id(b.dtype, b.n, b.k, b.n_slots, b.slot_stride, _p(b.data), _p(x), int(self.rows_per_expert),
                                 _p(ids), nei0, tokens, _p(out), _stream()))
        return out


@dataclass
class ExpertAct:
    """Silu (alpha/limit unused) or ClampedSwiglu with per-expert biases and padding."""
    kind: int = 0
    alpha: float = 1.702
    limit: float = 7.0
    gate_b: Optional[torch.Tensor] = None
    up_b: Optional[torch.Tensor] = None
    down_b: Optional[torch.Tensor] = None
    pad: int = 0

    @classmethod
    def silu(cls):
        return cls(0)

    @classmethod
    def clamped_swiglu(cls, alpha, limit, gate_b, up_b, down_b, pad=0):
        return cls(1, alpha, limit, gate_b, up_b, down_b, pad)


class MoeLayer:
    """A MoE layer whose experts are resident in device banks (gate, up, down).

    ``slot_table`` (device u32 expert -> slot, NO_SLOT when absent) switches to the bank
    variant: picks resolve through the table and picks without a slot are counted."""

    def __init__(self, gate: ExpertBank, up: ExpertBank, down: ExpertBank, n_experts: int, top_k: int,
                 norm_topk_prob: bool = True, act: ExpertAct = None, slot_table: torch.Tensor = None):
        self.banks = (gate, up, down)
        self.n_experts, self.top_k, self.norm = n_experts, top_k, norm_topk_prob
        self.act = act or ExpertAct.silu()
        self.slot_table = slot_table
        self.hidden, self.inter = gate.k, gate.n
        d = MoeDesc()
        d.n_experts, d.top_k, d.hidden, d.inter = n_experts, top_k, self.hidden, self.inter
        d.norm, d.act = int(norm_topk_prob), self.act.kind
        d.alpha, d.limit, d.pad = self.act.alpha, self.act.limit, self.act.pad
        for m, b in enumerate(self.banks):
            d.dtype[m] = b.dtype
            d.w[m] = b.data.data_ptr()
            d.slot_stride[m] = b.slot_stride
        for m, b in enumerate((self.act.gate_b, self.act.up_b, self.act.down_b)):
            d.bias[m] = None if b is None else b.data_ptr()
        d.slot_table = None if slot_table is None else slot_table.data_ptr()
        d.n_slots = gate.n_slots
        self.desc = d
        self._ws = None

    def workspace(self, tokens, device):
        need = lib().cw_moe_workspace_size(ctypes.byref(self.desc), tokens)
        if need == 0 and tokens > 0:
            raise CwError(CW_EINVAL, lib().cw_last_error().decode(errors="replace"))
        if self._ws is None or self._ws.numel() < need:
            # zero-filled once: the one-token layer keeps its sync state there, at zero between calls
            self._ws = torch.zeros(need, dtype=torch.uint8, device=device)
        return self._ws, need

    def status(self) -> int:
        """The workspace's status word (CW_MOE_STATUS_OFFSET): blocks of one-token calls whose
        barrier gave up or found an invalid sync state. Read on the current stream (the Python
        int waits for it)."""
        if self._ws is None:
            return 0
        word = self._ws[CW_MOE_STATUS_OFFSET:CW_MOE_STATUS_OFFSET + 4].cpu()
        return int(word.view(torch.int32)[0]) & 0xFFFFFFFF

    def forward(self, xs: torch.Tensor, logits: torch.Tensor, missing: torch.Tensor = None):
        """xs (T, hidden) f32, logits (T, E) f32 -> (out (T, hidden), ids (T, K), w (T, K))."""
        _need(xs, torch.float32, "xs")
        _need(logits, torch.float32, "logits")
        t = xs.shape[0]
        if xs.shape[1] != self.hidden or logits.shape != (t, self.n_experts):
            raise CwError(CW_EINVAL, "xs %s / logits %s do not fit the layer" % (tuple(xs.shape), tuple(logits.shape)))
        out = torch.empty((t, self.hidden), dtype=torch.float32, device=xs.device)
        ids = torch.empty((t, self.top_k), dtype=torch.int32, device=xs.device)
        w = torch.empty((t, self.top_k), dtype=torch.float32, device=xs.device)
        ws, need = self.workspace(t, xs.device)
        check(lib().cw_moe_layer(ctypes.byref(self.desc), _p(xs), _p(logits), t, _p(out), _p(ids), _p(w), _p(missing),
                                 _p(ws), need, _stream()))
        return out, ids, w
