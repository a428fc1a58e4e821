"""A layer's expert bank on the device, filled from host memory (cw_bank_* in include/cwmoe.h).

Mirrors the plain branch of ExpertStore (crates/engine/src/experts.rs: Bank 62-82, make_bank
1320-1378, ensure 1489-1641, prefetch 1004-1098): a forward first ``ensure``s the experts its
tokens picked, which copies the misses into least-recently-used slots and brings the device
table up to date on the current stream, then runs the layer through that table. The expert
store is host memory (pinned, so copies are DMA) instead of the SSD.
"""
import ctypes

import numpy as np
import torch

from . import formats as F
from . import ops
from ._lib import BankSource, BankStats, CW_EFULL, CW_EINVAL, CwError, MoeDesc, check, lib


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def pinned_copy(raw) -> torch.Tensor:
    """Host bytes as a pinned (page-locked) uint8 tensor, the form the bank copies by DMA."""
    raw = np.ascontiguousarray(np.asarray(raw, dtype=np.uint8).reshape(-1))
    t = torch.empty(raw.size, dtype=torch.uint8, pin_memory=True)
    t.numpy()[:] = raw
    return t


class Bank:
    """n_slots device slots of each of a layer's three expert matrices (gate, up, down).

    ``host`` holds three uint8 CPU tensors, matrix m of expert e at byte e * expert_bytes[m];
    ``shapes`` the (rows, cols) of one expert's matrix, ``dtypes`` their GGUF types. A matrix
    with ``shrink[m]`` (a Q3_K, Q4_K or Q5_K store) is held as Q2_K, shrunk on arrival, weighted
    by ``shape[m]`` (device f32, one per column) when given (ExpertStore::shrink_into,
    crates/engine/src/experts.rs:1245-1273)."""

    def __init__(self, host, dtypes, shapes, n_experts, n_slots, device="cuda", pin=True, shrink=(False, False, False),
                 shape=(None, None, None)):
        # numpy stores are copied to pinned memory (read by the fill kernel) unless pin is False
        # (then they are copied by DMA from where they are)
        as_tensor = pinned_copy if pin else (lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)))
        self.host = [h if isinstance(h, torch.Tensor) else as_tensor(h) for h in host]
        self.dtypes, self.shapes = tuple(dtypes), [tuple(s) for s in shapes]
        self.n_experts, self.n_slots = n_experts, n_slots
        self.expert_bytes = [F.matrix_bytes(d, r, c) for d, (r, c) in zip(self.dtypes, self.shapes)]
        src = BankSource()
        src.n_experts = n_experts
        for m in range(3):
            if self.host[m].device.type != "cpu" or self.host[m].numel() < n_experts * self.expert_bytes[m]:
                raise CwError(CW_EINVAL, "bank: host matrix %d holds %d bytes for %d experts of %d" %
                              (m, self.host[m].numel(), n_experts, self.expert_bytes[m]))
            src.dtype[m] = self.dtypes[m]
            src.rows[m], src.cols[m] = self.shapes[m]
            src.expert_bytes[m] = self.expert_bytes[m]
            src.host[m] = self.host[m].data_ptr()
            src.shrink[m] = int(bool(shrink[m]))
            src.shape[m] = None if shape[m] is None else shape[m].data_ptr()
        self._shape = shape  # kept alive with the bank
        self._src = src
        need = lib().cw_bank_device_bytes(ctypes.byref(src), n_slots)
        if need == 0:
            raise CwError(CW_EINVAL, lib().cw_last_error().decode(errors="replace"))
        self.mem = torch.empty(need + 256, dtype=torch.uint8, device=device)
        base = (-self.mem.data_ptr()) % 256
        self._mem = self.mem[base:base + need]
        self._h = lib().cw_bank_new(ctypes.byref(src), n_slots, ctypes.c_void_p(self._mem.data_ptr()), need)
        if not self._h:
            raise CwError(CW_EINVAL, lib().cw_last_error().decode(errors="replace"))
        d = MoeDesc()
        check(lib().cw_bank_fill_desc(self._h, ctypes.byref(d)))
        self._desc = d
        root = self._mem.data_ptr()
        self.banks = []
        for m in range(3):  # slot dtype and stride from the bank (Q2_K for a shrunk matrix)
            off = d.w[m] - root
            data = self._mem[off:off + n_slots * d.slot_stride[m]]
            rows, cols = self.shapes[m]
            self.banks.append(ops.ExpertBank(data, d.dtype[m], rows, cols, n_slots, d.slot_stride[m]))
        off = d.slot_table - root
        self.table = self._mem[off:off + 4 * n_experts].view(torch.int32)

    def close(self):
        if getattr(self, "_h", None):
            lib().cw_bank_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library may already be gone
            pass

    def ensure(self, needed):
        """Places the experts in ``needed`` (any int array, duplicates ignored) on the current
        stream. Returns the number copied in, or None when the bank cannot hold them now."""
        needed = np.ascontiguousarray(np.asarray(needed).reshape(-1), dtype=np.uint32)
        loaded = ctypes.c_int(0)
        rc = lib().cw_bank_ensure(self._h, needed.ctypes.data_as(ctypes.c_void_p), needed.size, _stream(),
                                  ctypes.byref(loaded))
        if rc == CW_EFULL:
            return None
        check(rc)
        return loaded.value

    def prefetch(self, predicted):
        """Starts copying predicted experts into free slots on the bank's own stream; returns how many."""
        predicted = np.ascontiguousarray(np.asarray(predicted).reshape(-1), dtype=np.uint32)
        n = lib().cw_bank_prefetch(self._h, predicted.ctypes.data_as(ctypes.c_void_p), predicted.size)
        if n < 0:
            check(-n)
        return n

    def slot_of(self, expert):
        return lib().cw_bank_slot_of(self._h, int(expert))

    def stats(self):
        st = BankStats()
        lib().cw_bank_get_stats(self._h, ctypes.byref(st))
        return {name: getattr(st, name) for name, _ in BankStats._fields_}

    def moe_layer(self, top_k, norm_topk_prob=True, act=None):
        """The layer over this bank: picks resolve through the bank's table."""
        g, u, d = self.banks
        return ops.MoeLayer(g, u, d, self.n_experts, top_k, norm_topk_prob, act=act, slot_table=self.table)
