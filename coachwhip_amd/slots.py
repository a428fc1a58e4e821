"""Slots: the expert bank's bookkeeping without its memory (crates/engine/src/experts.rs:84-286),
implemented in C++ (cw_slots.cpp) behind the C ABI. Pure host code: no GPU needed."""
import ctypes

import numpy as np

from ._lib import NO_SLOT, lib


class Plan:
    """What one forward needs from the bank: (expert, slot) hits and misses, prefetch hits."""

    def __init__(self, hits, misses, prefetch_hits):
        self.hits, self.misses, self.prefetch_hits = hits, misses, prefetch_hits

    def __eq__(self, other):
        return (self.hits, self.misses, self.prefetch_hits) == (other.hits, other.misses, other.prefetch_hits)

    def __repr__(self):
        return "Plan(hits=%r, misses=%r, prefetch_hits=%d)" % (self.hits, self.misses, self.prefetch_hits)


def _ready_arr(ready, n):
    if ready is None:
        return None
    return np.array([1 if ready(s) else 0 for s in range(n)], dtype=np.uint8)


def _u32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class Slots:
    def __init__(self, n):
        self.n = n
        self._h = lib().cw_slots_new(n)
        if not self._h:
            raise ValueError("Slots: %d slots" % n)

    def __del__(self):
        if getattr(self, "_h", None):
            try:
                lib().cw_slots_free(self._h)
            except Exception:  # interpreter shutdown: the library may already be gone
                pass
            self._h = None

    def assign(self, needed, ready=None):
        """Plan, or None (and nothing changed) when too few slots are free."""
        needed = _u32(needed)
        k = len(needed)
        hits = np.empty(2 * max(k, 1), dtype=np.uint32)
        misses = np.empty(2 * max(k, 1), dtype=np.uint32)
        nh, nm, ph = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_uint64(0)
        ra = _ready_arr(ready, self.n)
        rc = lib().cw_slots_assign(self._h, _ptr(needed), k, _ptr(ra), _ptr(hits), ctypes.byref(nh), _ptr(misses),
                                   ctypes.byref(nm), ctypes.byref(ph))
        if rc < 0:
            raise ValueError("Slots.assign: bad argument")
        if rc == 0:
            return None
        pairs = lambda a, n: [(int(a[2 * i]), int(a[2 * i + 1])) for i in range(n)]
        return Plan(pairs(hits, nh.value), pairs(misses, nm.value), int(ph.value))

    def release(self, e):
        lib().cw_slots_release(self._h, e)

    def pop(self, used):
        used = _u32(used)
        lib().cw_slots_pop(self._h, _ptr(used), len(used))

    def reserve(self, predicted, ready=None):
        predicted = _u32(predicted)
        out = np.empty(2 * max(len(predicted), 1), dtype=np.uint32)
        n = lib().cw_slots_reserve(self._h, _ptr(predicted), len(predicted), _ptr(_ready_arr(ready, self.n)), _ptr(out))
        return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(n)]

    # views of the state, as the reference's fields
    @property
    def holder(self):
        return [None if (h := lib().cw_slots_holder(self._h, s)) == NO_SLOT else int(h) for s in range(self.n)]

    @property
    def lru(self):
        order = np.empty(self.n, dtype=np.int32)
        lib().cw_slots_lru(self._h, _ptr(order))
        return [int(v) for v in order]

    @property
    def slot_of(self):
        return {e: s for s, e in enumerate(self.holder) if e is not None}

    def is_prefetched(self, e):
        return bool(lib().cw_slots_is_prefetched(self._h, e))

    def table(self, n_experts):
        t = np.empty(n_experts, dtype=np.uint32)
        lib().cw_slots_table(self._h, _ptr(t), n_experts)
        return t
