"""ctypes binding of libcwmoe.so, the HIP library behind include/cwmoe.h.

The library must be built in-tree (``make -C coachwhip_amd/csrc``); there is no fallback: every
entry point of this package runs the HIP kernels or raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcwmoe.so")

CW_OK, CW_ENOTSUP, CW_EINVAL, CW_EHIP, CW_EFULL = 0, 1, 2, 3, 4
NO_SLOT = 0xFFFFFFFF
# include/cwmoe.h: the MoE-layer workspace's sync-state bytes and the offset of its status word
CW_MOE_STATE_BYTES, CW_MOE_STATUS_OFFSET = 8448, 8320


class CwError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("cwmoe error %d: %s" % (code, msg))
        self.code = code


class CwNotSupported(CwError):
    pass


_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_U32P = ctypes.POINTER(ctypes.c_uint32)


class MoeDesc(ctypes.Structure):
    """struct cw_moe_desc (include/cwmoe.h)."""
    _fields_ = [("n_experts", _I), ("top_k", _I), ("hidden", _I), ("inter", _I), ("norm", _I),
                ("act", _I), ("alpha", ctypes.c_float), ("limit", ctypes.c_float), ("pad", _I),
                ("dtype", _I * 3), ("w", _P * 3), ("slot_stride", _L * 3), ("bias", _P * 3),
                ("slot_table", _P), ("n_slots", _I)]


class SharedDesc(ctypes.Structure):
    """struct cw_shared_desc (include/cwmoe.h)."""
    _fields_ = [("hidden", _I), ("inter", _I), ("dtype", _I * 3), ("w", _P * 3), ("gate_inp", _P)]


class BankSource(ctypes.Structure):
    """struct cw_bank_source (include/cwmoe.h)."""
    _fields_ = [("n_experts", _I), ("dtype", _I * 3), ("rows", _L * 3), ("cols", _L * 3), ("expert_bytes", _L * 3),
                ("host", _P * 3), ("shrink", _I * 3), ("shape", _P * 3)]


class BankStats(ctypes.Structure):
    """struct cw_bank_stats (include/cwmoe.h)."""
    _fields_ = [(name, ctypes.c_uint64) for name in
                ("hits", "prefetch_hits", "loads", "bytes_loaded", "prefetch_copies", "crowded")]


# every symbol include/cwmoe.h declares, with its signature
SIGNATURES = {
    "cw_version": ([], ctypes.c_char_p),
    "cw_last_error": ([], ctypes.c_char_p),
    "cw_block_size": ([_I], _I),
    "cw_type_size": ([_I], _I),
    "cw_dequantize": ([_I, _P, _L, _P, _P], _I),
    "cw_qmatmul_workspace_size": ([_I, _L, _L, _L], ctypes.c_size_t),
    "cw_qmatmul": ([_I, _P, _L, _L, _P, _L, _P, _P, ctypes.c_size_t, _P], _I),
    "cw_route_topk": ([_P, _I, _I, _I, _I, _P, _P, _P], _I),
    "cw_router_logits": ([_I, _P, _I, _I, _P, _P, _I, _P, _P], _I),
    "cw_matvec_id": ([_I, _L, _L, _L, _L, _P, _P, _I, _P, _I, _I, _P, _P], _I),
    "cw_matmul_id_grouped_workspace_size": ([_I, _L, _L, _L, _L, _I, _I, _I], ctypes.c_size_t),
    "cw_matmul_id_grouped": ([_I, _L, _L, _L, _L, _P, _P, _I, _P, _I, _I, _P, _P, ctypes.c_size_t, _P], _I),
    "cw_rows16_bytes": ([_L, _L], _L),
    "cw_repack_rows16": ([_P, _L, _P, _L, _L, _L, _L, _P], _I),
    "cw_swiglu": ([_P, _P, _P, _L, _P], _I),
    "cw_clamped_swiglu": ([_P, _P, _P, _P, _P, _L, _I, _I, ctypes.c_float, ctypes.c_float, _P, _P], _I),
    "cw_weighted_sum": ([_P, _P, _P, _P, _I, _I, _I, _P, _P], _I),
    "cw_slots_resolve": ([_P, _P, _I, _P, _P, _P], _I),
    "cw_moe_workspace_size": ([ctypes.POINTER(MoeDesc), _I], ctypes.c_size_t),
    "cw_moe_layer": ([ctypes.POINTER(MoeDesc), _P, _P, _I, _P, _P, _P, _P, _P, ctypes.c_size_t, _P], _I),
    "cw_moe_layer_noalloc": ([ctypes.POINTER(MoeDesc), _P, _P, _I, _P, _P, _P, _P, _P], _I),
    "cw_shared_expert_workspace_size": ([ctypes.POINTER(SharedDesc), _I], ctypes.c_size_t),
    "cw_shared_expert": ([ctypes.POINTER(SharedDesc), _P, _I, _P, _I, _P, ctypes.c_size_t, _P], _I),
    "cw_gguf_open": ([ctypes.c_char_p], _P),
    "cw_gguf_close": ([_P], None),
    "cw_gguf_version": ([_P], _I),
    "cw_gguf_n_tensors": ([_P], _L),
    "cw_gguf_find": ([_P, ctypes.c_char_p], _L),
    "cw_gguf_tensor": ([_P, _L, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_I), ctypes.POINTER(_I),
                        ctypes.POINTER(_L), ctypes.POINTER(_L), ctypes.POINTER(_L)], _I),
    "cw_gguf_data": ([_P, _L], _P),
    "cw_gguf_meta_int": ([_P, ctypes.c_char_p, ctypes.POINTER(_L)], _I),
    "cw_gguf_meta_float": ([_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)], _I),
    "cw_gguf_meta_str": ([_P, ctypes.c_char_p], ctypes.c_char_p),
    "cw_gguf_experts": ([_P, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_L), ctypes.POINTER(_L), ctypes.POINTER(_L),
                         ctypes.POINTER(_L), ctypes.POINTER(_P)], _I),
    "cw_device_errors": ([], ctypes.c_uint32),
    "cw_slots_new": ([_I], _P),
    "cw_slots_free": ([_P], None),
    "cw_slots_assign": ([_P, _P, _I, _P, _P, ctypes.POINTER(_I), _P, ctypes.POINTER(_I),
                         ctypes.POINTER(ctypes.c_uint64)], _I),
    "cw_slots_release": ([_P, ctypes.c_uint32], None),
    "cw_slots_pop": ([_P, _P, _I], None),
    "cw_slots_reserve": ([_P, _P, _I, _P, _P], _I),
    "cw_slots_holder": ([_P, _I], ctypes.c_uint32),
    "cw_slots_slot_of": ([_P, ctypes.c_uint32], _I),
    "cw_slots_lru": ([_P, _P], None),
    "cw_slots_is_prefetched": ([_P, ctypes.c_uint32], _I),
    "cw_slots_table": ([_P, _P, _I], None),
    "cw_requant_q2k": ([_I, _P, _L, _P, _L, _P, _P], _I),
    "cw_bank_device_bytes": ([ctypes.POINTER(BankSource), _I], ctypes.c_size_t),
    "cw_bank_new": ([ctypes.POINTER(BankSource), _I, _P, ctypes.c_size_t], _P),
    "cw_bank_free": ([_P], None),
    "cw_bank_ensure": ([_P, _P, _I, _P, ctypes.POINTER(_I)], _I),
    "cw_bank_prefetch": ([_P, _P, _I], _I),
    "cw_bank_fill_desc": ([_P, ctypes.POINTER(MoeDesc)], _I),
    "cw_bank_table": ([_P], _P),
    "cw_bank_slot_of": ([_P, ctypes.c_uint32], _I),
    "cw_bank_get_stats": ([_P, ctypes.POINTER(BankStats)], None),
}

_lib = None


def lib():
    """The loaded library; raises when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError("libcwmoe.so is not built: run `make -C %s/csrc` (or __graft_entry__.build())" % HERE)
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def check(rc):
    if rc != CW_OK:
        msg = lib().cw_last_error().decode(errors="replace")
        raise (CwNotSupported if rc == CW_ENOTSUP else CwError)(rc, msg)
    return rc
