"""The C ABI library loads and exports every entry point include/cwmoe.h declares; argument
errors come back as status codes before any GPU work (CPU only)."""
import ctypes
import os
import re

import pytest

import coachwhip_amd as cw
from coachwhip_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "cwmoe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cw_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    L = cw.lib()
    names = declared_symbols()
    assert len(names) >= 25
    for name in names:
        assert hasattr(L, name), name
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_header_constants_match_the_binding():
    """The workspace constants the header publishes (the one-token layer's sync-state bytes and its
    status word's offset) are the ones the Python binding uses."""
    text = open(os.path.join(ROOT, "include", "cwmoe.h")).read()
    consts = dict(re.findall(r"#define (CW_MOE_[A-Z_]+) (\d+)\b", text))
    assert int(consts["CW_MOE_STATE_BYTES"]) == _lib.CW_MOE_STATE_BYTES
    assert int(consts["CW_MOE_STATUS_OFFSET"]) == _lib.CW_MOE_STATUS_OFFSET
    assert _lib.CW_MOE_STATUS_OFFSET + 4 <= _lib.CW_MOE_STATE_BYTES


def test_format_sizes():
    L = cw.lib()
    for dt in cw.formats.WEIGHT_TYPES:
        assert L.cw_block_size(dt) == cw.formats.block_size(dt)
        assert L.cw_type_size(dt) == cw.formats.type_size(dt)
    assert L.cw_block_size(2) == 0 and L.cw_type_size(99) == 0


def test_argument_errors_are_status_codes():
    L = cw.lib()
    # unsupported dtype (Q4_0) is a capability "no", not a crash
    assert L.cw_qmatmul(2, None, 16, 32, None, 1, None, None, 0, None) == _lib.CW_ENOTSUP
    assert b"dtype" in L.cw_last_error()
    # k not a whole number of blocks
    assert L.cw_qmatmul(cw.formats.Q4_K, None, 16, 100, None, 1, None, None, 0, None) == _lib.CW_EINVAL
    assert L.cw_route_topk(None, 1, 2048, 8, 1, None, None, None, None) == _lib.CW_EINVAL
    assert L.cw_route_topk(None, 1, 16, 17, 1, None, None, None, None) == _lib.CW_EINVAL
    assert L.cw_matvec_id(cw.formats.IQ2_XXS, 16, 256, 4, 10, None, None, 0, None, 1, 1, None, None) == _lib.CW_EINVAL
    # zero-sized work is a no-op that needs no device
    assert L.cw_route_topk(None, 0, 16, 2, 1, None, None, None, None) == _lib.CW_OK
    assert L.cw_dequantize(cw.formats.Q8_0, None, 0, None, None) == _lib.CW_OK


def test_moe_descriptor_validation():
    L = cw.lib()
    d = _lib.MoeDesc()
    d.n_experts, d.top_k, d.hidden, d.inter = 256, 8, 2048, 512
    d.dtype[0] = d.dtype[1] = cw.formats.IQ2_XXS
    d.dtype[2] = cw.formats.IQ2_S
    for m in range(3):
        d.w[m] = 0x1000
    d.slot_stride[0] = d.slot_stride[1] = 512 * 8 * 66
    d.slot_stride[2] = 2048 * 2 * 82
    assert L.cw_moe_workspace_size(ctypes.byref(d), 1) > 0
    # the decode's sync state leads every layout, so one workspace serves calls of any size
    assert L.cw_moe_workspace_size(ctypes.byref(d), 1) < L.cw_moe_workspace_size(ctypes.byref(d), 1500)
    d.slot_stride[2] = 100
    assert L.cw_moe_workspace_size(ctypes.byref(d), 1) == 0 and b"stride" in L.cw_last_error()


def test_matmul_id_grouped_probe_and_checks():
    """cw_matmul_id_grouped answers "not supported" (the reference's Ok(false), mv_id.rs:298-307) for
    shapes without a grouped kernel, so the caller falls back to cw_matvec_id; shape errors are
    CW_EINVAL; no GPU is needed to see either."""
    L = cw.lib()
    F = cw.formats
    stride = F.matrix_bytes(F.IQ2_XXS, 512, 2048)
    ws = L.cw_matmul_id_grouped_workspace_size(F.IQ2_XXS, 512, 2048, 256, stride, 0, 8, 1500)
    # piles and tiles for 12,000 picks, the x rows in fp16 and their scales
    assert ws >= 12000 * 8 + 1500 * 2048 * 2 + 1500 * 4
    assert L.cw_matmul_id_grouped_workspace_size(F.IQ2_XXS, 512, 2048, 256, stride, 1, 8, 1500) > ws
    assert L.cw_matmul_id_grouped_workspace_size(F.IQ2_XXS, 512, 2048, 2048, stride, 0, 8, 20) == 0  # > 1024 slots
    assert b"1024" in L.cw_last_error()
    assert L.cw_matmul_id_grouped(F.F16, 512, 2048, 8, stride, None, None, 0, None, 8, 20, None, None, 0,
                                  None) == _lib.CW_ENOTSUP
    assert L.cw_matmul_id_grouped(F.IQ2_XXS, 512, 2048, 8, 100, None, None, 0, None, 8, 20, None, None, 0,
                                  None) == _lib.CW_EINVAL                 # slot stride below the matrix
    assert L.cw_matmul_id_grouped(F.IQ2_XXS, 512, 2048, 8, stride, None, None, 0, None, 8, 0, None, None, 0,
                                  None) == _lib.CW_OK                     # no tokens, no work


def test_next_row_entry_points_reject_bad_arguments():
    """The shrink, the router GEMV, the shared expert and the banks check their arguments before
    any device work (no GPU is needed to see the status codes)."""
    L = cw.lib()
    F = cw.formats
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails its checks first
    # the shrink: Q3_K/Q4_K/Q5_K only; weights need a row length; no work, no device
    assert L.cw_requant_q2k(F.Q8_0, fake, 4, None, 0, fake, None) == _lib.CW_ENOTSUP
    assert b"Q3_K" in L.cw_last_error()
    assert L.cw_requant_q2k(F.Q4_K, None, 4, None, 0, fake, None) == _lib.CW_EINVAL
    assert L.cw_requant_q2k(F.Q4_K, fake, 4, ctypes.c_void_p(0x1000), 0, fake, None) == _lib.CW_EINVAL
    assert L.cw_requant_q2k(F.Q4_K, fake, -1, None, 0, fake, None) == _lib.CW_EINVAL
    assert L.cw_requant_q2k(F.Q4_K, None, 0, None, 0, None, None) == _lib.CW_OK
    # router logits: aligned pointers, f32/f16 weights, hidden a multiple of 4
    assert L.cw_router_logits(0, fake, 8, 64, None, ctypes.c_void_p(0x1004), 1, fake, None) == _lib.CW_EINVAL
    assert L.cw_router_logits(0, None, 8, 64, None, fake, 1, fake, None) == _lib.CW_EINVAL
    assert L.cw_router_logits(0, fake, 8, 64, None, fake, 0, fake, None) == _lib.CW_OK
    # banks: a matrix that is neither readable nor shrinkable, or shrink of a readable non-K type
    src = _lib.BankSource()
    src.n_experts = 4
    for m in range(3):
        src.dtype[m] = F.Q8_0
        src.rows[m], src.cols[m] = 32, 64
        src.expert_bytes[m] = F.matrix_bytes(F.Q8_0, 32, 64)
        src.host[m] = 0x1000
    assert L.cw_bank_device_bytes(ctypes.byref(src), 2) > 0
    src.shrink[0] = 1                                                     # Q8_0 cannot be shrunk
    assert L.cw_bank_device_bytes(ctypes.byref(src), 2) == 0 and b"cannot be shrunk" in L.cw_last_error()
    src.shrink[0] = 0
    src.shape[1] = 0x2000                                                 # weights on a matrix kept as it is
    assert L.cw_bank_device_bytes(ctypes.byref(src), 2) == 0
    src.shape[1] = None
    src.dtype[2], src.rows[2], src.cols[2] = F.Q3_K, 64, 256              # Q3_K is read only through the shrink
    src.expert_bytes[2] = F.matrix_bytes(F.Q3_K, 64, 256)
    assert L.cw_bank_device_bytes(ctypes.byref(src), 2) == 0
    src.shrink[2] = 1                                                     # ... and then its slots are Q2_K
    q2 = F.matrix_bytes(F.Q2_K, 64, 256)
    al = lambda v: (v + 255) // 256 * 256
    want = 2 * al(2 * src.expert_bytes[0]) + al(2 * q2) + 2 * al(8 * src.expert_bytes[2]) + al(4 * 4)
    assert L.cw_bank_device_bytes(ctypes.byref(src), 2) == want
    # a GGUF handle that does not exist
    assert not L.cw_gguf_open(b"/nonexistent/model.gguf")
    assert L.cw_gguf_n_tensors(None) == 0 and L.cw_gguf_find(None, b"x") == -1
