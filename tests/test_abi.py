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
    d.slot_stride[2] = 100
    assert L.cw_moe_workspace_size(ctypes.byref(d), 1) == 0 and b"stride" in L.cw_last_error()
