"""cw_moe_layer_noalloc (the layer on the library's static per-device scratch) against cw_moe_layer
(the same layer on a caller's workspace), through the C ABI: two calls in a row, the second with a
smaller input, each equal to the workspace entry point's output bit for bit (ids, weights, output,
missing count); a call too large for the scratch is refused before any device work."""
import ctypes

import numpy as np
import pytest
import torch

import coachwhip_amd as cw
from coachwhip_amd import _lib
from coachwhip_amd import formats as F
from coachwhip_amd import ops, synth

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _layer(rng, E, K, dts, n_slots):
    layer = synth.moe_weights(E, K, 2048, 512, dts, rng, n_slots=n_slots)
    banks = [ops.ExpertBank.from_blocks(layer.host[m], layer.dtypes[m], *shape, n_slots)
             for m, shape in enumerate([(512, 2048), (512, 2048), (2048, 512)])]
    return banks


def _run(entry, desc, x, logits, K, ws=None):
    T, H = x.shape
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    ids = torch.empty((T, K), dtype=torch.int32, device="cuda")
    w = torch.empty((T, K), dtype=torch.float32, device="cuda")
    missing = torch.zeros(1, dtype=torch.int32, device="cuda")
    L = cw.lib()
    if entry == "noalloc":
        rc = L.cw_moe_layer_noalloc(ctypes.byref(desc), _p(x), _p(logits), T, _p(out), _p(ids), _p(w), _p(missing), None)
    else:
        need = L.cw_moe_workspace_size(ctypes.byref(desc), T)
        rc = L.cw_moe_layer(ctypes.byref(desc), _p(x), _p(logits), T, _p(out), _p(ids), _p(w), _p(missing), _p(ws), need,
                            None)
    _lib.check(rc)
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in (out, ids, w, missing)]


def test_noalloc_layer_equals_the_workspace_layer():
    print("noalloc: two calls, the second smaller", flush=True)
    rng = np.random.default_rng(101)
    E, K, S = 512, 10, 56
    banks = _layer(rng, E, K, (F.IQ3_S, F.IQ3_S, F.Q4_K), S)
    table = np.full(E, 0xFFFFFFFF, dtype=np.uint32)
    table[rng.choice(E, size=S, replace=False)] = rng.permutation(S).astype(np.uint32)
    tab = torch.from_numpy(table.view(np.int32)).cuda()
    moe = ops.MoeLayer(*banks, n_experts=E, top_k=K, norm_topk_prob=True, slot_table=tab)
    desc = moe.desc
    L = cw.lib()
    ws = torch.zeros(L.cw_moe_workspace_size(ctypes.byref(desc), 40), dtype=torch.uint8, device="cuda")
    # 40 tokens (the grouped MFMA path), then 1 token (the one-launch decode, whose barrier state
    # lives in the scratch), then 40 again: unmasked logits, so some picks are missing
    for T in (40, 1, 40):
        x = torch.from_numpy(rng.standard_normal((T, 2048)).astype(np.float32)).cuda()
        lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda()
        a = _run("noalloc", desc, x, lg, K)
        b = _run("workspace", desc, x, lg, K, ws)
        print("  T", T, "missing", int(a[3][0]), flush=True)
        for got, want in zip(a, b):
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        assert np.all(np.isfinite(a[0]))


def test_noalloc_layer_refuses_what_does_not_fit():
    print("noalloc: refusal", flush=True)
    rng = np.random.default_rng(102)
    E, K = 64, 8
    banks = _layer(rng, E, K, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), E)
    moe = ops.MoeLayer(*banks, n_experts=E, top_k=K, norm_topk_prob=True)
    L = cw.lib()
    T = 1500
    assert L.cw_moe_workspace_size(ctypes.byref(moe.desc), T) > _lib_noalloc_bytes()
    x = torch.zeros((T, 2048), dtype=torch.float32, device="cuda")
    lg = torch.zeros((T, E), dtype=torch.float32, device="cuda")
    out = torch.full((T, 2048), 7.0, dtype=torch.float32, device="cuda")
    rc = L.cw_moe_layer_noalloc(ctypes.byref(moe.desc), _p(x), _p(lg), T, _p(out), None, None, None, None)
    assert rc == _lib.CW_EINVAL and b"scratch" in L.cw_last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())                   # nothing ran


def _lib_noalloc_bytes():
    return 8 << 20
