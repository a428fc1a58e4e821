"""MoE layers at BASELINE.json's full prefill sizes: config 3 (256 experts, top-8, hidden 2048, FFN
512, IQ2_XXS / IQ2_S, 1,500 tokens) and config 4 (128 experts, top-4, hidden and FFN 2880, MXFP4,
clamped SwiGLU, 2,048 tokens), on the grouped MFMA path.

The oracle cannot run a whole batch of this size in test time, so the checks rest on a property
of the computation: each token's output depends only on its own activations and logits (its
picks' rows are computed independently inside their tiles, and summed per token in pick order).
Hence:
- a sample of tokens from the full batch equals the oracle run on those tokens alone (rel-L2
  <= 1e-3, the north-star tolerance; ids identical);
- permuting the batch permutes the outputs, bit for bit;
- a token's output is bit-identical in another batch that shares only part of its tokens."""
import zlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CONFIGS = [
    # name, E, K, h, I, dtypes, act, T
    ("config3_prefill", 256, 8, 2048, 512, "iq2", 0, 1500),
    ("config4_prefill", 128, 4, 2880, 2880, "mxfp4", 1, 2048),          # block-scaled MFMA (FP4 x FP6 terms)
    ("config4_prefill_fp16", 128, 4, 2880, 2880, "mxfp4", 1, 2048),     # CWMOE_MXFP4_F16=1: the fp16 MFMA path
]


def _layer(name, E, K, h, I, kind, act):
    import torch
    from coachwhip_amd import formats as F
    from coachwhip_amd import ops, synth
    dts = (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S) if kind == "iq2" else (F.MXFP4,) * 3
    gen = torch.Generator(device="cuda")
    gen.manual_seed(zlib.crc32(name.replace("_fp16", "").encode()))
    shapes = [(I, h), (I, h), (h, I)]
    banks = []
    for m, (n, k) in enumerate(shapes):
        raw = synth.device_blocks(dts[m], E * n * k, gen)
        banks.append(ops.ExpertBank(raw, dts[m], n, k, E, F.matrix_bytes(dts[m], n, k)))
    ea = ops.ExpertAct.silu()
    bias = None
    if act == 1:
        bias = [torch.randn((E, I), generator=gen, device="cuda") * 0.02, torch.randn((E, I), generator=gen, device="cuda") * 0.02,
                torch.randn((E, h), generator=gen, device="cuda") * 0.02]
        ea = ops.ExpertAct.clamped_swiglu(1.702, 7.0, *bias)
    moe = ops.MoeLayer(*banks, n_experts=E, top_k=K, norm_topk_prob=True, act=ea)
    host = synth.MoeWeights(E, K, h, I, dts, [b.data.cpu().numpy() for b in banks], [b.slot_stride for b in banks], E,
                            act=act, bias=None if bias is None else [b.cpu().numpy() for b in bias])
    return moe, host


@pytest.mark.parametrize("name,E,K,h,I,kind,act,T", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_full_size_prefill(name, E, K, h, I, kind, act, T, monkeypatch):
    import torch
    from coachwhip_amd import synth
    from oracle import oracle as O
    monkeypatch.delenv("CWMOE_PREFILL_MIN_TOKENS", raising=False)
    monkeypatch.setenv("CWMOE_MXFP4_F16", "1" if name.endswith("_fp16") else "0")
    print("full size", name, T, "tokens", flush=True)
    moe, host = _layer(name, E, K, h, I, kind, act)
    rng = np.random.default_rng(zlib.crc32(name.replace("_fp16", "").encode()) + 1)
    x = rng.standard_normal((T, h)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    out, ids, _ = moe.forward(torch.from_numpy(x).cuda(), torch.from_numpy(logits).cuda())
    out = out.cpu().numpy()
    ids = ids.cpu().numpy().view(np.uint32)

    # a sample of tokens against the oracle on those tokens alone
    sample = rng.choice(T, 6, replace=False)
    assert not synth.near_ties_within_top_k(logits[sample], K)
    want, wids, _, _ = O.moe_layer(host, x[sample], logits[sample])
    assert np.array_equal(ids[sample], wids)
    err = O.rel_l2(out[sample], want)
    print("  sampled rel_l2", err, flush=True)
    assert err <= 1e-3

    # a permuted batch: outputs permuted bit for bit
    perm = rng.permutation(T)
    out_p = moe.forward(torch.from_numpy(x[perm]).cuda(), torch.from_numpy(logits[perm]).cuda())[0].cpu().numpy()
    assert np.array_equal(out_p, out[perm])

    # another batch sharing the first half of the tokens: those rows bit-identical
    x2, l2 = x.copy(), logits.copy()
    x2[T // 2:] = rng.standard_normal((T - T // 2, h)).astype(np.float32)
    l2[T // 2:] = rng.standard_normal((T - T // 2, E)).astype(np.float32)
    out_2 = moe.forward(torch.from_numpy(x2).cuda(), torch.from_numpy(l2).cuda())[0].cpu().numpy()
    assert np.array_equal(out_2[:T // 2], out[:T // 2])
    assert np.all(np.isfinite(out))
