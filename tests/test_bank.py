"""The device expert bank (cw_bank_*): bookkeeping, copies, the device table, prefetch, and a
layer run through it.

What pins it: the bookkeeping must follow Slots (the C++ port pinned by the reference's bank.rs
cases in test_slots.py) call for call; every slot must hold its expert's bytes exactly as the
host store (a GGUF file's ffn_*_exps slices) has them; the device table must equal the
bookkeeping's expert -> slot map (the reference's sync_table, crates/engine/src/experts.rs:
73-81); and a layer run through the bank must match the resident oracle (the experts'
arithmetic does not depend on which slot holds them)."""
import ctypes
import zlib

import numpy as np
import pytest

from coachwhip_amd import CwError
from coachwhip_amd import formats as F
from coachwhip_amd._lib import NO_SLOT, BankSource, lib

SHAPES = [(256, 256), (256, 256), (256, 256)]
DTYPES = (F.IQ2_XXS, F.IQ2_XXS, F.Q4_K)


def _source(n_experts=40, expert_bytes=None):
    src = BankSource()
    src.n_experts = n_experts
    for m in range(3):
        src.dtype[m] = DTYPES[m]
        src.rows[m], src.cols[m] = SHAPES[m]
        src.expert_bytes[m] = F.matrix_bytes(DTYPES[m], *SHAPES[m]) if expert_bytes is None else expert_bytes
        src.host[m] = 4096  # never read: these tests only size and check the source
    return src


def test_device_bytes_and_source_checks():
    src = _source()
    eb = [F.matrix_bytes(d, *s) for d, s in zip(DTYPES, SHAPES)]
    align = lambda x: (x + 255) // 256 * 256
    assert lib().cw_bank_device_bytes(ctypes.byref(src), 8) == sum(align(8 * b) for b in eb) + align(4 * 40)
    assert lib().cw_bank_device_bytes(ctypes.byref(_source(expert_bytes=100)), 8) == 0       # wrong size
    assert b"expected" in lib().cw_last_error()
    assert lib().cw_bank_device_bytes(ctypes.byref(src), 0) == 0                              # no slots
    bad = _source()
    bad.cols[2] = 200                                                                          # not whole blocks
    assert lib().cw_bank_device_bytes(ctypes.byref(bad), 8) == 0
    bad = _source()
    bad.host[1] = None
    assert lib().cw_bank_device_bytes(ctypes.byref(bad), 8) == 0
    assert not lib().cw_bank_new(ctypes.byref(src), 8, None, 1 << 20)                         # no device memory


# ------------------------------------------------------------------------------ on the GPU

def _random_store(rng, n_experts):
    from coachwhip_amd import synth
    return [synth.random_blocks(d, n_experts * r * c, rng) for d, (r, c) in zip(DTYPES, SHAPES)]


def _check_bank(bank, mirror, raw, needed, skip=()):
    import torch
    torch.cuda.synchronize()
    table, want = bank.table.cpu().numpy().view(np.uint32).copy(), mirror.table(bank.n_experts)
    table[list(skip)] = want[list(skip)]
    assert np.array_equal(table, want)
    for e in set(int(v) for v in needed):
        slot = mirror.slot_of[e]
        assert bank.slot_of(e) == slot
        for m in range(3):
            eb = bank.expert_bytes[m]
            got = bank.banks[m].data[slot * eb:(slot + 1) * eb].cpu().numpy()
            assert np.array_equal(got, raw[m][e * eb:(e + 1) * eb]), (e, m, slot)


@pytest.mark.gpu
@pytest.mark.parametrize("pin", [True, False], ids=["pinned_fill_kernel", "pageable_dma"])
def test_bank_follows_slots_and_holds_the_bytes(pin):
    from coachwhip_amd.bank import Bank
    from coachwhip_amd.slots import Slots
    print("bank: 80 seeded ensure calls, pinned", pin, flush=True)
    rng = np.random.default_rng(5)
    E, S = 40, 8
    raw = _random_store(rng, E)
    bank = Bank(raw, DTYPES, SHAPES, E, S, pin=pin)
    mirror = Slots(S)
    hot = rng.choice(E, 10, replace=False)
    loads = hits = refused = 0
    for step in range(80):
        size = int(rng.integers(1, S + 2))                 # S + 1 needs more than the bank holds
        pool = hot if rng.random() < 0.7 and size <= len(hot) else np.arange(E)
        needed = rng.choice(pool, size, replace=False).astype(np.uint32)
        if step % 9 == 4:
            needed = np.concatenate([needed, needed[:2]])  # duplicates are ignored
        got = bank.ensure(needed)
        uniq = list(dict.fromkeys(int(v) for v in needed))
        if len(uniq) > S:
            assert got is None
            refused += 1
            continue
        plan = mirror.assign(uniq)
        assert plan is not None                            # nothing is being filled: always placeable
        assert got == len(plan.misses)
        loads += len(plan.misses)
        hits += len(plan.hits)
        _check_bank(bank, mirror, raw, uniq)
    st = bank.stats()
    assert (st["loads"], st["hits"], st["crowded"], st["prefetch_copies"]) == (loads, hits, 0, 0)
    assert st["bytes_loaded"] == loads * sum(bank.expert_bytes)
    assert refused > 0 and hits > 0 and loads > S


@pytest.mark.gpu
def test_bank_prefetch_keeps_the_placed_slots():
    import torch
    from coachwhip_amd.bank import Bank
    from coachwhip_amd.slots import Slots
    print("bank: prefetch", flush=True)
    rng = np.random.default_rng(6)
    E, S = 32, 8
    raw = _random_store(rng, E)
    bank = Bank(raw, DTYPES, SHAPES, E, S)
    mirror = Slots(S)
    assert bank.ensure([0, 1, 2]) == 3 and mirror.assign([0, 1, 2]) is not None
    # 1 is held; 5, 6, 7 go to free slots without waiting for anything on the stream
    assert bank.prefetch([5, 6, 7, 1]) == 3
    assert mirror.reserve([5, 6, 7, 1]) == [(e, bank.slot_of(e)) for e in (5, 6, 7)]
    assert bank.ensure([5, 6, 3]) == 1                     # 5, 6 were prefetched, 3 is a miss
    plan = mirror.assign([5, 6, 3])
    assert plan.prefetch_hits == 2 and len(plan.misses) == 1
    torch.cuda.synchronize()
    table = bank.table.cpu().numpy().view(np.uint32)
    assert table[7] in (NO_SLOT, mirror.slot_of[7])        # listed once its copy has landed
    _check_bank(bank, mirror, raw, [5, 6, 3], skip=[7])
    placed = {e: bank.slot_of(e) for e in (5, 6, 3)}
    # eight predictions, but the three slots the last ensure placed are not taken
    n = bank.prefetch(list(range(10, 18)))
    assert n == S - 3
    for e, s in placed.items():
        assert bank.slot_of(e) == s
    ready = [0 if s in placed.values() else 1 for s in range(S)]
    mirror.reserve(list(range(10, 18)), ready=lambda s: ready[s])
    torch.cuda.synchronize()
    assert bank.ensure([]) == 0                            # the copies are done: the table lists them all
    _check_bank(bank, mirror, raw, [5, 6, 3] + list(range(10, 10 + n)))
    st = bank.stats()
    assert (st["prefetch_copies"], st["prefetch_hits"], st["loads"]) == (3 + n, 2, 4)


@pytest.mark.gpu
def test_bank_prefetch_unlists_its_victims():
    """A prefetch that takes the slots of held experts takes those experts out of the device table
    in the ensure stream's order before it copies (the reference's not-ready mark and table sync,
    crates/engine/src/experts.rs:1052-1058): work queued after it counts them missing instead of
    reading a slot being overwritten. The prefetched experts are listed by the next ensure."""
    import torch
    from coachwhip_amd.bank import Bank
    from coachwhip_amd.slots import Slots
    print("bank: prefetch victims", flush=True)
    rng = np.random.default_rng(7)
    E, S = 32, 8
    raw = _random_store(rng, E)
    bank = Bank(raw, DTYPES, SHAPES, E, S)
    mirror = Slots(S)
    assert bank.ensure(list(range(S))) == S and mirror.assign(list(range(S))) is not None
    assert bank.ensure([0, 1]) == 0 and mirror.assign([0, 1]) is not None
    held = {e: bank.slot_of(e) for e in range(S)}
    ready = [0 if s in (held[0], held[1]) else 1 for s in range(S)]
    want = mirror.reserve([20, 21, 22], ready=lambda s: ready[s])
    assert bank.prefetch([20, 21, 22]) == 3
    assert want == [(e, bank.slot_of(e)) for e in (20, 21, 22)]
    taken = {s for _, s in want}
    victims = [e for e in range(S) if held[e] in taken]
    assert len(victims) == 3 and not {0, 1} & set(victims)
    torch.cuda.synchronize()
    table = bank.table.cpu().numpy().view(np.uint32)
    for e in range(S):
        assert table[e] == (NO_SLOT if e in victims else held[e]), e
    for e in (20, 21, 22):
        assert table[e] == NO_SLOT                         # listed by the next ensure
    assert bank.ensure([20, 21, 22]) == 0                  # all three were prefetched
    assert mirror.assign([20, 21, 22]).prefetch_hits == 3
    _check_bank(bank, mirror, raw, [20, 21, 22])


@pytest.mark.gpu
def test_bank_ensure_on_another_stream_follows_the_prefetch_patches():
    """A prefetch takes its victims out of the table on the previous ensure's stream. An ensure on
    a different stream that places a victim again must list it after that removal, not before:
    the previous stream is held back by a long kernel here, so without the ordering the victim's
    new entry would be overwritten by the late removal and the expert counted missing."""
    import torch
    from coachwhip_amd.bank import Bank
    from coachwhip_amd.slots import Slots
    print("bank: ensure on another stream", flush=True)
    rng = np.random.default_rng(8)
    E, S = 32, 8
    raw = _random_store(rng, E)
    bank = Bank(raw, DTYPES, SHAPES, E, S)
    mirror = Slots(S)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(s1):
        assert bank.ensure(list(range(S))) == S and mirror.assign(list(range(S))) is not None
        assert bank.ensure([0, 1]) == 0 and mirror.assign([0, 1]) is not None
        held = {e: bank.slot_of(e) for e in range(S)}
        ready = [0 if s in (held[0], held[1]) else 1 for s in range(S)]
        torch.cuda._sleep(50_000_000)                      # s1 busy: the removal patches wait behind it
        want = mirror.reserve([20, 21, 22], ready=lambda s: ready[s])
        assert bank.prefetch([20, 21, 22]) == 3
    victims = [e for e in range(S) if held[e] in {s for _, s in want}]
    assert len(victims) == 3
    with torch.cuda.stream(s2):
        back = victims[:2]
        loaded = bank.ensure(back + [20])
        plan = mirror.assign(back + [20])
        assert plan is not None and loaded == len(plan.misses) == 2
    torch.cuda.synchronize()
    # 21 and 22 are prefetched but not asked for: listed once their copies have landed
    table = bank.table.cpu().numpy().view(np.uint32)
    assert all(table[e] in (NO_SLOT, mirror.slot_of[e]) for e in (21, 22))
    _check_bank(bank, mirror, raw, back + [20], skip=(21, 22))


@pytest.mark.gpu
def test_bank_rejects_bad_calls():
    from coachwhip_amd.bank import Bank
    print("bank: errors", flush=True)
    rng = np.random.default_rng(7)
    E, S = 16, 4
    raw = _random_store(rng, E)
    bank = Bank(raw, DTYPES, SHAPES, E, S)
    assert bank.ensure([0, 1, 2, 3, 4]) is None             # more than the slots
    with pytest.raises(CwError):
        bank.ensure([E])                                    # no such expert
    with pytest.raises(CwError):
        bank.prefetch([E + 3])
    assert bank.stats()["loads"] == 0
    with pytest.raises(CwError):
        Bank([r[:100] for r in raw], DTYPES, SHAPES, E, S)  # host store too small


BANK_LAYERS = [
    # name, E, K, h, I, dtypes, slots, tokens per step
    ("c5_shape", 128, 10, 2048, 512, (F.IQ3_S, F.IQ3_S, F.Q4_K), 24, 1),
    ("iq2_prefill", 64, 8, 1024, 512, (F.IQ2_XXS, F.IQ2_XXS, F.IQ2_S), 48, 4),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,E,K,h,I,dts,S,T", BANK_LAYERS, ids=[c[0] for c in BANK_LAYERS])
def test_layer_through_a_bank_matches_the_oracle(tmp_path, name, E, K, h, I, dts, S, T):
    """Experts from a GGUF file, S slots; each step routes, ensures the picks, and runs the
    layer through the bank's table: no pick missing, ids identical, outputs within 1e-3
    relative L2 of the resident oracle."""
    import torch
    from coachwhip_amd import ops, synth
    from coachwhip_amd.gguf import GGUFFile
    from oracle import oracle as O
    from tests import gguf_write as G
    print("bank layer", name, flush=True)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    layer = synth.moe_weights(E, K, h, I, dts, rng)
    tensors = [("blk.0.ffn_gate_exps.weight", dts[0], (E, I, h), layer.host[0]),
               ("blk.0.ffn_up_exps.weight", dts[1], (E, I, h), layer.host[1]),
               ("blk.0.ffn_down_exps.weight", dts[2], (E, h, I), layer.host[2])]
    path = tmp_path / (name + ".gguf")
    G.write_gguf(path, [], tensors)
    with GGUFFile(path) as g:
        bank = g.bank(0, S)
    moe = bank.moe_layer(K)
    missing = torch.zeros(1, dtype=torch.int32, device="cuda")
    loaded = 0
    for step in range(5):
        x = rng.standard_normal((T, h)).astype(np.float32)
        logits = rng.standard_normal((T, E)).astype(np.float32)
        assert not synth.near_ties_within_top_k(logits, K)
        dl = ops.to_device(logits)
        ids, _ = ops.route(dl, K, True)
        n = bank.ensure(ids.cpu().numpy())
        assert n is not None
        loaded += n
        out, got_ids, w = moe.forward(ops.to_device(x), dl, missing)
        want, wids, ww, _ = O.moe_layer(layer, x, logits)
        assert np.array_equal(got_ids.cpu().numpy().view(np.uint32), wids)
        assert np.max(np.abs(w.cpu().numpy() - ww)) < 1e-5
        err = O.rel_l2(out.cpu().numpy(), want)
        print("  step", step, "loaded", n, "rel_l2", err, flush=True)
        assert err <= 1e-3
    assert int(missing.cpu()[0]) == 0
    assert bank.stats()["loads"] == loaded


# ------------------------------------------------------------------------------ shrink on arrival

SHRINK_MATS = [(F.Q3_K, 256, 512), (F.Q4_K, 256, 512), (F.Q5_K, 512, 256)]


@pytest.mark.gpu
@pytest.mark.parametrize("pin", [True, False], ids=["pinned_fill_kernel", "pageable_dma"])
def test_bank_shrinks_misses_into_q2_k_slots(pin):
    """Gate and up (Q3_K, Q4_K) shrunk on arrival, gate with column weights; down (Q5_K) shrunk
    too in one bank and kept as Q4_K bytes in another. Every slot equals the oracle's shrink of
    its expert (cw_requant_q2k's bytes), through calls that miss more experts than one staging
    chunk (8) holds, and through prefetch."""
    import torch
    from coachwhip_amd.bank import Bank
    from coachwhip_amd.slots import Slots
    from oracle import oracle as O
    print("bank shrink, pinned", pin, flush=True)
    rng = np.random.default_rng(21 + pin)
    E, S = 30, 12
    for keep_down in (False, True):
        mats = SHRINK_MATS if not keep_down else SHRINK_MATS[:2] + [(F.Q4_K, 512, 256)]
        raw = [synth_blocks(dt, E * r * c, rng) for dt, r, c in mats]
        w_gate = (rng.uniform(0, 2, 512) ** 2).astype(np.float32)
        shape = (torch.from_numpy(w_gate).cuda(), None, None)
        shrink = (True, True, not keep_down)
        bank = Bank(raw, [m[0] for m in mats], [(r, c) for _, r, c in mats], E, S, pin=pin, shrink=shrink, shape=shape)
        mirror = Slots(S)
        eb = [F.matrix_bytes(dt, r, c) for dt, r, c in mats]
        want = []
        for m, (dt, r, c) in enumerate(mats):
            if shrink[m]:
                want.append(O.requant_q2k(dt, raw[m], E * r * c // 256, w_gate if m == 0 else None, c // 256).reshape(E, -1))
            else:
                want.append(raw[m].reshape(E, -1))

        def check(needed):
            torch.cuda.synchronize()
            assert np.array_equal(bank.table.cpu().numpy().view(np.uint32), mirror.table(E))
            for e in needed:
                slot = mirror.slot_of[int(e)]
                for m in range(3):
                    st = bank.banks[m].slot_stride
                    got = bank.banks[m].data[slot * st:(slot + 1) * st].cpu().numpy()
                    assert np.array_equal(got, want[m][e]), (keep_down, e, m)

        for needed in ([0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10], [3, 11, 12, 13], list(range(14, 26)), [0, 26, 27]):
            assert bank.ensure(needed) == len(mirror.assign(needed).misses)
            check(needed)
        n = bank.prefetch([28, 29, 1, 2])
        mirror.reserve([28, 29, 1, 2], ready=lambda s, keep=[mirror.slot_of[e] for e in (0, 26, 27)]: s not in keep)
        torch.cuda.synchronize()
        assert n >= 2 and bank.ensure([28, 29]) == 0
        mirror.assign([28, 29])
        check([28, 29])
        assert bank.banks[0].dtype == F.Q2_K and bank.banks[2].dtype == (F.Q4_K if keep_down else F.Q2_K)


def synth_blocks(dtype, n, rng):
    from coachwhip_amd import synth
    return synth.random_blocks(dtype, n, rng)


@pytest.mark.gpu
def test_layer_through_a_shrinking_bank_matches_the_oracle(monkeypatch):
    """Config-5-shaped experts stored as Q3_K (gate, up) and Q5_K (down), held as Q2_K: each
    step's picks are ensured (misses shrunk on arrival) and the layer runs through the bank; it
    matches the oracle's layer over the oracle's shrink of every expert. Then a 40-token batch
    over 20 resident experts takes the grouped MFMA path over the same Q2_K slots."""
    import torch
    from coachwhip_amd import ops, synth
    from coachwhip_amd.bank import Bank
    from oracle import oracle as O
    print("shrinking bank layer", flush=True)
    rng = np.random.default_rng(33)
    E, K, H, I, S = 64, 10, 2048, 512, 24
    mats = [(F.Q3_K, I, H), (F.Q3_K, I, H), (F.Q5_K, H, I)]
    raw = [synth.random_blocks(dt, E * r * c, rng) for dt, r, c in mats]
    shrunk = [O.requant_q2k(dt, raw[m], E * r * c // 256) for m, (dt, r, c) in enumerate(mats)]
    layer = synth.MoeWeights(E, K, H, I, (F.Q2_K,) * 3, shrunk, [F.matrix_bytes(F.Q2_K, r, c) for _, r, c in mats], E)
    bank = Bank(raw, [m[0] for m in mats], [(r, c) for _, r, c in mats], E, S, shrink=(True, True, True))
    moe = bank.moe_layer(K)
    missing = torch.zeros(1, dtype=torch.int32, device="cuda")
    for step in range(4):
        x = rng.standard_normal((1, H)).astype(np.float32)
        logits = rng.standard_normal((1, E)).astype(np.float32)
        assert not synth.near_ties_within_top_k(logits, K)
        dl = ops.to_device(logits)
        ids, _ = ops.route(dl, K, True)
        assert bank.ensure(ids.cpu().numpy()) is not None
        out, got_ids, _ = moe.forward(ops.to_device(x), dl, missing)
        want, wids, _, _ = O.moe_layer(layer, x, logits)
        assert np.array_equal(got_ids.cpu().numpy().view(np.uint32), wids)
        err = O.rel_l2(out.cpu().numpy(), want)
        print("  step", step, "rel_l2", err, flush=True)
        assert err <= 2e-5
    assert int(missing.cpu()[0]) == 0

    # prefill: the grouped path rounds activations to fp16 once, so the 1e-3 gate
    monkeypatch.setenv("CWMOE_PREFILL_MIN_TOKENS", "1")
    live = rng.choice(E, 20, replace=False)
    assert bank.ensure(live) is not None
    mask = np.full(E, -1e30, np.float32)
    mask[live] = 0.0
    T = 40
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32) + mask
    assert not synth.near_ties_within_top_k(logits, K)
    out, got_ids, _ = moe.forward(ops.to_device(x), ops.to_device(logits), missing)
    want, wids, _, _ = O.moe_layer(layer, x, logits)
    assert np.array_equal(got_ids.cpu().numpy().view(np.uint32), wids)
    err = O.rel_l2(out.cpu().numpy(), want)
    print("  prefill rel_l2", err, flush=True)
    assert err <= 1e-3
    assert int(missing.cpu()[0]) == 0
