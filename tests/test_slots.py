"""The bank's slot bookkeeping (C++ Slots behind the C ABI): the reference's own cases,
crates/engine/tests/bank.rs, ported. No GPU."""
from coachwhip_amd import Plan, Slots


def check_consistent(s, n):
    assert sorted(s.lru) == list(range(n)), "the use order lists every slot exactly once"
    for e, slot in s.slot_of.items():
        assert s.holder[slot] == e
    assert sum(h is not None for h in s.holder) == len(s.slot_of)


def test_a_fresh_bank_misses_everything_and_fills_slots_in_order():      # bank.rs:24-30
    s = Slots(4)
    assert s.assign([7, 3]) == Plan([], [(7, 0), (3, 1)], 0)
    check_consistent(s, 4)


def test_a_second_ask_is_a_hit_in_the_same_slot():                       # bank.rs:32-39
    s = Slots(4)
    s.assign([7, 3])
    plan = s.assign([3])
    assert plan.hits == [(3, 1)] and plan.misses == []


def test_the_least_recently_used_expert_is_evicted():                     # bank.rs:41-50
    s = Slots(2)
    s.assign([1])
    s.assign([2])
    s.assign([1])
    plan = s.assign([3])
    assert plan.misses == [(3, 1)], "3 takes 2's slot"
    assert 2 not in s.slot_of and 1 in s.slot_of


def test_never_evicts_an_expert_the_same_word_needs():                     # bank.rs:52-60
    s = Slots(3)
    s.assign([1, 2, 3])
    plan = s.assign([4, 1, 2])
    assert plan.misses == [(4, 2)] and len(plan.hits) == 2
    check_consistent(s, 3)


def test_never_hands_out_a_slot_still_being_filled():                      # bank.rs:62-67
    s = Slots(3)
    plan = s.assign([9], lambda slot: slot != 0)
    assert plan.misses == [(9, 1)]


def test_a_crowded_bank_says_none_and_changes_nothing():                   # bank.rs:69-79
    s = Slots(2)
    s.assign([1, 2])
    holder, lru = s.holder, s.lru
    assert s.assign([3, 4], lambda _: False) is None, "no slot is ready"
    assert s.assign([1, 3, 4]) is None, "three experts cannot fit two slots"
    assert s.holder == holder and s.lru == lru


def test_reserve_skips_what_is_held_and_never_evicts_another_guess():      # bank.rs:81-92
    s = Slots(3)
    s.assign([1, 2])
    got = s.reserve([2, 5, 6])
    assert len(got) == 2 and all(e in (5, 6) for e, _ in got)
    assert 2 in s.slot_of
    assert s.is_prefetched(5) and s.is_prefetched(6)
    check_consistent(s, 3)


def test_reserve_stops_when_no_slot_is_free():                             # bank.rs:94-100
    s = Slots(2)
    got = s.reserve([1, 2, 3])
    assert [e for e, _ in got] == [1, 2]


def test_a_used_guess_counts_as_a_prefetch_hit_once():                     # bank.rs:102-110
    s = Slots(4)
    s.reserve([8])
    assert s.assign([8]).prefetch_hits == 1
    assert s.assign([8]).prefetch_hits == 0


def test_an_unused_guess_that_is_evicted_is_forgotten():                   # bank.rs:112-118
    s = Slots(1)
    s.reserve([8])
    s.assign([9])
    assert not s.is_prefetched(8)
    check_consistent(s, 1)


def test_matches_a_reference_lru_over_a_long_random_run():                 # bank.rs:120-154
    n = 8
    s = Slots(n)
    reference = []
    x = [42]

    def nxt(m):
        x[0] = (x[0] * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        return (x[0] >> 33) % m

    for _ in range(5000):
        k = 1 + nxt(4)
        needed = []
        while len(needed) < k:
            e = nxt(20)
            if e not in needed:
                needed.append(e)
        plan = s.assign(needed)
        for e in needed:
            was_held = e in reference
            assert any(h[0] == e for h in plan.hits) == was_held
            if was_held:
                reference.remove(e)
            elif len(reference) == n:
                victim = next(r for r in reference if r not in needed)
                reference.remove(victim)
            reference.append(e)
        check_consistent(s, n)


def test_release_and_pop_move_slots_to_the_front():                        # experts.rs:251-269
    s = Slots(3)
    s.assign([1, 2, 3])
    s.pop([3])
    assert s.lru[0] == 2
    s.release(2)
    assert s.lru[0] == 1 and s.holder[1] is None
    assert list(s.table(4)) == [0xFFFFFFFF, 0, 0xFFFFFFFF, 2]  # expert 1 in slot 0, 3 in slot 2
