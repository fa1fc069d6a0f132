"""The expert cache's policy on the CPU (no device): the reference's
ExpertCache (spm-granite-moe/src/expert_cache.rs:20-90) -- a miss counts an
observation, the second observation admits, the least recently used resident
expert makes room -- and mmid-cache's layer-aware victims
(tools/llama-logits/mmid-cache.hpp:134-173).  Expected outcomes are worked
out by hand in each test."""
import numpy as np

from emufpga_amd.expert_cache import policy_trace

HIT, ADMIT, STREAM = 0, 1, 2


def run(n_slots, aware, seq):
    """seq: list of calls, each a list of (layer, expert)."""
    calls, layers, experts = [], [], []
    for c, call in enumerate(seq):
        for layer, expert in call:
            calls.append(c)
            layers.append(layer)
            experts.append(expert)
    return [list(x) for x in policy_trace(n_slots, aware, calls, layers, experts)]


def test_admit_on_second_use_then_hit():
    out, slot = run(2, False, [[(0, 5)], [(0, 5)], [(0, 5)]])
    assert out == [STREAM, ADMIT, HIT] and slot == [-1, 0, 0]


def test_least_recently_used_is_evicted():
    # A, B admitted on their second use; A touched again; C's second use evicts B (older than A);
    # B's next miss is its third observation, so it is admitted at once (the seen count outlives
    # an eviction, expert_cache.rs:54-56), evicting the least recent of A and C: A
    seq = [[(0, 1)], [(0, 1)], [(0, 2)], [(0, 2)], [(0, 1)], [(0, 3)], [(0, 3)], [(0, 2)], [(0, 2)]]
    out, slot = run(2, False, seq)
    assert out == [STREAM, ADMIT, STREAM, ADMIT, HIT, STREAM, ADMIT, ADMIT, HIT]
    assert slot[6] == slot[3]  # C took B's slot
    assert slot[7] == slot[1]  # B took A's


def test_layer_aware_prefers_a_victim_of_the_incoming_layer():
    # slots hold layer 0 expert 1 (older) and layer 1 expert 1 (newer); layer 1 expert 2 is admitted
    seq = [[(0, 1)], [(0, 1)], [(1, 1)], [(1, 1)], [(1, 2)], [(1, 2)]]
    lru, lru_slot = run(2, False, seq)
    aware, aware_slot = run(2, True, seq)
    assert lru[-1] == ADMIT and lru_slot[-1] == lru_slot[1]        # plain LRU evicts layer 0's older entry
    assert aware[-1] == ADMIT and aware_slot[-1] == aware_slot[3]  # layer-aware evicts the same layer's


def test_experts_of_the_call_in_progress_are_not_evicted():
    # one slot, held by expert 1; a call using 1 and (second use of) 2 cannot evict 1: 2 streams through
    seq = [[(0, 1)], [(0, 1)], [(0, 2)], [(0, 1), (0, 2)]]
    out, slot = run(1, False, seq)
    assert out == [STREAM, ADMIT, STREAM, HIT, STREAM]
    # in a later call of its own, 2 takes the slot
    out, _ = run(1, False, seq + [[(0, 2)]])
    assert out[-1] == ADMIT


def test_no_slots_streams_everything():
    out, slot = run(0, True, [[(0, 1)], [(0, 1)], [(0, 1)]])
    assert out == [STREAM] * 3 and slot == [-1] * 3


def test_experts_of_a_call_are_in_use_from_its_start():
    """mmid-cache.hpp's acquire/release: every expert of a call is in use
    from the call's start, whatever order the call looks them up in.  One
    slot; expert 5 is admitted on its second use; expert 3 seen once.  A
    call of {3, 5} looks 3 up first: its second use wants a slot, but the
    only one holds 5, which the same call uses, so 3 streams through and 5
    hits (evicting 5 would upload it again for this very call)."""
    out, slot = policy_trace(1, False, [0, 1, 2, 3, 3], [0] * 5, [5, 5, 3, 3, 5])
    assert list(out) == [2, 1, 2, 2, 0]
    assert list(slot) == [-1, 0, -1, -1, 0]
