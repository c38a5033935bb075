"""The order form of the device replay (k_replay_tree in kernels.hip)
against the slot loop it replaces, on random node tables numbered as the
level planner numbers them: identical output trees and status wherever the
order form applies (distinct candidate keys), and a hand-made tie that it
must hand to the slot loop.  CPU only (tests/replay_model.py)."""
import numpy as np
import pytest

from replay_model import random_table, replay_ordered, replay_slots


@pytest.mark.parametrize("seed", range(6))
def test_order_form_equals_slot_loop(seed):
    rng = np.random.default_rng(seed)
    agree = 0
    for it in range(500):
        ties = it % 5 == 0
        G, left, kept, ls = random_table(rng, int(rng.integers(1, 9)),
                                         p_expand=rng.uniform(0.5, 1.0),
                                         p_kept=rng.uniform(0.6, 1.0), ties=ties)
        ml = int(rng.integers(2, 64))
        gamma = float(rng.choice([0.0, -1.0, 0.5, -np.inf] if not ties else [0.0, 2.0]))
        a = replay_slots(G, left, kept, ls, ml, gamma)
        b = replay_ordered(G, left, kept, ls, ml, gamma)
        if b is None:
            continue
        assert a[3] == b[3], it
        if a[3]:
            continue
        nc = a[2]
        assert b[2] == nc, it
        np.testing.assert_array_equal(a[0][:nc], b[0][:nc], err_msg=str(it))
        np.testing.assert_array_equal(a[1][:nc], b[1][:nc], err_msg=str(it))
        agree += 1
    assert agree > 250


def test_full_trees_without_unexpanded_nodes():
    """Tables like the planner's: every node the loop can pop is expanded
    (the deepest nodes are at max_depth and have no split), so the replay
    never fails."""
    rng = np.random.default_rng(11)
    for it in range(300):
        G, left, kept, ls = random_table(rng, int(rng.integers(2, 8)), p_expand=1.0,
                                         p_kept=0.95)
        G[left < 0] = -np.inf
        ml = int(rng.integers(2, 80))
        a = replay_slots(G, left, kept, ls, ml, 0.0)
        b = replay_ordered(G, left, kept, ls, ml, 0.0)
        assert b is not None and a[3] == 0 and b[3] == 0
        assert a[2] == b[2]
        np.testing.assert_array_equal(a[0][:a[2]], b[0][:b[2]])
        np.testing.assert_array_equal(a[1][:a[2]], b[1][:b[2]])


def test_equal_keys_go_to_the_slot_loop():
    # Root 5 -> children 3, 3 (equal keys among candidates).
    G = np.array([5.0, 3.0, 3.0])
    left = np.array([1, -1, -1])
    kept = np.array([True, True, True])
    ls = np.array([True, True, True])
    assert replay_ordered(G, left, kept, ls, 4, 0.0) is None
    # Equal keys at or below gamma never matter.
    G2 = np.array([5.0, -1.0, -1.0])
    assert replay_ordered(G2, left, kept, ls, 4, 0.0) is not None
