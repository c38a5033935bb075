"""The bagging stream's host parts: MT19937 draws (vector and scalar paths,
every starting position), the final RandomState, and the list/chain form of
the Fisher-Yates swaps that the GPU uses.  CPU only."""
import os
import subprocess
import sys

import numpy as np
import pytest

from bsscl_gbm import _native
import fy_model

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _state_after(seed, doubles):
    rng = np.random.RandomState(seed)
    if doubles:
        rng.random_sample(doubles)   # two 32-bit words each
    return rng


@pytest.mark.parametrize("doubles", [0, 1, 311, 312, 313, 400])
def test_rs_draws_match_numpy_shuffle(doubles):
    for n in (1, 2, 3, 17, 1000, 70_001):
        rng = _state_after(5, doubles)
        d, key, pos = _native.rs_draws(rng.get_state(), n)
        assert len(d) == max(n - 1, 0)
        assert np.all(d <= np.arange(n - 1, 0, -1))
        a = np.arange(n)
        rng.shuffle(a)
        np.testing.assert_array_equal(fy_model.fisher_yates_sequential(np.arange(n), d), a)
        st = rng.get_state()
        np.testing.assert_array_equal(key, st[1])
        assert pos == st[2]


@pytest.mark.parametrize("doubles", [0, 1, 311, 312, 400])
def test_sampler_starting_positions_and_final_state(doubles):
    """Host-rows sampler against rng.shuffle from every kind of starting
    position (fresh state pos=624, mid-block, exactly at a block end)."""
    n, F, rounds = 300_007, 11, 3
    n_sub, f_sub = n // 2, 7
    rng = _state_after(11, doubles)
    s = _native.Sampler(rng.get_state(), n, n_sub, True, F, f_sub, True, rounds)
    rows = np.arange(n, dtype=np.int64)
    feats = np.arange(F, dtype=np.int32)
    for _ in range(rounds):
        rng.shuffle(rows)
        rng.shuffle(feats)
        r, f = s.next()
        np.testing.assert_array_equal(r, rows[:n_sub])
        np.testing.assert_array_equal(f, np.sort(feats[:f_sub]))
    key, pos = s.state()
    st = rng.get_state()
    np.testing.assert_array_equal(key, st[1])
    assert pos == st[2]
    s.close()


@pytest.mark.parametrize("doubles", [0, 7, 312])
def test_parallel_draws_match_numpy_over_mask_ranges(doubles):
    """Rounds long enough for the counting pass and the draw workers (about
    100 chunks of words each, crossing the masks 2^21-1 .. 1), against
    RandomState.shuffle, and the state after them."""
    n, F, rounds = 2_000_003, 5, 3
    rng = _state_after(23, doubles)
    s = _native.Sampler(rng.get_state(), n, n - 1, True, F, 3, True, rounds)
    rows = np.arange(n, dtype=np.int64)
    feats = np.arange(F, dtype=np.int32)
    for _ in range(rounds):
        rng.shuffle(rows)
        rng.shuffle(feats)
        r, f = s.next()
        np.testing.assert_array_equal(r, rows[:n - 1])
        np.testing.assert_array_equal(f, np.sort(feats[:3]))
    key, pos = s.state()
    st = rng.get_state()
    np.testing.assert_array_equal(key, st[1])
    assert pos == st[2]
    s.close()


@pytest.mark.parametrize("window", ["1", "0", "6"])
def test_parallel_transfer_functions_and_word_by_word_chunks(monkeypatch, window):
    """The chunk transfer functions of the parallel form (default entry
    windows; windows of width 0, so nearly every chunk is counted word by
    word; windows six times wider, with many merges per chunk) give the
    stream of RandomState.shuffle exactly."""
    monkeypatch.setenv("BSSCL_SAMPLER_WINDOW", window)
    n, F, rounds = 1_500_007, 7, 3
    rng = _state_after(31, 5)
    s = _native.Sampler(rng.get_state(), n, n // 3, True, F, 4, True, rounds)
    rows = np.arange(n, dtype=np.int64)
    feats = np.arange(F, dtype=np.int32)
    for _ in range(rounds):
        rng.shuffle(rows)
        rng.shuffle(feats)
        r, f = s.next()
        np.testing.assert_array_equal(r, rows[:n // 3])
        np.testing.assert_array_equal(f, np.sort(feats[:4]))
    key, pos = s.state()
    st = rng.get_state()
    np.testing.assert_array_equal(key, st[1])
    assert pos == st[2]
    stats = s.stats()
    s.close()
    chunks = stats["spec_chunks"] + stats["seq_chunks"]
    assert chunks >= rounds * 100
    if window == "0":
        assert stats["seq_chunks"] > 0.9 * chunks
    else:
        assert stats["spec_chunks"] > 0.7 * chunks


def test_sampler_scalar_path_matches():
    """The same stream with the AVX-512 draws switched off (the switch is
    read once per process, so this runs in a child)."""
    code = (
        "import sys, numpy as np; sys.path[:0] = [%r, %r];"
        "from bsscl_gbm import _native;"
        "rng = np.random.RandomState(3); n, F = 100_003, 9;"
        "s = _native.Sampler(rng.get_state(), n, 60_000, True, F, 5, True, 2);"
        "rows = np.arange(n); feats = np.arange(F);"
        "ok = True\n"
        "for _ in range(2):\n"
        "    rng.shuffle(rows); rng.shuffle(feats); r, f = s.next()\n"
        "    ok = ok and np.array_equal(r, rows[:60_000]) and np.array_equal(f, np.sort(feats[:5]))\n"
        "key, pos = s.state(); st = rng.get_state()\n"
        "ok = ok and np.array_equal(key, st[1]) and pos == st[2]\n"
        "s.close(); print('OK' if ok else 'MISMATCH')\n"
    ) % (os.path.join(ROOT, "bsscl-gbm_amd"), os.path.join(ROOT, "tests"))
    env = dict(os.environ, BSSCL_SAMPLER_SCALAR="1")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip().endswith("OK"), out.stdout


def test_device_rows_sampler_refuses_host_rows():
    rng = np.random.RandomState(0)
    if _native.device_count() == 0:
        # Row draws go to a GPU: without one the sampler cannot be made.
        with pytest.raises(ValueError):
            _native.Sampler(rng.get_state(), 1000, 500, True, 4, 4, False, 2, device_rows=True)
    else:
        s = _native.Sampler(rng.get_state(), 1000, 500, True, 4, 4, False, 2, device_rows=True)
        with pytest.raises(ValueError):
            s.next()
        s.close()
    # Without row bagging a device-rows sampler still delivers features.
    s = _native.Sampler(rng.get_state(), 1000, 1000, False, 6, 3, True, 1, device_rows=True)
    r, f = s.next()
    np.testing.assert_array_equal(r, np.arange(1000))
    assert len(f) == 3 and np.all(np.diff(f) > 0)
    s.close()


def _adversarial_draws(n):
    steps = np.arange(n - 1, 0, -1)
    rng = np.random.default_rng(n)
    return {
        "zeros": np.zeros(n - 1, np.uint32),                  # one list of length n-1
        "self": steps.astype(np.uint32),                      # no swaps
        "previous": (steps - 1).astype(np.uint32),            # a chain through every step
        "half": (steps // 2).astype(np.uint32),
        "random": np.array([rng.integers(0, k + 1) for k in steps], np.uint32),
    }


@pytest.mark.parametrize("n", [2, 3, 5, 64, 257, 1000, 4099])
def test_fisher_yates_sorted_key_form_equals_sequential(n):
    """The sorted (position, step) key form of the device kernels."""
    a0 = np.random.default_rng(2).permutation(n).astype(np.int32)
    for name, d in _adversarial_draws(n).items():
        np.testing.assert_array_equal(fy_model.fisher_yates_sorted_keys(a0, d),
                                      fy_model.fisher_yates_sequential(a0, d), err_msg=name)


@pytest.mark.parametrize("n", [1, 2, 3, 5, 64, 1000, 4099])
def test_fisher_yates_list_form_equals_sequential(n):
    a0 = np.random.default_rng(1).permutation(n).astype(np.int32)
    if n == 1:
        np.testing.assert_array_equal(fy_model.fisher_yates_lists(a0, np.zeros(0, np.uint32)), a0)
        return
    for name, d in _adversarial_draws(n).items():
        np.testing.assert_array_equal(fy_model.fisher_yates_lists(a0, d),
                                      fy_model.fisher_yates_sequential(a0, d), err_msg=name)


def test_fisher_yates_list_form_on_mt_draws():
    for n in (10, 999, 200_003):
        d, _, _ = _native.rs_draws(np.random.RandomState(n).get_state(), n)
        a0 = np.arange(n, dtype=np.int32)[::-1].copy()
        np.testing.assert_array_equal(fy_model.fisher_yates_lists(a0, d),
                                      fy_model.fisher_yates_sequential(a0, d))
