"""Pin the numpy HiSparse swap-in oracle.

Known answers from the reference's tests/test_hisparse.py, a brute-force
exactness invariant, and the 200-step golden trace written by
tests/golden/make_golden.py from the reference implementation.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import hisparse as oh
from tests.conftest import load_golden


def test_unique_first_occurrence():
    assert oh.unique_first_occurrence(np.array([5, 3, 5, 1, 3, 9])).tolist() == [5, 3, 1, 9]
    assert oh.unique_first_occurrence(np.array([], dtype=np.int64)).size == 0


def test_lru_replacement_order_known_answer():
    """reference tests/test_hisparse.py:108-129: buf=4, prefill 10."""
    st = oh.HiSparseState(num_layers=1, max_reqs=1, buf=4, top_k=2, max_ctx=32)
    st.admit(0, np.arange(1, 11))

    def select(pos, positions):
        if pos > 10:
            st.backup(0, pos - 1, 100 + pos)
        st.swap_in(0, [0], [pos + 1], np.array([positions]))

    select(10, [5, 10])
    assert st.buffer_tokens[0, 0].tolist() == [5, 1, 2, 3]
    assert st.lru_slots[0, 0].tolist() == [1, 2, 3, 0]
    select(11, [1, 5])
    assert (st.hits, st.misses) == (2, 1)
    assert st.lru_slots[0, 0].tolist() == [2, 3, 1, 0]
    select(12, [7, 8])
    assert st.buffer_tokens[0, 0].tolist() == [5, 1, 7, 8]
    assert st.lru_slots[0, 0].tolist() == [1, 0, 2, 3]
    assert (st.hits, st.misses) == (2, 3)


def test_fast_path_rows_are_slots():
    st = oh.HiSparseState(1, 2, buf=16, top_k=16, max_ctx=32)
    rows, _ = st.swap_in(0, [1], [7], np.arange(16)[None])
    assert rows[0, :7].tolist() == list(range(17, 24)) and np.all(rows[0, 7:] == -1)
    assert st.fast_path_calls == 1


@pytest.mark.parametrize(("prefill_len", "buf", "top_k"), [(10, 16, 8), (40, 16, 8), (5, 32, 32)])
def test_swap_in_is_exact_under_random_selections(prefill_len, buf, top_k):
    """Brute force: simulate slot contents; every row must hold the requested position."""
    total = 120
    st = oh.HiSparseState(1, 1, buf=buf, top_k=top_k, max_ctx=256)
    st.admit(0, np.arange(prefill_len))
    content = np.full(buf + 1, -1, dtype=np.int64)
    content[: min(prefill_len, buf)] = np.arange(min(prefill_len, buf))
    rng = np.random.default_rng(7)
    for pos in range(prefill_len, total):
        if pos > prefill_len:
            st.backup(0, pos - 1, pos - 1)
            if pos - 1 < buf:
                content[pos - 1] = pos - 1
        content[min(pos, buf)] = pos  # the newest token's slot
        s = pos + 1
        n = min(s, top_k)
        if s <= top_k:
            sel = np.arange(n)
        else:
            sel = rng.integers(0, s, n)
            sel[-1] = s - 1
            sel[0] = sel[1]
        rows, copies = st.swap_in(0, [0], [s], sel[None])
        for slot, host in copies[0]:
            content[slot] = host  # host row == position here
        assert np.array_equal(content[rows[0, :n]], sel)
        if s > top_k:
            assert rows[0, 0] == rows[0, 1]
    assert st.misses > 0


def test_victim_shortage_and_missing_host_row_raise():
    tokens, lru = np.arange(4), np.arange(4)
    with pytest.raises(RuntimeError):
        oh.swap_in_long(tokens, lru, np.array([10, 11, 12, 13, 14, 20]), 21, np.arange(32))
    with pytest.raises(AssertionError):
        oh.swap_in_long(tokens, lru, np.array([9, 20]), 21, np.full(32, -1))


def test_golden_200_step_trace():
    g = load_golden("swap_trace.npz")
    layers, buf, top_k, ctx, prefill = g["meta"].tolist()
    st = oh.HiSparseState(layers, 1, buf=buf, top_k=top_k, max_ctx=ctx)
    host = g["host_rows_final"]
    st.admit(0, host[:prefill])
    i = 0
    for step in range(200):
        pos = prefill + step
        if pos > prefill:
            st.backup(0, pos - 1, host[pos - 1])
        for layer in range(layers):
            sel = g["selections"][i]
            rows, _ = st.swap_in(layer, [0], [pos + 1], sel[None])
            assert np.array_equal(rows[0], g["rows"][i]), f"step {step} layer {layer}"
            assert np.array_equal(st.buffer_tokens[layer, 0], g["tokens"][i])
            assert np.array_equal(st.lru_slots[layer, 0], g["lru"][i])
            assert [st.hits, st.misses] == g["stats"][i].tolist()
            i += 1
