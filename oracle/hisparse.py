"""numpy restatement of the HiSparse hot-buffer swap-in (reference
``src/qwenquest/hisparse/coordinator.py``).  Test infrastructure only.

State per (layer, request), exactly as the reference keeps it:
``tokens[buf]`` - position cached by each LRU slot (-1 = none);
``lru[buf]``    - slots ordered least -> most recently used.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def unique_first_occurrence(x: np.ndarray) -> np.ndarray:
    """coordinator.py:62-71: unique values ordered by first occurrence."""
    x = np.asarray(x, dtype=np.int64)
    if x.size == 0:
        return x
    _, first = np.unique(x, return_index=True)
    return x[np.sort(first)]


@dataclass
class SwapPlan:
    slots: np.ndarray  # [n] slot per requested entry (buf = reserved newest slot)
    tokens: np.ndarray  # new tokens[buf]
    lru: np.ndarray  # new lru[buf]
    copies: list[tuple[int, int]]  # (victim slot, host row) in miss order
    hits: int
    misses: int


def swap_in_long(
    tokens: np.ndarray,
    lru: np.ndarray,
    positions: np.ndarray,
    seq_len: int,
    host_rows: np.ndarray,
) -> SwapPlan:
    """coordinator.py:259-304 for one (layer, request) with ``seq_len > buf``.

    ``host_rows``: the request's ``req_to_host_pool`` row (position -> host row, -1 = none).
    Raises RuntimeError / AssertionError exactly where the reference does
    (coordinator.py:278-279, 285-286).
    """
    tokens = np.asarray(tokens, dtype=np.int64).copy()
    lru = np.asarray(lru, dtype=np.int64)
    positions = np.asarray(positions, dtype=np.int64)
    buf = tokens.shape[0]
    slots = np.empty_like(positions)
    is_newest = positions == seq_len - 1
    slots[is_newest] = buf  # coordinator.py:264-265
    wanted = positions[~is_newest]
    uniq = unique_first_occurrence(wanted)  # coordinator.py:267-268
    hit_in_lru = np.isin(tokens[lru], uniq)  # coordinator.py:273
    hit_slots = lru[hit_in_lru]
    evictable = lru[~hit_in_lru]
    misses = uniq[~np.isin(uniq, tokens)]  # coordinator.py:276
    num_miss = int(misses.size)
    if num_miss > evictable.size:
        raise RuntimeError("device_buffer_size too small for this top-k")
    victims = evictable[:num_miss]
    copies: list[tuple[int, int]] = []
    if num_miss:
        hidx = np.asarray(host_rows, dtype=np.int64)[misses]
        if bool((hidx < 0).any()):
            raise AssertionError("positions without host backup were selected")
        copies = [(int(s), int(h)) for s, h in zip(victims, hidx)]
        tokens[victims] = misses  # coordinator.py:291
    new_lru = np.concatenate([evictable[num_miss:], victims, hit_slots])  # coordinator.py:295
    order = np.argsort(tokens, kind="stable")  # coordinator.py:298-300
    slot = order[np.searchsorted(tokens[order], wanted)]
    slots[~is_newest] = slot
    return SwapPlan(slots, tokens, new_lru, copies, int(uniq.size) - num_miss, num_miss)


class HiSparseState:
    """Per-request LRU bookkeeping of ``HiSparseCoordinator`` (coordinator.py:124-134, 138-174,
    232-257, 308-316) without the KV payload: enough to check row maps and LRU state."""

    def __init__(self, num_layers: int, max_reqs: int, buf: int, top_k: int, max_ctx: int):
        if buf < top_k:
            raise ValueError("device_buffer_size must be >= top_k")
        self.buf, self.top_k = buf, top_k
        self.buffer_tokens = np.full((num_layers, max_reqs, buf), -1, dtype=np.int64)
        self.lru_slots = np.tile(np.arange(buf, dtype=np.int64), (num_layers, max_reqs, 1))
        self.req_to_host_pool = np.full((max_reqs, max_ctx), -1, dtype=np.int64)
        self.hits = self.misses = self.fast_path_calls = 0

    def admit(self, req: int, host_rows: np.ndarray) -> None:
        """coordinator.py:154-167 (bookkeeping part)."""
        n = len(host_rows)
        self.req_to_host_pool[req, :n] = host_rows
        self.buffer_tokens[:, req, :] = np.arange(self.buf)
        self.lru_slots[:, req, :] = np.arange(self.buf)

    def backup(self, req: int, pos: int, host_row: int) -> None:
        """coordinator.py:211-212."""
        self.req_to_host_pool[req, pos] = host_row

    def swap_in(self, layer: int, reqs, seq_lens, positions) -> tuple[np.ndarray, list]:
        """coordinator.py:232-257.  Returns (rows [bs, top_k] int64, copies per request)."""
        bs = len(reqs)
        out = np.full((bs, self.top_k), -1, dtype=np.int64)
        all_copies = []
        for i in range(bs):
            req, s = int(reqs[i]), int(seq_lens[i])
            n = min(s, self.top_k)
            pos = np.asarray(positions[i, :n], dtype=np.int64)
            base = req * (self.buf + 1)
            if s <= self.buf:
                self.fast_path_calls += 1
                out[i, :n] = base + pos
                all_copies.append([])
                continue
            plan = swap_in_long(
                self.buffer_tokens[layer, req], self.lru_slots[layer, req], pos, s,
                self.req_to_host_pool[req],
            )
            self.buffer_tokens[layer, req] = plan.tokens
            self.lru_slots[layer, req] = plan.lru
            self.hits += plan.hits
            self.misses += plan.misses
            out[i, :n] = base + plan.slots
            all_copies.append(plan.copies)
        return out, all_copies

    def release(self, req: int) -> None:
        """coordinator.py:308-316 (bookkeeping part)."""
        self.req_to_host_pool[req] = -1
        self.buffer_tokens[:, req, :] = -1
        self.lru_slots[:, req, :] = np.arange(self.buf)
