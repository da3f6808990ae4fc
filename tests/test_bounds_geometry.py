"""CPU model of prefill_bounds_wave_kernel's geometry (bounds.hip): the launch covers every
page of the prompt exactly once, each wave folds its page's rows [begin, end) once each and
in order (64-row index chunks, batches of 32 loads), and every index it reads lies in
[0, n_tokens).  Mirrors the kernel's loops; no GPU."""

from __future__ import annotations

import pytest

WAVES_PER_BLOCK = 2  # 128-thread blocks
PAGES_PER_WAVE = 1
BATCH = 32
CHUNK = 64


def ceil_div(a, b):
    return (a + b - 1) // b


def fold_order(n, P):
    pages = max(1, ceil_div(n, P))
    blocks = ceil_div(pages, WAVES_PER_BLOCK * PAGES_PER_WAVE)
    seen_pages, order, reads = [], [], []
    for blk in range(blocks):
        for wave in range(WAVES_PER_BLOCK):
            page0 = (blk * WAVES_PER_BLOCK + wave) * PAGES_PER_WAVE
            if page0 * P >= n:
                continue
            for j in range(PAGES_PER_WAVE):
                page = page0 + j
                begin, end = page * P, min(page * P + P, n)
                if begin >= end:
                    break
                seen_pages.append(page)
                rows = []
                for t0 in range(begin, end, CHUNK):
                    cnt = min(CHUNK, end - t0)
                    reads.extend(t0 + lane for lane in range(64) if lane < cnt)
                    for tb in range(0, cnt, BATCH):
                        rows.extend(t0 + tb + i for i in range(BATCH) if tb + i < cnt)
                order.append((page, rows))
    return pages, seen_pages, order, reads


@pytest.mark.parametrize("P", [16, 64, 128, 200])
@pytest.mark.parametrize("n", [1, 63, 64, 65, 255, 256, 777, 4097, 131071])
def test_every_page_and_row_folded_once_in_order(n, P):
    pages, seen, order, reads = fold_order(n, P)
    full = n // P
    assert sorted(seen) == list(range(ceil_div(n, P)))  # each page once (the partial tail too)
    assert len(seen) == len(set(seen))
    for page, rows in order:
        assert rows == list(range(page * P, min(page * P + P, n)))  # row order = sequential fold
    assert all(0 <= r < n for r in reads)
    assert full <= pages
