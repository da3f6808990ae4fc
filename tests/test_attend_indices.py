"""CPU model of the fused attention kernels' index arithmetic (qwenquest_amd/csrc/decode.hip).

For every launch shape the host code can choose, it checks that

* every row-table entry a wave reads lies inside its block's table and was written by the
  table fill (entries past the request's real slots hold row 0, never stale LDS),
* the real slots [0, n) of a request are attended exactly once over all parts and waves,
* the selection reads only score entries below the candidate limit, its survivor array and
  page list fit, and the page index of every selected slot is < k (the page list's length),
* every partial and counter index stays inside the workspace and the sync buffer,
* the LDS a launch allocates covers the larger of its row table and its selection.

The first fused attention kernel faulted the GPU on a recent-window-only flow (top_k 64,
k_sel 0, seq_len < 64): its table fill wrote only the real slots, while a step reads all of
its 16 (or 32) entries (the ones past n are masked in the softmax only), so uninitialised
LDS words became pool-row indices.  The fill now covers the block's whole share; this
model is the check that found it, kept for every geometry the host code can pick.
"""

from __future__ import annotations

import itertools
import math

import pytest

# geometry of decode.hip (kept in step with its constants and host helpers)
W4_WAVES, W4_PARTS, W4_ROWCAP = 4, 8, 1024
HEAD_WAVES, HEAD_TILES, HEAD_ROWCAP = 8, 2, 4096
MAX_SEL, MAX_TOPK, MAX_G, KV = 64, 4096, 16, 4
KPT_FORMS = (2, 4, 6, 8, 9, 12, 16, 24)


def ceil_div(a, b):
    return -(-a // b)


def step_parts(top_k):
    return max(1, min(W4_PARTS, ceil_div(top_k, W4_WAVES * 32)))


def step_per_wave(top_k, parts):
    return ceil_div(top_k, parts * W4_WAVES * 32) * 32


def dense_parts(max_rows):
    return max(1, ceil_div(max_rows, MAX_TOPK))


def kpt_form(max_pages, k_sel):
    n_max = max(max_pages, k_sel)
    for kpt in KPT_FORMS:
        if n_max <= kpt * 256:
            return kpt
    return None


def select_smem_bytes(kpt, nt=256):
    # SelectSmem<KPT, NT>: cand[NT*KPT+64] u64, gmax[64] u64, grank[64], crank[64], wcnt[NT/64],
    # tau u64 (8-aligned), order[64]
    b = (nt * kpt + 64) * 8 + 64 * 8 + 64 * 4 + 64 * 4 + (nt // 64) * 4
    b = ceil_div(b, 8) * 8 + 8 + 64 * 4
    return ceil_div(b, 8) * 8


def head_smem_bytes(waves, rowcap):
    # HeadSmem<W, ROWCAP>: rows[ROWCAP] i32, m[W][16], l[W][16], o[W][16][128] f32
    return rowcap * 4 + 2 * waves * MAX_G * 4 + waves * MAX_G * 128 * 4


def attend_block(n, slot_base, per_wave, waves, step_rows):
    """Reads of one block's row table and the real slots its waves attend."""
    per_block = waves * per_wave
    written = set()
    threads = 64 * waves
    for i0 in range(0, per_block, threads * 4):  # the fill: 4 slots per thread per pass
        for tid in range(threads):
            for u in range(4):
                i = i0 + tid + threads * u
                if i < per_block:
                    written.add(i)
    reads, real = set(), []
    for w in range(waves):
        r0 = w * per_wave
        r_end = max(r0, min(r0 + per_wave, n - slot_base))
        for i in range(ceil_div(r_end - r0, step_rows)):
            t0 = r0 + step_rows * i
            tiles = step_rows // 16
            reads.update(t0 + t * 16 + lo for t in range(tiles) for lo in range(16))
            reads.update(t0 + u * 16 + hi * 4 + j for u in range(tiles) for hi in range(4) for j in range(4))
            valid = r_end - t0
            assert valid > 0
            real.extend(slot_base + t0 + x for x in range(min(valid, step_rows)))
    return per_block, written, reads, real


def check_launch(top_k, n, parts, per_wave, waves, step_rows, rowcap):
    per_block = waves * per_wave
    assert per_block <= rowcap, f"table of {per_block} slots > {rowcap}"
    assert parts * per_block >= min(n, top_k)
    seen = []
    for part in range(parts):
        pb, written, reads, real = attend_block(n, part * per_block, per_wave, waves, step_rows)
        assert written == set(range(pb)), "the fill leaves table entries unwritten"
        assert not reads or max(reads) < pb, "a step reads past the block's table"
        assert reads <= written, "a step reads an entry the fill did not write"
        seen.extend(real)
    assert sorted(seen) == list(range(n)), "real slots not attended exactly once"


def check_selection(top_k, page, max_pages, lim):
    k = top_k // page - 1
    kpt = kpt_form(max_pages, k)
    assert kpt is not None
    n_eff = max(lim, k)
    assert n_eff <= kpt * 256
    score_reads = [tid + 256 * i for tid in range(256) for i in range(kpt) if tid + 256 * i < lim]
    assert not score_reads or max(score_reads) < min(lim, max_pages)
    assert k <= MAX_SEL
    # survivors <= n_eff fit cand[NT*KPT + 64]; slots < k*P read s_pages[slot // P] < k
    assert n_eff <= 256 * kpt + 64
    assert all(slot // page < k for slot in range(k * page))
    smem = max(head_smem_bytes(W4_WAVES, W4_ROWCAP), select_smem_bytes(kpt))
    assert smem <= 64 * 1024


TOPKS = (64, 128, 192, 256, 1024, 2048, 2112, 4032, 4096)
SEQS = (1, 2, 15, 16, 31, 33, 63, 64, 65, 127, 2047, 2048, 2049, 4095, 4096, 4097, 9000, 131072)


@pytest.mark.parametrize("top_k", TOPKS)
def test_fused_attention_row_table_and_slots(top_k):
    parts = step_parts(top_k)
    per_wave = step_per_wave(top_k, parts)
    for s in SEQS:
        n = min(max(s, 0), top_k)
        check_launch(top_k, n, parts, per_wave, W4_WAVES, 16, W4_ROWCAP)


@pytest.mark.parametrize("top_k", TOPKS)
def test_rows_mode_actual_lengths(top_k):
    """quest_hisparse's rows mode: n = clamp(actual, 0, slots) for any given actual length."""
    parts = step_parts(top_k)
    per_wave = step_per_wave(top_k, parts)
    for actual in (-3, 0, 1, 17, top_k - 1, top_k, top_k + 5):
        check_launch(top_k, min(max(actual, 0), top_k), parts, per_wave, W4_WAVES, 16, W4_ROWCAP)


@pytest.mark.parametrize("max_pages", (2, 64, 512, 513, 1024, 2049, 2050, 2304, 2305, 3072, 4096, 6144))
def test_selection_forms(max_pages):
    """The KPT form the host picks holds every candidate page: 2304 (9 keys per thread,
    contexts just past 128K), 3072 (12), 6144 (24) pages and the forms between."""
    for top_k, page in ((64, 64), (128, 64), (2048, 64), (4096, 64), (4160, 64)):
        if top_k // page - 1 > MAX_SEL:
            continue
        for lim in sorted({0, 1, max_pages // 2, max_pages - 1, max_pages}):
            check_selection(top_k, page, max_pages, lim)


def test_largest_form_is_the_fused_limit():
    assert kpt_form(24 * 256, 63) == 24 and kpt_form(24 * 256 + 1, 63) is None
    assert kpt_form(2304, 31) == 9 and kpt_form(2305, 31) == 12


@pytest.mark.parametrize("max_rows", (1, 64, 4096, 4097, 9100, 65536, 131071, 131072 + 64))
def test_dense_attention_geometry(max_rows):
    """Dense decode: the 8-wave kernel over req_to_token[:seq_len], 32-row steps, up to
    4096 slots per block, as many parts as the table's width needs."""
    parts = dense_parts(max_rows)
    per_wave = ceil_div(max_rows, parts * HEAD_WAVES * 32) * 32
    for s in sorted({1, 31, 33, max_rows // 3, max_rows - 1, max_rows}):
        if s <= 0:
            continue
        n = min(s, max_rows)
        if parts > 12:  # the full model is quadratic in the slots: sample the parts' first and last blocks
            per_block = HEAD_WAVES * per_wave
            assert per_block <= HEAD_ROWCAP and parts * per_block >= n
            for part in (0, parts // 2, parts - 1):
                pb, written, reads, _ = attend_block(n, part * per_block, per_wave, HEAD_WAVES, 32)
                assert written == set(range(pb)) and (not reads or max(reads) < pb)
            continue
        check_launch(max_rows, n, parts, per_wave, HEAD_WAVES, 32, HEAD_ROWCAP)


@pytest.mark.parametrize("bs,top_k,G", list(itertools.product((1, 3, 16, 64), (64, 2048, 4096), (1, 8, 16))))
def test_partials_and_counters_in_bounds(bs, top_k, G):
    parts = step_parts(top_k)
    ws_floats = bs * KV * parts * G * (128 + 2)
    o_floats = bs * KV * parts * G * 128
    last_o = ((bs * KV - 1) * parts + parts - 1) * G + (G - 1)
    assert (last_o + 1) * 128 <= o_floats
    assert o_floats + (last_o + 1) * 2 <= ws_floats
    sync_words = bs * KV * 32
    assert (bs * KV - 1) * 32 < sync_words
    assert math.isfinite(ws_floats)


def test_model_catches_a_fill_of_the_real_slots_only():
    """The first fused kernel's fill (real slots only) fails the model at the faulting
    flow's shape: top_k 64, recent window only, 31 real slots."""
    top_k, n = 64, 31
    parts = step_parts(top_k)
    per_wave = step_per_wave(top_k, parts)
    _, _, reads, _ = attend_block(n, 0, per_wave, W4_WAVES, 16)
    written_real_only = set(range(n))
    assert not reads <= written_real_only
