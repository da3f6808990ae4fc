"""CPU model of the fused attention kernels' index arithmetic (qwenquest_amd/csrc/decode.hip).

The Quest step's attention (quest_attend_unit_kernel) works in units of 64 layout slots
(one selected page, the recent window, or 64 slots of the dense layout): wave w of part p
takes units p*W + w, p*W + w + W*parts, ...  For every launch shape the host can choose
the model checks that every unit's slots lie inside the layout, that the real slots
[0, n) of a request are attended exactly once, that each wave's row shuffles stay inside
the wave, that the selection reads only score entries of the request's row, keeps its
survivors inside its LDS array and asks for ranks < k, that partial and counter indices
stay inside their buffers, and that the LDS a launch allocates fits the CU.

Dense decode (quest_attend_part_kernel) still stages rows in an LDS row table; its model
checks that every table entry a step reads lies inside the block's table and was written
by the fill.  The first fused attention kernel of this library faulted the GPU on a
recent-window-only flow (top_k 64, k_sel 0, seq_len < 64): its table fill wrote only the
real slots, while a step reads all 16 (or 32) entries of its tile (the ones past n are
masked in the softmax only), so uninitialised LDS words became pool-row indices.  The
fill now covers the block's whole share; test_model_catches_a_fill_of_the_real_slots_only
keeps the model honest about that case.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest

# geometry of decode.hip (kept in step with its constants and host helpers)
PARTS_MAX = 8
HEAD_WAVES, HEAD_TILES, HEAD_ROWCAP = 8, 2, 4096
MAX_SEL, MAX_TOPK, MAX_G, KV, UNIT = 64, 4096, 16, 4, 64
KPT_FORMS = (2, 4, 5, 6, 8, 9, 12, 16, 24)
KPT_MAX = {4: 32, 8: 24}  # the last form of each block width
CUS = 256


def ceil_div(a, b):
    return -(-a // b)


def unit_shape(bs, top_k, cus=CUS):
    """(waves per block, parts per (request, KV head)) as decode.hip's unit_shape picks them."""
    units, pairs = top_k // UNIT, bs * KV
    cap8 = max(1, min(PARTS_MAX, ceil_div(units, 8)))
    cap4 = max(1, min(PARTS_MAX, ceil_div(units, 4)))
    if pairs * units < 8 * cus:
        return 4, cap4
    if pairs <= cus:
        return 8, max(1, min(cap8, cus // pairs))
    return 4, max(1, min(cap4, ceil_div(2 * cus, pairs)))


def dense_parts(max_rows):
    return max(1, ceil_div(max_rows, MAX_TOPK))


def kpt_form(max_pages, k_sel, nt):
    n_max = max(max_pages, k_sel)
    for kpt in KPT_FORMS:
        if n_max <= kpt * nt:
            return kpt
    return KPT_MAX[nt // 64]


def rank_select_smem_bytes(kpt, nt):
    # RankSelectSmem<KPT, NT>: gmax[64] u32, gcnt[NT/64][64] i32, cand[NT*KPT+64] u64 (8-aligned),
    # crank[NT/64][64] i32, count, order[64]
    b = 64 * 4 + (nt // 64) * 64 * 4
    b = ceil_div(b, 8) * 8 + (nt * kpt + 64) * 8
    b += (nt // 64) * 64 * 4 + 4 + 64 * 4
    return ceil_div(b, 8) * 8


def unit_smem_bytes(kpt, waves):
    comb = 2 * waves * MAX_G * 4 + waves * MAX_G * 128 * 4
    return max(rank_select_smem_bytes(kpt, 64 * waves), comb)


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


def check_units(top_k, n, bs):
    """The unit kernel's slot coverage for one request of a batch of bs."""
    waves, parts = unit_shape(bs, top_k)
    units = top_k // UNIT
    seen = []
    for part in range(parts):
        for w in range(waves):
            for u in range(part * waves + w, units, parts * waves):
                assert 0 <= u < units
                for lane in range(64):
                    slot = u * UNIT + lane
                    assert slot < top_k
                    if slot < n:
                        seen.append(slot)
                # shuffle sources of the K tiles (16t + lo) and V steps (16t + 4hi + j)
                srcs = {t * 16 + lo for t in range(4) for lo in range(16)} | {
                    t * 16 + hi * 4 + j for t in range(4) for hi in range(4) for j in range(4)}
                assert max(srcs) < 64
    assert sorted(seen) == list(range(n)), "real slots not attended exactly once"
    return waves, parts


def sel_page(tid, i, nt, spread=True):
    """Page whose score thread tid holds in slot i (qq_quest_dev.h sel_page): page
    blocks (page tid + nt*i, as the scores are loaded) or, spread (fewer candidates
    than threads), page nt*i + g + 64*m with group g of nt/64 consecutive threads."""
    gs = nt // 64
    return nt * i + tid // gs + 64 * (tid % gs) if spread else tid + nt * i


def kernel_page(tid, i, nt, lim):
    """The mapping the selections use for a request with lim candidates."""
    return sel_page(tid, i, nt, lim < nt)


def check_selection(top_k, page, max_pages, lim, waves):
    nt = 64 * waves
    k = top_k // page - 1
    kpt = kpt_form(max_pages, k, nt)
    n_eff = max(lim, k)
    assert n_eff <= kpt * nt
    # every page slot of the block is held by exactly one (thread, slot), in both mappings;
    # the spread moves slot 0 only, inside the block's first nt pages
    for spread in (False, True):
        assert sorted(sel_page(t, i, nt, spread) for t in range(nt) for i in range(kpt)) == list(range(nt * kpt))
    assert sorted(sel_page(t, 0, nt, True) for t in range(nt)) == list(range(nt))
    # score reads (page blocks) clamp to the request's row of max_pages entries
    reads = {min(tid + nt * i, max_pages - 1) for tid in range(nt) for i in range(kpt)}
    assert max(reads) < max_pages and min(reads) >= 0
    assert k <= MAX_SEL
    # survivors are a subset of the block's nt*kpt keys: cand holds nt*kpt + 64
    assert nt * kpt <= nt * kpt + 64
    smem = unit_smem_bytes(kpt, waves)
    assert smem <= (80 * 1024 if waves == 4 else 160 * 1024)  # two 4-wave blocks share a CU's 160 KiB


TOPKS = (64, 128, 192, 256, 1024, 2048, 2112, 4032, 4096)
SEQS = (1, 2, 15, 16, 31, 33, 63, 64, 65, 127, 2047, 2048, 2049, 4095, 4096, 4097, 9000, 131072)


@pytest.mark.parametrize("top_k", TOPKS)
@pytest.mark.parametrize("bs", (1, 4, 16, 32, 48, 64, 96, 128, 256))
def test_unit_attention_slots(top_k, bs):
    for s in SEQS:
        check_units(top_k, min(max(s, 0), top_k), bs)


def test_benchmark_shape_runs_one_unit_per_wave():
    """Batch 16 x top_k 2048: 8-wave blocks, 4 parts per (request, KV head), 256 blocks
    (one per CU), each wave one 64-row unit."""
    waves, parts = check_units(2048, 2048, 16)
    assert (waves, parts) == (8, 4) and 16 * KV * parts == CUS
    assert unit_shape(8, 2048) == (4, 8)


def test_larger_batches_fill_one_round_of_blocks():
    """Past batch 16 (2048 slots) a wave takes several units one after the other so that
    the grid is about one round of resident blocks: 8-wave blocks up to one (request, KV
    head) pair per CU, then two 4-wave blocks per CU."""
    for bs, shape, units_per_wave in ((32, (8, 2), 2), (48, (8, 1), 4), (64, (8, 1), 4), (96, (4, 2), 4),
                                      (128, (4, 1), 8), (256, (4, 1), 8)):
        waves, parts = check_units(2048, 2048, bs)
        assert (waves, parts) == shape
        assert ceil_div(2048 // UNIT, waves * parts) == units_per_wave
        assert bs * KV * parts <= 4 * CUS


@pytest.mark.parametrize("top_k", TOPKS)
def test_rows_mode_actual_lengths(top_k):
    """quest_hisparse's rows mode: n = clamp(actual, 0, slots) for any given actual length."""
    for actual in (-3, 0, 1, 17, top_k - 1, top_k, top_k + 5):
        check_units(top_k, min(max(actual, 0), top_k), 16)


@pytest.mark.parametrize("max_pages", (2, 64, 512, 513, 1024, 2049, 2050, 2304, 2305, 2560, 2561, 3072, 4096, 6144,
                                       6145, 7040, 8192))
@pytest.mark.parametrize("waves", (4, 8))
def test_selection_forms(max_pages, waves):
    """The KPT form the host picks holds every candidate page: 2304 / 2560 (contexts just
    past 128K at 4 / 8 waves), 3072, 6144, 8192 pages (the fused step's limit) and the
    forms between."""
    for top_k, page in ((64, 64), (128, 64), (2048, 64), (4096, 64), (4160, 64)):
        if top_k // page - 1 > MAX_SEL:
            continue
        for lim in sorted({0, 1, max_pages // 2, max_pages - 1, max_pages}):
            check_selection(top_k, page, max_pages, lim, waves)


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


@pytest.mark.parametrize("bs,top_k,G", list(itertools.product((1, 3, 16, 64, 128), (64, 2048, 4096), (1, 8, 16))))
def test_partials_and_counters_in_bounds(bs, top_k, G):
    parts = unit_shape(bs, top_k)[1]
    assert parts <= PARTS_MAX  # one merge pass
    ws_floats = bs * KV * parts * G * (128 + 2)
    o_floats = bs * KV * parts * G * 128
    last_o = ((bs * KV - 1) * parts + parts - 1) * G + (G - 1)
    assert (last_o + 1) * 128 <= o_floats
    assert o_floats + (last_o + 1) * 2 <= ws_floats
    # the caller's workspace: qq_decode_attention_workspace_bytes(bs, top_k, H, D) floats
    assert ws_floats <= bs * ceil_div(top_k, 64) * (G * KV) * (128 + 2)
    sync_words = bs * KV * 32
    assert (bs * KV - 1) * 32 < sync_words
    assert math.isfinite(ws_floats)


def test_model_catches_a_fill_of_the_real_slots_only():
    """The first fused kernel's fill (real slots only) fails the table model at the faulting
    flow's shape: top_k 64, recent window only, 31 real slots, 4 waves of 32 rows in
    16-row steps."""
    n = 31
    _, _, reads, _ = attend_block(n, 0, 32, 4, 16)
    written_real_only = set(range(n))
    assert not reads <= written_real_only


# ------------------------------------------------------------- selection model
# select_ranked / select_topk_block (qq_quest_dev.h) on the CPU: keys ordered by score,
# then lower page; tau = the k-th largest maximum of 64 groups of nt/64 consecutive
# threads; the keys >= tau survive and are ranked.  The model checks the two-stage
# algorithm against an exact top-k (np.lexsort) and the survivor count that decides
# between the 64-survivor ranking and the quadratic one.


def model_select(scores, lim, n_eff, k, nt, kpt, mapping):
    """(pages in rank order, survivor count) of the block selection; mapping(tid, i, nt)
    gives the page a thread's slot holds."""
    gs = nt // 64
    keys = np.zeros((nt, kpt), dtype=object)
    for tid in range(nt):
        for i in range(kpt):
            p = mapping(tid, i, nt)
            if p < n_eff:
                sc = scores[p] if p < lim else -np.inf
                keys[tid, i] = (sc, -p)  # larger = higher score, then lower page
            else:
                keys[tid, i] = None  # not a page: below every key
    def kmax(a, b):
        if a is None:
            return b
        if b is None:
            return a
        return max(a, b)
    gmax = []
    for g in range(64):
        m = None
        for t in range(g * gs, (g + 1) * gs):
            for i in range(kpt):
                m = kmax(m, keys[t, i])
        gmax.append(m)
    real = sorted((m for m in gmax if m is not None), reverse=True)
    tau = real[k - 1] if len(real) >= k else None  # None: every key survives
    surv = [key for key in keys.flat if key is not None and (tau is None or key >= tau)]
    surv.sort(reverse=True)
    return [-key[1] for key in surv[:k]], len(surv)


def exact_topk(scores, lim, n_eff, k):
    sc = np.array([scores[p] if p < lim else -np.inf for p in range(n_eff)])
    order = np.lexsort((np.arange(n_eff), -sc))  # score desc, page asc
    return [int(p) for p in order[:k]]


@pytest.mark.parametrize("lim,nt,kpt", [(31, 256, 2), (40, 256, 2), (63, 256, 2), (127, 256, 2), (127, 512, 2),
                                        (255, 512, 2), (300, 256, 2), (1023, 512, 2), (2047, 512, 5)])
def test_selection_model_matches_exact_topk(lim, nt, kpt):
    rng = np.random.default_rng(lim * 7 + nt)
    k = 31
    n_eff = max(lim, k)
    for trial in range(3):
        scores = rng.standard_normal(lim).astype(np.float32)
        if trial == 1:  # heavy ties: a few distinct values
            scores = rng.integers(0, 4, lim).astype(np.float32)
        pages, total = model_select(scores, lim, n_eff, k, nt, kpt, lambda t, i, n: kernel_page(t, i, n, lim))
        assert pages == exact_topk(scores, lim, n_eff, k)
        if trial == 0 and lim >= 64:
            # distinct scores: the threshold keeps the ranking on its 64-survivor path
            assert total <= 64, (lim, nt, total)


def test_page_blocks_would_take_the_quadratic_ranking():
    """Page blocks alone (page tid + nt*i) fill 16 of 64 groups with 127 candidates at
    nt = 512: every key passes the threshold.  Spread, the same candidates keep the
    ranking on its 64-survivor path; from nt candidates on, blocks fill every group."""
    rng = np.random.default_rng(5)
    scores = rng.standard_normal(127).astype(np.float32)
    block = lambda tid, i, nt: sel_page(tid, i, nt, False)  # noqa: E731
    pages, total = model_select(scores, 127, 127, 31, 512, 2, block)
    assert pages == exact_topk(scores, 127, 127, 31)
    assert total == 127
    _, total_rr = model_select(scores, 127, 127, 31, 512, 2, sel_page)
    assert total_rr <= 64
    for nt in (256, 512):
        gs = nt // 64
        filled = {sel_page(t, 0, nt, False) // gs for t in range(nt)}  # groups with a page < nt
        assert len(filled) == 64
