"""Pin the numpy oracle for Quest (bounds, layout, GQA mean, scores, top-k).

Each check is one the oracle could fail with a plausible mistake: the
reference's own known answers (tests/test_quest_algorithm.py of the
reference), closed forms, brute force, and golden vectors written by
tests/golden/make_golden.py from the reference implementation.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bf16
from oracle import quest as oq
from tests.conftest import bf16_bits, load_golden

TOP_K, PAGE, KV, D, LAYERS, MAX_REQS, MAX_CTX = 256, 64, 4, 32, 2, 8, 2048


def make_state(top_k=TOP_K, page=PAGE, kv=KV, d=D, **kw) -> oq.QuestState:
    s = oq.QuestState(top_k, page, **kw)
    s.init_storage(0, LAYERS, MAX_REQS, MAX_CTX, kv, d)
    return s


def make_k(n, seed=0, kv=KV, d=D) -> np.ndarray:
    gen = torch.Generator().manual_seed(seed)
    return bf16_bits(torch.randn(n, kv, d, generator=gen).to(torch.bfloat16))


def prefill(s, req, pool, n):
    for layer in range(LAYERS):
        s.update_prefill_representations(layer, req, pool, np.arange(n))


def decode(s, req, pool, locs):
    for loc in locs:
        for layer in range(LAYERS):
            s.update_decode_representations(layer, [req], pool, [loc])
        s.maybe_finalize_decode_representations([req])


def retrieve(s, q, reqs, seq_lens, layer=0, q_is_bf16=False):
    s.prepare_step(seq_lens)
    pos, actual, _ = s.retrieve_topk(np.asarray(q, dtype=np.float32), layer, reqs, q_is_bf16=q_is_bf16)
    return pos, actual


# ----------------------------------------------------------------- bf16 helpers


def test_bf16_conversion_matches_torch_rne():
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(100000, generator=gen) * 10
    # exact ties at the rounding boundary, both parities, plus specials
    ties = torch.tensor([1.0 + 2**-8, 1.0 + 3 * 2**-8, -(1.0 + 2**-8), 3.4e38, -3.4e38, 0.0, -0.0,
                         float("inf"), float("-inf"), 1e-40])
    x = torch.cat([x, ties])
    ref = bf16_bits(x.to(torch.bfloat16))
    assert np.array_equal(bf16.from_f32(x.numpy()), ref)
    assert np.array_equal(bf16.to_f32(ref), x.to(torch.bfloat16).float().numpy())


def test_orderable_key_is_monotone_and_folds_signed_zero():
    vals = np.array([-np.inf, -3.0, -1e-30, -0.0, 0.0, 1e-30, 2.0, np.inf], dtype=np.float32)
    keys = bf16.orderable_u32(vals)
    assert np.all(np.diff(keys.astype(np.int64)[[0, 1, 2, 3, 5, 6, 7]]) > 0)
    assert keys[3] == keys[4]
    assert bf16.orderable_u32(np.array([np.nan], dtype=np.float32))[0] == 0xFFFFFFFF


# -------------------------------------------------------- storage + bounds


def test_invalid_top_k_page_size_combo_rejected():
    with pytest.raises(ValueError):
        oq.QuestState(100, 64)
    with pytest.raises(ValueError):
        oq.QuestState(64, 0)


def test_init_storage_shapes_and_sentinels():
    s = make_state()
    assert s.page_k_bounds.shape == (LAYERS, MAX_REQS, MAX_CTX // PAGE, KV, D, 2)
    assert not s.page_valid.any()
    assert np.all(bf16.to_f32(s.running_k_min) == torch.finfo(torch.bfloat16).max)
    assert np.all(bf16.to_f32(s.running_k_max) == torch.finfo(torch.bfloat16).min)


def test_prefill_bounds_full_pages_only():
    s, pool = make_state(), make_k(512)
    prefill(s, 2, pool, 192)
    assert s.page_valid[:, 2, :3].all() and not s.page_valid[:, 2, 3:].any()
    f = bf16.to_f32(pool)
    for layer in range(LAYERS):
        for p in range(3):
            slab = f[p * PAGE : (p + 1) * PAGE]
            assert np.array_equal(bf16.to_f32(s.page_k_bounds[layer, 2, p, ..., 0]), slab.min(0))
            assert np.array_equal(bf16.to_f32(s.page_k_bounds[layer, 2, p, ..., 1]), slab.max(0))
    assert s.running_token_count[2] == 0 and s.running_page_idx[2] == 3


def test_prefill_bounds_partial_last_page_seeds_running():
    s, pool = make_state(), make_k(512)
    prefill(s, 1, pool, 200)
    f = bf16.to_f32(pool)
    for layer in range(LAYERS):
        assert np.array_equal(bf16.to_f32(s.running_k_min[layer, 1]), f[192:200].min(0))
        assert np.array_equal(bf16.to_f32(s.running_k_max[layer, 1]), f[192:200].max(0))
    assert s.running_token_count[1] == 8 and s.running_page_idx[1] == 3


def test_prefill_of_fp32_keys_rounds_like_bf16_storage():
    gen = torch.Generator().manual_seed(4)
    k32 = torch.randn(128, KV, D, generator=gen)
    s1, s2 = make_state(), make_state()
    prefill(s1, 0, k32.numpy(), 128)
    prefill(s2, 0, bf16_bits(k32.to(torch.bfloat16)), 128)
    assert np.array_equal(s1.page_k_bounds, s2.page_k_bounds)


def test_decode_bounds_finalise_completed_page_equals_prefill_of_same_tokens():
    s, pool = make_state(), make_k(512, seed=11)
    prefill(s, 3, pool, 64)
    decode(s, 3, pool, range(64, 128))
    ref = make_state()
    prefill(ref, 3, pool, 128)
    assert np.array_equal(s.page_k_bounds, ref.page_k_bounds)
    assert s.running_token_count[3] == 0 and s.running_page_idx[3] == 2
    assert np.all(s.running_k_min[:, 3] == bf16.BF16_MAX_BITS)


def test_page_is_not_valid_until_its_last_token_arrives():
    s, pool = make_state(), make_k(256)
    prefill(s, 0, pool, 64)
    decode(s, 0, pool, range(64, 127))
    assert not s.page_valid[:, 0, 1].any()
    decode(s, 0, pool, [127])
    assert s.page_valid[:, 0, 1].all()


def test_invalidate_request_resets_one_slot_only():
    s, pool = make_state(), make_k(512)
    for r in (1, 2, 3):
        prefill(s, r, pool, 150)
    s.invalidate_request(2)
    assert s.page_valid[:, 1, :2].all() and s.page_valid[:, 3, :2].all()
    assert not s.page_valid[:, 2].any()
    assert s.running_token_count[2] == 0 and s.running_page_idx[2] == 0


# -------------------------------------------------------------- layout


def test_step_layout_closed_form():
    lay = oq.step_layout([1, 5, 64, 70, 2048, 2049, 10000], 64, 2048, False)
    assert lay.actual_lens.tolist() == [1, 5, 64, 70, 2048, 2048, 2048]
    assert lay.is_short.tolist() == [True] * 5 + [False] * 2
    assert lay.candidate_limit.tolist() == [0, 0, 1, 1, 32, 32, 156]
    assert lay.recent_positions[6].tolist() == list(range(9936, 10000))
    assert lay.recent_positions[1].tolist() == [0, 1, 2, 3, 4] + [4] * 59
    assert lay.short_layout[3, :72].tolist() == list(range(70)) + [69, 69]
    avoid = oq.step_layout([1, 64, 70, 10000], 64, 2048, True)
    assert avoid.candidate_limit.tolist() == [0, 0, 0, 155]


def test_retrieve_topk_long_seq_ends_with_recent_window():
    s, pool = make_state(), make_k(2048, seed=99)
    prefill(s, 0, pool, 800)
    q = torch.randn(1, KV, D).numpy()
    pos, actual = retrieve(s, q, [0], [800])
    assert pos.shape == (1, TOP_K) and pos.dtype == np.int32 and actual.dtype == np.int32
    assert pos[0, -PAGE:].tolist() == list(range(800 - PAGE, 800))
    assert pos.min() >= 0 and pos.max() < 800


def test_retrieve_topk_short_seq_is_dense():
    s, pool = make_state(), make_k(256, seed=77)
    prefill(s, 0, pool, 128)
    pos, actual = retrieve(s, torch.randn(1, KV, D).numpy(), [0], [128])
    assert int(actual[0]) == 128
    assert pos[0, :128].tolist() == list(range(128))
    assert int(pos[0, 128:].max()) == 127


def test_retrieve_topk_picks_high_score_pages_and_breaks_ties_low():
    s = make_state()
    pool = np.zeros((2048, KV, D), dtype=np.uint16)
    pool[320:384] = bf16.from_f32(np.float32(5.0))
    prefill(s, 0, pool, 640)
    pos, _ = retrieve(s, np.ones((1, KV, D)), [0], [640])
    # page 5 wins, the remaining 2 picks are the tied zero pages with the lowest index
    assert pos[0, :192].tolist() == list(range(320, 384)) + list(range(0, 128))


def test_score_upper_bounds_every_token_of_the_page():
    s = make_state(top_k=128, page=16)
    pool = make_k(512, seed=5)
    prefill(s, 0, pool, 512)
    f = bf16.to_f32(pool).astype(np.float64)
    for seed in range(5):
        q = torch.randn(1, KV, D, generator=torch.Generator().manual_seed(seed)).numpy()
        scores = oq.page_scores(q, s.page_k_bounds[0, [0]])[0, :32]
        per_token = np.einsum("hd,thd->t", q[0].astype(np.float64), f)
        assert np.all(scores >= per_token.reshape(32, 16).max(1) - 1e-3)


def test_scores_match_a_naive_loop():
    s = make_state(top_k=128, page=16)
    pool = make_k(256, seed=6)
    prefill(s, 0, pool, 256)
    q = torch.randn(1, KV, D, generator=torch.Generator().manual_seed(1)).numpy()
    fast = oq.page_scores(q, s.page_k_bounds[1, [0]])[0, :16]
    for p in range(16):
        kmin = bf16.to_f32(s.page_k_bounds[1, 0, p, ..., 0])
        kmax = bf16.to_f32(s.page_k_bounds[1, 0, p, ..., 1])
        naive = sum(max(float(q[0, h, d]) * float(kmin[h, d]), float(q[0, h, d]) * float(kmax[h, d]))
                    for h in range(KV) for d in range(D))
        assert abs(float(fast[p]) - naive) < 1e-3


def test_canonical_score_order_is_the_lane_tree():
    """A plausible wrong order (a plain left-to-right sum) gives a different fp32 result."""
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 4, 128)).astype(np.float32) * 1000
    b = bf16.from_f32(rng.standard_normal((1, 64, 4, 128, 2)).astype(np.float32))
    got = oq.page_scores(q, b)[0]
    prod = (q[:, None] * np.where(q[:, None] >= 0, bf16.to_f32(b[..., 1]), bf16.to_f32(b[..., 0])))
    prod = prod.reshape(64, 512).astype(np.float32)
    lane = prod.reshape(64, 64, 8)
    acc = lane[..., 0]
    for j in range(1, 8):
        acc = (acc + lane[..., j]).astype(np.float32)
    tree = acc
    while tree.shape[1] > 1:
        h = tree.shape[1] // 2
        tree = (tree[:, :h] + tree[:, h:]).astype(np.float32)
    assert np.array_equal(got, tree[:, 0])
    seq = np.zeros(64, dtype=np.float32)
    for c in range(512):
        seq = (seq + prod[:, c]).astype(np.float32)
    assert not np.array_equal(got, seq)
    assert np.allclose(got, prod.astype(np.float64).sum(1), rtol=1e-5)


def test_gqa_queries_are_averaged_per_kv_group():
    q = torch.randn(3, 4 * KV, D).numpy()
    g = oq.group_queries(q.reshape(3, -1), KV, D, is_bf16=False)
    for h in range(KV):
        assert np.allclose(g[:, h], q[:, 4 * h : 4 * h + 4].mean(1), atol=1e-6)
    with pytest.raises(ValueError):
        oq.group_queries(np.zeros((3, 6, D)), KV, D, is_bf16=False)


def test_gqa_mean_matches_torch_bf16_mean_bitwise():
    gen = torch.Generator().manual_seed(8)
    q = torch.randn(64, 32, 128, generator=gen).to(torch.bfloat16)
    ref = q.view(64, 4, 8, 128).mean(dim=2)
    got = oq.group_queries(q.float().numpy(), 4, 128, is_bf16=True)
    assert np.array_equal(bf16.from_f32(got), bf16_bits(ref))


def test_unfinished_and_out_of_range_pages_are_never_selected():
    s = make_state(top_k=128, page=16)
    pool = make_k(1024, seed=3)
    big = 100 * torch.randn(1, KV, D, generator=torch.Generator().manual_seed(0)).numpy()
    prefill(s, 0, pool, 176)
    decode(s, 0, pool, range(176, 191))
    pos, _ = retrieve(s, big, [0], [192])
    assert int(pos[0, : 128 - 16].max()) < 176
    prefill(s, 1, pool, 1000)
    pos, _ = retrieve(s, big, [1], [300])
    assert int(pos[0, : 128 - 16].max()) < (300 // 16) * 16


def test_recent_window_overlap_upstream_vs_avoid():
    pool = np.zeros((2048, KV, D), dtype=np.uint16)
    pool[48:64] = bf16.from_f32(np.float32(3.0))
    q = np.ones((1, KV, D))
    up = make_state(top_k=32, page=16)
    prefill(up, 0, pool, 70)
    pos, _ = retrieve(up, q, [0], [70])
    assert sorted(pos[0].tolist()) != sorted(set(pos[0].tolist()))
    assert set(range(54, 64)) <= set(pos[0, :16].tolist())
    fixed = make_state(top_k=32, page=16, avoid_recent_overlap=True)
    prefill(fixed, 0, pool, 70)
    pos, actual = retrieve(fixed, q, [0], [70])
    assert len(set(pos[0].tolist())) == int(actual[0]) == 32
    assert pos[0, -16:].tolist() == list(range(54, 70))


def test_mixed_batch_of_short_and_long_requests():
    s, pool = make_state(top_k=64, page=16), make_k(1024, seed=8)
    prefill(s, 0, pool, 40)
    prefill(s, 1, pool, 300)
    pos, actual = retrieve(s, torch.randn(2, KV, D).numpy(), [0, 1], [40, 300])
    assert actual.tolist() == [40, 64]
    assert pos[0, :40].tolist() == list(range(40))
    assert pos[1, -16:].tolist() == list(range(284, 300))
    assert int(pos[1, :48].max()) < 288


# ------------------------------------------------------ golden vectors


def _assert_selection_matches(ours, ref, scores, limit, k, page):
    """Same page set as the reference; any difference must be an exact-score tie."""
    ours_pages = ours[: k * page : page] // page
    ref_pages = ref[: k * page : page] // page
    if set(ours_pages.tolist()) == set(ref_pages.tolist()):
        assert np.array_equal(ours[k * page :], ref[k * page :])
        return True
    s = scores.copy()
    s[limit:] = -np.inf
    diff = set(ours_pages.tolist()) ^ set(ref_pages.tolist())
    kth = np.sort(s)[::-1][k - 1]
    assert all(s[p] == kth for p in diff), "selection differs beyond a tie"
    return False


def test_golden_c1_scores_and_selection():
    g = load_golden("c1_selection.npz")
    q = bf16.to_f32(g["queries"])
    qbar = oq.group_queries(q, 4, 128, is_bf16=True)
    assert np.array_equal(bf16.from_f32(qbar), g["qbar"])
    bounds = np.broadcast_to(g["bounds"], (16,) + g["bounds"].shape)
    ours = oq.page_scores(qbar, bounds)
    ref = g["scores"][0]
    # the reference's fp32 order is torch's; ours is canonical: a few ulps apart at most
    assert np.allclose(ours, ref, rtol=0, atol=4 * np.spacing(np.abs(ref).max()))
    exact = 0
    for avoid in (0, 1):
        for si, s in enumerate(g["seq_lens"]):
            lay = oq.step_layout(np.full(16, s), 64, 2048, bool(avoid))
            pos, actual, _ = oq.retrieve_topk(qbar, bounds, lay, 64, 2048)
            refpos = g[f"positions_avoid{avoid}"][si]
            for i in range(16):
                n = int(actual[i])
                if lay.is_short[i]:
                    assert np.array_equal(pos[i, :n], refpos[i, :n])
                else:
                    exact += _assert_selection_matches(
                        pos[i], refpos[i], ours[i], int(lay.candidate_limit[i]), 31, 64)
    assert exact >= 150  # with random keys every long selection agrees exactly


def test_golden_small_shapes_fp32_and_bf16_queries():
    g = load_golden("small_selection.npz")
    for c in range(4):
        top_k, page, heads, is_bf16, _ = g[f"c{c}_meta"].tolist()
        q, seq = g[f"c{c}_q"], g[f"c{c}_seq"]
        qbar = oq.group_queries(q, 4, 32, is_bf16=bool(is_bf16))
        assert np.allclose(qbar, g[f"c{c}_qbar"], rtol=0, atol=2e-7 * max(1, np.abs(qbar).max()))
        bounds = np.broadcast_to(g[f"c{c}_bounds"], (4,) + g[f"c{c}_bounds"].shape)
        scores = oq.page_scores(qbar, bounds)
        ref_scores = g[f"c{c}_scores"]
        finite = np.isfinite(ref_scores)
        assert np.array_equal(np.isfinite(scores), finite)
        assert np.allclose(scores[finite], ref_scores[finite], rtol=1e-5, atol=1e-4)
        lay = oq.step_layout(seq, page, top_k, False)
        pos, actual, _ = oq.retrieve_topk(qbar, bounds, lay, page, top_k)
        assert np.array_equal(actual, g[f"c{c}_actual"])
        k = top_k // page - 1
        for i in range(4):
            n = int(actual[i])
            ref = g[f"c{c}_positions"][i]
            if lay.is_short[i]:
                assert np.array_equal(pos[i, :n], ref[:n])
            else:
                _assert_selection_matches(pos[i], ref, scores[i], int(lay.candidate_limit[i]), k, page)
