"""GPU parity of the Quest path (bounds, GQA mean, scores, selection, attention)
against the CPU oracle on identical seeded inputs.

Bounds, scores (canonical order), positions: bit-exact.  Attention: 1e-4 abs in fp32;
in bf16 the stated 2e-2 abs, tightened to 1e-3 + 1% of the largest output
(tests.conftest.attn_tol).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import bf16
from oracle import quest as oq
from tests.conftest import assert_attn_close, bf16_bits, load_golden

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def rand_bf16(shape, seed, scale=1.0, mean=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    if mean is not None:
        x = x + mean
    return x.to(torch.bfloat16)


def new_quest(top_k, page, layers, reqs, ctx, kv, d, avoid=False):
    from qwenquest_amd.quest import QuestAlgorithm

    q = QuestAlgorithm(top_k=top_k, page_size=page, device=DEV, avoid_recent_overlap=avoid)
    q.init_storage(0, layers, reqs, ctx, kv, d)
    st = oq.QuestState(top_k, page, avoid_recent_overlap=avoid)
    st.init_storage(0, layers, reqs, ctx, kv, d)
    return q, st


def assert_state_equal(q, st):
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(q.page_k_bounds), st.page_k_bounds)
    assert np.array_equal(bf16_bits(q.running_k_min), st.running_k_min)
    assert np.array_equal(bf16_bits(q.running_k_max), st.running_k_max)
    assert np.array_equal(q.running_token_count.cpu().numpy(), st.running_token_count)
    assert np.array_equal(q.running_page_idx.cpu().numpy(), st.running_page_idx)


# ------------------------------------------------------------------ bounds


def test_init_storage_sentinels_match_oracle():
    q, st = new_quest(256, 64, 2, 3, 1000, 4, 32)
    assert_state_equal(q, st)
    assert not q.page_valid.any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n", [0, 30, 64, 192, 200, 777])
@pytest.mark.parametrize("d,idx_dtype", [(32, torch.int32), (128, torch.int32), (128, torch.int64)])
def test_prefill_bounds_bit_exact(dtype, n, d, idx_dtype):
    """KV*D = 128 (the 16-byte block fold), 512 (one wave per page, bf16), fp32 keys (the
    per-element fold); partial pages, gathered rows, int32 and int64 indices."""
    q, st = new_quest(256, 64, 2, 4, 1024, 4, d)
    pool = rand_bf16((1100, 4, d), seed=n).to(dtype)
    idx = torch.randperm(1100, generator=torch.Generator().manual_seed(1))[:n].to(idx_dtype)
    host = pool.float().numpy() if dtype == torch.float32 else bf16_bits(pool)
    for layer in range(2):
        q.update_prefill_representations(layer, 2, pool.to(DEV), idx.to(DEV))
        st.update_prefill_representations(layer, 2, host, idx.numpy())
    assert_state_equal(q, st)


@pytest.mark.parametrize("page", [16, 128, 256])
@pytest.mark.parametrize("n", [100, 777])
def test_prefill_bounds_other_page_sizes_bit_exact(page, n):
    """The wave-per-page fold at KV*D = 512 with pages shorter and longer than its 64-row index
    chunks (bf16 keys, gathered rows, a partial last page)."""
    q, st = new_quest(256, page, 1, 4, 1024, 4, 128)
    pool = rand_bf16((1100, 4, 128), seed=n + page)
    idx = torch.randperm(1100, generator=torch.Generator().manual_seed(2))[:n].to(torch.int32)
    q.update_prefill_representations(0, 1, pool.to(DEV), idx.to(DEV))
    st.update_prefill_representations(0, 1, bf16_bits(pool), idx.numpy())
    assert_state_equal(q, st)


def test_prefill_bounds_special_values_fold_in_row_order():
    """bf16 keys at KV*D = 512 (one wave per page: batches without NaN or zero fold as
    16-bit key min / max, the others element by element) against the same keys as fp32
    (the per-element fold): NaN, +-0 and +-inf scattered over the rows, bit-identical
    bounds and running bounds."""
    n, d = 777, 128
    pool = rand_bf16((1100, 4, d), seed=5)
    bits = pool.view(torch.int16)
    g = torch.Generator().manual_seed(6)
    for val in (0x7FC0, 0x0000, 0x8000, 0x7F80, 0xFF80):
        for _ in range(25):
            r = int(torch.randint(0, 1100, (1,), generator=g))
            c = int(torch.randint(0, 4 * d, (1,), generator=g))
            bits[r].view(-1)[c] = val - 65536 if val >= 32768 else val
    idx = torch.randperm(1100, generator=torch.Generator().manual_seed(1))[:n].to(torch.int32)
    qb, _ = new_quest(256, 64, 1, 4, 1024, 4, d)
    qf, _ = new_quest(256, 64, 1, 4, 1024, 4, d)
    qb.update_prefill_representations(0, 2, pool.to(DEV), idx.to(DEV))
    qf.update_prefill_representations(0, 2, pool.float().to(DEV), idx.to(DEV))
    torch.cuda.synchronize()
    for name in ("page_k_bounds", "running_k_min", "running_k_max"):
        assert torch.equal(getattr(qb, name).view(torch.int16), getattr(qf, name).view(torch.int16)), name
    assert torch.isnan(qb.page_k_bounds.float()).any()


def test_prefill_fused_over_layers_equals_per_layer():
    from qwenquest_amd.memory import MHATokenToKVPool

    kvp = MHATokenToKVPool(600, 3, 2, 16, torch.bfloat16, DEV)
    kvp.k_all.copy_(rand_bf16((3, 601, 2, 16), seed=3).to(DEV))
    idx = torch.arange(1, 517, device=DEV)
    a, _ = new_quest(64, 16, 3, 2, 600, 2, 16)
    b, _ = new_quest(64, 16, 3, 2, 600, 2, 16)
    a.update_prefill_representations_fused(1, kvp.k_all, idx)
    for layer in range(3):
        b.update_prefill_representations(layer, 1, kvp.k_buffer[layer], idx)
    torch.cuda.synchronize()
    assert torch.equal(a.page_k_bounds, b.page_k_bounds)
    assert torch.equal(a.running_k_min, b.running_k_min)
    assert torch.equal(a.running_token_count, b.running_token_count)


def test_fused_bounds_with_start_layer_read_the_model_layers():
    """A backend covering model layers 2..3 of a 4-layer pool: the fused prefill and decode
    fold read k_all[2] and k_all[3] (the pool is indexed by model layer id), equal to the
    per-layer calls; a k_all holding fewer layers than end_layer is refused."""
    from qwenquest_amd.memory import MHATokenToKVPool
    from qwenquest_amd.quest import QuestAlgorithm

    kvp = MHATokenToKVPool(600, 4, 2, 16, torch.bfloat16, DEV)
    kvp.k_all.copy_(rand_bf16((4, 601, 2, 16), seed=13).to(DEV))
    a = QuestAlgorithm(top_k=64, page_size=16, device=DEV)
    b = QuestAlgorithm(top_k=64, page_size=16, device=DEV)
    for qa in (a, b):
        qa.init_storage(2, 4, 2, 600, 2, 16)
    idx = torch.arange(1, 300, device=DEV)
    a.update_prefill_representations_fused(1, kvp.k_all, idx)
    for layer in (2, 3):
        b.update_prefill_representations(layer, 1, kvp.k_buffer[layer], idx)
    reqs = torch.tensor([1], device=DEV)
    for step in range(20):
        locs = torch.tensor([300 + step], device=DEV)
        a.update_decode_representations_fused(reqs, kvp.k_all, locs)
        for layer in (2, 3):
            b.update_decode_representations(layer, reqs, kvp.k_buffer[layer], locs)
        b.maybe_finalize_decode_representations(reqs)
    torch.cuda.synchronize()
    assert torch.equal(a.page_k_bounds, b.page_k_bounds)
    assert torch.equal(a.running_k_min, b.running_k_min) and torch.equal(a.running_k_max, b.running_k_max)
    assert torch.equal(a.running_token_count, b.running_token_count)
    assert torch.equal(a.running_page_idx, b.running_page_idx)
    with pytest.raises(ValueError, match="layers"):
        a.update_prefill_representations_fused(0, kvp.k_all[:3].contiguous(), idx)


@pytest.mark.parametrize("fused", [False, True])
def test_decode_fold_and_finalize_bit_exact_across_page_boundaries(fused):
    from qwenquest_amd.memory import MHATokenToKVPool

    L, KV, D, P = 2, 4, 32, 16
    kvp = MHATokenToKVPool(400, L, KV, D, torch.bfloat16, DEV)
    kvp.k_all.copy_(rand_bf16((L, 401, KV, D), seed=5).to(DEV))
    host = bf16_bits(kvp.k_all.cpu())
    q, st = new_quest(64, P, L, 3, 400, KV, D)
    for r, n in ((0, 50), (2, 64)):
        q.update_prefill_representations_fused(r, kvp.k_all, torch.arange(1 + 100 * r, 1 + 100 * r + n, device=DEV))
        for layer in range(L):
            st.update_prefill_representations(layer, r, host[layer], np.arange(1 + 100 * r, 1 + 100 * r + n))
    reqs = torch.tensor([0, 2], device=DEV)
    for step in range(40):
        locs = torch.tensor([1 + 50 + step, 201 + 64 + step], device=DEV)
        if fused:
            q.update_decode_representations_fused(reqs, kvp.k_all, locs)
        else:
            for layer in range(L):
                q.update_decode_representations(layer, reqs, kvp.k_buffer[layer], locs)
            q.maybe_finalize_decode_representations(reqs)
        for layer in range(L):
            st.update_decode_representations(layer, [0, 2], host[layer], locs.cpu().numpy())
        st.maybe_finalize_decode_representations([0, 2])
    assert_state_equal(q, st)
    assert q.page_valid[:, 0, :5].all() and not q.page_valid[:, 0, 5:].any()


def test_decode_skip_rows_are_left_untouched():
    from qwenquest_amd.memory import MHATokenToKVPool

    kvp = MHATokenToKVPool(100, 1, 2, 8, torch.bfloat16, DEV)
    kvp.k_all.copy_(rand_bf16((1, 101, 2, 8), seed=6).to(DEV))
    q, _ = new_quest(16, 4, 1, 2, 64, 2, 8)
    q.update_prefill_representations_fused(0, kvp.k_all, torch.arange(1, 4, device=DEV))
    before = (q.running_k_min.clone(), q.running_token_count.clone())
    q.update_decode_representations_fused(torch.tensor([0], device=DEV), kvp.k_all, torch.tensor([-1], device=DEV))
    torch.cuda.synchronize()
    assert torch.equal(before[0], q.running_k_min) and torch.equal(before[1], q.running_token_count)


def test_invalidate_request_resets_one_slot():
    q, st = new_quest(64, 16, 2, 4, 512, 4, 32)
    pool = rand_bf16((512, 4, 32), seed=7)
    for r in (1, 2, 3):
        for layer in range(2):
            q.update_prefill_representations(layer, r, pool.to(DEV), torch.arange(150, device=DEV))
            st.update_prefill_representations(layer, r, bf16_bits(pool), np.arange(150))
    q.invalidate_request(2)
    st.invalidate_request(2)
    assert_state_equal(q, st)


# ----------------------------------------------------------- GQA mean + scores


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("heads,kv", [(32, 4), (16, 4), (4, 4), (8, 2)])
def test_group_queries_bit_exact(dtype, heads, kv):
    from qwenquest_amd.quest import QuestAlgorithm

    d = 32
    quest = QuestAlgorithm(top_k=64, page_size=16, device=DEV)
    quest.init_storage(0, 1, 1, 64, kv, d)
    qv = rand_bf16((5, heads, d), seed=heads).to(dtype)
    got = quest.group_queries(qv.to(DEV)).float().cpu().numpy()
    ref = oq.group_queries(qv.float().numpy(), kv, d, is_bf16=dtype == torch.bfloat16)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("kv,d", [(4, 128), (4, 32), (2, 8), (5, 32), (8, 128), (1, 24)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_page_scores_bit_exact_in_canonical_order(kv, d, dtype):
    P = 8
    q, st = new_quest(32, P, 1, 2, 512, kv, d)
    pool = rand_bf16((512, kv, d), seed=kv * d)
    q.update_prefill_representations(0, 1, pool.to(DEV), torch.arange(400, device=DEV))
    st.update_prefill_representations(0, 1, bf16_bits(pool), np.arange(400))
    qbar = (rand_bf16((3, kv, d), seed=9) * 3).to(dtype)
    got = q.page_scores(qbar.to(DEV), 0, torch.tensor([1, 1, 0], device=DEV)).cpu().numpy()
    ref = oq.page_scores(qbar.float().numpy(), st.page_k_bounds[0, [1, 1, 0]])
    assert np.array_equal((got + np.float32(0)).view(np.uint32), (ref + np.float32(0)).view(np.uint32))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))


@pytest.mark.parametrize("kv,d,group", [(4, 128, 4), (4, 128, 1), (4, 128, 2), (4, 128, 8), (4, 128, 16), (8, 128, 4),
                                         (4, 64, 4), (2, 32, 4), (5, 32, 4), (3, 8, 4)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_retrieve_scores_bit_exact_in_canonical_order(kv, d, group, dtype):
    """The scores retrieve_topk ranks (its scoring launch, fused with the GQA mean) equal
    the oracle's bit for bit on every candidate page, for the 16-byte lane-load shapes
    (KV*D = 256, 512, 1024; at 4 x 128 with bf16 queries and GQA groups of 2 .. 8 the
    4-pages-per-wave kernel, other groups the general one) and the general shapes;
    3 requests of different limits (partial page tiles)."""
    P, heads = 16, kv * group
    q, st = new_quest(64, P, 1, 3, 4096, kv, d)
    pool = rand_bf16((4096, kv, d), seed=kv * d + 1, mean=rand_bf16((4096, 1, 1), seed=3, scale=0.5))
    lens = (4000, 1500, 700)
    for r, n in enumerate(lens):
        q.update_prefill_representations(0, r, pool.to(DEV), torch.arange(n, device=DEV))
        st.update_prefill_representations(0, r, bf16_bits(pool), np.arange(n))
    queries = (rand_bf16((3, heads, d), seed=kv + d) * 2).to(dtype)
    reqs, seqs = [2, 0, 1], [701, 4001, 1501]
    q.prepare_step(torch.tensor(seqs, device=DEV))
    q.retrieve_topk(queries.to(DEV), 0, torch.tensor(reqs, device=DEV), torch.tensor(seqs, device=DEV))
    got = q._scores_ws[:3].cpu().numpy()
    qbar = oq.group_queries(queries.float().numpy(), kv, d, is_bf16=dtype == torch.bfloat16)
    lay = st.prepare_step(seqs)
    for i, r in enumerate(reqs):
        lim = int(lay.candidate_limit[i])
        ref = oq.page_scores(qbar[i : i + 1], st.page_k_bounds[0, [r], :lim])[0]
        assert np.array_equal((got[i, :lim] + np.float32(0)).view(np.uint32), (ref + np.float32(0)).view(np.uint32))


# ------------------------------------------------------------------ selection


def run_retrieve(q, st, queries, reqs, seqs, layer=0):
    seq_t = torch.tensor(seqs, device=DEV)
    q.prepare_step(seq_t)
    pos, actual = q.retrieve_topk(queries.to(DEV), layer, torch.tensor(reqs, device=DEV), seq_t)
    st.prepare_step(seqs)
    ref_pos, ref_actual, _ = st.retrieve_topk(queries.float().numpy(), layer, reqs,
                                              q_is_bf16=queries.dtype == torch.bfloat16)
    pos, actual = pos.cpu().numpy(), actual.cpu().numpy()
    assert np.array_equal(actual, ref_actual)
    for i in range(len(seqs)):
        n = int(actual[i])
        assert np.array_equal(pos[i, :n], ref_pos[i, :n]), f"request {i} seq {seqs[i]}"
    return pos, actual


@pytest.mark.parametrize("avoid", [False, True])
@pytest.mark.parametrize("top_k,P,heads", [(256, 64, 4), (128, 16, 16), (64, 16, 32), (32, 8, 8), (16, 16, 4)])
def test_retrieve_topk_positions_bit_exact(avoid, top_k, P, heads):
    kv, d = 4, 32
    q, st = new_quest(top_k, P, 2, 4, 2048, kv, d, avoid)
    pool = rand_bf16((2048, kv, d), seed=top_k + P)
    lens = (2000, 800, top_k, 300)
    for r, n in enumerate(lens):
        for layer in range(2):
            q.update_prefill_representations(layer, r, pool.to(DEV), torch.arange(n, device=DEV))
            st.update_prefill_representations(layer, r, bf16_bits(pool), np.arange(n))
    for dtype in (torch.bfloat16, torch.float32):
        queries = rand_bf16((4, heads, d), seed=heads).to(dtype)
        run_retrieve(q, st, queries, [0, 1, 2, 3], [2001, 801, top_k, 301], layer=1)
        run_retrieve(q, st, queries[:2], [3, 0], [300 + P, 1999])


def test_retrieve_topk_ties_break_to_lowest_page():
    q, st = new_quest(256, 64, 1, 1, 2048, 4, 32)
    pool = torch.zeros(2048, 4, 32, dtype=torch.bfloat16)
    pool[320:384] = 5.0
    q.update_prefill_representations(0, 0, pool.to(DEV), torch.arange(640, device=DEV))
    st.update_prefill_representations(0, 0, bf16_bits(pool), np.arange(640))
    pos, _ = run_retrieve(q, st, torch.ones(1, 4, 32), [0], [640])
    assert pos[0, :192].tolist() == list(range(320, 384)) + list(range(0, 128))


def test_recent_window_overlap_known_answer():
    pool = torch.zeros(2048, 4, 32, dtype=torch.bfloat16)
    pool[48:64] = 3.0
    for avoid in (False, True):
        q, st = new_quest(32, 16, 1, 1, 2048, 4, 32, avoid)
        q.update_prefill_representations(0, 0, pool.to(DEV), torch.arange(70, device=DEV))
        st.update_prefill_representations(0, 0, bf16_bits(pool), np.arange(70))
        pos, actual = run_retrieve(q, st, torch.ones(1, 4, 32), [0], [70])
        if avoid:
            assert len(set(pos[0].tolist())) == 32 and pos[0, -16:].tolist() == list(range(54, 70))
        else:
            assert set(range(54, 64)) <= set(pos[0, :16].tolist())


def test_large_selection_count_and_stale_bounds():
    """top_k / P - 1 = 255 selected pages (page size 1) and stale bounds past seq_len."""
    q, st = new_quest(256, 1, 1, 2, 1024, 2, 16)
    pool = rand_bf16((1024, 2, 16), seed=11)
    for r in range(2):
        q.update_prefill_representations(0, r, pool.to(DEV), torch.arange(1000, device=DEV))
        st.update_prefill_representations(0, r, bf16_bits(pool), np.arange(1000))
    run_retrieve(q, st, rand_bf16((2, 8, 16), seed=12), [0, 1], [1001, 600])


def test_outlier_channels_stress_ties_and_overflow():
    """Keys with x10 outlier channels and huge queries (sentinel pages -> -inf scores)."""
    kv, d = 4, 128
    pool = rand_bf16((4096, kv, d), seed=13).float()
    pool[:, :, :4] *= 10
    pool = pool.to(torch.bfloat16)
    for avoid in (False, True):
        q, st = new_quest(2048, 64, 1, 2, 4200, kv, d, avoid)
        q.update_prefill_representations(0, 0, pool.to(DEV), torch.arange(4000, device=DEV))
        st.update_prefill_representations(0, 0, bf16_bits(pool), np.arange(4000))
        queries = rand_bf16((2, 32, d), seed=14, scale=50)
        run_retrieve(q, st, queries, [0, 1], [4090, 2100])


def test_golden_c1_selection_through_the_kernel():
    """The reference's own positions (tests/golden, C1 shape): identical page sets."""
    from qwenquest_amd.quest import QuestAlgorithm

    g = load_golden("c1_selection.npz")
    queries = torch.from_numpy(g["queries"].view(np.int16)).view(torch.bfloat16)
    agree = 0
    for avoid in (0, 1):
        quest = QuestAlgorithm(top_k=2048, page_size=64, device=DEV, avoid_recent_overlap=bool(avoid))
        quest.init_storage(0, 1, 16, 8192, 4, 128)
        b = torch.from_numpy(g["bounds"].view(np.int16)).view(torch.bfloat16).to(DEV)
        quest.page_k_bounds[0].copy_(b.expand(16, *b.shape))
        for si, s in enumerate(g["seq_lens"].tolist()):
            seq = torch.full((16,), s, device=DEV)
            quest.prepare_step(seq)
            pos, actual = quest.retrieve_topk(queries.to(DEV), 0, torch.arange(16, device=DEV), seq)
            pos = pos.cpu().numpy()
            ref = g[f"positions_avoid{avoid}"][si]
            for i in range(16):
                n = int(actual[i])
                if s <= 2048:
                    assert np.array_equal(pos[i, :n], ref[i, :n])
                else:
                    assert sorted(pos[i, :1984:64].tolist()) == sorted(ref[i, :1984:64].tolist())
                    assert np.array_equal(pos[i, 1984:], ref[i, 1984:])
                    agree += 1
    assert agree == 160


# ------------------------------------------------------------------ attention


def attention_case(dtype, heads, kv, d, n_rows, seed, dup=False):
    from qwenquest_amd.attention.ops import decode_attention_rows

    pool = 3000
    k = rand_bf16((pool, kv, d), seed=seed).to(dtype)
    v = rand_bf16((pool, kv, d), seed=seed + 1).to(dtype)
    q = rand_bf16((len(n_rows), heads, d), seed=seed + 2).to(dtype)
    width = max(n_rows)
    gen = torch.Generator().manual_seed(seed)
    rows = torch.randint(0, pool, (len(n_rows), width), generator=gen)
    if dup:
        rows[:, 1] = rows[:, 0]
    actual = torch.tensor(n_rows, dtype=torch.int32)
    out = decode_attention_rows(q.to(DEV), k.to(DEV), v.to(DEV), rows.to(DEV), actual.to(DEV), d**-0.5)
    ref = oa.sparse_decode(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                           [rows[i, :n].numpy() for i, n in enumerate(n_rows)], d**-0.5)
    return out.float().cpu().numpy(), ref


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float32, 1e-4)])
@pytest.mark.parametrize("heads,kv,d", [(32, 4, 128), (8, 2, 16), (16, 4, 32), (4, 4, 8)])
def test_attention_matches_oracle(dtype, tol, heads, kv, d):
    out, ref = attention_case(dtype, heads, kv, d, [2048, 1, 65, 700], seed=heads + d, dup=True)
    if dtype == torch.bfloat16:
        assert_attn_close(out, ref, f"{heads}/{kv} heads x {d}")
    assert np.abs(out - ref).max() < tol


def test_decode_attention_single_request_api():
    from qwenquest_amd.attention.ops import decode_attention

    q = rand_bf16((8, 16), seed=1).float()
    k = rand_bf16((40, 2, 16), seed=2).float()
    v = rand_bf16((40, 2, 16), seed=3).float()
    rows = [0, 1, 2, 2, 39]
    out = decode_attention(q.to(DEV), k[rows].to(DEV), v[rows].to(DEV), 0.25).cpu().numpy()
    ref = oa.decode_attention(q.numpy(), k[rows].numpy(), v[rows].numpy(), 0.25)
    assert np.abs(out - ref).max() < 1e-5


# ------------------------------------------------------------ full backend


def test_quest_backend_decode_steps_match_oracle():
    """QuestOnlyBackend over 70 decode steps (pages complete and get selected) vs the oracle."""
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    L, H, KV, D, P, TOP_K, CTX = 2, 8, 2, 16, 8, 32, 256
    rtp = ReqToTokenPool(3, CTX, DEV)
    kvp = MHATokenToKVPool(3 * CTX, L, KV, D, torch.bfloat16, DEV)
    be = QuestOnlyBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P})
    st = oq.QuestState(TOP_K, P)
    st.init_storage(0, L, 3, CTX, KV, D)
    kk = rand_bf16((L, 3 * CTX + 1, KV, D), seed=21)
    vv = rand_bf16((L, 3 * CTX + 1, KV, D), seed=22)
    kb, vb = bf16.to_f32(bf16_bits(kk)), bf16.to_f32(bf16_bits(vv))
    kvp.k_all.copy_(kk.to(DEV))
    kvp.v_all.copy_(vv.to(DEV))
    prompt = {0: 45, 2: 20}
    for r, n in prompt.items():
        rtp.req_to_token[r] = torch.arange(1 + r * CTX, 1 + (r + 1) * CTX, dtype=torch.int32)
        be.quest.update_prefill_representations_fused(r, kvp.k_all, rtp.req_to_token[r, :n])
        be._skip_first_decode_update[r] = True
        for layer in range(L):
            st.update_prefill_representations(layer, r, bf16_bits(kk[layer]), np.arange(1 + r * CTX, 1 + r * CTX + n))
    reqs = [0, 2]
    first = {0: True, 2: True}

    class Layer:
        def __init__(self, i):
            self.layer_id, self.scaling = i, D**-0.5

    for step in range(70):
        seqs = [prompt[r] + step + 1 for r in reqs]
        batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.tensor(reqs, device=DEV),
                             torch.tensor(seqs, device=DEV), None, rtp, kvp, be)
        be.init_forward_metadata(batch)
        active = [r for r in reqs if not first[r]]
        for r in reqs:
            first[r] = False
        if active:
            for layer in range(L):
                locs = [1 + r * CTX + prompt[r] + step - 1 for r in active]
                st.update_decode_representations(layer, active, bf16_bits(kk[layer]), locs)
            st.maybe_finalize_decode_representations(active)
        st.prepare_step(seqs)
        q = rand_bf16((2, H, D), seed=100 + step)
        for layer in range(L):
            pos, actual = be.quest.retrieve_topk(q.to(DEV), layer, batch.req_pool_indices, batch.seq_lens)
            out = be.sparse_attention(q.to(DEV), Layer(layer), batch.req_pool_indices, pos, actual, 2)
            ref_pos, ref_actual, _ = st.retrieve_topk(q.float().numpy(), layer, reqs)
            pos = pos.cpu().numpy()
            for i, r in enumerate(reqs):
                n = int(ref_actual[i])
                assert np.array_equal(pos[i, :n], ref_pos[i, :n]), f"step {step} layer {layer} req {r}"
            rows = [1 + r * CTX + ref_pos[i, : int(ref_actual[i])] for i, r in enumerate(reqs)]
            ref = oa.sparse_decode(q.float().numpy(), kb[layer], vb[layer], rows, D**-0.5)
            assert_attn_close(out.float().cpu().numpy(), ref, f"step {step} layer {layer}")
    assert_state_equal(be.quest, st)


def test_determinism_bitwise():
    q, _ = new_quest(2048, 64, 1, 4, 32768, 4, 128)
    pool = rand_bf16((32768, 4, 128), seed=31).to(DEV)
    for r in range(4):
        q.update_prefill_representations(0, r, pool, torch.arange(32768 - 1000 * r, device=DEV))
    queries = rand_bf16((4, 32, 128), seed=32).to(DEV)
    seq = torch.tensor([32768, 31000, 30000, 29001], device=DEV)
    q.prepare_step(seq)
    a, _ = q.retrieve_topk(queries, 0, torch.arange(4, device=DEV), seq)
    a = a.clone()
    b, _ = q.retrieve_topk(queries, 0, torch.arange(4, device=DEV), seq)
    assert torch.equal(a, b)


def step_counters(be, bs):
    """The fused layer step's sync buffer: counters only, zero between calls."""
    return be._step_sync


# (layers, q heads, kv heads, head_dim, page, top_k, ctx, prompts, steps).  Flows with
# bf16, 4 KV heads x 128, page 64 and at most 64 selected pages run the two-launch fused
# layer step; the others the four-launch path.  Fused: the benchmark's shape with long,
# short, exactly-top_k and one-past requests; top_k 256 (one attention tile per head);
# top_k 64 (recent window only); top_k 4160 (64 selected pages, 17 tiles, G = 16); G = 1
# with a request reaching a multiple of 64 (its newest page becomes a candidate).
# Four-launch: head_dim 16; page 16 with top_k 48; G = 1 with page 8; 8 KV heads.
ENGINE_FLOWS = [
    (2, 8, 2, 16, 8, 32, 256, {1: 37, 2: 60}, 40),
    (1, 32, 4, 128, 64, 2048, 9000, {0: 8800, 1: 2046, 2: 2047, 3: 1000}, 4),
    (1, 32, 4, 128, 64, 256, 3000, {0: 2900, 1: 255, 2: 700}, 6),
    (1, 4, 4, 128, 64, 64, 700, {0: 650, 1: 63}, 4),
    (2, 64, 4, 128, 64, 4160, 9000, {0: 8900, 1: 4000, 2: 4159}, 3),
    (1, 4, 4, 128, 64, 2048, 6000, {0: 4094, 1: 5000}, 4),
    (1, 16, 4, 128, 16, 48, 600, {0: 500, 1: 40, 2: 47}, 12),
    (1, 4, 4, 128, 8, 64, 700, {0: 650, 2: 63}, 6),
    (1, 64, 8, 128, 32, 256, 1500, {0: 1400, 1: 255}, 4),
    (1, 64, 4, 128, 64, 2048, 6000, {0: 5900, 1: 2100, 2: 300}, 3),  # 16 q heads per KV head, fused
]


@pytest.mark.parametrize("flow", range(len(ENGINE_FLOWS)))
def test_forward_decode_fused_path_engine_flow(flow):
    """QuestOnlyBackend.forward_decode (one C call: new K/V store + select + attention) over
    decode steps whose K/V only arrives through forward_decode, vs the oracle; with trace."""
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool
    from qwenquest_amd.quest import QuestTrace

    L, H, KV, D, P, TOP_K, CTX, prompt, steps = ENGINE_FLOWS[flow]
    nreq = max(prompt) + 1
    for avoid in (False, True):
        rtp = ReqToTokenPool(nreq, CTX, DEV)
        kvp = MHATokenToKVPool(nreq * CTX, L, KV, D, torch.bfloat16, DEV)
        be = QuestOnlyBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P,
                                         "avoid_recent_overlap": avoid})
        be.quest.trace = QuestTrace()
        st = oq.QuestState(TOP_K, P, avoid_recent_overlap=avoid)
        st.init_storage(0, L, nreq, CTX, KV, D)
        kk = rand_bf16((L, nreq * CTX + 1, KV, D), seed=41)
        vv = rand_bf16((L, nreq * CTX + 1, KV, D), seed=42)
        kb, vb = bf16.to_f32(bf16_bits(kk)), bf16.to_f32(bf16_bits(vv))
        for r, n in prompt.items():
            rows = torch.arange(1 + r * CTX, 1 + r * CTX + n)
            rtp.req_to_token[r] = torch.arange(1 + r * CTX, 1 + (r + 1) * CTX, dtype=torch.int32)
            kvp.k_all[:, rows] = kk[:, rows].to(DEV)
            kvp.v_all[:, rows] = vv[:, rows].to(DEV)
            be.quest.update_prefill_representations_fused(r, kvp.k_all, rtp.req_to_token[r, :n])
            be._skip_first_decode_update[r] = True
            for layer in range(L):
                st.update_prefill_representations(layer, r, bf16_bits(kk[layer]), rows.numpy())
        reqs = sorted(prompt)

        class Layer:
            def __init__(self, i):
                self.layer_id, self.scaling = i, D**-0.5

        for step in range(steps):
            seqs = [prompt[r] + step + 1 for r in reqs]
            locs = torch.tensor([1 + r * CTX + s - 1 for r, s in zip(reqs, seqs)], device=DEV)
            batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.tensor(reqs, device=DEV),
                                 torch.tensor(seqs, device=DEV), locs, rtp, kvp, be)
            be.init_forward_metadata(batch)
            if step > 0:
                for layer in range(L):
                    st.update_decode_representations(layer, reqs, bf16_bits(kk[layer]), (locs - 1).cpu().numpy())
                st.maybe_finalize_decode_representations(reqs)
            st.prepare_step(seqs)
            q = rand_bf16((len(reqs), H, D), seed=300 + step)
            for layer in range(L):
                lc = locs.cpu()
                out = be.forward_decode(q.to(DEV), kk[layer, lc].to(DEV), vv[layer, lc].to(DEV), Layer(layer), batch)
                ref_pos, ref_actual, _ = st.retrieve_topk(q.float().numpy(), layer, reqs)
                rec = be.quest.trace.records[-len(reqs):]
                for i, r in enumerate(reqs):
                    n = int(ref_actual[i])
                    assert np.array_equal(rec[i].positions.numpy(), ref_pos[i, :n]), f"step {step} L{layer} r{r}"
                rows = [1 + r * CTX + ref_pos[i, : int(ref_actual[i])] for i, r in enumerate(reqs)]
                ref = oa.sparse_decode(q.float().numpy(), kb[layer], vb[layer], rows, D**-0.5)
                assert_attn_close(out.float().cpu().numpy(), ref, f"step {step} layer {layer}")
        assert_state_equal(be.quest, st)
        # the new tokens really went to the pool
        torch.cuda.synchronize()
        last = [1 + r * CTX + prompt[r] + steps - 1 for r in reqs]
        assert torch.equal(kvp.k_all[:, last].cpu(), kk[:, last])
        assert not step_counters(be, len(reqs)).any()  # the fused path leaves its counters at zero


R2T_LAYOUTS = ("page_runs", "scattered", "mixed")


@pytest.mark.parametrize("layout,ctx", [(lay, 3200) for lay in R2T_LAYOUTS] +
                         [("page_runs", 147456), ("scattered", 196608)])
def test_fused_step_req_to_token_layouts(layout, ctx):
    """The fused layer step over req_to_token layouts that are not one run per request:
    pages as runs at shuffled bases, scattered rows, and page runs broken by swapped rows.
    Positions bit-exact vs the oracle, outputs within attn_tol of the oracle's attention over
    r2t[req, positions].  The long tables (2304 and 3072 pages) take the selection's 9- and
    12-keys-per-thread forms."""
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    H, KV, D, P, TOP_K, CTX = 32, 4, 128, 64, 1024, ctx
    prompt = {0: CTX - 200, 1: CTX * 15 // 32, 2: CTX * 21 // 32}
    steps = 4
    nreq = len(prompt)
    rows_total = nreq * CTX + 1
    gen = np.random.default_rng(R2T_LAYOUTS.index(layout) + 11)
    if layout == "scattered":
        r2t = (gen.permutation(nreq * CTX) + 1).astype(np.int32).reshape(nreq, CTX)
    else:
        bases = gen.permutation(nreq * CTX // P)[: nreq * (CTX // P)] * P + 1
        r2t = (bases[:, None] + np.arange(P)[None]).reshape(nreq, CTX).astype(np.int32)
        if layout == "mixed":
            for r in range(nreq):
                for pg in range(r, CTX // P, 3):  # every third page: two rows swapped
                    a, b = pg * P + 5, pg * P + 40
                    r2t[r, a], r2t[r, b] = r2t[r, b], r2t[r, a]
    rtp = ReqToTokenPool(nreq, CTX, DEV)
    rtp.req_to_token.copy_(torch.from_numpy(r2t).to(DEV))
    kvp = MHATokenToKVPool(rows_total - 1, 1, KV, D, torch.bfloat16, DEV)
    be = QuestOnlyBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P})
    st = oq.QuestState(TOP_K, P)
    st.init_storage(0, 1, nreq, CTX, KV, D)
    kk = rand_bf16((1, rows_total, KV, D), seed=81)
    vv = rand_bf16((1, rows_total, KV, D), seed=82)
    kb, vb = bf16.to_f32(bf16_bits(kk)), bf16.to_f32(bf16_bits(vv))
    for r, n in prompt.items():
        rows = torch.from_numpy(r2t[r, :n].astype(np.int64))
        kvp.k_all[:, rows] = kk[:, rows].to(DEV)
        kvp.v_all[:, rows] = vv[:, rows].to(DEV)
        be.quest.update_prefill_representations_fused(r, kvp.k_all, rtp.req_to_token[r, :n])
        be._skip_first_decode_update[r] = True
        st.update_prefill_representations(0, r, bf16_bits(kk[0]), rows.numpy())
    reqs = sorted(prompt)

    class Layer:
        layer_id, scaling = 0, D**-0.5

    for step in range(steps):
        seqs = [prompt[r] + step + 1 for r in reqs]
        locs = torch.tensor([int(r2t[r, s - 1]) for r, s in zip(reqs, seqs)], device=DEV)
        batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.tensor(reqs, device=DEV),
                             torch.tensor(seqs, device=DEV), locs, rtp, kvp, be)
        be.init_forward_metadata(batch)
        if step > 0:
            prev = np.array([r2t[r, s - 2] for r, s in zip(reqs, seqs)])
            st.update_decode_representations(0, reqs, bf16_bits(kk[0]), prev)
            st.maybe_finalize_decode_representations(reqs)
        st.prepare_step(seqs)
        q = rand_bf16((len(reqs), H, D), seed=400 + step)
        lc = locs.cpu()
        out = be.forward_decode(q.to(DEV), kk[0, lc].to(DEV), vv[0, lc].to(DEV), Layer(), batch)
        pos = be._positions[: len(reqs)].clone()
        ref_pos, ref_actual, _ = st.retrieve_topk(q.float().numpy(), 0, reqs)
        got_pos = pos.cpu().numpy()
        rows = []
        for i, r in enumerate(reqs):
            n = int(ref_actual[i])
            assert np.array_equal(got_pos[i, :n], ref_pos[i, :n]), f"step {step} r{r}"
            rows.append(r2t[r, ref_pos[i, :n]].astype(np.int64))
        ref = oa.sparse_decode(q.float().numpy(), kb[0], vb[0], rows, D**-0.5)
        assert_attn_close(out.float().cpu().numpy(), ref, f"step {step}")
    assert not step_counters(be, len(reqs)).any()



@pytest.mark.parametrize("case", ["equal_keys", "wide_selection"])
def test_fused_step_ties_and_wide_selection(case):
    """The fused step's in-block selection on its slow paths, through QuestOnlyBackend:
    every key equal (all page scores tie, so every candidate passes the threshold - more
    than 64 survivors - and the ties break to the lowest page), and top_k 4096 (63 selected
    pages: the threshold is the 63rd largest of 64 group maxima, so hundreds of pages survive
    and the ranking counts).  Positions bit-exact vs the oracle over three decode steps,
    outputs within attn_tol of the oracle's attention over r2t[req, positions]."""
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    H, KV, D, P = 32, 4, 128, 64
    TOP_K, CTX = (2048, 40000) if case == "equal_keys" else (4096, 20000)
    prompt = {0: CTX - 100, 1: CTX * 2 // 3, 2: TOP_K + 300}
    steps, nreq = 3, 3
    rows_total = nreq * CTX + 1
    r2t = (1 + np.arange(nreq * CTX)).astype(np.int32).reshape(nreq, CTX)
    rtp = ReqToTokenPool(nreq, CTX, DEV)
    rtp.req_to_token.copy_(torch.from_numpy(r2t).to(DEV))
    kvp = MHATokenToKVPool(rows_total - 1, 1, KV, D, torch.bfloat16, DEV)
    be = QuestOnlyBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P})
    from qwenquest_amd import _lib

    bf = _lib.DTYPE_BF16  # the shape takes the fused (two-launch) layer step
    assert _lib.load().qq_quest_fused_step(bf, bf, bf, H, KV, D, P, TOP_K, be.quest.max_pages_per_req) == 1
    st = oq.QuestState(TOP_K, P)
    st.init_storage(0, 1, nreq, CTX, KV, D)
    if case == "equal_keys":
        kk = torch.zeros((1, rows_total, KV, D), dtype=torch.bfloat16)
    else:
        kk = rand_bf16((1, rows_total, KV, D), seed=91)
    vv = rand_bf16((1, rows_total, KV, D), seed=92)
    kb, vb = bf16.to_f32(bf16_bits(kk)), bf16.to_f32(bf16_bits(vv))
    kvp.k_all.copy_(kk.to(DEV))
    kvp.v_all.copy_(vv.to(DEV))
    for r, n in prompt.items():
        rows = torch.from_numpy(r2t[r, :n].astype(np.int64))
        be.quest.update_prefill_representations_fused(r, kvp.k_all, rtp.req_to_token[r, :n])
        be._skip_first_decode_update[r] = True
        st.update_prefill_representations(0, r, bf16_bits(kk[0]), rows.numpy())
    reqs = sorted(prompt)

    class Layer:
        layer_id, scaling = 0, D**-0.5

    for step in range(steps):
        seqs = [prompt[r] + step + 1 for r in reqs]
        locs = torch.tensor([int(r2t[r, s - 1]) for r, s in zip(reqs, seqs)], device=DEV)
        batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.tensor(reqs, device=DEV),
                             torch.tensor(seqs, device=DEV), locs, rtp, kvp, be)
        be.init_forward_metadata(batch)
        if step > 0:
            prev = np.array([r2t[r, s - 2] for r, s in zip(reqs, seqs)])
            st.update_decode_representations(0, reqs, bf16_bits(kk[0]), prev)
            st.maybe_finalize_decode_representations(reqs)
        st.prepare_step(seqs)
        q = rand_bf16((len(reqs), H, D), seed=500 + step)
        lc = locs.cpu()
        out = be.forward_decode(q.to(DEV), kk[0, lc].to(DEV), vv[0, lc].to(DEV), Layer(), batch)
        pos = be._positions[: len(reqs)].clone()
        ref_pos, ref_actual, _ = st.retrieve_topk(q.float().numpy(), 0, reqs)
        got_pos = pos.cpu().numpy()
        rows = []
        for i, r in enumerate(reqs):
            n = int(ref_actual[i])
            assert np.array_equal(got_pos[i, :n], ref_pos[i, :n]), f"{case} step {step} r{r}"
            rows.append(r2t[r, ref_pos[i, :n]].astype(np.int64))
        if case == "equal_keys":  # ties: the lowest pages first, then the recent window
            s0 = seqs[0]
            want = np.concatenate([np.arange(TOP_K - P), np.arange(s0 - P, s0)])
            assert np.array_equal(got_pos[0, :TOP_K], want)
        ref = oa.sparse_decode(q.float().numpy(), kb[0], vb[0], rows, D**-0.5)
        assert_attn_close(out.float().cpu().numpy(), ref, f"{case} step {step}")
    assert not step_counters(be, len(reqs)).any()

def test_positions_and_rows_entries_are_bit_identical():
    """qq_quest_decode_attention (positions through req_to_token) and
    qq_decode_attention_rows (rows given) on the same rows give the same bits, with
    ragged lengths (0, 1, 31, 2048), duplicated and out-of-range positions."""
    from qwenquest_amd.attention.ops import decode_attention_rows
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    H, KV, D, CTX, W = 32, 4, 128, 3000, 2048
    rtp = ReqToTokenPool(5, CTX, DEV)
    kvp = MHATokenToKVPool(5 * CTX, 1, KV, D, torch.bfloat16, DEV)
    be = QuestOnlyBackend(rtp, kvp, {"algorithm": "quest", "top_k": W, "quest_page_size": 64})
    gen = torch.Generator().manual_seed(5)
    kvp.k_all.copy_(rand_bf16(tuple(kvp.k_all.shape), seed=51).to(DEV))
    kvp.v_all.copy_(rand_bf16(tuple(kvp.v_all.shape), seed=52).to(DEV))
    r2t = torch.randperm(5 * CTX, generator=gen)[: 5 * CTX].view(5, CTX).to(torch.int32) + 1
    rtp.req_to_token.copy_(r2t.to(DEV))
    reqs = torch.tensor([4, 0, 2, 3], dtype=torch.int64)
    actual = torch.tensor([2048, 0, 1, 31], dtype=torch.int32)
    pos = torch.randint(0, CTX, (4, W), generator=gen, dtype=torch.int32)
    pos[0, 5] = pos[0, 4]
    pos[3, 7] = CTX + 5  # outside req_to_token: row 0
    q = rand_bf16((4, H, D), seed=53)

    class Layer:
        layer_id, scaling = 0, D**-0.5

    out_pos = be.sparse_attention(q.to(DEV), Layer(), reqs.to(DEV), pos.to(DEV), actual.to(DEV), 4)
    p64 = pos.to(torch.int64)
    rows = torch.where(p64 < CTX, r2t[reqs[:, None], p64.clamp(max=CTX - 1)].to(torch.int64), 0)
    out_rows = decode_attention_rows(q.to(DEV), kvp.k_buffer[0], kvp.v_buffer[0], rows.to(DEV), actual.to(DEV), D**-0.5)
    assert torch.equal(out_pos, out_rows)
    kb = bf16.to_f32(bf16_bits(kvp.k_all[0].cpu()))
    vb = bf16.to_f32(bf16_bits(kvp.v_all[0].cpu()))
    got = out_rows.float().cpu().numpy()
    for i in (0, 2, 3):
        r = rows[i, : int(actual[i])].numpy()
        ref = oa.decode_attention(q[i].float().numpy(), kb[r], vb[r], D**-0.5)
        assert_attn_close(got[i], ref, f"request {i}")
    assert not got[1].any()  # no rows: zeros


def test_fused_layer_step_graph_replay_eager_and_four_launch_agree():
    """The fused (two-launch) layer step replayed from a HIP graph equals its eager run bit for bit
    (positions and outputs, every replay), the four-launch path gives the same positions
    and outputs within attn_tol, and the sync counters are back at zero after each step."""
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    L, H, KV, D, P, TOP_K, CTX = 2, 32, 4, 128, 64, 2048, 6200
    prompts = [6000, 4095, 2047, 1000]
    B = len(prompts)
    kk = rand_bf16((L, B * CTX + 1, KV, D), seed=71)
    vv = rand_bf16((L, B * CTX + 1, KV, D), seed=72)
    qs = rand_bf16((L, B, H, D), seed=73)
    kn = rand_bf16((L, B, KV, D), seed=74)
    vn = rand_bf16((L, B, KV, D), seed=75)

    class Layer:
        def __init__(self, i):
            self.layer_id, self.scaling = i, D**-0.5

    def setup(four_launch):
        rtp = ReqToTokenPool(B, CTX, DEV)
        kvp = MHATokenToKVPool(B * CTX, L, KV, D, torch.bfloat16, DEV)
        kvp.k_all.copy_(kk.to(DEV))
        kvp.v_all.copy_(vv.to(DEV))
        base = 1 + torch.arange(B, device=DEV, dtype=torch.int64) * CTX
        rtp.req_to_token.copy_((base[:, None] + torch.arange(CTX, device=DEV)[None]).to(torch.int32))
        be = QuestOnlyBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P})
        if four_launch:
            be._step_sync = None
        for r, n in enumerate(prompts):
            be.quest.update_prefill_representations_fused(r, kvp.k_all, rtp.req_to_token[r, :n])
            be._skip_first_decode_update[r] = True
        seq = torch.tensor([n + 1 for n in prompts], device=DEV)
        loc = torch.empty(B, device=DEV, dtype=torch.int64)
        batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.arange(B, device=DEV), seq, loc, rtp, kvp, be)
        outs = torch.empty((L, B, H * D), dtype=torch.bfloat16, device=DEV)
        pos = torch.empty((L, B, TOP_K), dtype=torch.int32, device=DEV)
        qd, knd, vnd = qs.to(DEV), kn.to(DEV), vn.to(DEV)

        def step():
            torch.add(base, seq - 1, out=loc)
            be.init_forward_metadata(batch)
            for layer in range(L):
                outs[layer].copy_(be.forward_decode(qd[layer], knd[layer], vnd[layer], Layer(layer), batch))
                pos[layer].copy_(be._positions[:B])
            seq.add_(1)

        return be, step, outs, pos

    runs = {}
    for name in ("eager", "graph", "four"):
        be, step, outs, pos = setup(name == "four")
        step()  # first decode step after prefill, eager
        run = step
        if name == "graph":
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step()
            run = g.replay
        res = []
        for _ in range(70):  # crosses page boundaries: bounds finalized inside the steps
            run()
            torch.cuda.synchronize()
            if be._step_sync is not None:
                assert not step_counters(be, B).any()
            res.append((outs.clone(), pos.clone()))
        runs[name] = res
    for i, ((oe, pe), (og, pg), (of, pf)) in enumerate(zip(runs["eager"], runs["graph"], runs["four"])):
        assert torch.equal(pe, pg) and torch.equal(oe, og), f"graph replay {i} differs from eager"
        assert torch.equal(pe, pf), f"step {i}: four-launch positions differ"
        assert_attn_close(of.float().cpu().numpy(), oe.float().cpu().numpy(), f"step {i}: four-launch vs fused")


def test_decode_step_row_lookup():
    """qq_quest_decode_step_locs (quest_only.py:84-97): the previous token's pool row
    req_to_token[r, max(seq - 2, 0)] per listed request, -1 on a request's first decode step
    (its flag read before any clear, also when the request is listed twice) and for requests
    or positions outside the table; every listed request's flag is cleared."""
    from qwenquest_amd import _lib

    R, W = 4, 16
    r2t = (torch.arange(R * W, dtype=torch.int32) * 7 + 3).view(R, W).to(DEV)
    skip = torch.tensor([1, 0, 1, 1], dtype=torch.uint8, device=DEV)
    rpi = torch.tensor([0, 2, 0, 1, 5, -1, 1], dtype=torch.int64, device=DEV)
    seq = torch.tensor([10, 5, 10, 1, 9, 9, 40], dtype=torch.int64, device=DEV)
    out = torch.full((rpi.numel(),), 99, dtype=torch.int64, device=DEV)
    _lib.call("qq_quest_decode_step_locs", _lib.ptr(rpi), _lib.ptr(seq), rpi.numel(), _lib.ptr(skip), _lib.ptr(r2t),
              R, W, W, _lib.ptr(out), _lib.stream(DEV))
    torch.cuda.synchronize()
    t = r2t.cpu().long()
    expected = [-1, -1, -1, int(t[1, 0]), -1, -1, -1]  # r 0 and 2 skipped; r 1 at p = 0; r 5, -1 outside; p 38 >= W
    assert out.cpu().tolist() == expected
    assert skip.cpu().tolist() == [0, 0, 0, 1]
    skip.zero_()
    _lib.call("qq_quest_decode_step_locs", _lib.ptr(rpi[:2]), _lib.ptr(seq[:2]), 2, _lib.ptr(skip), _lib.ptr(r2t),
              R, W, W, _lib.ptr(out), _lib.stream(DEV))
    torch.cuda.synchronize()
    assert out[:2].cpu().tolist() == [int(t[0, 8]), int(t[2, 3])]
    # a view of the first 6 columns of the table: positions past its width give -1, not the
    # next row's entries
    view = r2t[:, :6]
    seq2 = torch.tensor([8, 8, 7, 3], dtype=torch.int64, device=DEV)  # p = 6, 6, 5, 1
    rpi2 = torch.tensor([0, 1, 2, 3], dtype=torch.int64, device=DEV)
    _lib.call("qq_quest_decode_step_locs", _lib.ptr(rpi2), _lib.ptr(seq2), 4, _lib.ptr(skip), _lib.ptr(view),
              R, view.shape[1], view.stride(0), _lib.ptr(out), _lib.stream(DEV))
    torch.cuda.synchronize()
    assert out[:4].cpu().tolist() == [-1, -1, int(t[2, 5]), int(t[3, 1])]


def test_one_launch_decode_step_equals_the_three_stages():
    """qq_quest_decode_step (QuestAlgorithm.decode_step): the row lookup, the fold of every
    layer with finalize, and the step layout in one launch equal qq_quest_decode_step_locs,
    update_decode_representations_fused and prepare_step bit for bit - bounds, running
    bounds, counters, first-step flags, rows, actual lengths and candidate limits - over 40
    steps that cross page boundaries, with requests on their first step, a row past the pool
    and a pool index past the table; the bounds equal the oracle's."""
    from qwenquest_amd import _lib
    from qwenquest_amd.memory import MHATokenToKVPool

    L, KV, D, P, R, W = 3, 4, 32, 16, 6, 200
    rows = R * W
    kvp = MHATokenToKVPool(rows, L, KV, D, torch.bfloat16, DEV)
    kvp.k_all.copy_(rand_bf16((L, rows + 1, KV, D), seed=21).to(DEV))
    host = bf16_bits(kvp.k_all.cpu())
    perm = torch.randperm(rows, generator=torch.Generator().manual_seed(3)) + 1
    table = perm.view(R, W).to(torch.int32)
    table[3, 70] = rows + 500  # a row past the pool: no key folded, counters still advance
    r2t = table.to(DEV)
    a, st = new_quest(64, P, L, R, W, KV, D)
    b, _ = new_quest(64, P, L, R, W, KV, D)
    prompts = {2: 40, 0: 17, 5: 64, 3: 63}
    skip_a = torch.zeros(R, dtype=torch.bool, device=DEV)
    for r, n in prompts.items():
        idx = r2t[r, :n]
        a.update_prefill_representations_fused(r, kvp.k_all, idx)
        b.update_prefill_representations_fused(r, kvp.k_all, idx)
        for layer in range(L):
            st.update_prefill_representations(layer, r, host[layer], table[r, :n].numpy())
        skip_a[r] = r != 3  # request 3 decodes without the first-step skip
    skip_b = skip_a.clone().to(torch.uint8)
    skip_a = skip_a.to(torch.uint8)
    rpi = torch.tensor([2, 0, 5, 3, 9], dtype=torch.int64, device=DEV)  # 9: past the table's rows
    seq = torch.tensor([prompts[2] + 1, prompts[0] + 1, prompts[5] + 1, prompts[3] + 1, 30], dtype=torch.int64,
                       device=DEV)
    sync = torch.zeros(int(_lib.load().qq_quest_decode_step_sync_bytes(5)), dtype=torch.uint8, device=DEV)
    locs_a = torch.empty(5, dtype=torch.int64, device=DEV)
    locs_b = torch.empty(5, dtype=torch.int64, device=DEV)
    skip_host = {r: r != 3 for r in prompts}
    for step in range(40):
        lay_a = a.decode_step(rpi, seq, kvp.k_all, r2t, skip_a, sync, locs_a)
        _lib.call("qq_quest_decode_step_locs", _lib.ptr(rpi), _lib.ptr(seq), 5, _lib.ptr(skip_b), _lib.ptr(r2t),
                  R, W, W, _lib.ptr(locs_b), _lib.stream(DEV))
        b.update_decode_representations_fused(rpi, kvp.k_all, locs_b)
        lay_b = b.prepare_step(seq)
        torch.cuda.synchronize()
        assert torch.equal(locs_a, locs_b), step
        assert torch.equal(skip_a, skip_b), step
        assert torch.equal(lay_a.actual_lens, lay_b.actual_lens) and torch.equal(
            lay_a.candidate_limit_i32, lay_b.candidate_limit_i32), step
        # the oracle folds the same rows
        want = []
        for i, r in enumerate(rpi.tolist()):
            if r >= R or skip_host.get(r, False):
                want.append(-1)
            else:
                want.append(int(table[r, max(int(seq[i]) - 2, 0)]))
        for r in prompts:
            skip_host[r] = False
        assert locs_a.cpu().tolist() == want, step
        # entries with a row fold it (a row past the pool folds nothing); all of them advance
        live = [(r, row) for r, row in zip(rpi.tolist(), want) if 0 <= r < R and row >= 0]
        folded = [(r, row) for r, row in live if row <= rows]
        if folded:
            for layer in range(L):
                st.update_decode_representations(layer, [r for r, _ in folded], host[layer],
                                                 np.array([row for _, row in folded]))
        st.maybe_finalize_decode_representations([r for r, _ in live])
        seq += 1
    assert sync.count_nonzero().item() == 0
    for x, y in ((a.page_k_bounds, b.page_k_bounds), (a.running_k_min, b.running_k_min),
                 (a.running_k_max, b.running_k_max), (a.running_token_count, b.running_token_count),
                 (a.running_page_idx, b.running_page_idx)):
        assert torch.equal(x, y)
    assert_state_equal(a, st)
