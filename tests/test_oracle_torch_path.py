"""The CPU PyTorch layer-step (oracle/torch_path.py, the bench's CPU baseline) agrees with
the numpy oracle: the same layout, the same selected positions on tie-free inputs, and the
attention within bf16 rounding of the float64 oracle."""

from __future__ import annotations

import numpy as np
import torch

from oracle import attention as oa
from oracle import bf16
from oracle import quest as oq
from oracle import torch_path as tp
from tests.conftest import bf16_bits


def test_layout_matches_oracle():
    seqs = [1, 63, 64, 65, 200, 2048, 2049, 9000]
    for avoid in (False, True):
        ref = oq.step_layout(seqs, 64, 2048, avoid)
        recent, short, is_short, actual, limit = tp.step_layout(torch.tensor(seqs), 64, 2048, avoid)
        assert np.array_equal(recent.numpy(), ref.recent_positions)
        assert np.array_equal(actual.numpy(), ref.actual_lens)
        assert np.array_equal(limit[:, 0].numpy(), ref.candidate_limit)


def test_layer_step_matches_oracle():
    H, KV, D, P, TOP_K = 32, 4, 128, 64, 512
    seqs = [3000, 511, 1800]
    R, MP, rows = 3, 64, 3 * 3100 + 1
    g = torch.Generator().manual_seed(9)
    k = torch.randn(rows, KV, D, generator=g).to(torch.bfloat16)
    v = torch.randn(rows, KV, D, generator=g).to(torch.bfloat16)
    r2t = (torch.randperm(rows - 1, generator=g)[: R * 3100].view(R, 3100) + 1).to(torch.int32)
    st = oq.QuestState(TOP_K, P)
    st.init_storage(0, 1, R, 3100, KV, D)
    kbits = bf16_bits(k)
    for r, s in enumerate(seqs):
        st.update_prefill_representations(0, r, kbits, r2t[r, : s - 1].numpy())
    st.prepare_step(seqs)
    q = torch.randn(3, H, D, generator=g).to(torch.bfloat16)
    ref_pos, ref_actual, _ = st.retrieve_topk(q.float().numpy(), 0, [0, 1, 2])
    bounds = torch.from_numpy(st.page_k_bounds[0].view(np.int16)).view(torch.bfloat16)
    pos, actual, out = tp.layer_step(q, bounds, torch.arange(3), torch.tensor(seqs), r2t, k, v, P, TOP_K, D**-0.5)
    assert np.array_equal(actual.numpy(), ref_actual)
    for i in range(3):
        n = int(ref_actual[i])
        assert np.array_equal(pos[i, :n].numpy(), ref_pos[i, :n])
    kf, vf = bf16.to_f32(kbits), bf16.to_f32(bf16_bits(v))
    ref = oa.sparse_decode(q.float().numpy(), kf, vf,
                           [r2t[i, ref_pos[i, : int(ref_actual[i])]].numpy().astype(np.int64) for i in range(3)], D**-0.5)
    err = np.abs(out.float().numpy() - ref).max()
    assert err <= 1e-3 + 8e-3 * np.abs(ref).max(), err


def test_torch_swap_in_equals_the_numpy_oracle():
    """oracle/torch_path.swap_in_long (the reference's torch op sequence, used by the bench's
    swap-in CPU baseline) gives the numpy oracle's slots, copies, LRU state and counts over a
    random multi-step run with duplicates, the newest position and misses."""
    import numpy as np

    from oracle import hisparse as oh
    from oracle import torch_path as tp

    rng = np.random.default_rng(5)
    buf, top_k, seq0 = 48, 32, 200
    host_rows = torch.arange(1, 1000, dtype=torch.int64)
    tok_np = np.arange(buf, dtype=np.int64)
    lru_np = np.arange(buf, dtype=np.int64)
    tok_t, lru_t = torch.from_numpy(tok_np.copy()), torch.from_numpy(lru_np.copy())
    for step in range(40):
        s = seq0 + step
        pos = rng.integers(0, s, size=top_k)
        pos[-1] = s - 1
        pos[3] = pos[4]
        plan = oh.swap_in_long(tok_np, lru_np, pos, s, host_rows.numpy())
        slots, victims, hidx, hits, misses = tp.swap_in_long(tok_t, lru_t, torch.from_numpy(pos), s, host_rows)
        assert np.array_equal(slots.numpy(), plan.slots), step
        assert [(int(a), int(b)) for a, b in zip(victims, hidx)] == [tuple(c) for c in plan.copies], step
        assert np.array_equal(tok_t.numpy(), plan.tokens) and np.array_equal(lru_t.numpy(), plan.lru), step
        assert (hits, misses) == (plan.hits, plan.misses)
        tok_np, lru_np = plan.tokens, plan.lru


def test_batched_torch_swap_in_equals_the_per_request_one():
    """oracle/torch_path.swap_in_batch (all requests of a layer at once, the bench's swap-in
    CPU baseline) gives, request by request, swap_in_long's slots, copies and LRU state, over
    a random multi-step run with duplicates, the newest position, hits and misses."""
    from oracle import torch_path as tp

    g = torch.Generator().manual_seed(11)
    bs, buf, top_k, max_ctx = 5, 40, 24, 400
    host = torch.arange(1, bs * max_ctx + 1, dtype=torch.int64).view(bs, max_ctx)
    tok_a = torch.arange(buf).repeat(bs, 1)
    tok_a[2, 30:] = -1  # a request admitted with a prompt shorter than the buffer: empty slots
    tok_a[4, ::3] = -1
    lru_a = torch.arange(buf).repeat(bs, 1)
    tok_b, lru_b = tok_a.clone(), lru_a.clone()
    for step in range(30):
        seqs = torch.tensor([200 + step + 7 * r for r in range(bs)])
        pos = (torch.rand(bs, top_k, generator=g) * seqs.unsqueeze(1)).long()
        pos[:, -1] = seqs - 1
        pos[:, 2] = pos[:, 3]
        slots, mreq, vic, hidx = tp.swap_in_batch(tok_b, lru_b, pos, seqs, host)
        for r in range(bs):
            s_r, v_r, h_r, _, _ = tp.swap_in_long(tok_a[r], lru_a[r], pos[r], int(seqs[r]), host[r])
            assert torch.equal(slots[r], s_r), (step, r)
            sel = mreq == r
            assert torch.equal(vic[sel], v_r) and torch.equal(hidx[sel], h_r), (step, r)
        assert torch.equal(tok_a, tok_b) and torch.equal(lru_a, lru_b), step
