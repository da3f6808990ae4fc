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
