"""CPU PyTorch restatement of one Quest decode layer-step (TEST INFRASTRUCTURE ONLY).

The reference's own op sequence on the CPU, for ``bench.py``'s ``cpu_baseline`` leg and the
tests: ``group_queries`` -> ``page_scores`` -> masked ``torch.topk`` -> layout
(reference ``src/qwenquest/quest.py:366-464``), the ``req_to_token`` gather
(``src/qwenquest/attention/quest_only.py:149-151``) and ``decode_attention`` per request
(``src/qwenquest/attention/ops.py:48-66``).  The product package never imports it.
It uses torch's CPU kernels (multi-threaded), so torch's reduction order and top-k tie
order apply here, not the canonical ones the numpy oracle fixes.
"""

from __future__ import annotations

import torch


def step_layout(seq_lens: torch.Tensor, page: int, top_k: int, avoid_recent_overlap: bool = False):
    """prepare_step (quest.py:325-362): recent window, dense layout, actual lengths and the
    candidate limit, all from ``seq_lens`` [bs] int64."""
    s = seq_lens.to(torch.int64)
    last = (s - 1).clamp(min=0).unsqueeze(1)
    recent = torch.minimum((s - page).clamp(min=0).unsqueeze(1) + torch.arange(page), last)
    short = torch.minimum(torch.arange(top_k).unsqueeze(0), last)
    is_short = (s <= top_k).unsqueeze(1)
    actual = torch.minimum(s, torch.tensor(top_k)).to(torch.int32)
    limit = s // page
    if avoid_recent_overlap:
        limit = (limit - 1).clamp(min=0)
    return recent, short, is_short, actual, limit.unsqueeze(1)


def retrieve_topk(q: torch.Tensor, bounds: torch.Tensor, req_pool_indices: torch.Tensor,
                  seq_lens: torch.Tensor, page: int, top_k: int, avoid_recent_overlap: bool = False):
    """quest.py:366-464 for one layer: q [bs, H, D] (bf16), bounds [R, MP, KV, D, 2] (one
    layer's page_k_bounds) -> (positions int32 [bs, top_k], actual_lens int32 [bs])."""
    bs, heads, dim = q.shape
    kv = bounds.shape[2]
    recent, short, is_short, actual, limit = step_layout(seq_lens, page, top_k, avoid_recent_overlap)
    if bool(is_short.all()):
        return short.to(torch.int32), actual
    qbar = q.reshape(bs, kv, heads // kv, dim).mean(dim=2) if heads != kv else q  # quest.py:385-391
    kb = bounds[req_pool_indices.long()]  # [bs, MP, KV, D, 2]                       quest.py:402
    qq = qbar.unsqueeze(1)
    chosen = torch.where(qq >= 0, kb[..., 1], kb[..., 0])  # quest.py:404
    scores = (qq.float() * chosen.float()).sum(dim=(2, 3))  # quest.py:405
    k_sel = top_k // page - 1
    if k_sel > 0:
        page_idx = torch.arange(scores.shape[1]).unsqueeze(0)
        scores = scores.masked_fill(page_idx >= limit, float("-inf"))  # quest.py:450-451
        pages = torch.topk(scores, k=k_sel, dim=1).indices  # quest.py:452
        sel = (pages.unsqueeze(2) * page + torch.arange(page).view(1, 1, -1)).reshape(bs, k_sel * page)
    else:
        sel = torch.empty((bs, 0), dtype=torch.int64)
    long_layout = torch.cat([sel, recent], dim=1)
    return torch.where(is_short, short, long_layout).to(torch.int32), actual


def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scaling: float) -> torch.Tensor:
    """ops.py:48-66: q [H, D], k/v [n, KV, D] -> [H*D] in q's dtype (fp32 softmax)."""
    heads, dim = q.shape
    kv = k.shape[1]
    qg = q.view(kv, heads // kv, dim).float()
    scores = torch.einsum("hgd,nhd->hgn", qg, k.float()) * scaling
    probs = scores.softmax(dim=-1)
    out = torch.einsum("hgn,nhd->hgd", probs, v.float())
    return out.reshape(heads * dim).to(q.dtype)


def layer_step(q, bounds, req_pool_indices, seq_lens, req_to_token, k_buf, v_buf, page, top_k, scaling,
               avoid_recent_overlap: bool = False):
    """One Quest decode layer-step for a batch (no new-token store: the pool already holds
    it): selection, then per request the gather through req_to_token and the attention."""
    pos, actual = retrieve_topk(q, bounds, req_pool_indices, seq_lens, page, top_k, avoid_recent_overlap)
    outs = []
    for i in range(q.shape[0]):
        n = int(actual[i])
        rows = req_to_token[int(req_pool_indices[i]), pos[i, :n].long()].long()  # quest_only.py:149-151
        outs.append(decode_attention(q[i], k_buf[rows], v_buf[rows], scaling))
    return pos, actual, torch.stack(outs)
