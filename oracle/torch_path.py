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


def unique_first_occurrence(x: torch.Tensor) -> torch.Tensor:
    """coordinator.py:62-71: unique values of a 1-D tensor, ordered by first occurrence."""
    if x.numel() == 0:
        return x
    uniq, inverse = torch.unique(x, return_inverse=True)
    first = torch.full((uniq.numel(),), x.numel(), dtype=torch.int64)
    first = first.scatter_reduce(0, inverse, torch.arange(x.numel()), reduce="amin")
    return uniq[torch.argsort(first)]


def swap_in_long(tokens: torch.Tensor, lru: torch.Tensor, positions: torch.Tensor, seq_len: int,
                 host_rows: torch.Tensor):
    """coordinator.py:259-304 for one (layer, request) with seq_len > buf, the reference's torch
    op sequence on the CPU.  tokens / lru [buf] int64 are updated in place; host_rows is the
    request's req_to_host_pool row.  Returns (slots [n] int64 with buf = the reserved newest
    slot, victims, host rows to copy into them, hits, misses); raises where the reference raises
    (coordinator.py:278-279, 285-286)."""
    buf = tokens.numel()
    slots = torch.empty_like(positions)
    is_newest = positions == seq_len - 1
    slots[is_newest] = buf  # coordinator.py:264-265
    wanted = positions[~is_newest]
    uniq = unique_first_occurrence(wanted)  # coordinator.py:267
    hit_in_lru = torch.isin(tokens[lru], uniq)  # coordinator.py:273
    hit_slots = lru[hit_in_lru]
    evictable = lru[~hit_in_lru]
    misses = uniq[~torch.isin(uniq, tokens)]  # coordinator.py:276
    num_miss = int(misses.numel())
    if num_miss > evictable.numel():
        raise RuntimeError("device_buffer_size too small for this top-k")
    victims = evictable[:num_miss]
    host_idx = host_rows[misses]
    if num_miss and bool((host_idx < 0).any()):
        raise AssertionError("positions without host backup were selected")
    tokens[victims] = misses  # coordinator.py:291
    lru.copy_(torch.cat([evictable[num_miss:], victims, hit_slots]))  # coordinator.py:295
    sorted_tokens, order = torch.sort(tokens)  # coordinator.py:298-299
    slots[~is_newest] = order[torch.searchsorted(sorted_tokens, wanted)]
    return slots, victims, host_idx, int(uniq.numel()) - num_miss, num_miss


def swap_in_batch(tokens: torch.Tensor, lru: torch.Tensor, positions: torch.Tensor, seq_lens: torch.Tensor,
                  host_rows: torch.Tensor):
    """swap_in_long (coordinator.py:259-304) for a batch of long requests (seq_len > buf) at
    once, as batch-wide tensor ops so that torch's CPU kernels spread over the cores: keys
    request * 2^32 + position make unique / isin / sort act per request.  tokens / lru
    [bs, buf] int64 are the batch rows' states (updated in place), positions [bs, n] int64,
    host_rows [bs, max_ctx] their req_to_host_pool rows.  Returns (slots [bs, n], buf for the
    newest position; miss_req [m], victims [m], host_idx [m]): the copies, in each request's
    miss order.  Raises where the reference raises (coordinator.py:278-279, 285-286)."""
    bs, buf = tokens.shape
    n = positions.shape[1]
    K = 1 << 32
    req = torch.arange(bs, dtype=torch.int64)
    newest = positions == (seq_lens - 1).unsqueeze(1)
    wanted = torch.where(newest, torch.full_like(positions, -1), positions)
    flat = (req.unsqueeze(1) * K + wanted)[~newest]  # request-major, entry order kept
    uniq, inverse = torch.unique(flat, return_inverse=True)
    first = torch.full((uniq.numel(),), flat.numel(), dtype=torch.int64)
    first = first.scatter_reduce(0, inverse, torch.arange(flat.numel()), reduce="amin")
    uniq = uniq[torch.argsort(first)]  # coordinator.py:267: first-occurrence order per request
    tok_keys = req.unsqueeze(1) * K + tokens  # empty slots (-1) match no position
    # both sides hold distinct keys (a request's slots cache distinct positions; empty slots
    # differ by slot below), so isin may skip its own de-duplication
    tok_keys = torch.where(tokens < 0, -1 - (req.unsqueeze(1) * buf + torch.arange(buf)), tok_keys)
    hit = torch.isin(torch.gather(tok_keys, 1, lru), uniq, assume_unique=True)  # coordinator.py:273, LRU order
    misses = uniq[~torch.isin(uniq, tok_keys.reshape(-1), assume_unique=True)]  # coordinator.py:276
    miss_req = misses // K
    miss_pos = misses - miss_req * K
    num_miss = torch.bincount(miss_req, minlength=bs)
    ev = ~hit
    ev_rank = torch.cumsum(ev, dim=1) - 1
    if bool((num_miss > ev.sum(dim=1)).any()):
        raise RuntimeError("device_buffer_size too small for this top-k")
    ev_slot = torch.zeros((bs, buf), dtype=torch.int64)
    rr, jj = ev.nonzero(as_tuple=True)
    ev_slot[rr, ev_rank[rr, jj]] = lru[rr, jj]  # the e-th evictable slot of each request
    start = torch.cumsum(num_miss, 0) - num_miss
    miss_rank = torch.arange(misses.numel()) - start[miss_req]
    victims = ev_slot[miss_req, miss_rank]
    host_idx = host_rows[miss_req, miss_pos]
    if bool((host_idx < 0).any()):
        raise AssertionError("positions without host backup were selected")
    tokens[miss_req, victims] = miss_pos  # coordinator.py:291
    # coordinator.py:295: [evictable[m:], victims, hits], each group in LRU order
    group = torch.where(hit, 2, torch.where(ev_rank < num_miss.unsqueeze(1), 1, 0))
    lru.copy_(torch.gather(lru, 1, torch.sort(group * buf + torch.arange(buf), dim=1).indices))
    sorted_tok, order = torch.sort(tokens, dim=1)  # coordinator.py:298-299
    idx = torch.searchsorted(sorted_tok, wanted).clamp(max=buf - 1)
    slots = torch.where(newest, torch.full_like(positions, buf), torch.gather(order, 1, idx))
    return slots, miss_req, victims, host_idx
