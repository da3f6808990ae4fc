"""numpy restatement of ``QuestAlgorithm`` (reference ``src/qwenquest/quest.py``).

Test infrastructure only (see ``oracle/__init__.py``).  Bounds are kept as
uint16 bf16 bit patterns in exactly the reference layout::

    page_k_bounds [layers, max_reqs, max_pages, kv_heads, head_dim, 2]  (min, max)
    running_k_min / running_k_max [layers, max_reqs, kv_heads, head_dim]
    running_token_count / running_page_idx [max_reqs] int32
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle import bf16

LANES = 64  # lanes of the canonical per-page reduction


def _as_bits(k: np.ndarray) -> np.ndarray:
    """Keys as bf16 bits: uint16 input is already bf16, float input is rounded (RNE)."""
    k = np.asarray(k)
    if k.dtype == np.uint16:
        return k
    return bf16.from_f32(k.astype(np.float32))


def _bmin(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Elementwise min of bf16 bit arrays with NaN propagation (torch.minimum semantics)."""
    fa, fb = bf16.to_f32(a), bf16.to_f32(b)
    out = np.where(fb < fa, b, a)
    out = np.where(np.isnan(fb), b, out)
    return np.where(np.isnan(fa), a, out).astype(np.uint16)


def _bmax(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    fa, fb = bf16.to_f32(a), bf16.to_f32(b)
    out = np.where(fb > fa, b, a)
    out = np.where(np.isnan(fb), b, out)
    return np.where(np.isnan(fa), a, out).astype(np.uint16)


def _reduce_min(bits: np.ndarray, axis: int) -> np.ndarray:
    f = bf16.to_f32(bits)
    return bf16.from_f32(np.min(f, axis=axis))  # np.min propagates NaN like torch.amin


def _reduce_max(bits: np.ndarray, axis: int) -> np.ndarray:
    f = bf16.to_f32(bits)
    return bf16.from_f32(np.max(f, axis=axis))


@dataclass
class Layout:
    """``StepLayout`` (quest.py:61-75), computed by ``prepare_step`` (quest.py:325-362)."""

    seq_lens: np.ndarray  # [bs] int64
    recent_positions: np.ndarray  # [bs, P] int64
    short_layout: np.ndarray  # [bs, top_k] int64
    is_short: np.ndarray  # [bs] bool
    actual_lens: np.ndarray  # [bs] int32
    candidate_limit: np.ndarray  # [bs] int64


def step_layout(seq_lens, page_size: int, top_k: int, avoid_recent_overlap: bool) -> Layout:
    """quest.py:325-362 (prepare_step)."""
    P = page_size
    seq = np.asarray(seq_lens, dtype=np.int64)
    last_valid = np.maximum(seq - 1, 0)[:, None]
    recent_start = np.maximum(seq - P, 0)[:, None]
    recent = np.minimum(recent_start + np.arange(P, dtype=np.int64)[None], last_valid)
    short = np.minimum(np.arange(top_k, dtype=np.int64)[None], last_valid)
    is_short = seq <= top_k
    actual = np.minimum(seq, top_k).astype(np.int32)
    full = seq // P
    limit = np.maximum(full - 1, 0) if avoid_recent_overlap else full
    return Layout(seq, recent, short, is_short, actual, limit)


def group_queries(q: np.ndarray, kv_heads: int, head_dim: int, is_bf16: bool) -> np.ndarray:
    """quest.py:366-391.  ``q``: float32 values ``[bs, H*D]`` or ``[bs, H, D]``.

    Returns the GQA mean ``[bs, kv_heads, head_dim]`` as float32 values (already
    rounded to bf16 when ``is_bf16``).  Canonical order: sequential fp32 sum over
    the group, then one division by the group size, then one rounding.
    """
    q = np.asarray(q, dtype=np.float32)
    bs = q.shape[0]
    if q.ndim == 2:
        if q.shape[1] % head_dim != 0:
            raise ValueError(f"Query hidden {q.shape[1]} not divisible by head_dim {head_dim}")
        q = q.reshape(bs, q.shape[1] // head_dim, head_dim)
    elif q.ndim != 3:
        raise ValueError(f"Unsupported query shape {q.shape}")
    heads = q.shape[1]
    if heads == kv_heads:
        return q.copy()
    if heads % kv_heads != 0:
        raise ValueError(f"q_heads {heads} not divisible by kv_heads {kv_heads}")
    g = heads // kv_heads
    grouped = q.reshape(bs, kv_heads, g, head_dim)
    acc = np.zeros((bs, kv_heads, head_dim), dtype=np.float32)
    for i in range(g):
        acc = (acc + grouped[:, :, i]).astype(np.float32)
    mean = (acc / np.float32(g)).astype(np.float32)
    return bf16.round_f32(mean) if is_bf16 else mean


def page_scores(qbar: np.ndarray, bounds: np.ndarray) -> np.ndarray:
    """quest.py:393-405 in the canonical fp32 order.

    ``qbar``: ``[bs, KV, D]`` float32 values.  ``bounds``: ``[bs, pages, KV, D, 2]``
    bf16 bits.  Returns ``[bs, pages]`` float32.
    """
    qbar = np.asarray(qbar, dtype=np.float32)
    bs, n_pages = bounds.shape[0], bounds.shape[1]
    kmin = bf16.to_f32(bounds[..., 0])
    kmax = bf16.to_f32(bounds[..., 1])
    q = qbar[:, None]
    with np.errstate(over="ignore", invalid="ignore"):
        prod = (q * np.where(q >= 0, kmax, kmin)).astype(np.float32)
    c = prod.shape[2] * prod.shape[3]
    m = -(-c // LANES)
    flat = np.zeros((bs, n_pages, LANES * m), dtype=np.float32)
    flat[..., :c] = prod.reshape(bs, n_pages, c)
    lanes = flat.reshape(bs, n_pages, LANES, m)
    with np.errstate(over="ignore", invalid="ignore"):
        acc = lanes[..., 0].copy()
        for j in range(1, m):
            acc = (acc + lanes[..., j]).astype(np.float32)
        w = LANES
        while w > 1:
            w //= 2
            acc = (acc[..., :w] + acc[..., w : 2 * w]).astype(np.float32)
    return acc[..., 0]


def topk_pages(scores: np.ndarray, limit: int, k: int) -> np.ndarray:
    """quest.py:450-452: mask pages >= limit to -inf, take the k best.

    Order: descending score; ties -> lowest page index (the build's spec).
    """
    s = np.asarray(scores, dtype=np.float32).copy()
    s[limit:] = -np.inf
    key = bf16.orderable_u32(s).astype(np.int64)
    order = np.lexsort((np.arange(s.shape[0]), -key))
    return order[:k].astype(np.int64)


def retrieve_topk(
    qbar: np.ndarray,
    bounds_rows: np.ndarray,
    layout: Layout,
    page_size: int,
    top_k: int,
) -> tuple[np.ndarray, np.ndarray, np.ndarray | None]:
    """quest.py:409-464.  ``bounds_rows``: ``[bs, max_pages, KV, D, 2]`` bits of this
    layer for the batch's requests.  Returns (positions int32 [bs, top_k],
    actual_lens int32 [bs], masked scores [bs, max_pages] or None)."""
    P = page_size
    k = top_k // P - 1
    bs = layout.seq_lens.shape[0]
    if bool(layout.is_short.all()):
        return layout.short_layout.astype(np.int32), layout.actual_lens, None
    scores = page_scores(qbar, bounds_rows)
    masked = scores.copy()
    out = np.empty((bs, top_k), dtype=np.int64)
    for i in range(bs):
        masked[i, int(layout.candidate_limit[i]) :] = -np.inf
        if layout.is_short[i]:
            out[i] = layout.short_layout[i]
            continue
        if k > 0:
            pages = topk_pages(scores[i], int(layout.candidate_limit[i]), k)
            sel = (pages[:, None] * P + np.arange(P)[None]).reshape(-1)
        else:
            sel = np.empty(0, dtype=np.int64)
        out[i] = np.concatenate([sel, layout.recent_positions[i]])
    return out.astype(np.int32), layout.actual_lens, masked


class QuestState:
    """Storage + bounds lifecycle of ``QuestAlgorithm`` (quest.py:130-321, 468-479)."""

    def __init__(self, top_k: int, page_size: int, *, avoid_recent_overlap: bool = False):
        # quest.py:138-144
        if page_size <= 0:
            raise ValueError(f"quest page_size must be > 0, got {page_size}")
        if top_k % page_size != 0:
            raise ValueError(f"top_k ({top_k}) must be divisible by quest_page_size ({page_size})")
        self.top_k = top_k
        self.page_size = page_size
        self.top_k_pages = top_k // page_size
        self.avoid_recent_overlap = avoid_recent_overlap

    def init_storage(self, start_layer, end_layer, max_reqs, max_context_len, kv_heads, head_dim):
        """quest.py:171-209."""
        self.start_layer, self.end_layer = start_layer, end_layer
        self.num_layers = end_layer - start_layer
        self.max_reqs = max_reqs
        self.max_pages_per_req = (max_context_len + self.page_size - 1) // self.page_size
        self.kv_heads, self.head_dim = kv_heads, head_dim
        shape = (self.num_layers, max_reqs, self.max_pages_per_req, kv_heads, head_dim, 2)
        self.page_k_bounds = np.empty(shape, dtype=np.uint16)
        self.page_k_bounds[..., 0] = bf16.BF16_MAX_BITS
        self.page_k_bounds[..., 1] = bf16.BF16_MIN_BITS
        rshape = (self.num_layers, max_reqs, kv_heads, head_dim)
        self.running_k_min = np.full(rshape, bf16.BF16_MAX_BITS, dtype=np.uint16)
        self.running_k_max = np.full(rshape, bf16.BF16_MIN_BITS, dtype=np.uint16)
        self.running_token_count = np.zeros(max_reqs, dtype=np.int32)
        self.running_page_idx = np.zeros(max_reqs, dtype=np.int32)

    @property
    def page_valid(self) -> np.ndarray:
        """quest.py:220-223."""
        kmax = bf16.to_f32(self.page_k_bounds[..., 1])
        return (kmax > bf16.to_f32(bf16.BF16_MIN_BITS)).any(axis=(-1, -2))

    def update_prefill_representations(self, layer_id, req, k_buffer, prefill_indices):
        """quest.py:231-280.  ``k_buffer``: ``[pool, KV, D]`` bf16 bits or float."""
        lo = layer_id - self.start_layer
        idx = np.asarray(prefill_indices, dtype=np.int64)
        n = idx.shape[0]
        P = self.page_size
        full = n // P
        kb = _as_bits(k_buffer)
        if full > 0:
            paged = kb[idx[: full * P]].reshape(full, P, self.kv_heads, self.head_dim)
            self.page_k_bounds[lo, req, :full, ..., 0] = _reduce_min(paged, 1)
            self.page_k_bounds[lo, req, :full, ..., 1] = _reduce_max(paged, 1)
        partial = n - full * P
        if partial > 0:
            part = kb[idx[full * P :]]
            self.running_k_min[lo, req] = _reduce_min(part, 0)
            self.running_k_max[lo, req] = _reduce_max(part, 0)
        if layer_id == self.end_layer - 1:
            self.running_token_count[req] = partial
            self.running_page_idx[req] = full

    def update_decode_representations(self, layer_id, req_indices, k_buffer, device_locs):
        """quest.py:284-302."""
        lo = layer_id - self.start_layer
        reqs = np.asarray(req_indices, dtype=np.int64)
        new = _as_bits(k_buffer)[np.asarray(device_locs, dtype=np.int64)]
        self.running_k_min[lo, reqs] = _bmin(self.running_k_min[lo, reqs], new)
        self.running_k_max[lo, reqs] = _bmax(self.running_k_max[lo, reqs], new)

    def maybe_finalize_decode_representations(self, req_indices):
        """quest.py:304-321."""
        reqs = np.asarray(req_indices, dtype=np.int64)
        counts = self.running_token_count[reqs]
        completing = reqs[counts == self.page_size - 1]
        for r in completing:
            p = int(self.running_page_idx[r])
            self.page_k_bounds[:, r, p, ..., 0] = self.running_k_min[:, r]
            self.page_k_bounds[:, r, p, ..., 1] = self.running_k_max[:, r]
            self.running_k_min[:, r] = bf16.BF16_MAX_BITS
            self.running_k_max[:, r] = bf16.BF16_MIN_BITS
            self.running_page_idx[r] += 1
        self.running_token_count[reqs] = (counts + 1) % self.page_size

    def invalidate_request(self, req):
        """quest.py:468-479."""
        self.page_k_bounds[:, req, ..., 0] = bf16.BF16_MAX_BITS
        self.page_k_bounds[:, req, ..., 1] = bf16.BF16_MIN_BITS
        self.running_k_min[:, req] = bf16.BF16_MAX_BITS
        self.running_k_max[:, req] = bf16.BF16_MIN_BITS
        self.running_token_count[req] = 0
        self.running_page_idx[req] = 0

    def prepare_step(self, seq_lens) -> Layout:
        self.layout = step_layout(seq_lens, self.page_size, self.top_k, self.avoid_recent_overlap)
        return self.layout

    def retrieve_topk(self, q_values, layer_id, req_pool_indices, *, q_is_bf16=True):
        """quest.py:409-464 on this state; ``q_values`` float32 ``[bs, H, D]``."""
        lo = layer_id - self.start_layer
        qbar = group_queries(q_values, self.kv_heads, self.head_dim, q_is_bf16)
        rows = self.page_k_bounds[lo, np.asarray(req_pool_indices, dtype=np.int64)]
        return retrieve_topk(qbar, rows, self.layout, self.page_size, self.top_k)
