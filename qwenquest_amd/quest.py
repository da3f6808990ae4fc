"""QuestAlgorithm on MI355X (reference ``src/qwenquest/quest.py``).

Same class, method names, tensors and lifecycle as the reference; every
computation runs in the HIP kernels of ``libqwenquest_amd.so``:

=======================================  =====================================
reference (quest.py)                     kernel entry point
=======================================  =====================================
init_storage / invalidate_request        qq_quest_reset
update_prefill_representations  [Q2]     qq_quest_prefill_bounds (layer-fused)
update_decode_representations   [Q3]     qq_quest_decode_update (fused finalize)
maybe_finalize_decode_representations    qq_quest_decode_finalize
prepare_step                    [Q4]     qq_quest_prepare_step
group_queries / page_scores     [Q5]     qq_quest_group_queries / qq_quest_page_scores
retrieve_topk                   [Q6]     qq_quest_retrieve_topk (score + select + layout)
=======================================  =====================================

Selection order is pinned: page scores are fp32 sums in a fixed lane/tree
order and ties go to the lowest page index (the reference leaves both to torch).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from qwenquest_amd import _lib

__all__ = ["QuestAlgorithm", "QuestSelection", "QuestTrace", "StepLayout"]

_BF16_POS_INF = torch.finfo(torch.bfloat16).max
_BF16_NEG_INF = torch.finfo(torch.bfloat16).min


@dataclass
class StepLayout:
    """Layer-independent part of the selection (reference quest.py:61-75).

    The kernels consume ``seq_lens``, ``actual_lens`` and ``candidate_limit``;
    the other fields of the reference are derived on request.
    """

    seq_lens: torch.Tensor  # [bs] int64
    actual_lens: torch.Tensor  # [bs] int32  min(seq_len, top_k)
    candidate_limit_i32: torch.Tensor  # [bs] int32  pages >= this are never candidates
    page_size: int
    top_k: int

    @property
    def candidate_limit(self) -> torch.Tensor:
        return self.candidate_limit_i32.to(torch.int64).unsqueeze(1)

    @property
    def is_short(self) -> torch.Tensor:
        return (self.seq_lens <= self.top_k).unsqueeze(1)

    @property
    def recent_positions(self) -> torch.Tensor:
        P = self.page_size
        last = (self.seq_lens - 1).clamp(min=0).unsqueeze(1)
        start = (self.seq_lens - P).clamp(min=0).unsqueeze(1)
        off = torch.arange(P, device=self.seq_lens.device).unsqueeze(0)
        return torch.minimum(start + off, last)

    @property
    def short_layout(self) -> torch.Tensor:
        last = (self.seq_lens - 1).clamp(min=0).unsqueeze(1)
        return torch.minimum(torch.arange(self.top_k, device=self.seq_lens.device).unsqueeze(0), last)


@dataclass
class QuestSelection:
    """One ``retrieve_topk`` decision (reference quest.py:78-89)."""

    layer_id: int
    req_pool_idx: int
    seq_len: int
    dense: bool
    selected_pages: list[int]
    recent_window: tuple[int, int]
    page_scores: torch.Tensor | None
    positions: torch.Tensor


@dataclass
class QuestTrace:
    """Opt-in recorder (reference quest.py:92-104); recording synchronises the stream."""

    max_records: int | None = None
    records: list[QuestSelection] = field(default_factory=list)

    def add(self, record: QuestSelection) -> None:
        if self.max_records is None or len(self.records) < self.max_records:
            self.records.append(record)

    def for_layer(self, layer_id: int) -> list[QuestSelection]:
        return [r for r in self.records if r.layer_id == layer_id]


class QuestAlgorithm:
    """Quest page-wise sparse attention, bounds indexed by (layer, req_pool_idx, page).

    Storage (bf16), exactly the reference layout:
    ``page_k_bounds [num_layers, max_reqs, max_pages_per_req, kv_heads, head_dim, 2]``,
    ``running_k_min/max [num_layers, max_reqs, kv_heads, head_dim]``,
    ``running_token_count / running_page_idx [max_reqs]`` int32.
    """

    def __init__(
        self,
        top_k: int,
        page_size: int,
        device: torch.device | str,
        *,
        avoid_recent_overlap: bool = False,
    ):
        if page_size <= 0:
            raise ValueError(f"quest page_size must be > 0, got {page_size}")
        if top_k % page_size != 0:
            raise ValueError(
                f"top_k ({top_k}) must be divisible by quest_page_size ({page_size}); "
                "Quest emits whole pages worth of token positions."
            )
        self.top_k = top_k
        self.page_size = page_size
        self.top_k_pages = top_k // page_size
        self.device = torch.device(device)
        self.avoid_recent_overlap = avoid_recent_overlap
        self.start_layer = self.end_layer = self.num_layers = 0
        self.max_reqs = self.max_pages_per_req = self.kv_heads = self.head_dim = 0
        self._initialized = False
        self._step: StepLayout | None = None
        self.trace: QuestTrace | None = None

    # ------------------------------------------------------------------ setup

    def init_storage(
        self,
        start_layer: int,
        end_layer: int,
        max_reqs: int,
        max_context_len: int,
        kv_heads: int,
        head_dim: int,
    ) -> None:
        """Allocate and sentinel-fill bounds for layers ``[start_layer, end_layer)`` (quest.py:171-209)."""
        if self.device.type != "cuda":
            raise RuntimeError("qwenquest_amd.QuestAlgorithm needs a GPU device (no CPU path)")
        self.start_layer, self.end_layer = start_layer, end_layer
        self.num_layers = end_layer - start_layer
        self.max_reqs = max_reqs
        self.max_pages_per_req = (max_context_len + self.page_size - 1) // self.page_size
        self.kv_heads, self.head_dim = kv_heads, head_dim
        dev = self.device
        shape = (self.num_layers, max_reqs, self.max_pages_per_req, kv_heads, head_dim, 2)
        self.page_k_bounds = torch.empty(shape, dtype=torch.bfloat16, device=dev)
        rshape = (self.num_layers, max_reqs, kv_heads, head_dim)
        self.running_k_min = torch.empty(rshape, dtype=torch.bfloat16, device=dev)
        self.running_k_max = torch.empty(rshape, dtype=torch.bfloat16, device=dev)
        self.running_token_count = torch.empty(max_reqs, dtype=torch.int32, device=dev)
        self.running_page_idx = torch.empty(max_reqs, dtype=torch.int32, device=dev)
        # per-call workspace of retrieve_topk: the page scores of the batch
        self._scores_ws = torch.empty((max_reqs, max(self.max_pages_per_req, 1)), dtype=torch.float32, device=dev)
        self._reset(0, max_reqs)
        self._initialized = True

    def _reset(self, req_begin: int, req_count: int) -> None:
        _lib.call(
            "qq_quest_reset", _lib.ptr(self.page_k_bounds), _lib.ptr(self.running_k_min),
            _lib.ptr(self.running_k_max), _lib.ptr(self.running_token_count),
            _lib.ptr(self.running_page_idx), self.num_layers, self.max_reqs,
            self.max_pages_per_req, self.kv_heads, self.head_dim, req_begin, req_count,
            _lib.stream(self.device),
        )

    @property
    def page_k_min(self) -> torch.Tensor:
        """View ``[num_layers, max_reqs, max_pages, kv_heads, head_dim]`` (writes go through)."""
        return self.page_k_bounds[..., 0]

    @property
    def page_k_max(self) -> torch.Tensor:
        return self.page_k_bounds[..., 1]

    @property
    def page_valid(self) -> torch.Tensor:
        """``[num_layers, max_reqs, max_pages]`` bool, derived from the sentinel."""
        return (self.page_k_max > _BF16_NEG_INF).any(dim=(-1, -2))

    def storage_bytes(self) -> int:
        n = self.page_k_bounds.numel() + self.running_k_min.numel() + self.running_k_max.numel()
        return n * 2

    def _geometry(self) -> tuple[int, int, int, int, int, int]:
        return (self.num_layers, self.max_reqs, self.max_pages_per_req, self.kv_heads,
                self.head_dim, self.page_size)

    def _check_keys(self, k: torch.Tensor) -> None:
        if k.dim() != 3 or k.shape[1] != self.kv_heads or k.shape[2] != self.head_dim:
            raise ValueError(f"key buffer must be [rows, {self.kv_heads}, {self.head_dim}], got {tuple(k.shape)}")
        if not k.is_contiguous():
            raise ValueError("key buffer must be contiguous")

    # ------------------------------------------------------ [Q2] prefill bounds

    def update_prefill_representations(
        self,
        layer_id: int,
        req_pool_idx: int,
        k_buffer: torch.Tensor,
        prefill_indices: torch.Tensor,
    ) -> None:
        """[Q2] Bounds of one request's prefill keys at one layer (quest.py:231-280)."""
        self._check_keys(k_buffer)
        lo = layer_id - self.start_layer
        self._prefill(k_buffer, 0, k_buffer.shape[0], int(req_pool_idx), prefill_indices, lo, 1,
                      layer_id == self.end_layer - 1)

    def update_prefill_representations_fused(
        self, req_pool_idx: int, k_all: torch.Tensor, prefill_indices: torch.Tensor
    ) -> None:
        """[Q2] All Quest layers in one launch; ``k_all`` is the pool's ``[model_layers, rows,
        KV, D]`` tensor (``MHATokenToKVPool.k_all``) indexed by model layer id, so Quest layer
        ``start_layer + i`` reads ``k_all[start_layer + i]``."""
        self._check_k_all(k_all)
        stride = k_all.stride(0)
        self._prefill(k_all[self.start_layer], stride, k_all.shape[1], int(req_pool_idx),
                      prefill_indices, 0, self.num_layers, True)

    def _check_k_all(self, k_all: torch.Tensor) -> None:
        if k_all.dim() != 4 or not k_all.is_contiguous():
            raise ValueError("k_all must be a contiguous [model_layers, rows, KV, D] tensor")
        if k_all.shape[0] < self.end_layer:
            raise ValueError(
                f"k_all holds {k_all.shape[0]} layers but the Quest layers run to {self.end_layer}: "
                "pass the pool's full per-model-layer tensor"
            )
        self._check_keys(k_all[0])

    def _prefill(self, k0, stride, rows, req, idx, layer_begin, n_layers, set_counters) -> None:
        idx = idx.to(self.device)
        if idx.dtype not in (torch.int32, torch.int64):
            idx = idx.to(torch.int64)
        idx = idx.contiguous()
        _lib.call(
            "qq_quest_prefill_bounds", _lib.ptr(k0), stride, _lib.dtype_code(k0.dtype), rows,
            _lib.ptr(idx), int(idx.dtype == torch.int64), int(idx.numel()), req, layer_begin,
            n_layers, int(set_counters), _lib.ptr(self.page_k_bounds),
            _lib.ptr(self.running_k_min), _lib.ptr(self.running_k_max),
            _lib.ptr(self.running_token_count), _lib.ptr(self.running_page_idx),
            *self._geometry(), _lib.stream(self.device),
        )

    # ------------------------------------------------------- [Q3] decode bounds

    def update_decode_representations(
        self,
        layer_id: int,
        req_indices: torch.Tensor,
        k_buffer: torch.Tensor,
        device_locs: torch.Tensor,
    ) -> None:
        """[Q3] Fold the previous token's key into the running min/max (quest.py:284-302)."""
        self._check_keys(k_buffer)
        self._decode(k_buffer, 0, k_buffer.shape[0], req_indices, device_locs,
                     layer_id - self.start_layer, 1, False)

    def update_decode_representations_fused(
        self, req_indices: torch.Tensor, k_all: torch.Tensor, device_locs: torch.Tensor
    ) -> None:
        """[Q3] Fold for every layer and finalize completed pages in one pass
        (update_decode_representations x layers + maybe_finalize_decode_representations);
        ``k_all`` as for update_prefill_representations_fused (indexed by model layer id)."""
        self._check_k_all(k_all)
        self._decode(k_all[self.start_layer], k_all.stride(0), k_all.shape[1], req_indices,
                     device_locs, 0, self.num_layers, True)

    def _decode(self, k0, stride, rows, reqs, locs, layer_begin, n_layers, finalize) -> None:
        reqs = reqs.to(device=self.device, dtype=torch.int64).contiguous()
        locs = locs.to(device=self.device, dtype=torch.int64).contiguous()
        if reqs.numel() != locs.numel():
            raise ValueError("req_indices and device_locs differ in length")
        _lib.call(
            "qq_quest_decode_update", _lib.ptr(k0), stride, _lib.dtype_code(k0.dtype), rows,
            _lib.ptr(reqs), _lib.ptr(locs), int(reqs.numel()), layer_begin, n_layers,
            int(finalize), _lib.ptr(self.page_k_bounds), _lib.ptr(self.running_k_min),
            _lib.ptr(self.running_k_max), _lib.ptr(self.running_token_count),
            _lib.ptr(self.running_page_idx), *self._geometry(), _lib.stream(self.device),
        )

    def maybe_finalize_decode_representations(self, req_indices: torch.Tensor) -> None:
        """[Q3] Advance counters; finalize pages whose P-th token arrived (quest.py:304-321)."""
        reqs = req_indices.to(device=self.device, dtype=torch.int64).contiguous()
        _lib.call(
            "qq_quest_decode_finalize", _lib.ptr(reqs), int(reqs.numel()),
            _lib.ptr(self.page_k_bounds), _lib.ptr(self.running_k_min),
            _lib.ptr(self.running_k_max), _lib.ptr(self.running_token_count),
            _lib.ptr(self.running_page_idx), *self._geometry(), _lib.stream(self.device),
        )

    # ----------------------------------------------------- [Q4] per-step layout

    def prepare_step(self, seq_lens: torch.Tensor) -> StepLayout:
        """[Q4] Layer-independent selection inputs, once per decode step (quest.py:325-362)."""
        seq = seq_lens.to(device=self.device, dtype=torch.int64).contiguous()
        bs = int(seq.numel())
        actual = torch.empty(bs, dtype=torch.int32, device=self.device)
        limit = torch.empty(bs, dtype=torch.int32, device=self.device)
        _lib.call("qq_quest_prepare_step", _lib.ptr(seq), bs, self.page_size, self.top_k,
                  int(self.avoid_recent_overlap), _lib.ptr(actual), _lib.ptr(limit),
                  _lib.stream(self.device))
        self._step = StepLayout(seq, actual, limit, self.page_size, self.top_k)
        return self._step

    def decode_step(
        self,
        req_indices: torch.Tensor,
        seq_lens: torch.Tensor,
        k_all: torch.Tensor,
        req_to_token: torch.Tensor,
        skip_first: torch.Tensor,
        sync: torch.Tensor,
        device_locs_out: torch.Tensor | None = None,
    ) -> StepLayout:
        """[Q3] + [Q4] in one launch, as a backend's init_forward_metadata runs them
        (quest_only.py:84-97, quest.py:284-362): the previous token's row of each request
        (``req_to_token[req, seq_len - 2]``; none while ``skip_first[req]`` is set, which is
        then cleared) folded into every layer's running bounds with completed pages
        finalized, then the step layout.  Equal to the row lookup,
        update_decode_representations_fused and prepare_step in that order for a batch that
        lists each request once.  ``sync``: at least qq_quest_decode_step_sync_bytes(bs)
        zeroed bytes, left zeroed."""
        self._check_k_all(k_all)
        rpi = req_indices.to(device=self.device, dtype=torch.int64).contiguous()
        seq = seq_lens.to(device=self.device, dtype=torch.int64).contiguous()
        bs = int(seq.numel())
        if rpi.numel() != bs:
            raise ValueError("req_indices and seq_lens differ in length")
        if skip_first.dtype not in (torch.bool, torch.uint8) or not skip_first.is_contiguous():
            raise ValueError("skip_first must be a contiguous bool or uint8 tensor")
        if req_to_token.dtype != torch.int32 or req_to_token.dim() != 2 or req_to_token.stride(1) != 1:
            raise ValueError("req_to_token must be a 2-D int32 tensor with unit column stride")
        actual = torch.empty(bs, dtype=torch.int32, device=self.device)
        limit = torch.empty(bs, dtype=torch.int32, device=self.device)
        k0 = k_all[self.start_layer]
        _lib.call(
            "qq_quest_decode_step", _lib.ptr(rpi), _lib.ptr(seq), bs, _lib.ptr(skip_first), _lib.ptr(req_to_token),
            req_to_token.shape[0], req_to_token.shape[1], req_to_token.stride(0),
            _lib.ptr(device_locs_out) if device_locs_out is not None else None,
            _lib.ptr(k0), k_all.stride(0), _lib.dtype_code(k0.dtype), k_all.shape[1],
            _lib.ptr(self.page_k_bounds), _lib.ptr(self.running_k_min), _lib.ptr(self.running_k_max),
            _lib.ptr(self.running_token_count), _lib.ptr(self.running_page_idx), *self._geometry(),
            self.top_k, int(self.avoid_recent_overlap), _lib.ptr(actual), _lib.ptr(limit),
            _lib.ptr(sync), sync.numel() * sync.element_size(), _lib.stream(self.device),
        )
        self._step = StepLayout(seq, actual, limit, self.page_size, self.top_k)
        return self._step

    # ---------------------------------------------------- [Q5] page criticality

    def _queries_3d(self, queries: torch.Tensor) -> torch.Tensor:
        """Validate like group_queries (quest.py:374-388); returns contiguous ``[bs, H, D]``."""
        bs = queries.shape[0]
        if queries.dim() == 2:
            if queries.shape[1] % self.head_dim != 0:
                raise ValueError(f"Query hidden {queries.shape[1]} not divisible by head_dim {self.head_dim}")
            q = queries.view(bs, queries.shape[1] // self.head_dim, self.head_dim)
        elif queries.dim() == 3:
            q = queries
        else:
            raise ValueError(f"Unsupported query shape {tuple(queries.shape)}")
        if q.shape[2] != self.head_dim:
            raise ValueError(f"query head_dim {q.shape[2]} != {self.head_dim}")
        if q.shape[1] % self.kv_heads != 0:
            raise ValueError(f"q_heads {q.shape[1]} not divisible by kv_heads {self.kv_heads}")
        if q.dtype not in (torch.bfloat16, torch.float32):
            q = q.float()
        return q.contiguous()

    def group_queries(self, queries: torch.Tensor) -> torch.Tensor:
        """[Q5] ``[bs, H*D]`` or ``[bs, H, D]`` -> ``[bs, kv_heads, head_dim]`` GQA mean (quest.py:366-391)."""
        q = self._queries_3d(queries)
        bs = q.shape[0]
        out = torch.empty((bs, self.kv_heads, self.head_dim), dtype=q.dtype, device=q.device)
        _lib.call("qq_quest_group_queries", _lib.ptr(q), _lib.dtype_code(q.dtype), q.stride(0),
                  q.shape[1], self.kv_heads, self.head_dim, bs, _lib.ptr(out), _lib.stream(self.device))
        return out

    def page_scores(self, grouped_q: torch.Tensor, layer_id: int, req_pool_indices: torch.Tensor) -> torch.Tensor:
        """[Q5] Criticality of every page slot ``[bs, max_pages_per_req]`` fp32 (quest.py:393-405)."""
        q = grouped_q.reshape(grouped_q.shape[0], self.kv_heads * self.head_dim)
        if q.dtype not in (torch.bfloat16, torch.float32):
            q = q.float()
        q = q.contiguous()
        rpi = req_pool_indices.to(device=self.device, dtype=torch.int64).contiguous()
        bs = q.shape[0]
        out = torch.empty((bs, self.max_pages_per_req), dtype=torch.float32, device=self.device)
        _lib.call("qq_quest_page_scores", _lib.ptr(q), _lib.dtype_code(q.dtype), q.stride(0),
                  _lib.ptr(self.page_k_bounds), layer_id - self.start_layer, _lib.ptr(rpi), bs,
                  self.max_reqs, self.max_pages_per_req, self.kv_heads, self.head_dim,
                  _lib.ptr(out), _lib.stream(self.device))
        return out

    # ----------------------------------------------------------- [Q6] top-k

    def retrieve_topk(
        self,
        queries: torch.Tensor,
        layer_id: int,
        req_pool_indices: torch.Tensor,
        seq_lens: torch.Tensor,
        *,
        out: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """[Q6] Token positions this layer attends to (quest.py:409-464).

        Returns ``(positions [bs, top_k] int32, actual_lens [bs] int32)``; long
        requests get the ``top_k/P - 1`` best complete pages (descending score,
        ties to the lowest page) expanded to positions, then the recent window;
        short requests get ``0 .. seq_len-1``.  ``out`` may supply the positions
        buffer (``[>= bs, top_k]`` int32) to avoid an allocation.
        """
        step = self._step
        if step is None:
            raise RuntimeError("prepare_step() must be called once per decode step first")
        q = self._queries_3d(queries)
        bs = q.shape[0]
        if step.seq_lens.shape[0] != bs or seq_lens.shape[0] != bs:
            raise ValueError("batch size differs from the one given to prepare_step()")
        if bs > self.max_reqs:
            raise ValueError(f"batch {bs} exceeds max_reqs {self.max_reqs}")
        rpi = req_pool_indices
        if rpi.dtype != torch.int64 or rpi.device != self.device or not rpi.is_contiguous():
            rpi = rpi.to(device=self.device, dtype=torch.int64).contiguous()
        positions = out if out is not None else torch.empty((bs, self.top_k), dtype=torch.int32, device=self.device)
        _lib.call(
            "qq_quest_retrieve_topk", _lib.ptr(q), _lib.dtype_code(q.dtype), q.stride(0), q.shape[1],
            _lib.ptr(self.page_k_bounds), layer_id - self.start_layer, _lib.ptr(rpi),
            _lib.ptr(step.seq_lens), _lib.ptr(step.candidate_limit_i32), bs, self.max_reqs,
            self.max_pages_per_req, self.kv_heads, self.head_dim, self.page_size, self.top_k,
            _lib.ptr(self._scores_ws), _lib.ptr(positions), _lib.stream(self.device),
        )
        if self.trace is not None:
            self._record(layer_id, rpi, step, positions[:bs])
        return positions[:bs], step.actual_lens

    # ------------------------------------------------------ [Q8] request end

    def invalidate_request(self, req_pool_idx: int) -> None:
        """[Q8] Reset every per-request buffer of a freed slot (quest.py:468-479)."""
        self._reset(int(req_pool_idx), 1)

    # ----------------------------------------------------------- tracing

    def _record(self, layer_id, req_pool_indices, step: StepLayout, positions) -> None:
        """quest.py:483-515; scores are the kernel's, masked past candidate_limit."""
        assert self.trace is not None
        P, k = self.page_size, self.top_k_pages - 1
        seqs = step.seq_lens.tolist()
        actual = step.actual_lens.tolist()
        limits = step.candidate_limit_i32.tolist()
        pos_cpu = positions.to("cpu", torch.int64)
        scores_cpu = self._scores_ws[: len(seqs)].cpu()
        all_short = all(s <= self.top_k for s in seqs)
        for i, s in enumerate(seqs):
            dense = s <= self.top_k
            full = s // P
            page_scores = None
            if not dense:
                sc = scores_cpu[i, :full].clone()
                sc[limits[i]:] = float("-inf")
                page_scores = sc
            elif not all_short:
                page_scores = None
            pages = [] if dense or k <= 0 else sorted(int(p) // P for p in pos_cpu[i, : k * P : P].tolist())
            self.trace.add(
                QuestSelection(
                    layer_id=layer_id,
                    req_pool_idx=int(req_pool_indices[i]),
                    seq_len=s,
                    dense=dense,
                    selected_pages=pages,
                    recent_window=(max(s - P, 0), s),
                    page_scores=page_scores,
                    positions=pos_cpu[i, : actual[i]].clone(),
                )
            )
