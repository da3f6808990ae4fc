"""Mode 2 - Quest sparse decode, full KV pool on the GPU
(reference ``src/qwenquest/attention/quest_only.py``, SGLang ``flashinfer_quest``).

Per decode step::

    init_forward_metadata:  [Q3] fold the previous token's K into the running bounds of
                                 every layer + finalize completed pages (one fused kernel;
                                 skipped on the first decode step after prefill)
                            [Q4] prepare_step
    forward_decode (x L):   save new K/V -> [Q6] retrieve_topk (score + select + layout)
                            -> [Q7] req_to_token gather + split-K attention
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import TYPE_CHECKING, Any

import torch

from qwenquest_amd import _lib
from qwenquest_amd.attention.base import AttentionBackend
from qwenquest_amd.attention.ops import AttentionWorkspace
from qwenquest_amd.config import SparseConfig, parse_hisparse_config
from qwenquest_amd.quest import QuestAlgorithm

if TYPE_CHECKING:
    from qwenquest_amd.batch import ForwardBatch
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

__all__ = ["QuestOnlyBackend"]


class QuestOnlyBackend(AttentionBackend):
    name = "flashinfer_quest"

    def __init__(
        self,
        req_to_token_pool: ReqToTokenPool,
        token_to_kv_pool: MHATokenToKVPool,
        sparse_config: str | Mapping[str, Any] | SparseConfig | None,
        *,
        start_layer: int = 0,
        end_layer: int | None = None,
    ):
        super().__init__(req_to_token_pool, token_to_kv_pool)
        cfg = parse_hisparse_config(sparse_config)
        if cfg.algorithm != "quest" or cfg.quest_page_size is None:
            raise ValueError("Quest backends require hisparse_config with algorithm='quest'")
        self.sparse_config = cfg
        device = token_to_kv_pool.device
        self.quest = QuestAlgorithm(
            top_k=cfg.top_k, page_size=cfg.quest_page_size, device=device,
            avoid_recent_overlap=cfg.avoid_recent_overlap,
        )
        self.quest.init_storage(
            start_layer=start_layer,
            end_layer=token_to_kv_pool.num_layers if end_layer is None else end_layer,
            max_reqs=req_to_token_pool.size,
            max_context_len=req_to_token_pool.max_context_len,
            kv_heads=token_to_kv_pool.kv_heads,
            head_dim=token_to_kv_pool.head_dim,
        )
        self._skip_first_decode_update = torch.zeros(req_to_token_pool.size, dtype=torch.bool, device=device)
        self._step_locs = torch.empty(req_to_token_pool.size, dtype=torch.int64, device=device)
        self._positions = torch.empty((req_to_token_pool.size, cfg.top_k), dtype=torch.int32, device=device)
        self._attn_ws = AttentionWorkspace(device)
        # counters of the fused (two-launch) layer step: zeroed once, left zeroed by every
        # call (set to None to run the layer as four launches)
        sync_bytes = int(_lib.load().qq_quest_layer_step_sync_bytes(req_to_token_pool.size, token_to_kv_pool.kv_heads))
        self._step_sync = torch.zeros(max(sync_bytes, 4), dtype=torch.uint8, device=device)
        # counters of the one-launch decode-step bookkeeping, left zeroed by every call
        step_bytes = int(_lib.load().qq_quest_decode_step_sync_bytes(req_to_token_pool.size))
        self._decode_sync = torch.zeros(max(step_bytes, 4), dtype=torch.uint8, device=device)

    # ---------------------------------------------------------------- per step

    def init_forward_metadata(self, batch: ForwardBatch) -> None:
        """[Q3] + [Q4] for a decode batch in one launch (QuestAlgorithm.decode_step): the
        same results as _do_quest_decode_step_update followed by prepare_step."""
        if batch.forward_mode.is_decode():
            bs = int(batch.req_pool_indices.numel())
            if bs > self._step_locs.numel():
                raise ValueError(f"batch {bs} exceeds the request pool ({self._step_locs.numel()})")
            self.quest.decode_step(batch.req_pool_indices, batch.seq_lens, self.token_to_kv_pool.k_all,
                                   self.req_to_token, self._skip_first_decode_update, self._decode_sync,
                                   self._step_locs[:bs])

    def _do_quest_decode_step_update(self, req_pool_indices: torch.Tensor, seq_lens: torch.Tensor) -> None:
        """[Q3] The previous step's token sits at position ``seq_len - 2`` (quest_only.py:84-97).

        Requests on their first decode step after prefill get row -1, which the
        fused kernel skips (no fold, no counter advance), without a host sync: one
        kernel looks the rows up and clears the first-step flags.
        """
        dev = self.quest.device
        rpi = req_pool_indices.to(device=dev, dtype=torch.int64).contiguous()
        seq = seq_lens.to(device=dev, dtype=torch.int64).contiguous()
        bs = int(rpi.numel())
        if bs > self._step_locs.numel():
            raise ValueError(f"batch {bs} exceeds the request pool ({self._step_locs.numel()})")
        locs = self._step_locs[:bs]
        r2t = self.req_to_token
        _lib.call("qq_quest_decode_step_locs", _lib.ptr(rpi), _lib.ptr(seq), bs,
                  _lib.ptr(self._skip_first_decode_update), _lib.ptr(r2t), r2t.shape[0], r2t.shape[1], r2t.stride(0),
                  _lib.ptr(locs), _lib.stream(dev))
        self.quest.update_decode_representations_fused(rpi, self.token_to_kv_pool.k_all, locs)

    # ----------------------------------------------------------------- prefill

    def forward_extend(self, q, k, v, layer, batch: ForwardBatch) -> torch.Tensor:
        out = super().forward_extend(q, k, v, layer, batch)
        if layer.layer_id == self.quest.end_layer - 1:
            self._update_quest_for_extend(batch)
        return out

    def _update_quest_for_extend(self, batch: ForwardBatch) -> None:
        """[Q2] Per request: bounds of positions ``0 .. seq_len-1`` at every layer (quest_only.py:115-128)."""
        for req_idx, seq_len in zip(batch.req_pool_indices.tolist(), batch.seq_lens.tolist(), strict=True):
            prefill_indices = self.req_to_token[req_idx, :seq_len]
            self.quest.update_prefill_representations_fused(req_idx, self.token_to_kv_pool.k_all, prefill_indices)
            self._skip_first_decode_update[req_idx] = True

    # ------------------------------------------------------------------ decode

    def forward_decode(self, q, k, v, layer, batch: ForwardBatch) -> torch.Tensor:
        """quest_only.py:132-159 in one C call: save the new K/V, select, gather + attend."""
        return self.forward_decode_phase(q, k, v, layer, batch, 3)

    def forward_decode_phase(self, q, k, v, layer, batch: ForwardBatch, phase: int) -> torch.Tensor:
        """forward_decode's stages: 1 = scoring + selection + new-token store, 2 = layout +
        attention (after phase 1 of the same layer and batch), 3 = both.  Returns the output
        tensor (complete after phase 2)."""
        assert batch.out_cache_loc is not None
        quest = self.quest
        step = quest._step
        if step is None:
            raise RuntimeError("prepare_step() must be called once per decode step first")
        pool = self.token_to_kv_pool
        bs = batch.batch_size
        q3 = quest._queries_3d(q)
        heads, dim = q3.shape[1], pool.head_dim
        if step.seq_lens.shape[0] != bs:
            raise ValueError("batch size differs from the one given to prepare_step()")
        kn = k.reshape(bs, pool.kv_heads * dim)
        vn = v.reshape(bs, pool.kv_heads * dim)
        if kn.dtype != vn.dtype or kn.dtype not in (torch.bfloat16, torch.float32):
            kn, vn = kn.to(pool.dtype), vn.to(pool.dtype)
        kn, vn = kn.contiguous(), vn.contiguous()
        loc = batch.out_cache_loc
        if loc.dtype != torch.int64 or not loc.is_contiguous():
            loc = loc.to(torch.int64).contiguous()
        rpi = batch.req_pool_indices
        if rpi.dtype != torch.int64 or not rpi.is_contiguous():
            rpi = rpi.to(torch.int64).contiguous()
        k_buf, v_buf = pool.get_kv_buffer(layer.layer_id)
        buf = self._attn_ws.get(bs, quest.top_k, heads, dim)
        out = torch.empty((bs, heads * dim), dtype=q3.dtype, device=q3.device)
        r2t = self.req_to_token
        sync = self._step_sync  # None: the four-launch path
        _lib.call(
            "qq_quest_forward_decode_phase", _lib.ptr(q3), _lib.dtype_code(q3.dtype), q3.stride(0), heads,
            _lib.ptr(kn), _lib.ptr(vn), _lib.dtype_code(kn.dtype), _lib.ptr(loc), _lib.ptr(k_buf),
            _lib.ptr(v_buf), _lib.dtype_code(k_buf.dtype), k_buf.shape[0], _lib.ptr(quest.page_k_bounds),
            layer.layer_id - quest.start_layer, _lib.ptr(rpi), _lib.ptr(step.seq_lens),
            _lib.ptr(step.candidate_limit_i32), _lib.ptr(step.actual_lens), bs, quest.max_reqs,
            quest.max_pages_per_req, quest.kv_heads, quest.head_dim, quest.page_size, quest.top_k,
            _lib.ptr(r2t), r2t.stride(0), r2t.shape[0], float(layer.scaling), _lib.ptr(quest._scores_ws),
            _lib.ptr(self._positions), _lib.ptr(out), _lib.ptr(buf), buf.numel(), _lib.ptr(sync),
            0 if sync is None else sync.numel(), int(phase), _lib.stream(q3.device),
        )
        if quest.trace is not None and phase & 2:
            quest._record(layer.layer_id, rpi, step, self._positions[:bs])
        return out

    def sparse_attention(self, q, layer, req_pool_indices, positions, actual, bs) -> torch.Tensor:
        """[Q7] rows = req_to_token[req, positions[:n]] -> attention over exactly those rows."""
        heads = q.shape[1] if q.dim() == 3 else q.shape[1] // self.token_to_kv_pool.head_dim
        dim = self.token_to_kv_pool.head_dim
        q3 = q.reshape(bs, heads, dim).contiguous()
        k_buf, v_buf = self.token_to_kv_pool.get_kv_buffer(layer.layer_id)
        rpi = req_pool_indices
        if rpi.dtype != torch.int64 or rpi.device != q3.device:
            rpi = rpi.to(device=q3.device, dtype=torch.int64)
        rpi = rpi.contiguous()
        buf = self._attn_ws.get(bs, positions.shape[1], heads, dim)
        out = torch.empty((bs, heads * dim), dtype=q3.dtype, device=q3.device)
        r2t = self.req_to_token
        _lib.call(
            "qq_quest_decode_attention", _lib.ptr(q3), _lib.dtype_code(q3.dtype), q3.stride(0), heads,
            _lib.ptr(k_buf), _lib.ptr(v_buf), _lib.dtype_code(k_buf.dtype), k_buf.shape[0],
            self.token_to_kv_pool.kv_heads, dim, _lib.ptr(r2t), r2t.stride(0), r2t.shape[0], _lib.ptr(rpi),
            _lib.ptr(positions), positions.stride(0), _lib.ptr(actual), bs, float(layer.scaling),
            _lib.ptr(out), _lib.ptr(buf), buf.numel(), _lib.stream(q3.device),
        )
        return out

    # --------------------------------------------------------------- lifecycle

    def on_request_finished(self, req_pool_idx: int) -> None:
        """[Q8] quest_only.py:163-167."""
        self.quest.invalidate_request(req_pool_idx)
        self._skip_first_decode_update[req_pool_idx] = False
