"""Mode 3 - Quest selection + HiSparse hierarchical KV cache
(reference ``src/qwenquest/attention/quest_hisparse.py``, SGLang ``flashinfer_hisparse``).

Per decode step::

    init_forward_metadata:  [H2] fold the previous token into the bounds + back it up to
                                 the pinned host tier; [Q4] prepare_step
    forward_decode (x L):   new K/V -> hot buffer newest slot; [Q6] retrieve_topk;
                            [H3] swap-in (plan + host->device copy of misses);
                            [Q7] attention over the returned hot-buffer rows
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import TYPE_CHECKING, Any

import torch

from qwenquest_amd.attention.base import AttentionBackend
from qwenquest_amd.attention.ops import AttentionWorkspace, decode_attention_rows
from qwenquest_amd.config import SparseConfig, parse_hisparse_config
from qwenquest_amd.hisparse.coordinator import HiSparseCoordinator
from qwenquest_amd.quest import QuestAlgorithm

if TYPE_CHECKING:
    from qwenquest_amd.batch import ForwardBatch
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

__all__ = ["QuestHiSparseBackend"]


class QuestHiSparseBackend(AttentionBackend):
    name = "flashinfer_hisparse"
    uses_token_pool_for_decode = False
    frees_prefill_kv_after_admission = True

    def __init__(
        self,
        req_to_token_pool: ReqToTokenPool,
        token_to_kv_pool: MHATokenToKVPool,
        sparse_config: str | Mapping[str, Any] | SparseConfig | None,
        *,
        host_pool_size: int,
        start_layer: int = 0,
        end_layer: int | None = None,
        host_device: torch.device | str = "cpu",
    ):
        super().__init__(req_to_token_pool, token_to_kv_pool)
        cfg = parse_hisparse_config(sparse_config)
        if cfg.algorithm != "quest" or cfg.quest_page_size is None:
            raise ValueError("Quest backends require hisparse_config with algorithm='quest'")
        self.sparse_config = cfg
        device = token_to_kv_pool.device
        num_layers = token_to_kv_pool.num_layers
        self.quest = QuestAlgorithm(
            top_k=cfg.top_k, page_size=cfg.quest_page_size, device=device,
            avoid_recent_overlap=cfg.avoid_recent_overlap,
        )
        self.quest.init_storage(
            start_layer=start_layer,
            end_layer=num_layers if end_layer is None else end_layer,
            max_reqs=req_to_token_pool.size,
            max_context_len=req_to_token_pool.max_context_len,
            kv_heads=token_to_kv_pool.kv_heads,
            head_dim=token_to_kv_pool.head_dim,
        )
        self.coord = HiSparseCoordinator(
            quest=self.quest,
            num_layers=num_layers,
            kv_heads=token_to_kv_pool.kv_heads,
            head_dim=token_to_kv_pool.head_dim,
            max_reqs=req_to_token_pool.size,
            max_context_len=req_to_token_pool.max_context_len,
            top_k=cfg.top_k,
            device_buffer_size=cfg.device_buffer_size,
            host_pool_size=host_pool_size,
            dtype=token_to_kv_pool.dtype,
            device=device,
            host_device=host_device,
        )
        self._positions = torch.empty((req_to_token_pool.size, cfg.top_k), dtype=torch.int32, device=device)
        self._attn_ws = AttentionWorkspace(device)

    def init_forward_metadata(self, batch: ForwardBatch) -> None:
        if batch.forward_mode.is_decode():
            self.coord.prepare_decode_step(batch.req_pool_indices, batch.seq_lens)
            self.quest.prepare_step(batch.seq_lens)

    def on_extend_finished(self, batch: ForwardBatch) -> None:
        """[H1] quest_hisparse.py:103-108."""
        for req_idx, seq_len in zip(batch.req_pool_indices.tolist(), batch.seq_lens.tolist(), strict=True):
            prefill_indices = self.req_to_token[req_idx, :seq_len]
            self.coord.admit_request(req_idx, seq_len, self.token_to_kv_pool, prefill_indices)

    def forward_decode(self, q, k, v, layer, batch: ForwardBatch) -> torch.Tensor:
        """quest_hisparse.py:112-133."""
        reqs, seq_lens = batch.req_pool_indices, batch.seq_lens
        self.coord.write_new_token(layer.layer_id, reqs, seq_lens, k, v)
        positions, actual = self.quest.retrieve_topk(q, layer.layer_id, reqs, seq_lens, out=self._positions)
        rows = self.coord.swap_in_selected_pages(reqs, seq_lens, positions, layer.layer_id, actual_lens=actual)
        bs = batch.batch_size
        q3 = self.quest._queries_3d(q)
        return decode_attention_rows(
            q3, self.coord.device_k[layer.layer_id], self.coord.device_v[layer.layer_id], rows, actual,
            layer.scaling, workspace=self._attn_ws,
        ).view(bs, -1)

    def on_request_finished(self, req_pool_idx: int) -> None:
        self.coord.request_finished(req_pool_idx)
