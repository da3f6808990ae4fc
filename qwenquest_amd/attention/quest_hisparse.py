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

from qwenquest_amd import _lib
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
        swap_route: str = "kernel",
        async_admission: bool = False,
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
            swap_route=swap_route,
            async_admission=async_admission,
        )
        # with the admission backup on a side stream the prompt's pool rows are read after
        # on_extend_finished returns: the engine frees them once coord.admission_done(req)
        self.frees_prefill_kv_after_admission = not async_admission
        self._positions = torch.empty((req_to_token_pool.size, cfg.top_k), dtype=torch.int32, device=device)
        self._attn_ws = AttentionWorkspace(device)
        # QuestOnlyBackend runs its fused layer step for some shapes; the attention over the
        # hot-buffer rows then runs the same kernel (counters in this zeroed buffer), so the
        # two modes give the same bits
        sync_bytes = int(_lib.load().qq_quest_layer_step_sync_bytes(req_to_token_pool.size, token_to_kv_pool.kv_heads))
        self._attn_sync = torch.zeros(max(sync_bytes, 4), dtype=torch.uint8, device=device)
        self._fused_cache: dict[tuple, bool] = {}

    def init_forward_metadata(self, batch: ForwardBatch) -> None:
        if batch.forward_mode.is_decode():
            self.coord.prepare_decode_step(batch.req_pool_indices, batch.seq_lens)
            self.quest.prepare_step(batch.seq_lens)

    def on_extend_finished(self, batch: ForwardBatch) -> None:
        """[H1] quest_hisparse.py:103-108."""
        for req_idx, seq_len in zip(batch.req_pool_indices.tolist(), batch.seq_lens.tolist(), strict=True):
            prefill_indices = self.req_to_token[req_idx, :seq_len]
            self.coord.admit_request(req_idx, seq_len, self.token_to_kv_pool, prefill_indices)

    def _fused_attention(self, q3: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
        """Whether QuestOnlyBackend.forward_decode would run the fused layer step for these
        tensors (its new K/V dtype rule: k's dtype if k and v share bf16 or fp32, else the pool's)."""
        pool_dtype = self.token_to_kv_pool.dtype
        new_dtype = k.dtype if k.dtype == v.dtype and k.dtype in (torch.bfloat16, torch.float32) else pool_dtype
        key = (q3.dtype, new_dtype, q3.shape[1])
        if key not in self._fused_cache:
            qa, pool = self.quest, self.token_to_kv_pool
            self._fused_cache[key] = bool(_lib.load().qq_quest_fused_step(
                _lib.dtype_code(q3.dtype), _lib.dtype_code(pool_dtype), _lib.dtype_code(new_dtype), q3.shape[1],
                pool.kv_heads, pool.head_dim, qa.page_size, qa.top_k, qa.max_pages_per_req))
        return self._fused_cache[key]

    def forward_decode(self, q, k, v, layer, batch: ForwardBatch) -> torch.Tensor:
        """quest_hisparse.py:112-133."""
        reqs, seq_lens = batch.req_pool_indices, batch.seq_lens
        coord = self.coord
        # the new token rides with the swap-in launch when it needs no conversion
        # (the selection does not read the hot buffer, the attention reads it after the swap-in)
        fused_new = coord.swap_route == "kernel" and k.dtype == coord.dtype and v.dtype == coord.dtype
        if not fused_new:
            coord.write_new_token(layer.layer_id, reqs, seq_lens, k, v)
        positions, actual = self.quest.retrieve_topk(q, layer.layer_id, reqs, seq_lens, out=self._positions)
        rows = coord.swap_in_selected_pages(reqs, seq_lens, positions, layer.layer_id, actual_lens=actual,
                                            new_k=k if fused_new else None, new_v=v if fused_new else None)
        bs = batch.batch_size
        q3 = self.quest._queries_3d(q)
        return decode_attention_rows(
            q3, self.coord.device_k[layer.layer_id], self.coord.device_v[layer.layer_id], rows, actual,
            layer.scaling, workspace=self._attn_ws,
            sync=self._attn_sync if self._fused_attention(q3, k, v) else None,
        ).view(bs, -1)

    def on_request_finished(self, req_pool_idx: int) -> None:
        self.coord.request_finished(req_pool_idx)

    def poll_errors(self) -> None:
        """The swap-in's and the eager backup's errors (coordinator.py:278-279, 285-286;
        memory.py:62-66) from the pinned mirror of the device error word, without a
        synchronisation: an error surfaces at the first poll after the kernel that detected it
        has finished (after a synchronisation, at once).  A failed request's attention output
        is NaN in the step that failed.  Eager decode steps poll at the next step's
        init_forward_metadata; a caller that replays a captured step polls after each replay."""
        self.coord.check_errors(sync=False)
