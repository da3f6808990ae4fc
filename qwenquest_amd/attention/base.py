"""Attention-backend interface (reference ``src/qwenquest/attention/base.py:20-112``).

The drop-in boundary: per forward the engine calls ``init_forward_metadata``
once, then the model calls ``forward`` once per layer.  ``layer`` is any object
with ``layer_id`` and ``scaling`` (the reference's ``RadixAttention``).
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TYPE_CHECKING, Any

import torch

from qwenquest_amd.attention.ops import extend_attention

if TYPE_CHECKING:
    from qwenquest_amd.batch import ForwardBatch
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

__all__ = ["AttentionBackend"]


class AttentionBackend(ABC):
    #: SGLang backend this class stands in for.
    name: str = ""
    #: Whether a decode token's K/V goes to the shared device token pool.
    uses_token_pool_for_decode: bool = True
    #: Whether the engine may free the prefill's token-pool slots after on_extend_finished.
    frees_prefill_kv_after_admission: bool = False

    def __init__(self, req_to_token_pool: ReqToTokenPool, token_to_kv_pool: MHATokenToKVPool):
        self.req_to_token_pool = req_to_token_pool
        self.token_to_kv_pool = token_to_kv_pool

    @property
    def req_to_token(self) -> torch.Tensor:
        return self.req_to_token_pool.req_to_token

    def init_forward_metadata(self, batch: ForwardBatch) -> None:  # noqa: B027 - optional hook
        """Per-forward preparation (once, before layer 0)."""

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer: Any, batch: ForwardBatch) -> torch.Tensor:
        if batch.forward_mode.is_decode():
            return self.forward_decode(q, k, v, layer, batch)
        return self.forward_extend(q, k, v, layer, batch)

    def forward_extend(self, q, k, v, layer, batch: ForwardBatch) -> torch.Tensor:
        """Dense causal prefill: save the new K/V, then attend per request (base.py:65-93)."""
        assert batch.out_cache_loc is not None and batch.extend_prefix_lens is not None
        self.token_to_kv_pool.set_kv_buffer(layer.layer_id, batch.out_cache_loc, k, v)
        k_buf, v_buf = self.token_to_kv_pool.get_kv_buffer(layer.layer_id)
        offsets = batch.extend_token_offsets()
        outputs = []
        for i in range(batch.batch_size):
            req = int(batch.req_pool_indices[i])
            seq_len = int(batch.seq_lens[i])
            locs = self.req_to_token[req, :seq_len].long()
            outputs.append(
                extend_attention(q[offsets[i] : offsets[i + 1]], k_buf[locs], v_buf[locs],
                                 prefix_len=int(batch.extend_prefix_lens[i]), scaling=layer.scaling)
            )
        return torch.cat(outputs, dim=0)

    @abstractmethod
    def forward_decode(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer: Any, batch: ForwardBatch) -> torch.Tensor:
        """``q [bs, H, D]``, ``k/v [bs, KV, D]`` of the new tokens -> ``[bs, H*D]``."""

    def on_extend_finished(self, batch: ForwardBatch) -> None:  # noqa: B027 - optional hook
        """Called by the engine after a whole prefill forward (all layers)."""

    def on_request_finished(self, req_pool_idx: int) -> None:  # noqa: B027 - optional hook
        """Called by the engine before a request slot is reused."""

    def poll_errors(self) -> None:  # noqa: B027 - optional hook
        """Raise an error the device detected in a decode step whose kernels have finished,
        without a synchronisation.  A caller that replays a captured decode step calls it after
        each replay, since no Python check runs inside a replay.  Backends without
        device-detected errors have nothing to raise."""
