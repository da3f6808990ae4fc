"""Per-forward batch carrier (reference ``src/qwenquest/batch.py:27-64``)."""

from __future__ import annotations

import enum
from dataclasses import dataclass
from typing import TYPE_CHECKING, Any

import torch

if TYPE_CHECKING:
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

__all__ = ["ForwardBatch", "ForwardMode"]


class ForwardMode(enum.Enum):
    EXTEND = "extend"
    DECODE = "decode"

    def is_extend(self) -> bool:
        return self is ForwardMode.EXTEND

    def is_decode(self) -> bool:
        return self is ForwardMode.DECODE


@dataclass
class ForwardBatch:
    """``seq_lens`` counts the token being decoded (its K/V lands at ``seq_len - 1``)."""

    forward_mode: ForwardMode
    input_ids: torch.Tensor | None
    positions: torch.Tensor | None
    req_pool_indices: torch.Tensor  # [bs] int64
    seq_lens: torch.Tensor  # [bs] int64
    out_cache_loc: torch.Tensor | None
    req_to_token_pool: ReqToTokenPool
    token_to_kv_pool: MHATokenToKVPool
    attn_backend: Any
    extend_prefix_lens: torch.Tensor | None = None
    extend_seq_lens: torch.Tensor | None = None

    @property
    def batch_size(self) -> int:
        return int(self.req_pool_indices.shape[0])

    def extend_token_offsets(self) -> list[int]:
        assert self.extend_seq_lens is not None
        offsets = [0]
        for n in self.extend_seq_lens.tolist():
            offsets.append(offsets[-1] + int(n))
        return offsets
