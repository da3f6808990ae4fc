"""``--hisparse-config`` parsing (reference ``src/qwenquest/config.py:267-358``).

Same JSON keys, defaults and validation as the reference (which mirrors
SGLang's ``SparseConfig``); unknown keys land in ``sparse_extra_config``, from
which ``avoid_recent_overlap`` is read.
"""

from __future__ import annotations

import json
from collections.abc import Mapping
from dataclasses import dataclass, field
from typing import Any

__all__ = ["SparseConfig", "parse_hisparse_config"]

_DEFAULT_TOP_K = 2048
_DEFAULT_HOST_TO_DEVICE_RATIO = 2
_DEFAULT_SWAP_IN_BLOCK = 960
_DEFAULT_QUEST_PAGE = 64
_MAX_SWAP_IN_BLOCK = 1024


@dataclass(frozen=True)
class SparseConfig:
    """Reference ``SparseConfig`` (config.py:267-295).

    ``top_k``, ``device_buffer_size``, ``algorithm`` and ``quest_page_size``
    drive the kernels; ``host_to_device_ratio`` and ``swap_in_block_size`` are
    carried so a real config string round-trips.
    """

    top_k: int = _DEFAULT_TOP_K
    device_buffer_size: int = 2 * _DEFAULT_TOP_K
    host_to_device_ratio: int = _DEFAULT_HOST_TO_DEVICE_RATIO
    swap_in_block_size: int = _DEFAULT_SWAP_IN_BLOCK
    algorithm: str | None = None
    backend: str | None = None
    page_size: int | None = None
    min_sparse_prompt_len: int | None = None
    quest_page_size: int | None = None
    sparse_extra_config: dict[str, Any] = field(default_factory=dict, hash=False)

    @property
    def avoid_recent_overlap(self) -> bool:
        return bool(self.sparse_extra_config.get("avoid_recent_overlap", False))


def _load(config: str | Mapping[str, Any] | None) -> dict[str, Any]:
    if config is None:
        return {}
    if isinstance(config, str):
        try:
            return dict(json.loads(config))
        except json.JSONDecodeError as e:
            raise ValueError(f"Failed to parse hisparse_config: {e}") from e
    return dict(config)


def parse_hisparse_config(config: str | Mapping[str, Any] | SparseConfig | None) -> SparseConfig:
    """Reference ``parse_hisparse_config`` (config.py:298-358)."""
    if isinstance(config, SparseConfig):
        return config
    d = _load(config)
    top_k = d.pop("top_k", _DEFAULT_TOP_K)
    device_buffer_size = d.pop("device_buffer_size", 2 * top_k)
    host_to_device_ratio = d.pop("host_to_device_ratio", _DEFAULT_HOST_TO_DEVICE_RATIO)
    swap_in_block_size = d.pop("swap_in_block_size", _DEFAULT_SWAP_IN_BLOCK)
    if device_buffer_size < top_k:
        raise ValueError(
            f"device_buffer_size ({device_buffer_size}) must be no smaller than top_k ({top_k})"
        )
    if isinstance(swap_in_block_size, bool) or not isinstance(swap_in_block_size, int):
        raise ValueError(f"swap_in_block_size must be an integer, got {swap_in_block_size!r}")
    if not 0 < swap_in_block_size <= _MAX_SWAP_IN_BLOCK:
        raise ValueError(
            f"swap_in_block_size ({swap_in_block_size}) must be in the range [1, {_MAX_SWAP_IN_BLOCK}]"
        )
    algorithm = d.pop("algorithm", None)
    backend = d.pop("backend", None)
    min_sparse_prompt_len = d.pop("min_sparse_prompt_len", None)
    page_size = d.pop("page_size", None)
    quest_page_size = d.pop("quest_page_size", None)
    if algorithm == "quest":
        if quest_page_size is None:
            quest_page_size = _DEFAULT_QUEST_PAGE
        if quest_page_size <= 0 or top_k % quest_page_size != 0:
            raise ValueError(
                f"hisparse_config: top_k ({top_k}) must be divisible by "
                f"quest_page_size ({quest_page_size}) for algorithm='quest'."
            )
    return SparseConfig(
        top_k=top_k,
        device_buffer_size=device_buffer_size,
        host_to_device_ratio=host_to_device_ratio,
        swap_in_block_size=swap_in_block_size,
        algorithm=algorithm,
        backend=backend,
        page_size=page_size,
        min_sparse_prompt_len=min_sparse_prompt_len,
        quest_page_size=quest_page_size,
        sparse_extra_config=d,
    )
