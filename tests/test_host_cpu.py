"""Host logic that needs no GPU: config parsing (reference tests/test_config.py:132-175)
and the argument validation of the host classes."""

from __future__ import annotations

import pytest
import torch

from qwenquest_amd.config import SparseConfig, parse_hisparse_config
from qwenquest_amd.quest import QuestAlgorithm


def test_hisparse_defaults_match_upstream():
    cfg = parse_hisparse_config('{"algorithm": "quest"}')
    assert (cfg.top_k, cfg.quest_page_size, cfg.device_buffer_size) == (2048, 64, 4096)
    assert (cfg.host_to_device_ratio, cfg.swap_in_block_size) == (2, 960)
    assert cfg.avoid_recent_overlap is False
    assert parse_hisparse_config(None).quest_page_size is None


def test_hisparse_full_config_round_trips():
    cfg = parse_hisparse_config(
        '{"top_k": 2048, "device_buffer_size": 6144, "host_to_device_ratio": 10, '
        '"swap_in_block_size": 960, "algorithm": "quest", "quest_page_size": 32}'
    )
    assert cfg.device_buffer_size == 6144 and cfg.quest_page_size == 32
    assert parse_hisparse_config(cfg) is cfg


def test_unknown_keys_go_to_extra_config():
    cfg = parse_hisparse_config({"algorithm": "quest", "avoid_recent_overlap": True, "foo": 1})
    assert cfg.avoid_recent_overlap is True
    assert cfg.sparse_extra_config == {"avoid_recent_overlap": True, "foo": 1}


@pytest.mark.parametrize(
    "raw",
    [
        '{"algorithm": "quest", "top_k": 100}',
        '{"top_k": 2048, "device_buffer_size": 1024}',
        '{"swap_in_block_size": 2048}',
        '{"swap_in_block_size": true}',
        '{"swap_in_block_size": 0}',
        "{not json",
    ],
)
def test_hisparse_validation(raw):
    with pytest.raises(ValueError):
        parse_hisparse_config(raw)


def test_sparse_config_is_frozen():
    cfg = SparseConfig()
    with pytest.raises(AttributeError):
        cfg.top_k = 1  # type: ignore[misc]


def test_invalid_top_k_page_size_combo_rejected():
    with pytest.raises(ValueError):
        QuestAlgorithm(top_k=100, page_size=64, device="cpu")
    with pytest.raises(ValueError):
        QuestAlgorithm(top_k=64, page_size=0, device="cpu")


def test_quest_storage_refuses_the_cpu():
    q = QuestAlgorithm(top_k=64, page_size=16, device="cpu")
    with pytest.raises(RuntimeError, match="GPU"):
        q.init_storage(0, 2, 2, 256, 4, 32)


def test_retrieve_topk_requires_prepare_step():
    q = QuestAlgorithm(top_k=64, page_size=16, device="cpu")
    with pytest.raises(RuntimeError):
        q.retrieve_topk(torch.randn(1, 4, 32), 0, torch.tensor([0]), torch.tensor([5]))
