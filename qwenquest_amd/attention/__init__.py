"""Attention backends (reference ``src/qwenquest/attention/__init__.py``)."""

from qwenquest_amd.attention.base import AttentionBackend
from qwenquest_amd.attention.dense import DenseBackend
from qwenquest_amd.attention.quest_hisparse import QuestHiSparseBackend
from qwenquest_amd.attention.quest_only import QuestOnlyBackend

ATTENTION_MODES = ("dense", "quest", "quest_hisparse")

__all__ = ["ATTENTION_MODES", "AttentionBackend", "DenseBackend", "QuestHiSparseBackend", "QuestOnlyBackend"]
