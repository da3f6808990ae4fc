"""qwenquest_amd - the Quest sparse-decode path of QwenQuest, MI355X-native.

Host code mirrors the reference's attention-backend interface
(``AttentionBackend``, ``QuestOnlyBackend``, ``QuestHiSparseBackend``,
``QuestAlgorithm``, ``ReqToTokenPool``/``MHATokenToKVPool``); all computation
runs in hand-written gfx950 HIP kernels of ``libqwenquest_amd.so`` behind a C ABI
(``include/qwenquest_amd.h``).  There is no CPU path.
"""

from qwenquest_amd.batch import ForwardBatch, ForwardMode
from qwenquest_amd.config import SparseConfig, parse_hisparse_config
from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool, TokenToKVPoolAllocator
from qwenquest_amd.quest import QuestAlgorithm, QuestSelection, QuestTrace, StepLayout

__version__ = "0.1.0"

__all__ = [
    "ForwardBatch",
    "ForwardMode",
    "MHATokenToKVPool",
    "QuestAlgorithm",
    "QuestSelection",
    "QuestTrace",
    "ReqToTokenPool",
    "SparseConfig",
    "StepLayout",
    "TokenToKVPoolAllocator",
    "parse_hisparse_config",
]
