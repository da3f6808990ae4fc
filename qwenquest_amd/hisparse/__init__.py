"""HiSparse hierarchical KV cache (reference ``src/qwenquest/hisparse``)."""

from qwenquest_amd.hisparse.coordinator import HiSparseCoordinator, SwapInStats

__all__ = ["HiSparseCoordinator", "SwapInStats"]
