"""Two-level KV addressing (reference ``src/qwenquest/memory.py``).

``ReqToTokenPool.req_to_token[req, position]`` is the physical row of a
position; ``MHATokenToKVPool`` holds one ``[size + 1, KV, D]`` K and V buffer
per layer, row 0 reserved as padding.  The per-layer buffers are views into ONE
``[num_layers, size + 1, KV, D]`` allocation so kernels that fuse all layers
(bounds append, prefill bounds) address them as base + layer stride.
"""

from __future__ import annotations

import torch

from qwenquest_amd import _lib

__all__ = ["MHATokenToKVPool", "ReqToTokenPool", "TokenToKVPoolAllocator", "kv_pair_zeros"]

# A V buffer starts this many bytes past its allocation's start.  Two large
# allocations are equally aligned (2 MiB), so without it a row's K and V slices
# of one KV head would sit at the same address modulo 1 KiB, and the attention's
# gather fetches such pairs more slowly (Quest layer step at batch 16 x 128K:
# 38.1 us per layer-step with the pools at the same offset, 37.5 us at 256 or
# 512 bytes apart; 2048 bytes apart is no better than 0).
V_SHIFT_BYTES = 512


def kv_pair_zeros(shape: tuple, dtype: torch.dtype, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """Zeroed K and V tensors of ``shape``, contiguous, with V placed V_SHIFT_BYTES into
    its allocation (a view; the layout and strides are those of a plain tensor)."""
    k = torch.zeros(shape, dtype=dtype, device=device)
    off = V_SHIFT_BYTES // torch.empty((), dtype=dtype).element_size()
    n = 1
    for d in shape:
        n *= int(d)
    v = torch.zeros(n + off, dtype=dtype, device=device)[off:].view(shape)
    return k, v


class ReqToTokenPool:
    """``req_to_token[req_pool_idx, position] -> physical token row`` (memory.py:28-50)."""

    def __init__(self, size: int, max_context_len: int, device: torch.device | str):
        self.size = size
        self.max_context_len = max_context_len
        self.device = torch.device(device)
        self.req_to_token = torch.zeros((size, max_context_len), dtype=torch.int32, device=self.device)
        self._free_slots = list(range(size))

    def available_size(self) -> int:
        return len(self._free_slots)

    def alloc(self) -> int:
        if not self._free_slots:
            raise RuntimeError("ReqToTokenPool is full; lower the number of concurrent requests")
        return self._free_slots.pop(0)

    def free(self, req_pool_idx: int) -> None:
        self.req_to_token[req_pool_idx].zero_()
        self._free_slots.append(req_pool_idx)


class TokenToKVPoolAllocator:
    """Free list over physical rows ``[1, size]``; row 0 is padding (memory.py:53-76)."""

    def __init__(self, size: int, device: torch.device | str = "cpu"):
        self.size = size
        self.device = torch.device(device)
        self._free = torch.arange(1, size + 1, dtype=torch.int64, device=self.device)

    def available_size(self) -> int:
        return int(self._free.numel())

    def alloc(self, n: int) -> torch.Tensor:
        if n > self._free.numel():
            raise RuntimeError(f"KV pool out of memory: need {n} token slots, {self._free.numel()} free")
        out, self._free = self._free[:n], self._free[n:]
        return out

    def free(self, indices: torch.Tensor) -> None:
        idx = indices.to(device=self.device, dtype=torch.int64).flatten()
        idx = idx[idx > 0]
        if idx.numel():
            self._free = torch.cat([self._free, idx])


class MHATokenToKVPool:
    """Per-layer K/V buffers ``[size + 1, kv_heads, head_dim]`` (memory.py:79-120)."""

    def __init__(
        self,
        size: int,
        num_layers: int,
        kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device | str,
    ):
        self.size = size
        self.num_layers = num_layers
        self.kv_heads = kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = torch.device(device)
        shape = (num_layers, size + 1, kv_heads, head_dim)
        self.k_all, self.v_all = kv_pair_zeros(shape, dtype, self.device)
        self.k_buffer = list(self.k_all.unbind(0))
        self.v_buffer = list(self.v_all.unbind(0))

    @property
    def rows(self) -> int:
        return self.size + 1

    @property
    def layer_stride(self) -> int:
        """Elements between consecutive layers' buffers."""
        return (self.size + 1) * self.kv_heads * self.head_dim

    def get_key_buffer(self, layer_id: int) -> torch.Tensor:
        return self.k_buffer[layer_id]

    def get_value_buffer(self, layer_id: int) -> torch.Tensor:
        return self.v_buffer[layer_id]

    def get_kv_buffer(self, layer_id: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.k_buffer[layer_id], self.v_buffer[layer_id]

    def set_kv_buffer(self, layer_id: int, loc: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write ``k``/``v`` ``[n, kv_heads, head_dim]`` at rows ``loc`` (memory.py:114-120)."""
        kb, vb = self.k_buffer[layer_id], self.v_buffer[layer_id]
        loc = loc.to(device=self.device, dtype=torch.int64).contiguous()
        n = int(loc.numel())
        if n == 0:
            return
        k = k.reshape(n, self.kv_heads * self.head_dim).contiguous()
        v = v.reshape(n, self.kv_heads * self.head_dim).to(k.dtype).contiguous()
        _lib.call(
            "qq_kv_scatter", _lib.ptr(kb), _lib.ptr(vb), _lib.dtype_code(self.dtype), self.rows,
            _lib.ptr(k), _lib.ptr(v), _lib.dtype_code(k.dtype), _lib.ptr(loc), n,
            self.kv_heads * self.head_dim, _lib.stream(self.device),
        )
