"""Mode 1 - dense decode, the comparator of the Quest backends
(reference ``src/qwenquest/attention/dense.py``, SGLang ``flashinfer``).

Every decode step attends each request's whole KV history in the device token
pool.  bf16 with 4 KV heads x 128 runs one C call (``qq_dense_forward_decode``:
the new K/V store, then the attention kernel of the Quest layer step over all
of a request's rows); other shapes store the new K/V and run the split-K
attention over the explicit row list ``req_to_token[req, :seq_len]``.
"""

from __future__ import annotations

from typing import TYPE_CHECKING

import torch

from qwenquest_amd import _lib
from qwenquest_amd.attention.base import AttentionBackend
from qwenquest_amd.attention.ops import AttentionWorkspace, decode_attention_rows

if TYPE_CHECKING:
    from qwenquest_amd.batch import ForwardBatch
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

__all__ = ["DenseBackend"]


class DenseBackend(AttentionBackend):
    name = "flashinfer"

    def __init__(self, req_to_token_pool: ReqToTokenPool, token_to_kv_pool: MHATokenToKVPool):
        super().__init__(req_to_token_pool, token_to_kv_pool)
        device = token_to_kv_pool.device
        lib = _lib.load()
        # the attention's (request, KV head) counters: zeroed once, left zeroed by every call
        sync_bytes = int(lib.qq_quest_layer_step_sync_bytes(req_to_token_pool.size, token_to_kv_pool.kv_heads))
        self._sync = torch.zeros(max(sync_bytes, 4), dtype=torch.uint8, device=device)
        self._ws = torch.empty(0, dtype=torch.uint8, device=device)
        self._rows_ws = AttentionWorkspace(device)

    def _fast(self, q3: torch.Tensor) -> bool:
        pool = self.token_to_kv_pool
        heads = q3.shape[1]
        return (q3.dtype == torch.bfloat16 and pool.dtype == torch.bfloat16 and pool.kv_heads == 4
                and pool.head_dim == 128 and heads % 4 == 0 and heads // 4 <= 16)

    def forward_decode(self, q, k, v, layer, batch: ForwardBatch) -> torch.Tensor:
        """dense.py:26-42: set_kv_buffer, then attention over req_to_token[req, :seq_len]."""
        assert batch.out_cache_loc is not None
        pool = self.token_to_kv_pool
        bs = batch.batch_size
        dim = pool.head_dim
        q3 = q.reshape(bs, -1, dim)
        heads = q3.shape[1]
        rpi = batch.req_pool_indices.to(device=q3.device, dtype=torch.int64).contiguous()
        seq = batch.seq_lens.to(device=q3.device, dtype=torch.int64).contiguous()
        k_buf, v_buf = pool.get_kv_buffer(layer.layer_id)
        r2t = self.req_to_token
        if not self._fast(q3):
            pool.set_kv_buffer(layer.layer_id, batch.out_cache_loc, k, v)
            n_max = r2t.shape[1]
            rows = r2t[rpi].to(torch.int64)  # [bs, max_ctx]: the first seq_len entries are attended
            actual = seq.clamp(max=n_max).to(torch.int32)
            return decode_attention_rows(q3, k_buf, v_buf, rows, actual, float(layer.scaling),
                                         workspace=self._rows_ws)
        q3 = q3.contiguous()
        kn = k.reshape(bs, pool.kv_heads * dim).to(torch.bfloat16).contiguous()
        vn = v.reshape(bs, pool.kv_heads * dim).to(torch.bfloat16).contiguous()
        loc = batch.out_cache_loc.to(device=q3.device, dtype=torch.int64).contiguous()
        need = int(_lib.load().qq_dense_decode_workspace_bytes(bs, r2t.shape[1], heads, pool.kv_heads))
        if self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=q3.device)
        out = torch.empty((bs, heads * dim), dtype=q3.dtype, device=q3.device)
        _lib.call(
            "qq_dense_forward_decode", _lib.ptr(q3), _lib.dtype_code(q3.dtype), q3.stride(0), heads,
            _lib.ptr(kn), _lib.ptr(vn), _lib.dtype_code(kn.dtype), _lib.ptr(loc), _lib.ptr(k_buf),
            _lib.ptr(v_buf), _lib.dtype_code(k_buf.dtype), k_buf.shape[0], pool.kv_heads, dim, _lib.ptr(rpi),
            _lib.ptr(seq), bs, _lib.ptr(r2t), r2t.stride(0), r2t.shape[0], float(layer.scaling), _lib.ptr(out),
            _lib.ptr(self._ws) if need else None, need, _lib.ptr(self._sync), self._sync.numel(),
            _lib.stream(q3.device),
        )
        return out
