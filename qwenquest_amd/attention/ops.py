"""Attention math (reference ``src/qwenquest/attention/ops.py``).

``decode_attention`` runs the HIP split-K kernel over an explicit row list;
``extend_attention`` (dense causal prefill) is outside the accelerated path and
uses torch's SDPA on the device, in float32.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from qwenquest_amd import _lib

__all__ = ["decode_attention", "extend_attention", "AttentionWorkspace"]


class AttentionWorkspace:
    """Device workspace of the split-K attention kernels (per-chunk (m, l, o) partials)."""

    def __init__(self, device: torch.device):
        self.device = device
        self.buf = torch.empty(0, dtype=torch.uint8, device=device)

    def get(self, bs: int, max_rows: int, heads: int, head_dim: int) -> torch.Tensor:
        need = int(_lib.load().qq_decode_attention_workspace_bytes(bs, max_rows, heads, head_dim))
        if self.buf.numel() < need:
            self.buf = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self.buf


_workspaces: dict[torch.device, AttentionWorkspace] = {}


def _workspace(device: torch.device) -> AttentionWorkspace:
    ws = _workspaces.get(device)
    if ws is None:
        ws = _workspaces[device] = AttentionWorkspace(device)
    return ws


def decode_attention_rows(
    q: torch.Tensor,
    k_buf: torch.Tensor,
    v_buf: torch.Tensor,
    rows: torch.Tensor,
    actual_lens: torch.Tensor,
    scaling: float,
    *,
    workspace: AttentionWorkspace | None = None,
    out: torch.Tensor | None = None,
    sync: torch.Tensor | None = None,
) -> torch.Tensor:
    """Batched form: request ``i`` attends ``q[i] [H, D]`` over ``k_buf[rows[i, :actual_lens[i]]]``.

    ``rows`` ``[bs, >= max(actual_lens)]`` int64, ``k_buf``/``v_buf`` ``[rows, KV, D]``.
    Returns ``[bs, H*D]`` in q's dtype.  With ``sync`` (a zeroed uint8 buffer of at least
    ``qq_quest_layer_step_sync_bytes`` bytes) the bf16 KV*D = 4*128 shapes run the attention
    kernel of the fused Quest layer step, whose arithmetic QuestHiSparseBackend shares with
    QuestOnlyBackend.
    """
    bs, heads, dim = q.shape
    kv = k_buf.shape[1]
    q = q.contiguous()
    rows = rows.to(torch.int64).contiguous()
    actual = actual_lens.to(device=q.device, dtype=torch.int32).contiguous()
    ws = workspace or _workspace(q.device)
    buf = ws.get(bs, rows.shape[1], heads, dim)
    res = out if out is not None else torch.empty((bs, heads * dim), dtype=q.dtype, device=q.device)
    _lib.call(
        "qq_decode_attention_rows", _lib.ptr(q), _lib.dtype_code(q.dtype), q.stride(0), heads,
        _lib.ptr(k_buf), _lib.ptr(v_buf), _lib.dtype_code(k_buf.dtype), k_buf.shape[0], kv, dim,
        _lib.ptr(rows), rows.stride(0), _lib.ptr(actual), bs, float(scaling), _lib.ptr(res),
        _lib.ptr(buf), buf.numel(), _lib.ptr(sync) if sync is not None else None,
        sync.numel() if sync is not None else 0, _lib.stream(q.device),
    )
    return res


def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scaling: float) -> torch.Tensor:
    """One query ``[H, D]`` against the listed rows ``k, v [n, KV, D]`` -> ``[H*D]``
    (reference ops.py:48-66; duplicates counted, fp32 softmax and accumulation)."""
    n = k.shape[0]
    k = k.to(v.dtype).contiguous()
    v = v.contiguous()
    rows = torch.arange(n, dtype=torch.int64, device=q.device).unsqueeze(0)
    actual = torch.full((1,), n, dtype=torch.int32, device=q.device)
    return decode_attention_rows(q.unsqueeze(0), k, v, rows, actual, scaling)[0]


def extend_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, prefix_len: int, scaling: float) -> torch.Tensor:
    """Dense causal prefill of one request (reference ops.py:18-45), torch SDPA in float32."""
    n, num_heads, head_dim = q.shape
    kv_len, kv_heads, _ = k.shape
    group = num_heads // kv_heads
    qh = q.float().transpose(0, 1).unsqueeze(0)
    kh = k.float().repeat_interleave(group, dim=1).transpose(0, 1).unsqueeze(0).contiguous()
    vh = v.float().repeat_interleave(group, dim=1).transpose(0, 1).unsqueeze(0).contiguous()
    q_pos = prefix_len + torch.arange(n, device=q.device)
    mask = torch.arange(kv_len, device=q.device).unsqueeze(0) <= q_pos.unsqueeze(1)
    out = F.scaled_dot_product_attention(qh.contiguous(), kh, vh, attn_mask=mask, scale=scaling)
    return out[0].transpose(0, 1).reshape(n, num_heads * head_dim).to(q.dtype)
