"""numpy restatement of ``decode_attention`` (reference ``src/qwenquest/attention/ops.py:48-66``).

Test infrastructure only.  Computed in float64 (the reference computes in
float32); HIP results are compared within a tolerance, never bit-exactly.
"""

from __future__ import annotations

import numpy as np


def decode_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scaling: float) -> np.ndarray:
    """One query ``[H, D]`` against the listed rows ``k, v [n, KV, D]`` -> ``[H*D]`` float64.

    Query head ``h`` reads KV head ``h // (H // KV)``; rows are attended exactly as
    listed, so a row given twice is counted twice (ops.py:3-7).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    heads, dim = q.shape
    kv = k.shape[1]
    qg = q.reshape(kv, heads // kv, dim)
    s = np.einsum("hgd,nhd->hgn", qg, k) * scaling
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("hgn,nhd->hgd", p, v).reshape(heads * dim)


def sparse_decode(q, k_buf, v_buf, rows_per_req, scaling: float) -> np.ndarray:
    """forward_decode's per-request loop (quest_only.py:153-159): ``[bs, H*D]`` float64."""
    return np.stack(
        [decode_attention(q[i], k_buf[r], v_buf[r], scaling) for i, r in enumerate(rows_per_req)]
    )
