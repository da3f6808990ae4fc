"""Pin the numpy decode-attention oracle against torch SDPA on the expanded rows."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import attention as oa


def sdpa_reference(q, k, v, scale):
    h, d = q.shape
    kv = k.shape[1]
    g = h // kv
    kk = k.repeat_interleave(g, dim=1).transpose(0, 1)  # [H, n, D]
    vv = v.repeat_interleave(g, dim=1).transpose(0, 1)
    out = F.scaled_dot_product_attention(q[:, None].double(), kk.double(), vv.double(), scale=scale)
    return out[:, 0].reshape(-1).numpy()


def test_decode_attention_matches_sdpa():
    gen = torch.Generator().manual_seed(0)
    for h, kv, d, n in [(32, 4, 128, 300), (8, 2, 16, 7), (4, 4, 32, 1)]:
        q = torch.randn(h, d, generator=gen)
        k = torch.randn(n, kv, d, generator=gen)
        v = torch.randn(n, kv, d, generator=gen)
        got = oa.decode_attention(q.numpy(), k.numpy(), v.numpy(), d**-0.5)
        assert np.allclose(got, sdpa_reference(q, k, v, d**-0.5), atol=1e-12)


def test_duplicate_rows_are_counted_twice():
    gen = torch.Generator().manual_seed(1)
    q = torch.randn(4, 8, generator=gen).numpy()
    k = torch.randn(3, 2, 8, generator=gen).numpy()
    v = torch.randn(3, 2, 8, generator=gen).numpy()
    dup = oa.decode_attention(q, k[[0, 1, 2, 2]], v[[0, 1, 2, 2]], 0.3)
    single = oa.decode_attention(q, k, v, 0.3)
    assert not np.allclose(dup, single)
    # counting row 2 twice == adding log(2) to its logit
    qg = q.reshape(2, 2, 8)
    s = np.einsum("hgd,nhd->hgn", qg, k) * 0.3
    s[..., 2] += np.log(2.0)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    assert np.allclose(dup, np.einsum("hgn,nhd->hgd", p, v).reshape(-1), atol=1e-12)
