"""DenseBackend (reference ``src/qwenquest/attention/dense.py:26-42``): every decode step
attends each request's whole history ``req_to_token[req, :seq_len]``.  Compared with the
float64 oracle of ``decode_attention`` (ops.py:48-66) over the same rows, within attn_tol (2e-2 at most)
(bf16); the new tokens' K/V must land in the pool (memory.py:114-120)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import bf16
from tests.conftest import assert_attn_close, bf16_bits

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def rand_bf16(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


class Layer:
    def __init__(self, i, d):
        self.layer_id, self.scaling = i, d**-0.5


def run_dense(H, KV, D, dtype, ctx, prompts, steps, layers, seed):
    from qwenquest_amd.attention.dense import DenseBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    nreq = len(prompts)
    rtp = ReqToTokenPool(nreq, ctx, DEV)
    kvp = MHATokenToKVPool(nreq * ctx, layers, KV, D, dtype, DEV)
    gen = np.random.default_rng(seed)
    r2t = (gen.permutation(nreq * ctx) + 1).astype(np.int32).reshape(nreq, ctx)  # scattered rows
    rtp.req_to_token.copy_(torch.from_numpy(r2t).to(DEV))
    kk = rand_bf16((layers, nreq * ctx + 1, KV, D), seed + 1)
    vv = rand_bf16((layers, nreq * ctx + 1, KV, D), seed + 2)
    for r, n in enumerate(prompts):  # the prompts' K/V in the pool; decoded tokens arrive by forward_decode
        rows = torch.from_numpy(r2t[r, :n].astype(np.int64))
        kvp.k_all[:, rows] = kk[:, rows].to(DEV).to(dtype)
        kvp.v_all[:, rows] = vv[:, rows].to(DEV).to(dtype)
    kb = bf16.to_f32(bf16_bits(kk))
    vb = bf16.to_f32(bf16_bits(vv))
    be = DenseBackend(rtp, kvp)
    for step in range(steps):
        seqs = [n + step + 1 for n in prompts]
        locs = torch.tensor([int(r2t[r, s - 1]) for r, s in enumerate(seqs)], device=DEV)
        batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.arange(nreq, device=DEV),
                             torch.tensor(seqs, device=DEV), locs, rtp, kvp, be)
        be.init_forward_metadata(batch)
        q = rand_bf16((nreq, H, D), seed + 100 + step)
        lc = locs.cpu()
        for layer in range(layers):
            out = be.forward_decode(q.to(DEV).to(dtype), kk[layer, lc].to(DEV).to(dtype),
                                    vv[layer, lc].to(DEV).to(dtype), Layer(layer, D), batch)
            rows = [r2t[r, :s].astype(np.int64) for r, s in enumerate(seqs)]
            ref = oa.sparse_decode(q.float().numpy(), kb[layer], vb[layer], rows, D**-0.5)
            assert_attn_close(out.float().cpu().numpy(), ref, f"step {step} layer {layer}")
        assert torch.equal(kvp.k_all[:, lc].cpu().to(torch.bfloat16), kk[:, lc])
    return be


def test_dense_backend_ragged_scattered():
    """bf16, 32 q / 4 KV heads x 128: ragged contexts 1 … 9100 tokens over scattered pool
    rows, 3 decode steps x 2 layers, through qq_dense_forward_decode; counters left at 0."""
    be = run_dense(32, 4, 128, torch.bfloat16, 9300, [9100, 700, 1, 4095, 4096], 3, 2, 5)
    assert not be._sync.any()


def test_dense_backend_other_shape():
    """16 q / 2 KV heads x 64 (outside the dense kernel): the new K/V store and the
    split-K attention over the row list req_to_token[req, :seq_len]."""
    run_dense(16, 2, 64, torch.bfloat16, 3000, [2900, 40, 1500], 2, 1, 7)


def test_dense_backend_full_context():
    """One request at 131072 tokens (33 parts of 4096 rows per KV head, merged in two
    passes) and one at 70001, one layer, one step."""
    be = run_dense(32, 4, 128, torch.bfloat16, 131072 + 64, [131071, 70000], 1, 1, 9)
    assert not be._sync.any()
