"""Row sensitivity of the attention kernels: every attended slot counts.

A large value planted in one attended row's V (one KV head, one channel) must move the
output of that head's queries by the row's softmax weight - the oracle's attention over the
same rows with the same planted value is the reference, within the scaled bf16 tolerance of
tests.conftest.attn_tol, and the planted value is chosen so that the move is far above it.
Slots are picked at the kernels' seams: the first and last slot, 16-row step, wave and part
boundaries, the first recent-window slot and the newest token (whose V arrives through the
call itself), and for dense decode the part (4096-row) and merge-group (8-part) boundaries.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import bf16
from tests.conftest import assert_attn_close, bf16_bits

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
H, KV, D = 32, 4, 128
PLANT = 4096.0


class Layer:
    layer_id, scaling = 0, D**-0.5


def _pool(nreq, ctx, seed):
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    rtp = ReqToTokenPool(nreq, ctx, DEV)
    kvp = MHATokenToKVPool(nreq * ctx, 1, KV, D, torch.bfloat16, DEV)
    g = torch.Generator(device=DEV).manual_seed(seed)
    kvp.k_all.normal_(generator=g)
    kvp.v_all.normal_(generator=g)
    perm = torch.randperm(nreq * ctx, generator=torch.Generator().manual_seed(seed)) + 1
    rtp.req_to_token.copy_(perm.view(nreq, ctx).to(torch.int32).to(DEV))
    return rtp, kvp


def _check_planted(run, rows_of, kvp, new_v, new_rows, reqs_slots, q):
    """run(v_new) -> output [bs, H*D] bf16.  For each (request, slot): plant PLANT into the
    V of the slot's row (KV head slot % KV, one channel), run, and compare with the oracle
    over the same rows.  The planted channel of that head's queries moves by PLANT x the
    row's softmax weight (far above the error bound, which is relative there: bf16 rounds
    the output to 2^-9); every other output element is held to attn_tol."""
    G = H // KV
    base_v = kvp.v_all[0].clone()
    kb = bf16.to_f32(bf16_bits(kvp.k_all[0].cpu()))
    new_rows = new_rows.cpu().numpy()
    qn = q.float().cpu().numpy()
    for i, slot in reqs_slots:
        rows = rows_of()
        row = int(rows[i][slot])
        h, c = slot % KV, (slot * 37) % D
        vn = new_v.clone()
        if row == int(new_rows[i]):  # the newest token's V comes in through the call
            vn[i, h, c] = PLANT
        else:
            kvp.v_all[0, row, h, c] = PLANT
        out = run(vn).float().cpu().numpy()
        kvp.v_all[0].copy_(base_v)
        vb = bf16.to_f32(bf16_bits(kvp.v_all[0].cpu()))
        plain_vb = vb.copy()
        keep = new_rows >= 0
        vb[new_rows[keep]] = bf16.to_f32(bf16_bits(vn.cpu()))[keep]
        plain_vb[new_rows[keep]] = bf16.to_f32(bf16_bits(new_v.cpu()))[keep]
        vb[row, h, c] = PLANT
        ref = oa.sparse_decode(qn, kb, vb, rows, D**-0.5)
        plain = oa.sparse_decode(qn, kb, plain_vb, rows, D**-0.5)
        sel = np.zeros((len(rows), H, D), dtype=bool)
        sel[i, h * G:(h + 1) * G, c] = True
        sel = sel.reshape(len(rows), H * D)
        moved = np.abs(ref - plain)[sel]
        assert moved.max() > 0.05, f"slot {slot}: the planted value barely moves the output"
        err = np.abs(out - ref)[sel]
        bound = 2e-3 + 8e-3 * np.abs(ref[sel])
        assert np.all(err <= bound), (
            f"request {i} slot {slot} (row {row}, head {h}, channel {c}): planted channel off by "
            f"{err.max():.3e} (moved {moved.max():.3e})")
        assert_attn_close(out[~sel], ref[~sel], f"request {i} slot {slot}: other outputs")


def test_quest_fused_step_every_slot_counts():
    """QuestOnlyBackend.forward_decode (the fused layer step): a request with the dense
    layout (2048 real slots) and one with 31 selected pages + the recent window."""
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode

    CTX, TOP_K = 9100, 2048
    prompts = [2047, 8999]
    rtp, kvp = _pool(2, CTX, 11)
    be = QuestOnlyBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": 64})
    for r, n in enumerate(prompts):
        be.quest.update_prefill_representations_fused(r, kvp.k_all, rtp.req_to_token[r, :n])
        be._skip_first_decode_update[r] = True
    seqs = [n + 1 for n in prompts]
    r2t = rtp.req_to_token.cpu().numpy()
    locs = torch.tensor([int(r2t[r, s - 1]) for r, s in enumerate(seqs)], device=DEV)
    batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.arange(2, device=DEV),
                         torch.tensor(seqs, device=DEV), locs, rtp, kvp, be)
    be.init_forward_metadata(batch)
    g = torch.Generator(device=DEV).manual_seed(3)
    q = torch.randn((2, H, D), generator=g, device=DEV).to(torch.bfloat16)
    kn = torch.randn((2, KV, D), generator=g, device=DEV).to(torch.bfloat16)
    vn = torch.randn((2, KV, D), generator=g, device=DEV).to(torch.bfloat16)

    def run(v_new):
        return be.forward_decode(q, kn, v_new, Layer(), batch)

    run(vn)
    torch.cuda.synchronize()
    pos = be._positions[:2].cpu().numpy()

    def rows_of():
        return [r2t[r, pos[r, : min(s, TOP_K)]].astype(np.int64) for r, s in enumerate(seqs)]

    seams = [0, 15, 16, 63, 64, 255, 256, 511, 512, 1023, 1024, 1983, 1984, 2046, 2047]
    _check_planted(run, rows_of, kvp, vn, locs, [(i, s) for i in (0, 1) for s in seams], q)


def test_rows_attention_every_slot_counts():
    """decode_attention_rows with the sync buffer (quest_hisparse's attention over its
    hot-buffer rows: the fused step's kernel), ragged lengths."""
    from qwenquest_amd import _lib
    from qwenquest_amd.attention.ops import decode_attention_rows

    rtp, kvp = _pool(1, 6000, 17)
    lens = [2048, 1000]
    g = torch.Generator().manual_seed(4)
    rows = torch.randint(1, 6000, (2, 2048), generator=g, dtype=torch.int64)
    q = torch.randn((2, H, D), generator=torch.Generator(device=DEV).manual_seed(5), device=DEV).to(torch.bfloat16)
    sync = torch.zeros(int(_lib.load().qq_quest_layer_step_sync_bytes(2, KV)), dtype=torch.uint8, device=DEV)
    actual = torch.tensor(lens, dtype=torch.int32, device=DEV)
    no_new = torch.zeros((2, KV, D), dtype=torch.bfloat16, device=DEV)
    none_rows = torch.tensor([-1, -1])

    def run(_):
        return decode_attention_rows(q, kvp.k_buffer[0], kvp.v_buffer[0], rows.to(DEV), actual, D**-0.5, sync=sync)

    def rows_of():
        return [rows[i, :n].numpy() for i, n in enumerate(lens)]

    # distinct rows within and across the requests (a shared row would carry the planted value
    # into another output)
    perm = torch.randperm(5999, generator=g) + 1
    rows[0, : lens[0]] = perm[: lens[0]]
    rows[1, : lens[1]] = perm[lens[0]: lens[0] + lens[1]]
    seams = [(0, s) for s in (0, 16, 255, 256, 1024, 2047)] + [(1, s) for s in (0, 511, 999)]
    _check_planted(run, rows_of, kvp, no_new, none_rows, seams, q)


def test_dense_decode_every_part_counts():
    """DenseBackend: one 40000-token request = 10 parts of 4096 rows, merged in two passes
    (groups of 8 parts): part and group boundaries, the first and the newest row."""
    from qwenquest_amd.attention.dense import DenseBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode

    S = 40000
    rtp, kvp = _pool(1, S + 64, 23)
    be = DenseBackend(rtp, kvp)
    r2t = rtp.req_to_token.cpu().numpy()
    locs = torch.tensor([int(r2t[0, S - 1])], device=DEV)
    batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.zeros(1, dtype=torch.int64, device=DEV),
                         torch.tensor([S], device=DEV), locs, rtp, kvp, be)
    g = torch.Generator(device=DEV).manual_seed(6)
    q = torch.randn((1, H, D), generator=g, device=DEV).to(torch.bfloat16)
    kn = torch.randn((1, KV, D), generator=g, device=DEV).to(torch.bfloat16)
    vn = torch.randn((1, KV, D), generator=g, device=DEV).to(torch.bfloat16)

    def run(v_new):
        return be.forward_decode(q, kn, v_new, Layer(), batch)

    def rows_of():
        return [r2t[0, :S].astype(np.int64)]

    run(vn)
    seams = [0, 4095, 4096, 8191, 8192, 32767, 32768, 36863, 36864, S - 1]
    _check_planted(run, rows_of, kvp, vn, locs, [(0, s) for s in seams], q)
