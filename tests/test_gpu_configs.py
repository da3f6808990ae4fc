"""Parity at the path's own full-size configurations (Qwen3-30B-A3B shapes: 32 q / 4 KV
heads x 128, bf16, page 64, top_k 2048 = 31 selected pages + the recent 64):

* batch 8 x 32768 tokens, keys N(0,1) plus a per-(request, page) mean offset N(0, 0.5);
* a 48-layer ragged sweep, batch 16, contexts uniform in [8192, 131072], 64 decode steps
  (every step appends one token per request; pages complete and are finalized);
* batch 4 x 262144 tokens, 4 outlier channels per KV head scaled x10, 256 decode steps,
  both overlap modes, quest and quest_hisparse.

Inputs are generated on the device from fixed seeds and copied to the host for the
oracle; positions are compared bit for bit, attention within the bf16 tolerance of tests.conftest.attn_tol.  The
48-layer sweep checks the prefill bounds of every (layer, request) on the device against the
min / max of its K rows (exact operations) and starts the oracle from them, so that the oracle
follows every pair without copying the whole K pool to the host.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import bf16
from oracle import quest as oq
from tests.conftest import assert_attn_close, bf16_bits

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
H, KV, D, P, TOP_K = 32, 4, 128, 64, 2048
SCALE = D**-0.5


class Layer:
    def __init__(self, i):
        self.layer_id, self.scaling = i, SCALE


def dev_randn(shape, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(shape, generator=g, device=DEV, dtype=torch.float32)


def oracle_attention(q_row, k_rows, v_rows):
    """q_row [H, D] bf16, k_rows / v_rows [n, KV, D] bf16 (CPU) -> [H*D] float32."""
    kb = bf16.to_f32(bf16_bits(k_rows))
    vb = bf16.to_f32(bf16_bits(v_rows))
    return oa.decode_attention(q_row.float().numpy(), kb, vb, SCALE).reshape(-1)


def make_quest_backend(B, ctx, L, avoid=False, hisparse=False):
    from qwenquest_amd.attention.quest_hisparse import QuestHiSparseBackend
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    rtp = ReqToTokenPool(B, ctx, DEV)
    kvp = MHATokenToKVPool(B * ctx, L, KV, D, torch.bfloat16, DEV)
    cfg = {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P, "avoid_recent_overlap": avoid}
    if hisparse:
        be = QuestHiSparseBackend(rtp, kvp, cfg, host_pool_size=B * ctx)
    else:
        be = QuestOnlyBackend(rtp, kvp, cfg)
    base = 1 + torch.arange(B, device=DEV, dtype=torch.int64) * ctx
    rtp.req_to_token.copy_((base[:, None] + torch.arange(ctx, device=DEV)[None]).to(torch.int32))
    return rtp, kvp, be, base


def test_batch8_32k_per_page_offsets():
    """Batch 8 x 32768 tokens, one layer, 4 decode steps through QuestOnlyBackend (fused
    two-launch step): positions bit-exact vs the oracle, attention within attn_tol."""
    from qwenquest_amd.batch import ForwardBatch, ForwardMode

    B, S, steps = 8, 32768, 4
    ctx = S + steps + 64
    rtp, kvp, be, base = make_quest_backend(B, ctx, 1)
    # k = N(0,1) + mu[request, page], mu ~ N(0, 0.5); row 1 + r*ctx + p holds position p
    mu = dev_randn((B, (ctx + P - 1) // P), 11) * 0.5
    rows_pos = torch.arange(ctx, device=DEV)
    k = dev_randn((B, ctx, KV, D), 12) + mu[:, rows_pos // P][:, :, None, None]
    kvp.k_all[0, 1:].copy_(k.reshape(B * ctx, KV, D).to(torch.bfloat16))
    kvp.v_all[0, 1:].copy_(dev_randn((B * ctx, KV, D), 13).to(torch.bfloat16))
    del k
    prompt = S - 1
    for r in range(B):
        be.quest.update_prefill_representations_fused(r, kvp.k_all, rtp.req_to_token[r, :prompt])
        be._skip_first_decode_update[r] = True
    kk, vv = kvp.k_all[0].cpu(), kvp.v_all[0].cpu()
    kbits = bf16_bits(kk)
    st = oq.QuestState(TOP_K, P)
    st.init_storage(0, 1, B, ctx, KV, D)
    for r in range(B):
        st.update_prefill_representations(0, r, kbits, (1 + r * ctx + np.arange(prompt)))
    reqs = list(range(B))
    for step in range(steps):
        seq = torch.full((B,), S + step, device=DEV, dtype=torch.int64)
        loc = base + seq - 1
        batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.arange(B, device=DEV), seq, loc, rtp, kvp, be)
        be.init_forward_metadata(batch)
        if step > 0:
            st.update_decode_representations(0, reqs, kbits, (loc - 1).cpu().numpy())
            st.maybe_finalize_decode_representations(reqs)
        st.prepare_step(seq.cpu().numpy())
        q = dev_randn((B, H, D), 100 + step).to(torch.bfloat16)
        lc = loc.cpu()
        out = be.forward_decode(q, kk[lc].to(DEV), vv[lc].to(DEV), Layer(0), batch).float().cpu().numpy()
        pos = be._positions[:B].cpu().numpy()
        ref_pos, ref_actual, _ = st.retrieve_topk(q.float().cpu().numpy(), 0, reqs)
        qc = q.cpu()
        for i in range(B):
            n = int(ref_actual[i])
            assert n == TOP_K
            assert np.array_equal(pos[i, :n], ref_pos[i, :n]), f"step {step} request {i}"
            rows = torch.from_numpy(1 + i * ctx + ref_pos[i, :n].astype(np.int64))
            ref = oracle_attention(qc[i], kk[rows], vv[rows])
            assert_attn_close(out[i], ref, f"step {step} request {i}")


SENT_MIN = int(np.array([bf16.BF16_MAX_BITS], dtype=np.uint16).view(np.int16)[0])  # unset page minimum
SENT_MAX = int(np.array([bf16.BF16_MIN_BITS], dtype=np.uint16).view(np.int16)[0])  # unset page maximum


def check_prefill_state_on_device(qs, k_all, starts, prompts):
    """The backend's bounds after the prefill against their definition (quest.py:231-280),
    on the device for every (layer, request): each complete page's (min, max) over its 64 K
    rows, the partial page's running (min, max), the unset sentinels everywhere else, and the
    page / token counters.  min and max are exact, so the comparison is bit for bit."""
    L = qs.page_k_bounds.shape[0]
    for r, n in enumerate(prompts):
        full, part = divmod(int(n), P)
        assert int(qs.running_page_idx[r]) == full and int(qs.running_token_count[r]) == part, f"request {r}"
        for layer in range(L):
            rows = k_all[layer, int(starts[r]) : int(starts[r]) + int(n)]
            paged = rows[: full * P].view(full, P, KV, D)
            pkb = qs.page_k_bounds[layer, r].view(torch.int16)
            rmin = qs.running_k_min[layer, r].view(torch.int16)
            rmax = qs.running_k_max[layer, r].view(torch.int16)
            what = f"layer {layer} request {r}"
            assert torch.equal(pkb[:full, ..., 0], paged.amin(1).view(torch.int16)), what
            assert torch.equal(pkb[:full, ..., 1], paged.amax(1).view(torch.int16)), what
            assert bool((pkb[full:, ..., 0] == SENT_MIN).all()) and bool((pkb[full:, ..., 1] == SENT_MAX).all()), what
            if part:
                assert torch.equal(rmin, rows[full * P :].amin(0).view(torch.int16)), what
                assert torch.equal(rmax, rows[full * P :].amax(0).view(torch.int16)), what
            else:
                assert bool((rmin == SENT_MIN).all()) and bool((rmax == SENT_MAX).all()), what


def test_ragged_48_layer_sweep_every_pair():
    """48 layers, batch 16, contexts uniform in [8192, 131072] (seeded), 64 decode steps with
    one append per request per step, all layers through QuestOnlyBackend.  After the prefill,
    every (layer, request)'s bounds are checked on the device against the min / max of its own
    K rows; the oracle then starts from that state and follows all 768 (layer, request) pairs
    itself: every step's new K / V rows in the pool bit-exact for every pair; positions
    bit-exact for every pair at steps 0, 16, 31, 47 and 63, and for 19 sampled pairs (every
    request in one layer, the longest and the shortest request, request 5 in layer 47) at every
    step; attention within attn_tol for every pair at those five steps and for the sampled
    pairs at steps 1 and 62; after the last step every pair's page bounds, running bounds and the
    counters bit-exact (pages completed during the sweep included)."""
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    L, B, steps = 48, 16, 64
    gen = np.random.default_rng(2024)
    ctxs = gen.integers(8192, 131072, size=B, endpoint=True)
    ctx = int(ctxs.max()) + steps + 64
    # request r's rows are packed after r-1's: its context plus room for the decode steps
    span = ctxs + steps + 64
    starts = 1 + np.concatenate([[0], np.cumsum(span)[:-1]])
    pool = int(span.sum())
    rtp = ReqToTokenPool(B, ctx, DEV)
    kvp = MHATokenToKVPool(pool, L, KV, D, torch.bfloat16, DEV)
    be = QuestOnlyBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P})
    qs = be.quest
    base = torch.tensor(starts, device=DEV, dtype=torch.int64)
    rtp.req_to_token.copy_((base[:, None] + torch.arange(ctx, device=DEV)[None]).clamp(max=pool).to(torch.int32))
    for layer in range(L):
        kvp.k_all[layer].copy_(dev_randn((pool + 1, KV, D), 1000 + layer).to(torch.bfloat16))
        kvp.v_all[layer].copy_(dev_randn((pool + 1, KV, D), 2000 + layer).to(torch.bfloat16))
    prompts = [int(c) - 1 for c in ctxs]  # the first decode step has seq_len = ctxs[r]
    for r in range(B):
        qs.update_prefill_representations_fused(r, kvp.k_all, rtp.req_to_token[r, : prompts[r]])
        be._skip_first_decode_update[r] = True
    check_prefill_state_on_device(qs, kvp.k_all, starts, prompts)
    st = oq.QuestState(TOP_K, P)
    st.init_storage(0, L, B, ctx, KV, D)
    assert st.page_k_bounds.shape == tuple(qs.page_k_bounds.shape)
    for layer in range(L):
        st.page_k_bounds[layer] = bf16_bits(qs.page_k_bounds[layer])
    st.running_k_min[...] = bf16_bits(qs.running_k_min)
    st.running_k_max[...] = bf16_bits(qs.running_k_max)
    st.running_token_count[:] = qs.running_token_count.cpu().numpy()
    st.running_page_idx[:] = qs.running_page_idx.cpu().numpy()
    samples = sorted({(7 * r % L, r) for r in range(B)} | {(0, int(np.argmax(ctxs))), (23, int(np.argmin(ctxs))),
                                                          (47, 5)})
    every_pair_steps = {0, 16, 31, 47, 63}
    sampled_attention_steps = {1, 62}
    reqs = np.arange(B)
    seq = torch.tensor(ctxs, device=DEV, dtype=torch.int64)
    loc = torch.empty(B, device=DEV, dtype=torch.int64)
    batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.arange(B, device=DEV), seq, loc, rtp, kvp, be)
    for step in range(steps):
        torch.add(base, seq - 1, out=loc)
        be.init_forward_metadata(batch)
        kn = dev_randn((L, B, KV, D), 3000 + step).to(torch.bfloat16)
        vn = dev_randn((L, B, KV, D), 4000 + step).to(torch.bfloat16)
        q = dev_randn((L, B, H, D), 5000 + step).to(torch.bfloat16)
        seqs = seq.cpu().numpy()
        if step > 0:  # fold the previous decode token of every pair (checked in the pool last step)
            prev = bf16_bits(kvp.k_all[:, base + seq - 2])  # [L, B, KV, D]
            for layer in range(L):
                st.update_decode_representations(layer, reqs, prev[layer], reqs)
            st.maybe_finalize_decode_representations(reqs)
        st.prepare_step(seqs)
        every = step in every_pair_steps
        for layer in range(L):
            out = be.forward_decode(q[layer], kn[layer], vn[layer], Layer(layer), batch)
            mine = [r for (sl, r) in samples if sl == layer]
            if not every and not mine:
                continue
            pos = be._positions[:B].cpu().numpy()
            qf = q[layer].float().cpu().numpy()
            if every:
                ref_pos, ref_actual, _ = st.retrieve_topk(qf, layer, reqs)
                check = list(range(B))
            else:
                ref_pos = np.zeros((B, TOP_K), dtype=np.int32)
                ref_actual = np.zeros(B, dtype=np.int32)
                for r in mine:
                    lay = oq.step_layout(seqs[r : r + 1], P, TOP_K, False)
                    qbar = oq.group_queries(qf[r : r + 1], KV, D, True)
                    p1, a1, _ = oq.retrieve_topk(qbar, st.page_k_bounds[layer, [r]], lay, P, TOP_K)
                    ref_pos[r], ref_actual[r] = p1[0], a1[0]
                check = mine
            for r in check:
                n = int(ref_actual[r])
                assert n == TOP_K
                assert np.array_equal(pos[r, :n], ref_pos[r, :n]), f"step {step} layer {layer} request {r}"
            attend = check if every else (mine if step in sampled_attention_steps else [])
            if not attend:
                continue
            outs = out.float().cpu().numpy()
            rows = (base[attend][:, None] + torch.from_numpy(ref_pos[attend].astype(np.int64)).to(DEV))
            kr, vr = kvp.k_all[layer, rows].cpu(), kvp.v_all[layer, rows].cpu()
            qc = q[layer].cpu()
            for j, r in enumerate(attend):
                ref = oracle_attention(qc[r], kr[j], vr[j])
                assert_attn_close(outs[r], ref, f"step {step} layer {layer} request {r}")
        # the step's new token of every pair, as set_kv_buffer stored it (memory.py:114-120)
        assert torch.equal(kvp.k_all[:, loc].view(torch.int16), kn.view(torch.int16)), f"step {step}"
        assert torch.equal(kvp.v_all[:, loc].view(torch.int16), vn.view(torch.int16)), f"step {step}"
        seq.add_(1)
    torch.cuda.synchronize()
    for layer in range(L):
        assert np.array_equal(bf16_bits(qs.page_k_bounds[layer]), st.page_k_bounds[layer]), f"layer {layer}"
    assert np.array_equal(bf16_bits(qs.running_k_min), st.running_k_min)
    assert np.array_equal(bf16_bits(qs.running_k_max), st.running_k_max)
    assert np.array_equal(qs.running_page_idx.cpu().numpy(), st.running_page_idx)
    assert np.array_equal(qs.running_token_count.cpu().numpy(), st.running_token_count)
    del rtp, kvp, be, qs
    torch.cuda.empty_cache()


@pytest.mark.parametrize("avoid", [False, True])
def test_batch4_262k_outliers_quest_and_hisparse(avoid):
    """Batch 4 x 262144 tokens (4096+ pages), keys N(0,1) with 4 seeded outlier channels per
    KV head x10, 256 decode steps in one overlap mode: QuestOnlyBackend and
    QuestHiSparseBackend give bit-identical positions and outputs at every step; positions
    bit-exact vs the oracle on sampled steps, attention within attn_tol."""
    from qwenquest_amd.batch import ForwardBatch, ForwardMode

    B, S, steps = 4, 262144, 256
    ctx = S + steps + 64
    gen = torch.Generator().manual_seed(77)
    outl = torch.stack([torch.randperm(D, generator=gen)[:4] for _ in range(KV)])  # [KV, 4]
    scale = torch.ones(KV, D)
    scale[torch.arange(KV)[:, None], outl] = 10.0
    k = (dev_randn((B * ctx + 1, KV, D), 21) * scale.to(DEV)).to(torch.bfloat16)
    v = dev_randn((B * ctx + 1, KV, D), 22).to(torch.bfloat16)
    qs = dev_randn((steps, B, H, D), 23).to(torch.bfloat16)
    prompt = S - 1
    kk, vv = k.cpu(), v.cpu()
    kbits = bf16_bits(kk)
    st = oq.QuestState(TOP_K, P, avoid_recent_overlap=avoid)
    st.init_storage(0, 1, B, ctx, KV, D)
    for r in range(B):
        st.update_prefill_representations(0, r, kbits, 1 + r * ctx + np.arange(prompt))
    check_steps = set(range(0, steps, 16)) | {steps - 1}
    attn_steps = {0, 64, 255}
    reqs = list(range(B))
    results = {}
    for mode in ("quest", "quest_hisparse"):
        rtp, kvp, be, base = make_quest_backend(B, ctx, 1, avoid=avoid, hisparse=mode == "quest_hisparse")
        kvp.k_all[0].copy_(k)
        kvp.v_all[0].copy_(v)
        pre = ForwardBatch(ForwardMode.EXTEND, None, None, torch.arange(B), torch.full((B,), prompt), None,
                           rtp, kvp, be)
        if mode == "quest":
            be._update_quest_for_extend(pre)
        else:
            be.on_extend_finished(pre)
        outs, poss = [], []
        for step in range(steps):
            seq = torch.full((B,), S + step, device=DEV, dtype=torch.int64)
            loc = base + seq - 1
            batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.arange(B, device=DEV), seq,
                                 loc if mode == "quest" else None, rtp, kvp, be)
            be.init_forward_metadata(batch)
            out = be.forward_decode(qs[step], k[loc], v[loc], Layer(0), batch)
            outs.append(out.cpu())
            poss.append(be._positions[:B].cpu())
        results[mode] = (torch.stack(outs), torch.stack(poss))
        if mode == "quest_hisparse":
            s = be.coord.stats
            assert s.misses > 0 and s.hits > 0
        del rtp, kvp, be
        torch.cuda.empty_cache()
    assert torch.equal(results["quest"][1], results["quest_hisparse"][1])
    assert torch.equal(results["quest"][0], results["quest_hisparse"][0])
    outs, poss = results["quest"]
    for step in range(steps):
        seqs = np.full(B, S + step)
        if step > 0:
            st.update_decode_representations(0, reqs, kbits, 1 + np.arange(B) * ctx + seqs - 2)
            st.maybe_finalize_decode_representations(reqs)
        st.prepare_step(seqs)
        if step not in check_steps:
            continue
        ref_pos, ref_actual, _ = st.retrieve_topk(qs[step].float().cpu().numpy(), 0, reqs)
        for i in range(B):
            n = int(ref_actual[i])
            assert np.array_equal(poss[step, i, :n].numpy(), ref_pos[i, :n]), f"step {step} request {i}"
            if step in attn_steps:
                rows = torch.from_numpy(1 + i * ctx + ref_pos[i, :n].astype(np.int64))
                ref = oracle_attention(qs[step, i].cpu(), kk[rows], vv[rows])
                assert_attn_close(outs[step, i].float().numpy(), ref, f"step {step} request {i}")


@pytest.mark.parametrize("S,fused", [(450000, True), (540000, False)])
def test_contexts_past_384k(S, fused):
    """Batch 2 x 450000 tokens (7032 pages: the fused step's widest selection form, 32
    scores per thread) and 2 x 540000 (8438 pages, past the 8192 the fused step selects
    from, so QuestOnlyBackend runs the four-launch path), 80 decode steps that complete a
    page: QuestOnlyBackend and QuestHiSparseBackend give bit-identical positions and outputs
    at every step; positions bit-exact vs the oracle on sampled steps, attention within
    attn_tol."""
    from qwenquest_amd import _lib
    from qwenquest_amd.batch import ForwardBatch, ForwardMode

    B, steps = 2, 80
    ctx = S + steps + 64
    assert _lib.load().qq_quest_fused_step(_lib.DTYPE_BF16, _lib.DTYPE_BF16, _lib.DTYPE_BF16, H, KV, D, P, TOP_K,
                                           (ctx + P - 1) // P) == int(fused)
    k = dev_randn((B * ctx + 1, KV, D), 31).to(torch.bfloat16)
    v = dev_randn((B * ctx + 1, KV, D), 32).to(torch.bfloat16)
    qs = dev_randn((steps, B, H, D), 33).to(torch.bfloat16)
    prompt = S - 1
    kk, vv = k.cpu(), v.cpu()
    kbits = bf16_bits(kk)
    st = oq.QuestState(TOP_K, P)
    st.init_storage(0, 1, B, ctx, KV, D)
    for r in range(B):
        st.update_prefill_representations(0, r, kbits, 1 + r * ctx + np.arange(prompt))
    check_steps = {0, 1, 2, 30, 63, 64, 65, 79}
    attn_steps = {0, 65, 79}
    reqs = list(range(B))
    results = {}
    for mode in ("quest", "quest_hisparse"):
        rtp, kvp, be, base = make_quest_backend(B, ctx, 1, hisparse=mode == "quest_hisparse")
        kvp.k_all[0].copy_(k)
        kvp.v_all[0].copy_(v)
        pre = ForwardBatch(ForwardMode.EXTEND, None, None, torch.arange(B), torch.full((B,), prompt), None,
                           rtp, kvp, be)
        if mode == "quest":
            be._update_quest_for_extend(pre)
        else:
            be.on_extend_finished(pre)
        outs, poss = [], []
        for step in range(steps):
            seq = torch.full((B,), S + step, device=DEV, dtype=torch.int64)
            loc = base + seq - 1
            batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.arange(B, device=DEV), seq,
                                 loc if mode == "quest" else None, rtp, kvp, be)
            be.init_forward_metadata(batch)
            out = be.forward_decode(qs[step], k[loc], v[loc], Layer(0), batch)
            outs.append(out.cpu())
            poss.append(be._positions[:B].cpu())
        results[mode] = (torch.stack(outs), torch.stack(poss))
        del rtp, kvp, be
        torch.cuda.empty_cache()
    assert torch.equal(results["quest"][1], results["quest_hisparse"][1])
    assert torch.equal(results["quest"][0], results["quest_hisparse"][0])
    outs, poss = results["quest"]
    for step in range(steps):
        seqs = np.full(B, S + step)
        if step > 0:
            st.update_decode_representations(0, reqs, kbits, 1 + np.arange(B) * ctx + seqs - 2)
            st.maybe_finalize_decode_representations(reqs)
        st.prepare_step(seqs)
        if step not in check_steps:
            continue
        ref_pos, ref_actual, _ = st.retrieve_topk(qs[step].float().cpu().numpy(), 0, reqs)
        for i in range(B):
            n = int(ref_actual[i])
            assert n == TOP_K
            assert np.array_equal(poss[step, i, :n].numpy(), ref_pos[i, :n]), f"step {step} request {i}"
            if step in attn_steps:
                rows = torch.from_numpy(1 + i * ctx + ref_pos[i, :n].astype(np.int64))
                ref = oracle_attention(qs[step, i].cpu(), kk[rows], vv[rows])
                assert_attn_close(outs[step, i].float().numpy(), ref, f"step {step} request {i}")


@pytest.mark.parametrize("B", [32, 64, 96, 128])
def test_larger_batches_units_one_after_another(B):
    """Batches past 16 requests: the fused attention's grid is one round of resident blocks
    (batch 32: 8-wave blocks, 2 parts per (request, KV head); 64: one part, 4 units per wave
    one after another, no partial merge; 96: 4-wave blocks, 2 parts; 128: 4-wave blocks, one
    part, 8 units per wave); positions bit-exact vs the oracle on every request, attention
    within attn_tol on every 7th, over 3 decode steps."""
    from qwenquest_amd.batch import ForwardBatch, ForwardMode

    S, steps = (8192 if B <= 64 else 4096), 3
    ctx = S + steps + 64
    rtp, kvp, be, base = make_quest_backend(B, ctx, 1)
    kvp.k_all[0].copy_(dev_randn((B * ctx + 1, KV, D), 31).to(torch.bfloat16))
    kvp.v_all[0].copy_(dev_randn((B * ctx + 1, KV, D), 32).to(torch.bfloat16))
    prompt = S - 1
    for r in range(B):
        be.quest.update_prefill_representations_fused(r, kvp.k_all, rtp.req_to_token[r, :prompt])
        be._skip_first_decode_update[r] = True
    kk, vv = kvp.k_all[0].cpu(), kvp.v_all[0].cpu()
    kbits = bf16_bits(kk)
    st = oq.QuestState(TOP_K, P)
    st.init_storage(0, 1, B, ctx, KV, D)
    for r in range(B):
        st.update_prefill_representations(0, r, kbits, 1 + r * ctx + np.arange(prompt))
    reqs = list(range(B))
    for step in range(steps):
        seq = torch.full((B,), S + step, device=DEV, dtype=torch.int64)
        loc = base + seq - 1
        batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.arange(B, device=DEV), seq, loc, rtp, kvp, be)
        be.init_forward_metadata(batch)
        if step > 0:
            st.update_decode_representations(0, reqs, kbits, (loc - 1).cpu().numpy())
            st.maybe_finalize_decode_representations(reqs)
        st.prepare_step(seq.cpu().numpy())
        q = dev_randn((B, H, D), 400 + step).to(torch.bfloat16)
        lc = loc.cpu()
        out = be.forward_decode(q, kk[lc].to(DEV), vv[lc].to(DEV), Layer(0), batch).float().cpu().numpy()
        pos = be._positions[:B].cpu().numpy()
        ref_pos, ref_actual, _ = st.retrieve_topk(q.float().cpu().numpy(), 0, reqs)
        qc = q.cpu()
        for i in range(0, B, 7):
            n = int(ref_actual[i])
            assert np.array_equal(pos[i, :n], ref_pos[i, :n]), f"step {step} request {i}"
            rows = torch.from_numpy(1 + i * ctx + ref_pos[i, :n].astype(np.int64))
            ref = oracle_attention(qc[i], kk[rows], vv[rows])
            assert_attn_close(out[i], ref, f"step {step} request {i}")
        assert np.array_equal(pos[:, :TOP_K], ref_pos[:, :TOP_K])


def test_batch128_quest_and_hisparse_bit_identical():
    """Batch 128 x 8192 tokens (4-wave blocks, one part per (request, KV head), 8 units per
    wave): QuestOnlyBackend and QuestHiSparseBackend (whose attention over its hot-buffer
    rows takes the same launch shape) give the same positions and output bits over 4
    decode steps, with misses in the hot buffer."""
    from qwenquest_amd.batch import ForwardBatch, ForwardMode

    B, S, steps = 128, 8192, 4
    ctx = S + steps + 64
    k = dev_randn((B * ctx + 1, KV, D), 41).to(torch.bfloat16)
    v = dev_randn((B * ctx + 1, KV, D), 42).to(torch.bfloat16)
    qs = dev_randn((steps, B, H, D), 43).to(torch.bfloat16)
    prompt = S - 1
    results = {}
    for mode in ("quest", "quest_hisparse"):
        rtp, kvp, be, base = make_quest_backend(B, ctx, 1, hisparse=mode == "quest_hisparse")
        kvp.k_all[0].copy_(k)
        kvp.v_all[0].copy_(v)
        pre = ForwardBatch(ForwardMode.EXTEND, None, None, torch.arange(B), torch.full((B,), prompt), None,
                           rtp, kvp, be)
        if mode == "quest":
            be._update_quest_for_extend(pre)
        else:
            be.on_extend_finished(pre)
        outs, poss = [], []
        for step in range(steps):
            seq = torch.full((B,), S + step, device=DEV, dtype=torch.int64)
            loc = base + seq - 1
            batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.arange(B, device=DEV), seq,
                                 loc if mode == "quest" else None, rtp, kvp, be)
            be.init_forward_metadata(batch)
            out = be.forward_decode(qs[step], k[loc], v[loc], Layer(0), batch)
            outs.append(out.cpu())
            poss.append(be._positions[:B].cpu())
        results[mode] = (torch.stack(outs), torch.stack(poss))
        if mode == "quest_hisparse":
            assert be.coord.stats.misses > 0
        del rtp, kvp, be
        torch.cuda.empty_cache()
    assert torch.equal(results["quest"][1], results["quest_hisparse"][1])
    assert torch.equal(results["quest"][0], results["quest_hisparse"][0])


def test_c4_hisparse_batch16_128k_ar1_queries():
    """quest_hisparse at its benchmark configuration: batch 16 x 131072-token contexts, a hot
    buffer of 4096 + 1 rows per request and layer, the full history in pinned host memory,
    queries AR(1) across steps (q_t = 0.9 q_{t-1} + sqrt(0.19) e_t), 128 decode steps over 2
    layers (2 x 4.3 GB of pinned host tier; the per-layer work is the same for all 48).
    Every step: QuestOnlyBackend and QuestHiSparseBackend on the same pool and inputs give
    bit-identical positions and outputs, and the swap-in rows, buffer_tokens and lru_slots
    equal oracle/hisparse.py's; positions equal the Quest oracle's on sampled steps (page
    boundaries crossed at steps 1 and 65), and quest's attention outputs of requests 0, 7 and 15
    equal the float64 oracle's within attn_tol at steps 0 and 127 in both layers."""
    from oracle import hisparse as oh
    from qwenquest_amd.attention.quest_hisparse import QuestHiSparseBackend
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    B, S, L, steps, BUF = 16, 131072, 2, 128, 4096
    ctx = S + steps + 64
    prompt = S - 1
    rtp = ReqToTokenPool(B, ctx, DEV)
    kvp = MHATokenToKVPool(B * ctx, L, KV, D, torch.bfloat16, DEV)
    g = torch.Generator(device=DEV).manual_seed(4321)
    for layer in range(L):
        kvp.k_all[layer].normal_(generator=g)
        kvp.v_all[layer].normal_(generator=g)
    base = 1 + torch.arange(B, device=DEV, dtype=torch.int64) * ctx
    rtp.req_to_token.copy_((base[:, None] + torch.arange(ctx, device=DEV)[None]).to(torch.int32))
    cfg = {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P, "device_buffer_size": BUF}
    quest_be = QuestOnlyBackend(rtp, kvp, cfg)
    his_be = QuestHiSparseBackend(rtp, kvp, cfg, host_pool_size=B * ctx)
    pre = ForwardBatch(ForwardMode.EXTEND, None, None, torch.arange(B), torch.full((B,), prompt), None, rtp, kvp,
                       quest_be)
    quest_be._update_quest_for_extend(pre)
    his_be.on_extend_finished(pre)
    coord = his_be.coord
    swap_rows = []
    swap = coord.swap_in_selected_pages

    def recording_swap(reqs, seq_lens, top_k_result, layer_id, **kw):
        rows = swap(reqs, seq_lens, top_k_result, layer_id, **kw)
        swap_rows.append((top_k_result.clone(), rows))
        return rows

    coord.swap_in_selected_pages = recording_swap
    # oracles: Quest state from the same keys (host copies), LRU state per (layer, request)
    kbits = [bf16_bits(kvp.k_all[layer].cpu()) for layer in range(L)]
    st = oq.QuestState(TOP_K, P)
    st.init_storage(0, L, B, ctx, KV, D)
    for layer in range(L):
        for r in range(B):
            st.update_prefill_representations(layer, r, kbits[layer], 1 + r * ctx + np.arange(prompt))
    sh = oh.HiSparseState(L, B, buf=BUF, top_k=TOP_K, max_ctx=ctx)
    for r in range(B):
        sh.admit(r, np.arange(prompt))
    check_steps = {0, 1, 2, 64, 65, 127}
    q = dev_randn((L, B, H, D), 900)
    reqs = list(range(B))
    for step in range(steps):
        q = 0.9 * q + 0.19**0.5 * dev_randn((L, B, H, D), 1000 + step)
        qb = q.to(torch.bfloat16)
        kn = dev_randn((L, B, KV, D), 2000 + step).to(torch.bfloat16)
        vn = dev_randn((L, B, KV, D), 3000 + step).to(torch.bfloat16)
        seq = torch.full((B,), S + step, device=DEV, dtype=torch.int64)
        loc = base + seq - 1
        batches = [ForwardBatch(ForwardMode.DECODE, None, None, torch.arange(B, device=DEV), seq, loc, rtp, kvp, be)
                   for be in (quest_be, his_be)]
        outs = {}
        for be, batch in zip((quest_be, his_be), batches):
            be.init_forward_metadata(batch)
            outs[be.name] = [be.forward_decode(qb[layer], kn[layer], vn[layer], Layer(layer), batch)
                             for layer in range(L)]
        seqs = np.full(B, S + step)
        if step > 0:
            for r in range(B):
                sh.backup(r, S + step - 2, prompt + step - 1)
        for layer in range(L):
            # quest's positions buffer holds the last layer's: the four-launch retrieve gives each layer's
            pq, _ = quest_be.quest.retrieve_topk(qb[layer], layer, torch.arange(B, device=DEV), seq)
            ph, rows = swap_rows[layer]
            assert torch.equal(pq, ph), f"step {step} layer {layer}: positions differ"
            oq_out, oh_out = outs[quest_be.name][layer], outs[his_be.name][layer]
            assert torch.equal(oq_out.view(torch.int16), oh_out.view(torch.int16)), f"step {step} layer {layer}"
            rows_ref, _ = sh.swap_in(layer, reqs, seqs, ph.cpu().numpy())
            assert np.array_equal(rows.cpu().numpy(), rows_ref), f"step {step} layer {layer}: rows"
            assert np.array_equal(coord.buffer_tokens[layer].cpu().numpy(), sh.buffer_tokens[layer])
            assert np.array_equal(coord.lru_slots[layer].cpu().numpy(), sh.lru_slots[layer])
        swap_rows.clear()
        if step > 0:
            for layer in range(L):
                st.update_decode_representations(layer, reqs, kbits[layer], (loc - 1).cpu().numpy())
            st.maybe_finalize_decode_representations(reqs)
        st.prepare_step(seqs)
        if step in check_steps:
            for layer in range(L):
                ref_pos, ref_actual, _ = st.retrieve_topk(qb[layer].float().cpu().numpy(), layer, reqs)
                pq, _ = quest_be.quest.retrieve_topk(qb[layer], layer, torch.arange(B, device=DEV), seq)
                assert np.array_equal(pq.cpu().numpy(), ref_pos[:, :TOP_K]), f"step {step} layer {layer}: vs oracle"
                if step in (0, 127):
                    # the layer step's attention at this shape (the fused two-launch path)
                    # against the float64 oracle over the oracle's rows, new token included
                    out_q = outs[quest_be.name][layer].float().cpu().numpy()
                    for i in (0, 7, 15):
                        n = int(ref_actual[i])
                        rows = (base[i] + torch.from_numpy(ref_pos[i, :n].astype(np.int64)).to(DEV))
                        ref = oracle_attention(qb[layer, i].cpu(), kvp.k_all[layer][rows].cpu(),
                                               kvp.v_all[layer][rows].cpu())
                        assert_attn_close(out_q[i], ref, f"step {step} layer {layer} request {i}: attention")
        # the new token's keys join the oracle's copy of the pool (folded at the next step)
        for layer in range(L):
            kbits[layer][loc.cpu().numpy()] = bf16_bits(kn[layer].cpu())
    s = coord.stats
    assert (s.hits, s.misses) == (sh.hits, sh.misses) and s.misses > 0
    print(f"C4 hot-buffer hit rate {s.hit_rate:.3f} ({s.hits} hits, {s.misses} misses)")
