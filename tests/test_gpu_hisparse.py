"""GPU parity of the HiSparse hot buffer: exactness of the swap-in, the LRU state
machine (known answers + the reference's 200-step golden trace), eager backup,
release, error conditions, and quest_hisparse == quest bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import hisparse as oh
from qwenquest_amd import _lib
from tests.conftest import load_golden

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
LAYERS, KV, D = 2, 2, 8


def make(buf: int, top_k: int, page: int = 1, max_reqs: int = 2, max_ctx: int = 256, dtype=torch.float32,
         async_admission: bool = False):
    from qwenquest_amd.hisparse import HiSparseCoordinator
    from qwenquest_amd.memory import MHATokenToKVPool
    from qwenquest_amd.quest import QuestAlgorithm

    quest = QuestAlgorithm(top_k=top_k, page_size=page, device=DEV)
    quest.init_storage(0, LAYERS, max_reqs, max_ctx, KV, D)
    coord = HiSparseCoordinator(
        quest=quest, num_layers=LAYERS, kv_heads=KV, head_dim=D, max_reqs=max_reqs,
        max_context_len=max_ctx, top_k=top_k, device_buffer_size=buf,
        host_pool_size=max_reqs * max_ctx, dtype=dtype, device=DEV, async_admission=async_admission,
    )
    pool = MHATokenToKVPool(max_ctx, LAYERS, KV, D, dtype, DEV)
    return quest, coord, pool


def truth(total: int, seed: int = 0):
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(LAYERS, total, KV, D, generator=gen), torch.randn(LAYERS, total, KV, D, generator=gen)


def admit(coord, pool, req, n, k, v):
    locs = torch.arange(1, n + 1, device=DEV)
    for layer in range(LAYERS):
        pool.set_kv_buffer(layer, locs, k[layer, :n].to(DEV), v[layer, :n].to(DEV))
    coord.admit_request(req, n, pool, locs)


def decode_step(coord, req, pos, k, v):
    reqs, seq_lens = torch.tensor([req], device=DEV), torch.tensor([pos + 1], device=DEV)
    coord.prepare_decode_step(reqs, seq_lens)
    for layer in range(LAYERS):
        coord.write_new_token(layer, reqs, seq_lens, k[layer, pos : pos + 1].to(DEV), v[layer, pos : pos + 1].to(DEV))
    return reqs, seq_lens


@pytest.mark.parametrize(("prefill_len", "buf", "top_k"), [(10, 16, 8), (40, 16, 8), (5, 32, 32)])
def test_swap_in_is_exact_under_random_selections(prefill_len, buf, top_k):
    """reference tests/test_hisparse.py:65-90, plus the oracle's rows and LRU state each step."""
    total = 120
    k, v = truth(total)
    _, coord, pool = make(buf, top_k)
    admit(coord, pool, 1, prefill_len, k, v)
    st = oh.HiSparseState(LAYERS, 2, buf=buf, top_k=top_k, max_ctx=256)
    st.admit(1, np.arange(prefill_len))
    gen = torch.Generator().manual_seed(7)
    for pos in range(prefill_len, total):
        reqs, seq_lens = decode_step(coord, 1, pos, k, v)
        if pos > prefill_len:
            st.backup(1, pos - 1, pos - 1)
        seq_len = pos + 1
        n = min(seq_len, top_k)
        for layer in range(LAYERS):
            if seq_len <= top_k:
                sel = torch.arange(n)
            else:
                sel = torch.randint(0, seq_len, (n,), generator=gen)
                sel[-1] = seq_len - 1
                sel[0] = sel[1]
            rows = coord.swap_in_selected_pages(reqs, seq_lens, sel[None].int(), layer)
            got_k = coord.device_k[layer][rows[0, :n]].cpu()
            got_v = coord.device_v[layer][rows[0, :n]].cpu()
            assert torch.equal(got_k, k[layer, sel]), f"layer {layer} pos {pos}"
            assert torch.equal(got_v, v[layer, sel])
            ref_rows, _ = st.swap_in(layer, [1], [seq_len], sel[None].numpy())
            assert np.array_equal(rows.cpu().numpy()[0, :n], ref_rows[0, :n])
            assert np.array_equal(coord.buffer_tokens[layer, 1].cpu().numpy(), st.buffer_tokens[layer, 1])
            assert np.array_equal(coord.lru_slots[layer, 1].cpu().numpy(), st.lru_slots[layer, 1])
            if seq_len > top_k:
                assert rows[0, 0] == rows[0, 1]
    stats = coord.stats
    assert stats.misses > 0 and (stats.hits, stats.misses) == (st.hits, st.misses)


@pytest.mark.parametrize(("prefill_len", "buf", "top_k"),
                         [(1200, 1025, 512), (2000, 1500, 1024), (5000, 4096, 2048), (5000, 4097, 2048),
                          (7000, 6000, 3000)])
def test_swap_in_large_buffers_match_oracle(prefill_len, buf, top_k):
    """Hot buffers that are not a multiple of the plan block's 1024 threads and exceed it
    (each thread holds a run of ceil(buf / 1024) LRU entries, the last runs partial or empty),
    on both sides of the plan kernel's small form (top_k <= 2048 and buf <= 4096) and with
    more than two 1024-entry rounds (top_k 3000): rows, buffer_tokens, lru_slots and hit/miss
    counts equal the oracle's at every step, with duplicated and newest-token entries."""
    steps = 24
    total = prefill_len + steps
    k, v = truth(total, seed=3)
    _, coord, pool = make(buf, top_k, max_reqs=2, max_ctx=total + 8)
    admit(coord, pool, 1, prefill_len, k, v)
    st = oh.HiSparseState(LAYERS, 2, buf=buf, top_k=top_k, max_ctx=total + 8)
    st.admit(1, np.arange(prefill_len))
    gen = torch.Generator().manual_seed(17)
    for pos in range(prefill_len, total):
        reqs, seq_lens = decode_step(coord, 1, pos, k, v)
        if pos > prefill_len:
            st.backup(1, pos - 1, pos - 1)
        seq_len = pos + 1
        for layer in range(LAYERS):
            # a recent run, a few far pages, random picks and a duplicate, like a Quest layout
            sel = torch.randint(0, seq_len, (top_k,), generator=gen)
            sel[: top_k // 4] = torch.arange(seq_len - top_k // 4, seq_len)
            sel[top_k // 4] = sel[top_k // 4 + 1]
            rows = coord.swap_in_selected_pages(reqs, seq_lens, sel[None].int(), layer)
            ref_rows, _ = st.swap_in(layer, [1], [seq_len], sel[None].numpy())
            assert np.array_equal(rows.cpu().numpy()[0], ref_rows[0]), f"layer {layer} pos {pos}"
            assert np.array_equal(coord.buffer_tokens[layer, 1].cpu().numpy(), st.buffer_tokens[layer, 1])
            assert np.array_equal(coord.lru_slots[layer, 1].cpu().numpy(), st.lru_slots[layer, 1])
            assert torch.equal(coord.device_k[layer][rows[0]].cpu(), k[layer, sel])
    stats = coord.stats
    assert stats.misses > 0 and stats.hits > 0 and (stats.hits, stats.misses) == (st.hits, st.misses)


def test_every_decoded_token_is_backed_up_to_host():
    k, v = truth(64)
    _, coord, pool = make(buf=8, top_k=8)
    admit(coord, pool, 0, 20, k, v)
    for pos in range(20, 41):
        decode_step(coord, 0, pos, k, v)
    torch.cuda.synchronize()
    host_idx = coord.req_to_host_pool[0, :40].cpu()
    assert torch.all(host_idx >= 0)
    for layer in range(LAYERS):
        assert torch.equal(coord.host_k[layer][host_idx], k[layer, :40])
        assert torch.equal(coord.host_v[layer][host_idx], v[layer, :40])
    assert int(coord.req_to_host_pool[0, 40]) == -1


def test_lru_replacement_order_known_answer():
    """reference tests/test_hisparse.py:108-129."""
    k, v = truth(32)
    _, coord, pool = make(buf=4, top_k=2)
    admit(coord, pool, 0, 10, k, v)

    def select(pos, positions):
        reqs, seq_lens = decode_step(coord, 0, pos, k, v)
        coord.swap_in_selected_pages(reqs, seq_lens, torch.tensor([positions]).int(), 0)

    select(10, [5, 10])
    assert coord.buffer_tokens[0, 0].tolist() == [5, 1, 2, 3]
    assert coord.lru_slots[0, 0].tolist() == [1, 2, 3, 0]
    select(11, [1, 5])
    assert (coord.stats.hits, coord.stats.misses) == (2, 1)
    assert coord.lru_slots[0, 0].tolist() == [2, 3, 1, 0]
    select(12, [7, 8])
    assert coord.buffer_tokens[0, 0].tolist() == [5, 1, 7, 8]
    assert coord.lru_slots[0, 0].tolist() == [1, 0, 2, 3]
    assert (coord.stats.hits, coord.stats.misses) == (2, 3)


def test_fast_path_while_sequence_fits_the_buffer():
    k, v = truth(32)
    _, coord, pool = make(buf=16, top_k=16)
    admit(coord, pool, 0, 6, k, v)
    reqs, seq_lens = decode_step(coord, 0, 6, k, v)
    rows = coord.swap_in_selected_pages(reqs, seq_lens, torch.arange(16)[None].int(), 0)
    assert rows[0, :7].tolist() == coord.req_to_device_buffer[0, :7].tolist()
    assert torch.all(rows[0, 7:] == -1)
    assert coord.stats.fast_path_calls == 1 and coord.stats.misses == 0


def test_request_finished_releases_everything():
    k, v = truth(64)
    quest, coord, pool = make(buf=8, top_k=8, page=4)
    free_before = coord.host_allocator.available_size()
    admit(coord, pool, 1, 30, k, v)
    for pos in range(30, 36):
        decode_step(coord, 1, pos, k, v)
    assert quest.page_valid[:, 1].any()
    coord.request_finished(1)
    assert coord.host_allocator.available_size() == free_before
    assert torch.all(coord.req_to_host_pool[1] == -1)
    assert torch.all(coord.buffer_tokens[:, 1] == -1)
    assert not quest.page_valid[:, 1].any()


def test_coordinator_validates_sizes():
    from qwenquest_amd.hisparse import HiSparseCoordinator
    from qwenquest_amd.quest import QuestAlgorithm

    quest = QuestAlgorithm(top_k=8, page_size=4, device=DEV)
    quest.init_storage(0, LAYERS, 1, 64, KV, D)
    common = dict(quest=quest, num_layers=LAYERS, kv_heads=KV, head_dim=D, max_reqs=1, max_context_len=64,
                  host_pool_size=64, dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError):
        HiSparseCoordinator(top_k=8, device_buffer_size=4, **common)
    with pytest.raises(ValueError):
        HiSparseCoordinator(top_k=16, device_buffer_size=32, **common)


def test_error_conditions_are_raised():
    k, v = truth(64)
    _, coord, pool = make(buf=4, top_k=4)
    admit(coord, pool, 0, 10, k, v)
    reqs, seq_lens = decode_step(coord, 0, 10, k, v)
    # all wanted positions are backed up; 5 distinct misses cannot fit 4 slots... top_k=4 -> 3 + newest
    tokens_before = coord.buffer_tokens[0, 0].clone()
    # a position without host backup: position 30 was never decoded
    coord.req_to_host_pool[0, 9] = -1
    coord.swap_in_selected_pages(reqs, seq_lens, torch.tensor([[9, 6, 5, 10]]).int(), 0)
    with pytest.raises(AssertionError):
        coord.check_errors()
    assert torch.equal(coord.buffer_tokens[0, 0], tokens_before)  # state left unchanged


def test_golden_200_step_trace_through_the_kernels():
    """The reference's own 200-step trace (tests/golden/swap_trace.npz): identical rows,
    buffer_tokens, lru_slots and hit/miss counts at every layer of every step."""
    g = load_golden("swap_trace.npz")
    layers, buf, top_k, ctx, prefill = g["meta"].tolist()
    assert layers == LAYERS
    _, coord, pool = make(buf=buf, top_k=top_k, max_reqs=1, max_ctx=ctx)
    k, v = truth(ctx, seed=11)
    admit(coord, pool, 0, prefill, k, v)
    i = 0
    for step in range(200):
        pos = prefill + step
        reqs, seq_lens = decode_step(coord, 0, pos, k, v)
        for layer in range(layers):
            sel = torch.from_numpy(g["selections"][i])
            rows = coord.swap_in_selected_pages(reqs, seq_lens, sel[None].int(), layer)
            assert np.array_equal(rows[0].cpu().numpy(), g["rows"][i]), f"step {step} layer {layer}"
            assert np.array_equal(coord.buffer_tokens[layer, 0].cpu().numpy(), g["tokens"][i])
            assert np.array_equal(coord.lru_slots[layer, 0].cpu().numpy(), g["lru"][i])
            assert torch.equal(coord.device_k[layer][rows[0]].cpu(), k[layer, sel])
            i += 1
    s = coord.stats
    assert [s.hits, s.misses] == g["stats"][-1].tolist()


# (q heads, kv heads, head_dim, top_k, page, hot buffer, ctx, prompts, steps).  The last
# shape is the fused layer step's (32/4/128, page 64): quest runs the fused two-launch step,
# quest_hisparse the same attention kernel over its hot-buffer rows.
BIT_IDENTITY = [
    (8, 2, 16, 32, 8, 48, 256, {0: 90, 1: 107}, 60),
    (16, 2, 128, 32, 8, 48, 256, {0: 90, 1: 107}, 60),
    (32, 4, 128, 256, 64, 384, 1200, {0: 700, 1: 1003}, 40),
]


@pytest.mark.parametrize("avoid", [False, True])
@pytest.mark.parametrize("shape", range(len(BIT_IDENTITY)))
def test_quest_hisparse_is_bit_identical_to_quest(avoid, shape):
    """reference tests/test_engine.py:59-69 and test_bf16.py:27-43 at the backend boundary:
    the same q/k/v through QuestOnlyBackend and QuestHiSparseBackend over many decode steps
    (the hot buffer must swap) give bit-identical outputs and positions, also where quest
    runs the fused layer step; QuestHiSparseBackend with swap_route="memcpy", or with the
    admission backup on a side stream (async_admission), gives the same bits, the same
    hot-buffer state and the same host tier as with the in-kernel copy."""
    from qwenquest_amd.attention.quest_hisparse import QuestHiSparseBackend
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    H, KVH, DIM, TOP_K, P, BUF, CTX, prompts, steps = BIT_IDENTITY[shape]
    L = 3
    cfg = {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P, "device_buffer_size": BUF,
           "avoid_recent_overlap": avoid}
    gen = torch.Generator().manual_seed(3)
    total = max(prompts.values()) + steps + 1
    kk = torch.randn(L, 2, total, KVH, DIM, generator=gen).to(torch.bfloat16)
    vv = torch.randn(L, 2, total, KVH, DIM, generator=gen).to(torch.bfloat16)
    qq = torch.randn(steps, L, 2, H, DIM, generator=gen).to(torch.bfloat16)
    outs, poss, stats = {}, {}, {}
    for mode in ("quest", "quest_hisparse", "quest_hisparse_memcpy", "quest_hisparse_async"):
        rtp = ReqToTokenPool(2, CTX, DEV)
        kvp = MHATokenToKVPool(2 * CTX, L, KVH, DIM, torch.bfloat16, DEV)
        if mode == "quest":
            be = QuestOnlyBackend(rtp, kvp, cfg)
        else:
            be = QuestHiSparseBackend(rtp, kvp, cfg, host_pool_size=2 * CTX,
                                      swap_route="memcpy" if mode.endswith("memcpy") else "kernel",
                                      async_admission=mode.endswith("async"))
        for r, n in prompts.items():
            rtp.req_to_token[r] = torch.arange(1 + r * CTX, 1 + (r + 1) * CTX, dtype=torch.int32)
            rows = torch.arange(1 + r * CTX, 1 + r * CTX + n)
            kvp.k_all[:, rows] = kk[:, r, :n].to(DEV)
            kvp.v_all[:, rows] = vv[:, r, :n].to(DEV)
        batch = ForwardBatch(ForwardMode.EXTEND, None, None, torch.tensor([0, 1]), torch.tensor(list(prompts.values())),
                             None, rtp, kvp, be)
        if mode == "quest":
            be._update_quest_for_extend(batch)
        else:
            be.on_extend_finished(batch)

        class Layer:
            def __init__(self, i):
                self.layer_id, self.scaling = i, DIM**-0.5

        res, pos = [], []
        for step in range(steps):
            seqs = [prompts[r] + step + 1 for r in (0, 1)]
            locs = torch.tensor([1 + r * CTX + s - 1 for r, s in zip((0, 1), seqs)], device=DEV)
            b = ForwardBatch(ForwardMode.DECODE, None, None, torch.tensor([0, 1], device=DEV),
                             torch.tensor(seqs, device=DEV), locs if mode == "quest" else None, rtp, kvp, be)
            be.init_forward_metadata(b)
            for layer in range(L):
                kn = torch.stack([kk[layer, r, s - 1] for r, s in zip((0, 1), seqs)]).to(DEV)
                vn = torch.stack([vv[layer, r, s - 1] for r, s in zip((0, 1), seqs)]).to(DEV)
                res.append(be.forward_decode(qq[step, layer].to(DEV), kn, vn, Layer(layer), b).cpu())
                pos.append(be._positions[:2].cpu())
        outs[mode], poss[mode] = torch.stack(res), torch.stack(pos)
        if mode != "quest":
            st = be.coord.stats
            assert st.misses > 0 and st.hits > 0
            stats[mode] = (st, be.coord.buffer_tokens.cpu(), be.coord.lru_slots.cpu(), be.coord.device_k_all.cpu(),
                           be.coord.host_k_all.clone(), be.coord.host_v_all.clone())
            assert be.coord.admission_done(0) and be.coord.admission_done(1)
    fused = _lib.load().qq_quest_fused_step(_lib.DTYPE_BF16, _lib.DTYPE_BF16, _lib.DTYPE_BF16, H, KVH, DIM, P, TOP_K,
                                            (CTX + P - 1) // P)
    assert fused == (shape == len(BIT_IDENTITY) - 1)
    assert torch.equal(poss["quest"], poss["quest_hisparse"])
    assert torch.equal(outs["quest"], outs["quest_hisparse"])
    # the copy-engine swap-in route (plan kernel, hipMemcpyAsync per run of host rows on a side
    # stream, scatter) leaves the same hot buffers and gives the same bits
    assert torch.equal(poss["quest_hisparse_memcpy"], poss["quest_hisparse"])
    assert torch.equal(outs["quest_hisparse_memcpy"], outs["quest_hisparse"])
    for other in ("quest_hisparse_memcpy", "quest_hisparse_async"):
        a, b = stats["quest_hisparse"], stats[other]
        assert a[0] == b[0] and all(torch.equal(x, y) for x, y in zip(a[1:], b[1:])), other
    assert torch.equal(poss["quest_hisparse_async"], poss["quest_hisparse"])
    assert torch.equal(outs["quest_hisparse_async"], outs["quest_hisparse"])


def test_async_admission_waits_only_for_the_batch_members():
    """The admission backup on a side stream: pending per request until a decode step of a
    batch holding that request (host indices: only its members wait; device indices: every
    pending one), its release or an explicit wait; the host tier ends as a synchronous
    admission leaves it.  Requests 0 and 2 have their prompts in consecutive pool rows (the
    copy-engine backup), request 1 in scattered rows (more runs than the copy engines take:
    the copy kernel on the side stream)."""
    from qwenquest_amd.memory import MHATokenToKVPool

    CTX = 256
    prompts = {0: 120, 1: 90, 2: 60}
    truths = {r: truth(n, seed=10 + r) for r, n in prompts.items()}
    coords = {}
    for mode in (False, True):
        _, coord, _ = make(buf=16, top_k=8, max_reqs=3, max_ctx=CTX, async_admission=mode)
        pool = MHATokenToKVPool(3 * CTX, LAYERS, KV, D, torch.float32, DEV)
        for r, n in prompts.items():  # each prompt in rows of its own
            order = torch.randperm(n, generator=torch.Generator().manual_seed(r)) if r == 1 else torch.arange(n)
            locs = (1 + r * CTX + order).to(DEV)
            k, v = truths[r]
            for layer in range(LAYERS):
                pool.set_kv_buffer(layer, locs, k[layer].to(DEV), v[layer].to(DEV))
            coord.admit_request(r, n, pool, locs)
        coords[mode] = coord
    coord = coords[True]
    assert sorted(coord._adm_pending) == [0, 1, 2]
    locs1 = (1 + CTX + torch.randperm(90, generator=torch.Generator().manual_seed(1))).to(DEV)
    assert coord._row_runs(locs1, torch.arange(90, device=DEV), 3 * CTX + 1) is None
    assert coord._row_runs(torch.arange(5, 9, device=DEV), torch.arange(40, 44, device=DEV), 3 * CTX + 1) == [(5, 40, 4)]
    steps = [(torch.tensor([1]), torch.tensor([91])), ("release", 2),
             (torch.tensor([0, 1], device=DEV), torch.tensor([121, 92], device=DEV))]
    pending_after = [[0, 2], [0], []]
    for c in (coords[False], coord):
        for (what, arg), left in zip(steps, pending_after):
            if isinstance(what, str):
                c.request_finished(arg)
            else:
                c.prepare_decode_step(what, arg)
            if c is coord:
                assert sorted(c._adm_pending) == left
    torch.cuda.synchronize()
    assert all(coord.admission_done(r) for r in range(3))
    ref = coords[False]
    assert torch.equal(ref.req_to_host_pool.cpu(), coord.req_to_host_pool.cpu())
    rows = ref.req_to_host_pool[:2].flatten()
    rows = rows[rows >= 0].cpu()
    assert rows.numel() >= 120 + 90
    assert torch.equal(ref.host_k_all[:, rows], coord.host_k_all[:, rows])
    assert torch.equal(ref.host_v_all[:, rows], coord.host_v_all[:, rows])
    for r, n in ((0, 120), (1, 90)):  # the prompts themselves
        hr = coord.req_to_host_pool[r, :n].cpu()
        assert torch.equal(coord.host_k_all[:, hr], truths[r][0])
        assert torch.equal(coord.host_v_all[:, hr], truths[r][1])


def test_device_row_allocator_hands_out_rows_in_the_reference_order():
    """The host tier's free list kept on the device gives the rows TokenToKVPoolAllocator
    (reference memory.py:47-72) gives, over interleaved allocs and frees."""
    from qwenquest_amd.hisparse.coordinator import DeviceRowAllocator
    from qwenquest_amd.memory import TokenToKVPoolAllocator

    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    dev = DeviceRowAllocator(50, DEV, err, 0)
    ref = TokenToKVPoolAllocator(50, device="cpu")
    gen = torch.Generator().manual_seed(3)
    held = []
    for step in range(40):
        if held and torch.rand(1, generator=gen).item() < 0.4:
            rows = held.pop(int(torch.randint(0, len(held), (1,), generator=gen)))
            ref.free(rows)
            dev.free(rows.to(DEV))
        else:
            n = int(torch.randint(1, 6, (1,), generator=gen))
            if n > ref.available_size():
                with pytest.raises(RuntimeError):
                    dev.alloc(n)
                continue
            a, b = ref.alloc(n), dev.alloc(n).cpu()
            assert torch.equal(a, b), f"step {step}"
            held.append(a)
        assert dev.available_size() == ref.available_size()


def _his_coord(buf, top_k, ctx, host_pool, kv=2, d=8, dtype=torch.float32, max_reqs=2):
    from qwenquest_amd.hisparse import HiSparseCoordinator
    from qwenquest_amd.memory import MHATokenToKVPool
    from qwenquest_amd.quest import QuestAlgorithm

    quest = QuestAlgorithm(top_k=top_k, page_size=1, device=DEV)
    quest.init_storage(0, 1, max_reqs, ctx, kv, d)
    coord = HiSparseCoordinator(quest=quest, num_layers=1, kv_heads=kv, head_dim=d, max_reqs=max_reqs,
                                max_context_len=ctx, top_k=top_k, device_buffer_size=buf,
                                host_pool_size=host_pool, dtype=dtype, device=DEV)
    pool = MHATokenToKVPool(max_reqs * ctx, 1, kv, d, dtype, DEV)
    g = torch.Generator(device=DEV).manual_seed(8)
    pool.k_all.normal_(generator=g)
    pool.v_all.normal_(generator=g)
    return coord, pool


def test_host_pool_exhaustion_is_raised_from_the_device():
    """The eager backup takes its host rows on the device: with the pool exhausted the step
    backs nothing up and check_errors raises the allocator's RuntimeError (memory.py:62-66).
    The previous token is still folded into the Quest bounds, as the reference folds it
    (coordinator.py:204-208) before its alloc fails (:210): the bounds and counters equal
    those of a coordinator whose pool has room, for both requests of the batch."""
    coord, pool = _his_coord(buf=8, top_k=4, ctx=64, host_pool=42)
    roomy, _ = _his_coord(buf=8, top_k=4, ctx=64, host_pool=200)
    for c in (coord, roomy):
        for r in (0, 1):
            c.admit_request(r, 20, pool, torch.arange(1 + 64 * r, 21 + 64 * r, device=DEV))
    reqs = torch.tensor([0, 1], device=DEV)
    for pos in (20, 21):  # the first step is skipped, then one backup per request takes the last 2 rows
        for c in (coord, roomy):
            c.prepare_decode_step(reqs, torch.tensor([pos + 1, pos + 1], device=DEV))
            for r in (0, 1):  # the token decoded at this step, in its hot-buffer slot
                slot = r * 9 + min(pos, 8)
                c.device_k[0][slot] = pool.k_all[0, 1 + 64 * r + pos]
                c.device_v[0][slot] = pool.v_all[0, 1 + 64 * r + pos]
    coord.check_errors()
    assert coord.host_allocator.available_size() == 0
    for c in (coord, roomy):
        c.prepare_decode_step(reqs, torch.tensor([23, 23], device=DEV))  # position 21: no row left in coord
    with pytest.raises(RuntimeError, match="out of memory"):
        coord.check_errors()
    roomy.check_errors()
    assert int(coord.req_to_host_pool[0, 21]) == -1 and int(coord.req_to_host_pool[1, 21]) == -1
    assert int(coord.req_to_host_pool[0, 20]) >= 0 and int(roomy.req_to_host_pool[1, 21]) >= 0
    qa, qb = coord.quest, roomy.quest
    for name in ("page_k_bounds", "running_k_min", "running_k_max", "running_token_count", "running_page_idx"):
        assert torch.equal(getattr(qa, name), getattr(qb, name)), name


@pytest.mark.parametrize("fused", [True, False])
def test_failed_swap_in_poisons_only_that_request(fused):
    """A position without a host row (coordinator.py:284-286): the request's swap-in rows are
    all -1 and its state is unchanged, the rows attention (the fused layer step's kernel and
    the chunked one) outputs NaN for it and a finite output for the other request, and the
    host sees the error through the pinned mirror without a device synchronisation."""
    from qwenquest_amd.attention.ops import decode_attention_rows

    H4, KV4, D4, buf, top_k, ctx, n = 32, 4, 128, 256, 128, 600, 400
    coord, pool = _his_coord(buf, top_k, ctx, 2 * ctx, kv=KV4, d=D4, dtype=torch.bfloat16)
    for r in (0, 1):
        coord.admit_request(r, n, pool, torch.arange(1 + r * ctx, 1 + r * ctx + n, device=DEV))
    reqs = torch.tensor([0, 1], device=DEV)
    seq = torch.tensor([n + 1, n + 1], device=DEV)
    coord.prepare_decode_step(reqs, seq)
    newkv = torch.randn(2, KV4, D4, device=DEV).to(torch.bfloat16)
    coord.write_new_token(0, reqs, seq, newkv, newkv)
    coord.req_to_host_pool[1, 310] = -1
    sel = torch.arange(n - top_k, n, device=DEV).repeat(2, 1).int()  # misses beyond the buffer, all backed up
    tokens_before = coord.buffer_tokens[0, 1].clone()
    rows = coord.swap_in_selected_pages(reqs, seq, sel, 0)
    torch.cuda.synchronize()
    assert bool((rows[1] == -1).all()) and bool((rows[0] >= 0).all())
    assert torch.equal(coord.buffer_tokens[0, 1], tokens_before)
    with pytest.raises(AssertionError):
        coord.check_errors(sync=False)
    coord.check_errors()  # raised once: both the word and its mirror are cleared
    q = torch.randn(2, H4, D4, device=DEV).to(torch.bfloat16)
    actual = torch.full((2,), top_k, dtype=torch.int32, device=DEV)
    sync = torch.zeros(int(_lib.load().qq_quest_layer_step_sync_bytes(2, KV4)), dtype=torch.uint8, device=DEV)
    out = decode_attention_rows(q, coord.device_k[0], coord.device_v[0], rows, actual, D4**-0.5,
                                sync=sync if fused else None).float()
    assert bool(torch.isnan(out[1]).all()), "the failed request's output is not NaN"
    assert bool(torch.isfinite(out[0]).all())


def test_quest_hisparse_step_in_a_graph_equals_eager():
    """The quest_hisparse decode step has no host synchronisation: captured once in a HIP graph
    (bounds fold + eager backup + per layer new token, selection, swap-in, attention) and
    replayed, it gives the eager run's outputs, positions, LRU state, host rows and counters
    bit for bit over 12 steps, while the hot buffer swaps."""
    from qwenquest_amd.attention.quest_hisparse import QuestHiSparseBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    H4, KV4, D4, TOPK, PAGE, BUF, CTX, L4, steps = 32, 4, 128, 256, 64, 384, 1200, 2, 12
    prompts = {0: 700, 1: 1003}
    kk = torch.randn(L4, 2 * CTX + 1, KV4, D4, generator=torch.Generator().manual_seed(61)).to(torch.bfloat16)
    vv = torch.randn(L4, 2 * CTX + 1, KV4, D4, generator=torch.Generator().manual_seed(62)).to(torch.bfloat16)

    def setup():
        rtp = ReqToTokenPool(2, CTX, DEV)
        kvp = MHATokenToKVPool(2 * CTX, L4, KV4, D4, torch.bfloat16, DEV)
        kvp.k_all.copy_(kk.to(DEV))
        kvp.v_all.copy_(vv.to(DEV))
        for r in (0, 1):
            rtp.req_to_token[r] = torch.arange(1 + r * CTX, 1 + (r + 1) * CTX, dtype=torch.int32)
        be = QuestHiSparseBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOPK, "quest_page_size": PAGE,
                                             "device_buffer_size": BUF}, host_pool_size=2 * CTX)
        pre = ForwardBatch(ForwardMode.EXTEND, None, None, torch.tensor([0, 1]),
                           torch.tensor([prompts[0], prompts[1]]), None, rtp, kvp, be)
        be.on_extend_finished(pre)
        return rtp, kvp, be

    class Lay:
        def __init__(self, i):
            self.layer_id, self.scaling = i, D4**-0.5

    qs = torch.randn(steps, L4, 2, H4, D4, generator=torch.Generator().manual_seed(63)).to(torch.bfloat16).to(DEV)
    ks = torch.randn(steps, L4, 2, KV4, D4, generator=torch.Generator().manual_seed(64)).to(torch.bfloat16).to(DEV)
    results = {}
    for mode in ("eager", "graph"):
        rtp, kvp, be = setup()
        seq = torch.tensor([prompts[0] + 1, prompts[1] + 1], device=DEV, dtype=torch.int64)
        q_in = torch.empty_like(qs[0])
        k_in = torch.empty_like(ks[0])
        batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.tensor([0, 1], device=DEV), seq, None, rtp, kvp, be)
        outs_static, pos_static = [], []

        def step():
            be.init_forward_metadata(batch)
            res = []
            for layer in range(L4):
                res.append(be.forward_decode(q_in[layer], k_in[layer], k_in[layer], Lay(layer), batch))
            return res

        outs, poss = [], []
        graph = None
        for t in range(steps):
            q_in.copy_(qs[t])
            k_in.copy_(ks[t])
            if mode == "eager" or t < 2:  # two eager steps first (workspaces, first-step skips)
                res = step()
            else:
                if graph is None:
                    torch.cuda.synchronize()
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph):
                        outs_static = step()
                graph.replay()
                res = outs_static
            torch.cuda.synchronize()
            outs.append(torch.stack([o.clone() for o in res]).cpu())
            poss.append(be._positions[:2].clone().cpu())
            seq.add_(1)
        coord = be.coord
        results[mode] = (torch.stack(outs), torch.stack(poss), coord.buffer_tokens.cpu(), coord.lru_slots.cpu(),
                         coord.req_to_host_pool.cpu(), coord.host_k_all.clone(), coord._stats.cpu(),
                         coord.host_allocator.available_size())
        del rtp, kvp, be, coord
        torch.cuda.empty_cache()
    e, g = results["eager"], results["graph"]
    for t in range(steps):
        assert torch.equal(e[1][t], g[1][t]), f"step {t}: positions"
        assert torch.equal(e[0][t].view(torch.int16), g[0][t].view(torch.int16)), f"step {t}: outputs"
    for i, what in enumerate(("buffer_tokens", "lru_slots", "req_to_host_pool", "host tier", "counters"), start=2):
        assert torch.equal(e[i], g[i]), what
    assert e[7] == g[7]
    assert int(e[6][1]) > 0  # the hot buffer swapped


def test_swap_in_error_inside_a_replayed_graph_is_raised_by_the_poll():
    """A position without host backup (coordinator.py:284-286) met inside a replayed decode
    graph: no Python check runs during the replay, so the failed request shows as NaN outputs
    in every layer while the other request's stay finite, and the backend's non-blocking poll
    (poll_errors, the pinned error mirror) raises the reference's AssertionError once the
    replay has finished; the next poll is clean.  Request 1's hot buffer is emptied and its
    host rows cleared between two replays, so every position it selects is a miss without a
    host row."""
    from qwenquest_amd.attention.quest_hisparse import QuestHiSparseBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    H4, KV4, D4, TOPK, PAGE, BUF, CTX, L4 = 32, 4, 128, 256, 64, 384, 1200, 2
    prompts = (700, 1003)
    rtp = ReqToTokenPool(2, CTX, DEV)
    kvp = MHATokenToKVPool(2 * CTX, L4, KV4, D4, torch.bfloat16, DEV)
    g = torch.Generator(device=DEV).manual_seed(71)
    kvp.k_all.normal_(generator=g)
    kvp.v_all.normal_(generator=g)
    for r in (0, 1):
        rtp.req_to_token[r] = torch.arange(1 + r * CTX, 1 + (r + 1) * CTX, dtype=torch.int32)
    be = QuestHiSparseBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOPK, "quest_page_size": PAGE,
                                         "device_buffer_size": BUF}, host_pool_size=2 * CTX)
    be.on_extend_finished(ForwardBatch(ForwardMode.EXTEND, None, None, torch.tensor([0, 1]),
                                       torch.tensor(prompts), None, rtp, kvp, be))

    class Lay:
        def __init__(self, i):
            self.layer_id, self.scaling = i, D4**-0.5

    seq = torch.tensor([prompts[0] + 1, prompts[1] + 1], device=DEV, dtype=torch.int64)
    batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.tensor([0, 1], device=DEV), seq, None, rtp, kvp, be)
    q_in = torch.randn(L4, 2, H4, D4, generator=g, device=DEV).to(torch.bfloat16)
    k_in = torch.randn(L4, 2, KV4, D4, generator=g, device=DEV).to(torch.bfloat16)

    def step():
        be.init_forward_metadata(batch)
        return [be.forward_decode(q_in[i], k_in[i], k_in[i], Lay(i), batch) for i in range(L4)]

    for _ in range(2):  # eager steps first (workspaces, first-step skips)
        step()
        seq.add_(1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    graph.replay()
    torch.cuda.synchronize()
    be.poll_errors()  # a clean replay raises nothing
    assert all(bool(torch.isfinite(o).all()) for o in outs)
    seq.add_(1)
    coord = be.coord
    coord.buffer_tokens[:, 1] = -1
    coord.req_to_host_pool[1] = -1
    print("replay with request 1's host rows cleared", flush=True)
    graph.replay()
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        o = o.float().view(2, -1)
        assert bool(torch.isnan(o[1]).all()), f"layer {i}: the failed request's output is not NaN"
        assert bool(torch.isfinite(o[0]).all()), f"layer {i}: the other request's output is not finite"
    with pytest.raises(AssertionError, match="without host backup"):
        be.poll_errors()
    be.poll_errors()  # raised once: the mirror is cleared
    coord.check_errors()  # and so is the device word
