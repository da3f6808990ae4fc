"""qq_quest_forward_decode_noalloc (its scratch in a fixed per-device array)
against qq_quest_forward_decode with caller workspaces, both through the C ABI
on the same inputs: positions and attention outputs bit-identical, over two
calls in a row, the second with a smaller batch - for the fused layer-step
shape (bf16, 32 q / 4 KV heads x 128, page 64, top_k 2048) and for a shape the
four-launch path takes (8 q / 2 KV heads x 64, page 16, top_k 128)."""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)

# (q heads, kv heads, head_dim, page, top_k, ctx, prompt lengths per request)
SHAPES = [
    (32, 4, 128, 64, 2048, 9000, [8800, 2046, 5000, 3000]),
    (8, 2, 64, 16, 128, 1200, [1100, 127, 600, 900]),
]


def _setup(H, KV, D, P, TOP_K, CTX, prompts):
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    nreq = len(prompts)
    rtp = ReqToTokenPool(nreq, CTX, DEV)
    kvp = MHATokenToKVPool(nreq * CTX, 1, KV, D, torch.bfloat16, DEV)
    be = QuestOnlyBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P})
    g = torch.Generator(device=DEV).manual_seed(77)
    kvp.k_all.normal_(generator=g)
    kvp.v_all.normal_(generator=g)
    for r, n in enumerate(prompts):
        rtp.req_to_token[r] = torch.arange(1 + r * CTX, 1 + (r + 1) * CTX, dtype=torch.int32)
        be.quest.update_prefill_representations_fused(r, kvp.k_all, rtp.req_to_token[r, :n])
    return rtp, kvp, be


def _inputs(be, rtp, kvp, H, reqs, seqs, seed):
    """One layer's inputs, the step layout (prepare_step) and the output buffers (positions
    -7, outputs 3.0), kept alive in a dict; "head" is the argument list both entry points
    share."""
    from qwenquest_amd import _lib

    quest = be.quest
    bs = len(reqs)
    D, KV = kvp.head_dim, kvp.kv_heads
    g = torch.Generator(device=DEV).manual_seed(seed)
    t = {}
    t["q"] = torch.randn((bs, H, D), generator=g, device=DEV).to(torch.bfloat16)
    t["kn"] = torch.randn((bs, KV * D), generator=g, device=DEV).to(torch.bfloat16)
    t["vn"] = torch.randn((bs, KV * D), generator=g, device=DEV).to(torch.bfloat16)
    t["rpi"] = torch.tensor(reqs, device=DEV, dtype=torch.int64)
    seq = torch.tensor(seqs, device=DEV, dtype=torch.int64)
    t["loc"] = (1 + t["rpi"] * rtp.max_context_len + seq - 1).contiguous()
    t["step"] = step = quest.prepare_step(seq)
    t["positions"] = torch.full((bs, quest.top_k), -7, dtype=torch.int32, device=DEV)
    t["out"] = torch.full((bs, H * D), 3.0, dtype=torch.bfloat16, device=DEV)
    k_buf, v_buf = kvp.get_kv_buffer(0)
    r2t = rtp.req_to_token
    t["head"] = [
        _lib.ptr(t["q"]), _lib.DTYPE_BF16, t["q"].stride(0), H, _lib.ptr(t["kn"]), _lib.ptr(t["vn"]), _lib.DTYPE_BF16,
        _lib.ptr(t["loc"]), _lib.ptr(k_buf), _lib.ptr(v_buf), _lib.DTYPE_BF16, k_buf.shape[0],
        _lib.ptr(quest.page_k_bounds), 0, _lib.ptr(t["rpi"]), _lib.ptr(step.seq_lens),
        _lib.ptr(step.candidate_limit_i32), _lib.ptr(step.actual_lens), bs, quest.max_reqs,
        quest.max_pages_per_req, KV, D, quest.page_size, quest.top_k, _lib.ptr(r2t), r2t.stride(0),
        r2t.shape[0], float(D**-0.5),
    ]
    return t


def _launch(lib, noalloc, t, H, KV, D, quest):
    """Enqueue one call of either entry point on the current stream (no synchronisation)."""
    from qwenquest_amd import _lib

    bs = t["q"].shape[0]
    stream = _lib.stream(DEV)
    if noalloc:
        st = lib.qq_quest_forward_decode_noalloc(*t["head"], _lib.ptr(t["positions"]), _lib.ptr(t["out"]), stream)
    else:
        t["scores"] = torch.empty((bs, quest.max_pages_per_req), dtype=torch.float32, device=DEV)
        t["ws"] = torch.empty(int(lib.qq_decode_attention_workspace_bytes(bs, quest.top_k, H, D)),
                              dtype=torch.uint8, device=DEV)
        t["sync"] = torch.zeros(int(lib.qq_quest_layer_step_sync_bytes(bs, KV)), dtype=torch.uint8, device=DEV)
        st = lib.qq_quest_forward_decode(*t["head"], _lib.ptr(t["scores"]), _lib.ptr(t["positions"]),
                                         _lib.ptr(t["out"]), _lib.ptr(t["ws"]), t["ws"].numel(), _lib.ptr(t["sync"]),
                                         t["sync"].numel(), stream)
    _lib.check(st)


def _call(lib, noalloc, be, rtp, kvp, H, reqs, seqs, seed):
    """One layer through either entry point; returns (positions, out) after a sync."""
    t = _inputs(be, rtp, kvp, H, reqs, seqs, seed)
    _launch(lib, noalloc, t, H, kvp.kv_heads, kvp.head_dim, be.quest)
    torch.cuda.synchronize()
    return t["positions"].cpu(), t["out"].cpu()


def test_noalloc_first_call_inside_a_graph_capture():
    """The process's first call of the entry point (the scratch address lookup and the
    counter clear) made while a HIP graph is being captured: every replay, with eager work
    and synchronisations between them, gives the workspace entry point's positions and
    outputs bit for bit, and so does an eager call afterwards.  (No other test calls this
    entry point before it: this file is collected last and this test comes first in it.)"""
    from qwenquest_amd import _lib

    lib = _lib.load()
    H, KV, D, P, TOP_K, CTX, prompts = SHAPES[0]
    rtp, kvp, be = _setup(H, KV, D, P, TOP_K, CTX, prompts)
    reqs, seqs = [0, 1, 2, 3], [p + 1 for p in prompts]
    pos_ref, out_ref = _call(lib, False, be, rtp, kvp, H, reqs, seqs, 5)
    t = _inputs(be, rtp, kvp, H, reqs, seqs, 5)
    torch.cuda.synchronize()
    print("capture: first noalloc call inside torch.cuda.graph", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _launch(lib, True, t, H, KV, D, be.quest)
    for rep in range(3):
        t["positions"].fill_(-7)
        t["out"].fill_(3.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(t["positions"].cpu(), pos_ref), f"replay {rep}: positions differ"
        assert torch.equal(t["out"].cpu().view(torch.int16), out_ref.view(torch.int16)), f"replay {rep}: outputs differ"
        _call(lib, False, be, rtp, kvp, H, [3, 1], [prompts[3] + 2, prompts[1] + 2], 6)  # eager work between
    pos, out = _call(lib, True, be, rtp, kvp, H, reqs, seqs, 5)
    assert torch.equal(pos, pos_ref) and torch.equal(out.view(torch.int16), out_ref.view(torch.int16))
    del g


@pytest.mark.parametrize("shape", range(len(SHAPES)))
def test_noalloc_matches_workspace_entry_point(shape):
    from qwenquest_amd import _lib

    lib = _lib.load()
    H, KV, D, P, TOP_K, CTX, prompts = SHAPES[shape]
    rtp, kvp, be = _setup(H, KV, D, P, TOP_K, CTX, prompts)
    # two calls in a row, the second with a smaller batch (and other requests and lengths)
    for reqs, seqs, seed in (([0, 1, 2, 3], [p + 1 for p in prompts], 5), ([3, 1], [prompts[3] + 2, prompts[1] + 2], 6)):
        print(f"shape {shape} batch {len(reqs)} seqs {seqs}", flush=True)
        pos_ref, out_ref = _call(lib, False, be, rtp, kvp, H, reqs, seqs, seed)
        pos, out = _call(lib, True, be, rtp, kvp, H, reqs, seqs, seed)
        assert torch.equal(pos, pos_ref), f"positions differ (batch {len(reqs)})"
        assert torch.equal(out.view(torch.int16), out_ref.view(torch.int16)), f"outputs differ (batch {len(reqs)})"
        assert not torch.equal(out_ref, torch.full_like(out_ref, 3.0))


def test_noalloc_takes_four_launch_batches_past_the_counter_region():
    """The hand-off counters (64 KiB of the array) serve only the fused layer step (4 KV
    heads): a four-launch shape whose batch would need more counters than that (80 requests
    x 8 KV heads x 128 B = 80 KiB) is accepted and equals the workspace entry point."""
    from qwenquest_amd import _lib

    lib = _lib.load()
    H, KV, D, P, TOP_K, CTX = 8, 8, 64, 16, 128, 400
    prompts = [200 + 3 * i for i in range(80)]
    assert 80 * KV * 128 > 64 << 10
    rtp, kvp, be = _setup(H, KV, D, P, TOP_K, CTX, prompts)
    reqs, seqs = list(range(80)), [p + 1 for p in prompts]
    print(f"four-launch shape, batch {len(reqs)}", flush=True)
    pos_ref, out_ref = _call(lib, False, be, rtp, kvp, H, reqs, seqs, 9)
    pos, out = _call(lib, True, be, rtp, kvp, H, reqs, seqs, 9)
    assert torch.equal(pos, pos_ref)
    assert torch.equal(out.view(torch.int16), out_ref.view(torch.int16))


def test_noalloc_rejects_sizes_beyond_its_scratch():
    """Validation happens before any device call: a batch whose partials exceed the
    array is refused with QQ_EINVAL and a message naming the limit."""
    from qwenquest_amd import _lib

    lib = _lib.load()
    assert lib.qq_quest_forward_decode_noalloc_max_bytes() == 16 << 20
    fake = ctypes.c_void_p(16)
    args = [fake, 0, 4096, 32, None, None, 0, None, fake, fake, 0, 100, fake, 0, fake, fake, fake, fake,
            512, 512, 2049, 4, 128, 64, 2048, fake, 131072, 512, 0.088, fake, fake, None]
    st = lib.qq_quest_forward_decode_noalloc(*args)
    assert st == _lib.QQ_EINVAL and b"fixed scratch" in lib.qq_last_error()
