"""Write the golden vectors under tests/golden/ from the reference implementation.

Run in the development container only (the reference tree is not present on
the GPU machines)::

    PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_golden.py

It imports the reference (wengyinqi/QwenQuest at /root/reference/src) solely
for the functions no closed form or known answer pins:

* ``QuestAlgorithm.page_scores`` - its fp32 summation order is torch's;
* ``QuestAlgorithm.retrieve_topk`` - torch.topk's choice and order;
* ``HiSparseCoordinator._swap_in_long`` - the multi-step LRU evolution.

Only inputs and outputs are saved (``.npz``, bf16 as uint16 bit patterns).
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

REF_SRC = "/root/reference/src"
OUT = os.path.dirname(os.path.abspath(__file__))


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def score_cases() -> None:
    """C1-shaped selection: 1 request, 8192 context, 32 q / 4 KV heads, D=128, bf16."""
    from qwenquest.quest import QuestAlgorithm

    H, KV, D, P, TOP_K, CTX = 32, 4, 128, 64, 2048, 8192
    gen = torch.Generator().manual_seed(20240601)
    k = torch.randn(CTX, KV, D, generator=gen).to(torch.bfloat16)
    queries = torch.randn(16, H, D, generator=gen).to(torch.bfloat16)
    seq_lens = [8192, 8150, 8129, 4200, 2049, 2048, 700]
    out: dict[str, np.ndarray] = {"queries": bits(queries), "seq_lens": np.array(seq_lens)}
    for avoid in (False, True):
        quest = QuestAlgorithm(top_k=TOP_K, page_size=P, device="cpu", avoid_recent_overlap=avoid)
        quest.init_storage(0, 1, 1, CTX, KV, D)
        quest.update_prefill_representations(0, 0, k, torch.arange(CTX, dtype=torch.int32))
        out["bounds"] = bits(quest.page_k_bounds[0, 0])
        pos_all, scores_all = [], []
        for s in seq_lens:
            quest.prepare_step(torch.tensor([s] * 16))
            pos, _ = quest.retrieve_topk(queries, 0, torch.zeros(16, dtype=torch.int64), torch.tensor([s] * 16))
            pos_all.append(pos.numpy())
            qbar = quest.group_queries(queries)
            scores_all.append(quest.page_scores(qbar, 0, torch.zeros(16, dtype=torch.int64)).numpy())
        out[f"positions_avoid{int(avoid)}"] = np.stack(pos_all)
        out["scores"] = np.stack(scores_all)
        out["qbar"] = bits(quest.group_queries(queries))
    np.savez_compressed(os.path.join(OUT, "c1_selection.npz"), **out)


def small_cases() -> None:
    """Reference-test shapes: KV=4, D=32, fp32 and bf16 queries, group sizes 1/4/8."""
    from qwenquest.quest import QuestAlgorithm

    KV, D = 4, 32
    out: dict[str, np.ndarray] = {}
    for case, (top_k, P, H, qdtype, n) in enumerate(
        [(256, 64, 4, torch.float32, 800), (128, 16, 16, torch.float32, 512),
         (64, 16, 32, torch.bfloat16, 500), (32, 8, 8, torch.float32, 300)]
    ):
        gen = torch.Generator().manual_seed(1000 + case)
        k = torch.randn(n, KV, D, generator=gen).to(torch.bfloat16)
        q = torch.randn(4, H, D, generator=gen).to(qdtype)
        quest = QuestAlgorithm(top_k=top_k, page_size=P, device="cpu")
        quest.init_storage(0, 1, 1, 1024, KV, D)
        quest.update_prefill_representations(0, 0, k, torch.arange(n, dtype=torch.int32))
        seq = torch.tensor([n, n - 3, n - P + 1, n // 2])
        quest.prepare_step(seq)
        pos, actual = quest.retrieve_topk(q, 0, torch.zeros(4, dtype=torch.int64), seq)
        qbar = quest.group_queries(q)
        out[f"c{case}_meta"] = np.array([top_k, P, H, int(qdtype == torch.bfloat16), n])
        out[f"c{case}_bounds"] = bits(quest.page_k_bounds[0, 0])
        out[f"c{case}_q"] = q.float().numpy()
        out[f"c{case}_qbar"] = qbar.float().numpy()
        out[f"c{case}_seq"] = seq.numpy()
        out[f"c{case}_scores"] = quest.page_scores(qbar, 0, torch.zeros(4, dtype=torch.int64)).numpy()
        out[f"c{case}_positions"] = pos.numpy()
        out[f"c{case}_actual"] = actual.numpy()
    np.savez_compressed(os.path.join(OUT, "small_selection.npz"), **out)


def swap_trace() -> None:
    """200 decode steps of one request through HiSparse: buf 16, top_k 8, page 1, duplicates."""
    from qwenquest.hisparse import HiSparseCoordinator
    from qwenquest.memory import MHATokenToKVPool
    from qwenquest.quest import QuestAlgorithm

    layers, kv, d, buf, top_k, ctx, prefill = 2, 2, 8, 16, 8, 256, 20
    quest = QuestAlgorithm(top_k=top_k, page_size=1, device="cpu")
    quest.init_storage(0, layers, 1, ctx, kv, d)
    coord = HiSparseCoordinator(
        quest=quest, num_layers=layers, kv_heads=kv, head_dim=d, max_reqs=1,
        max_context_len=ctx, top_k=top_k, device_buffer_size=buf, host_pool_size=ctx,
        dtype=torch.float32, device="cpu",
    )
    pool = MHATokenToKVPool(ctx, layers, kv, d, torch.float32, "cpu")
    gen = torch.Generator().manual_seed(5)
    kk = torch.randn(layers, ctx, kv, d, generator=gen)
    vv = torch.randn(layers, ctx, kv, d, generator=gen)
    locs = torch.arange(1, prefill + 1)
    for layer in range(layers):
        pool.set_kv_buffer(layer, locs, kk[layer, :prefill], vv[layer, :prefill])
    coord.admit_request(0, prefill, pool, locs)
    sel_all, rows_all, tok_all, lru_all, stats_all, host_all = [], [], [], [], [], []
    for pos in range(prefill, prefill + 200):
        reqs, seq_lens = torch.tensor([0]), torch.tensor([pos + 1])
        coord.prepare_decode_step(reqs, seq_lens)
        for layer in range(layers):
            coord.write_new_token(layer, reqs, seq_lens, kk[layer, pos : pos + 1], vv[layer, pos : pos + 1])
        seq_len = pos + 1
        for layer in range(layers):
            sel = torch.randint(0, seq_len, (top_k,), generator=gen)
            sel[-1] = seq_len - 1
            sel[0] = sel[1]
            if pos % 7 == 0:  # a recent-window style run of consecutive positions
                sel[2:6] = torch.arange(seq_len - 5, seq_len - 1)
            rows = coord.swap_in_selected_pages(reqs, seq_lens, sel[None].int(), layer)
            assert torch.equal(coord.device_k[layer][rows[0]], kk[layer, sel])
            sel_all.append(sel.numpy())
            rows_all.append(rows[0].numpy())
            tok_all.append(coord.buffer_tokens[layer, 0].numpy().copy())
            lru_all.append(coord.lru_slots[layer, 0].numpy().copy())
            stats_all.append([coord.stats.hits, coord.stats.misses])
        host_all.append(coord.req_to_host_pool[0, :seq_len].numpy().copy())
    np.savez_compressed(
        os.path.join(OUT, "swap_trace.npz"),
        meta=np.array([layers, buf, top_k, ctx, prefill]),
        selections=np.stack(sel_all), rows=np.stack(rows_all), tokens=np.stack(tok_all),
        lru=np.stack(lru_all), stats=np.array(stats_all),
        host_rows_final=host_all[-1],
    )


def main() -> None:
    sys.path.insert(0, REF_SRC)
    torch.set_num_threads(1)
    score_cases()
    small_cases()
    swap_trace()
    for name in sorted(os.listdir(OUT)):
        if name.endswith(".npz"):
            print(name, os.path.getsize(os.path.join(OUT, name)))


if __name__ == "__main__":
    main()
