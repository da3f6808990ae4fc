"""Quest decode layer-step benchmark on one MI355X.

Workload (default): batch 16, every request at 128K context (131072 tokens),
Qwen3-30B-A3B attention shape (32 q heads, 4 KV heads, head_dim 128, bf16),
Quest page 64, top_k 2048 (31 pages + recent 64), quest mode: all 48 layers'
K/V pools (about 192 GiB) and page bounds (3 GiB) resident in HBM, inputs
synthetic N(0, 1) from fixed seeds.

One step = one decode step of all 48 layers through the drop-in backend:
bounds append (fused over layers) + per layer two launches: GQA-mean page
scoring + new K/V write, then per-request top-31 selection, layout,
req_to_token gather and attention.  The step is captured once in a HIP graph
and replayed; seq_lens advance by one token per replay, so pages complete and
get finalized during the run.  Reported value: microseconds per layer-step
(step time / 48).  The roofline's `traffic` is read from the committed
rocprofv3 PMC summary in profiles/ (copy-calibrated FETCH_SIZE + WRITE_SIZE),
and only when the summary records the hash of the HIP sources this build has.
After the timed region the same line gets `cpu_baseline` (the reference's op
sequence in torch on the host cores, on the GPU's own layer-0 tensors) and
`hisparse` (the quest_hisparse tier below, 4 layers, graph-replayed).

    python bench.py [--steps K] [--warmup W]

`--ragged` draws each request's context uniform in [8192, ctx] (seeded) instead.
`--hisparse` measures the quest_hisparse tier instead (batch 16, 128K context,
a hot buffer of 4096 + 1 rows per request and layer, the full K/V history in
pinned host memory, queries AR(1) with rho 0.9 across steps): swap-in rows per
layer-step, the swap-in's H2D rate next to the pinned hipMemcpy H2D peak
measured in the same run, and the decode time per layer-step.  Its pinned host
tier holds `--hisparse-layers` layers (default 4; the per-layer work is the
same for all 48).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
PROFILE = os.path.join(ROOT, "profiles", "quest_layer_step_kernels_b16_128k.md")


def sources_sha16() -> str:
    """Hash of the HIP sources the library is built from (qwenquest_amd/csrc)."""
    import glob
    import hashlib

    h = hashlib.sha256()
    for f in sorted(glob.glob(os.path.join(ROOT, "qwenquest_amd", "csrc", "*"))):
        if f.endswith((".hip", ".h")):
            h.update(os.path.basename(f).encode())
            h.update(open(f, "rb").read())
    return h.hexdigest()[:16]


def profiled_traffic() -> tuple[dict, dict]:
    """HBM bytes per launch of each layer-step kernel from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, copy-calibrated), and its provenance: the summary records the
    hash of the sources it was measured on, and the figures are used only when it matches the
    sources of this build ({} otherwise: a stale profile prints no traffic)."""
    traffic, recorded = {}, None
    try:
        for line in open(PROFILE):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = {k: int(v) for k, v in (kv.split("=") for kv in line.split(":", 1)[1].split())}
            elif line.startswith("sources_sha16:"):
                recorded = line.split(":", 1)[1].strip()
    except OSError:
        pass
    current = sources_sha16()
    source = {"file": os.path.relpath(PROFILE, ROOT), "sources_sha16": recorded, "build_sources_sha16": current,
              "sources_match": recorded == current}
    return (traffic if recorded == current else {}), source


class Layer:
    def __init__(self, layer_id: int, scaling: float):
        self.layer_id, self.scaling = layer_id, scaling


def algorithmic_bytes(seqs, page: int, top_k: int, row_bytes: int, page_bytes: int) -> dict:
    """Per layer-step: bounds of complete pages + K/V of the attended rows (+ small terms)."""
    bounds = sum((s // page) * page_bytes for s in seqs)
    kv = sum(min(s, top_k) * row_bytes for s in seqs)
    return {"bounds": bounds, "kv": kv, "headline": bounds + kv}


def time_graph(fn, reps: int, stream) -> float:
    """Average ms of one call of fn, from a graph holding `reps` calls, timed with HIP events."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(3):
        g.replay()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / (3 * reps)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(be, q, batch, top_k: int, page: int, scaling: float, reps: int = 20, warmup: int = 3) -> dict:
    """The reference's op sequence on the host cores (oracle/torch_path.py: group_queries ->
    page_scores -> masked topk -> req_to_token gather -> fp32 decode_attention, torch CPU
    kernels), on the same tensors the GPU holds for layer 0 (copied to host memory), with
    every core of this process's CPU set; the median of `reps` timed layer-steps after
    `warmup` untimed ones.  Also reports whether its positions equal the GPU's for that
    layer (torch.topk's tie order aside, they must)."""
    from oracle import torch_path as tp

    threads = max(1, min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "0")) or 1 << 30))
    torch.set_num_threads(threads)
    quest = be.quest
    pool = be.token_to_kv_pool
    bounds = quest.page_k_bounds[0].cpu()
    k_buf, v_buf = pool.k_all[0].cpu(), pool.v_all[0].cpu()
    r2t = be.req_to_token.cpu()
    qc = q.cpu()
    rpi = batch.req_pool_indices.cpu()
    seq = batch.seq_lens.cpu()
    times = []
    for i in range(warmup + reps):
        t0 = time.perf_counter()
        pos, actual, _ = tp.layer_step(qc, bounds, rpi, seq, r2t, k_buf, v_buf, page, top_k, scaling)
        if i >= warmup:
            times.append(time.perf_counter() - t0)
    gpu_pos = be._positions[: qc.shape[0]].cpu()
    same = all(torch.equal(pos[i, : int(actual[i])], gpu_pos[i, : int(actual[i])]) for i in range(qc.shape[0]))
    return {"us": float(np.median(times)) * 1e6, "threads": threads, "reps": reps, "warmup": warmup,
            "positions_equal_gpu": bool(same)}


def pinned_h2d_peak(nbytes: int = 1 << 30, reps: int = 5, d2h: bool = False) -> float:
    """GB/s of hipMemcpy (torch copy) from pinned host memory into device memory (d2h: the
    other way)."""
    src = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    if d2h:
        src, dst = dst, src
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src, non_blocking=True)
    e1.record()
    e1.synchronize()
    return nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9


def hisparse_measure(B: int, S: int, L: int, warmup: int, steps: int, event_steps: int, route: str = "kernel") -> dict:
    """quest_hisparse decode (QuestHiSparseBackend, the drop-in path) at batch B x S tokens, a
    hot buffer of 4096 + 1 rows per request and layer, the K/V history of L layers in pinned
    host memory, queries AR(1) with rho 0.9 across steps.  After `warmup` eager steps, one
    decode step (bounds fold + eager backup + per layer new token, selection, swap-in and
    attention) is captured in a HIP graph and replayed for `steps` timed steps (µs per
    layer-step); `event_steps` more steps run eagerly with HIP events around every swap-in
    call (plan + copy) on the launch stream, for the swap-in time and the missed rows.
    route "memcpy": the swap-in's copy through the copy engines (QuestHiSparseBackend
    swap_route="memcpy": a host synchronisation per swap-in, so no graph; the `steps` timed
    steps run eagerly with HIP events around each step)."""
    from qwenquest_amd.attention.quest_hisparse import QuestHiSparseBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    dev = torch.device("cuda", 0)
    H, KV, D, P, TOP_K, BUF = 32, 4, 128, 64, 2048, 4096
    total = warmup + steps + event_steps + 2
    max_ctx = S + total + 64
    t_setup = time.perf_counter()
    R = B + 1  # one more request slot: admitted while the B requests decode
    rtp = ReqToTokenPool(R, max_ctx, dev)
    kvp = MHATokenToKVPool(R * max_ctx, L, KV, D, torch.bfloat16, dev)
    gen = torch.Generator(device=dev).manual_seed(4321)
    for layer in range(L):
        kvp.k_all[layer].normal_(generator=gen)
        kvp.v_all[layer].normal_(generator=gen)
    base = 1 + torch.arange(R, device=dev, dtype=torch.int64) * max_ctx
    rtp.req_to_token.copy_((base[:, None] + torch.arange(max_ctx, device=dev)[None]).to(torch.int32))
    be = QuestHiSparseBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P,
                                         "device_buffer_size": BUF}, host_pool_size=R * max_ctx, swap_route=route,
                              async_admission=True)
    prompt = S - 1
    pre = ForwardBatch(ForwardMode.EXTEND, None, None, torch.arange(B), torch.full((B,), prompt), None, rtp, kvp, be)
    # admission of the B prompts: K/V backup to the pinned host tier (device -> host over
    # PCIe, on the admission stream), the first rows of the hot buffer, the bounds build
    # (coordinator.py:138-174); timed until the backups are done
    torch.cuda.synchronize()
    a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a0.record()
    be.on_extend_finished(pre)
    be.coord.wait_admission()
    a1.record()
    torch.cuda.synchronize()
    admit_ms = a0.elapsed_time(a1)
    setup_s = time.perf_counter() - t_setup

    coord = be.coord
    layers = [Layer(i, D**-0.5) for i in range(L)]
    rho = 0.9
    q = torch.randn((L, B, H, D), generator=gen, device=dev)
    q_in = torch.empty((L, B, H, D), dtype=torch.bfloat16, device=dev)
    kv_in = torch.empty((2, L, B, KV, D), dtype=torch.bfloat16, device=dev)
    seq = torch.full((B,), S, device=dev, dtype=torch.int64)
    batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.arange(B, device=dev), seq, None, rtp, kvp, be)

    def next_inputs():
        q.mul_(rho).add_(torch.randn((L, B, H, D), generator=gen, device=dev), alpha=(1 - rho**2) ** 0.5)
        q_in.copy_(q)
        kv_in.copy_(torch.randn((2, L, B, KV, D), generator=gen, device=dev))

    def step():
        be.init_forward_metadata(batch)
        return [be.forward_decode(q_in[i], kv_in[0, i], kv_in[1, i], layers[i], batch) for i in range(L)]

    for _ in range(warmup):
        next_inputs()
        step()
        seq.add_(1)
    torch.cuda.synchronize()
    use_graph = route == "kernel"
    graph = None
    if use_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    step_ms = []
    m0 = coord.stats.misses
    for _ in range(steps):
        next_inputs()
        e0.record(stream)
        if use_graph:
            graph.replay()
        else:
            step()
        e1.record(stream)
        e1.synchronize()
        step_ms.append(e0.elapsed_time(e1))
        seq.add_(1)
    graph_misses = coord.stats.misses - m0
    # eager steps with events around the swap-in calls
    swap = coord.swap_in_selected_pages
    events = []

    def timed_swap(*a, **kw):
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        rows = swap(*a, **kw)
        s1.record()
        events.append((s0, s1))
        return rows

    coord.swap_in_selected_pages = timed_swap
    swap_ms, misses = [], []
    for _ in range(event_steps):
        next_inputs()
        m0 = coord.stats.misses
        events.clear()
        step()
        torch.cuda.synchronize()
        swap_ms.append(sum(a.elapsed_time(b) for a, b in events))
        misses.append(coord.stats.misses - m0)
        seq.add_(1)
    coord.swap_in_selected_pages = swap
    overlap = None
    if use_graph:
        # one more request (slot B, a prompt of S-1 tokens) admitted while the B requests keep
        # decoding: its backup runs on the admission stream, the decode graph on this one
        torch.cuda.synchronize()
        side = coord._adm_stream
        b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        b0.record(side)
        coord.admit_request(B, prompt, kvp, rtp.req_to_token[B, :prompt])
        b1.record(side)
        ends = []
        for _ in range(16):
            next_inputs()
            s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s0.record(stream)
            graph.replay()
            s1.record(stream)
            ends.append((s0, s1))
            seq.add_(1)
        torch.cuda.synchronize()
        backup_ms = b0.elapsed_time(b1)
        during = [a.elapsed_time(b) for a, b in ends if b0.elapsed_time(b) <= backup_ms]
        coord.wait_admission(B)
        overlap = {
            "request_tokens": prompt,
            "layers": L,
            "backup_ms": round(backup_ms, 2),
            "backup_d2h_gbs": round(prompt * L * 2 * KV * D * 2 / (backup_ms * 1e-3) / 1e9, 2),
            "decode_steps_within_backup": len(during),
            "decode_us_per_layer_step_within_backup": round(float(np.mean(during)) * 1e3 / L, 2) if during else None,
            "decode_us_per_layer_step_alone": round(float(np.mean(step_ms)) * 1e3 / L, 2),
        }
    cpu_plan = hisparse_cpu_baseline(coord, be, step, next_inputs, seq, B, TOP_K, BUF)
    row_bytes = 2 * KV * D * 2  # K + V row
    miss_rows = float(np.mean(misses)) / L
    swap_us = float(np.mean(swap_ms)) * 1e3 / L
    h2d = miss_rows * row_bytes / (swap_us * 1e-6) / 1e9 if swap_us > 0 else 0.0
    peak = pinned_h2d_peak()
    d2h_peak = pinned_h2d_peak(d2h=True)
    admit_bytes = B * prompt * L * row_bytes
    admit_gbs = admit_bytes / (admit_ms * 1e-3) / 1e9
    st = coord.stats
    res = {
        "us_per_layer_step": round(float(np.mean(step_ms)) * 1e3 / L, 2),
        "graph": use_graph,
        "swap_route": route,
        "swap_in_rows_per_layer_step": round(miss_rows, 1),
        "graph_swap_in_rows_per_layer_step": round(graph_misses / steps / L, 1),
        "swap_in_us_per_layer_step": round(swap_us, 2),
        "h2d_gbs": round(h2d, 2),
        "h2d_pinned_memcpy_peak_gbs": round(peak, 2),
        "h2d_frac_of_memcpy_peak": round(h2d / peak, 4) if peak > 0 else None,
        "h2d_frac_of_64gbs_nominal": round(h2d / 64.0, 4),
        "hit_rate": round(st.hit_rate, 4),
        "cpu_baseline_swap_in": cpu_plan,
        "admission": {
            "requests": B,
            "tokens_per_request": prompt,
            "layers": L,
            "ms": round(admit_ms, 2),
            "d2h_gbs": round(admit_gbs, 2),
            "d2h_pinned_memcpy_peak_gbs": round(d2h_peak, 2),
            "d2h_frac_of_memcpy_peak": round(admit_gbs / d2h_peak, 4) if d2h_peak > 0 else None,
            "what": "on_extend_finished for the batch: every prompt's K and V rows backed up to the pinned host "
                    "tier through the copy engines on the admission stream (the d2h bytes), the first hot-buffer "
                    "rows and the page bounds built on the device, all inside the timed region; overlap: one more "
                    "prompt admitted while the batch's decode graph is replayed",
            "overlap": overlap,
        },
        "workload": f"quest_hisparse decode, batch {B}, {S}-token context, hot buffer {BUF}+1 rows, {L} layers' "
                    f"history in pinned host memory (the per-layer work is the same for all 48), AR(1) queries "
                    f"rho 0.9; {warmup} warm-up steps, {steps} {'graph-replayed' if use_graph else 'eager'} timed "
                    f"steps, {event_steps} eager steps with events around the swap-in; swap-in copy: "
                    f"{'copy kernel reading pinned host memory' if use_graph else 'hipMemcpyAsync per run of host rows on a side stream + scatter'}",
        "setup_s": round(setup_s, 1),
    }
    del be, coord, kvp, rtp, graph
    torch.cuda.empty_cache()
    return res


def hisparse_cpu_baseline(coord, be, step, next_inputs, seq, B: int, top_k: int, buf: int, reps: int = 20) -> dict:
    """The reference's swap-in on the host (coordinator.py:232-304 restated in numpy:
    oracle/hisparse.py's planner, then the misses' K and V rows copied host tier -> hot buffer
    with numpy) for one layer-step: the B requests of layer 0 in one decode step, from the
    state the GPU's swap-in started from (buffer_tokens, lru_slots, req_to_host_pool, the
    selected positions), median of `reps` after 3 warm-ups on the host cores.  The planned
    rows are checked against the GPU's."""
    from oracle import hisparse as oh

    cap = {}
    swap = coord.swap_in_selected_pages

    def capture(reqs, seqs, positions, layer_id, **kw):
        if layer_id == 0 and not cap:
            cap["tokens"] = coord.buffer_tokens[0].cpu().numpy().copy()
            cap["lru"] = coord.lru_slots[0].cpu().numpy().copy()
            cap["r2h"] = coord.req_to_host_pool.cpu().numpy()
            cap["pos"] = positions.cpu().numpy().astype(np.int64)
            cap["seq"] = seqs.cpu().numpy().astype(np.int64)
            cap["reqs"] = reqs.cpu().numpy().astype(np.int64)
            rows = swap(reqs, seqs, positions, layer_id, **kw)
            cap["rows"] = rows.cpu().numpy().copy()
            return rows
        return swap(reqs, seqs, positions, layer_id, **kw)

    coord.swap_in_selected_pages = capture
    next_inputs()
    step()
    torch.cuda.synchronize()
    seq.add_(1)
    coord.swap_in_selected_pages = swap
    host_k = coord.host_k_all[0].view(torch.int16).numpy()  # bf16 rows as raw 16-bit words
    host_v = coord.host_v_all[0].view(torch.int16).numpy()
    hot_k = np.empty((B * (buf + 1),) + host_k.shape[1:], dtype=host_k.dtype)
    hot_v = np.empty_like(hot_k)

    def plan_and_copy():
        rows = np.full((B, top_k), -1, dtype=np.int64)
        for b in range(B):
            req, s = int(cap["reqs"][b]), int(cap["seq"][b])
            n = min(s, top_k)
            plan = oh.swap_in_long(cap["tokens"][req], cap["lru"][req], cap["pos"][b, :n], s, cap["r2h"][req])
            base = req * (buf + 1)
            rows[b, :n] = base + plan.slots
            if plan.copies:
                victims = base + np.array([c[0] for c in plan.copies])
                hidx = np.array([c[1] for c in plan.copies])
                hot_k[victims] = host_k[hidx]
                hot_v[victims] = host_v[hidx]
        return rows

    for _ in range(3):
        rows = plan_and_copy()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        plan_and_copy()
        times.append(time.perf_counter() - t0)
    return {"value": round(float(np.median(times)) * 1e6, 1), "unit": "us per layer-step (16 requests' swap-in)",
            "cores": 1, "kind": "port", "rows_equal_gpu": bool(np.array_equal(rows, cap["rows"])),
            "sample": "one layer-step: the LRU planner of the reference (numpy restatement) and the misses' K/V "
                      "row copies (numpy) for all requests of layer 0 in one decode step, from the GPU's state "
                      f"before its swap-in; median of {reps} after 3 warm-ups, one thread"}


def hisparse_bench(args) -> int:
    torch.cuda.set_device(0)
    r = hisparse_measure(args.batch, args.ctx, args.hisparse_layers, args.warmup, args.steps, args.steps,
                         route=args.hisparse_route)
    print(json.dumps({
        "metric": "quest_hisparse decode @128K ctx, batch 16: swap-in H2D GB/s and us per layer-step",
        "value": r["h2d_gbs"], "unit": "GB/s (swap-in misses x 2 KiB / swap-in time)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
        "dtype": "bf16", "data": "synthetic N(0,1) K/V, AR(1) queries rho 0.9, fixed seeds",
        "config": {"workload": r["workload"], "batch": args.batch, "seq_len": args.ctx,
                   "layers": args.hisparse_layers},
        **{k: v for k, v in r.items() if k != "workload"},
    }))
    return 0


def dense_bench(args) -> int:
    """Dense decode (every request attends its whole context, attention/dense.py:26-42) on the
    same batch and contexts: the comparator the Quest layer step is measured against."""
    from qwenquest_amd import _lib
    from qwenquest_amd.attention.dense import DenseBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, S, L = args.batch, args.ctx, args.dense_layers
    H, KV, D = 32, 4, 128
    total_steps = args.warmup + args.steps + 2
    span = S + total_steps + 64
    max_ctx = span
    rows = B * span
    t_setup = time.perf_counter()
    rtp = ReqToTokenPool(B, max_ctx, dev)
    kvp = MHATokenToKVPool(rows, L, KV, D, torch.bfloat16, dev)
    gen = torch.Generator(device=dev).manual_seed(1234)
    for layer in range(L):
        kvp.k_all[layer].normal_(generator=gen)
        kvp.v_all[layer].normal_(generator=gen)
    base = 1 + torch.arange(B, device=dev, dtype=torch.int64) * span
    rtp.req_to_token.copy_((base[:, None] + torch.arange(max_ctx, device=dev)[None]).to(torch.int32))
    be = DenseBackend(rtp, kvp)
    q_all = torch.randn((L, B, H, D), generator=gen, device=dev).to(torch.bfloat16)
    k_new = torch.randn((L, B, KV, D), generator=gen, device=dev).to(torch.bfloat16)
    v_new = torch.randn((L, B, KV, D), generator=gen, device=dev).to(torch.bfloat16)
    layers = [Layer(i, D**-0.5) for i in range(L)]
    seq_lens = torch.full((B,), S, device=dev, dtype=torch.int64)
    out_loc = torch.empty(B, device=dev, dtype=torch.int64)
    batch = ForwardBatch(ForwardMode.DECODE, None, None, torch.arange(B, device=dev), seq_lens, out_loc, rtp, kvp, be)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup

    def step():
        torch.add(base, seq_lens - 1, out=out_loc)
        for layer in range(L):
            be.forward_decode(q_all[layer], k_new[layer], v_new[layer], layers[layer], batch)
        seq_lens.add_(1)

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    us_per_layer_step = (time.perf_counter() - t0) * 1e6 / args.steps / L
    seq_mid = S + 1 + args.warmup + args.steps // 2
    kv_bytes = B * seq_mid * 2 * KV * D * 2
    line = {
        "metric": "µs per dense decode layer-step @128K ctx, batch 16 (comparator of the Quest layer step)",
        "value": round(us_per_layer_step, 2),
        "unit": "us per layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "higher_is_better": False,
        "dtype": "bf16",
        "data": "synthetic N(0,1) q/k/v, fixed seeds",
        "config": {"workload": f"dense decode, batch {B}, {S}-token context, {L} layers cycled, "
                               f"32q/4kv heads x 128", "batch": B, "seq_len": S, "layers": L},
        "algorithmic_bytes_per_layer_step": kv_bytes,
        "hbm_frac_layer_step": round(kv_bytes / (us_per_layer_step * 1e-6) / (HBM_PEAK_GBS * 1e9), 4),
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(line))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--ctx", type=int, default=131072)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--cpu-reps", type=int, default=20, help="timed CPU-baseline layer-steps (0 = skip)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB three times (scale for the HBM byte counters)")
    ap.add_argument("--ragged", action="store_true",
                    help="contexts drawn uniform in [8192, ctx] per request (seeded) instead of all ctx")
    ap.add_argument("--hisparse", action="store_true", help="measure the quest_hisparse tier instead")
    ap.add_argument("--hisparse-layers", type=int, default=4)
    ap.add_argument("--hisparse-route", choices=("kernel", "memcpy"), default="kernel",
                    help="--hisparse: the swap-in's host -> device copy (memcpy: hipMemcpyAsync per run on a side stream)")
    ap.add_argument("--hisparse-steps", type=int, default=48,
                    help="graph-replayed quest_hisparse steps measured after the headline (0 = skip)")
    ap.add_argument("--dense", action="store_true",
                    help="measure dense decode (every request attends its whole context) instead")
    ap.add_argument("--dense-layers", type=int, default=8, help="K/V pools of the dense run (cycled)")
    args = ap.parse_args()
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        src.fill_(1)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "copies": 3}))
        return 0
    if args.gpus != 1:
        print("bench.py measures one GPU: the path shards by request with no cross-GPU traffic, "
              "and this build runs on a single MI355X; use --gpus 1", file=sys.stderr)
        return 2
    if args.hisparse:
        return hisparse_bench(args)
    if args.dense:
        return dense_bench(args)

    from qwenquest_amd import _lib
    from qwenquest_amd.attention.quest_only import QuestOnlyBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, S, L = args.batch, args.ctx, args.layers
    H, KV, D, P, TOP_K = 32, 4, 128, 64, 2048
    total_steps = args.warmup + args.steps + 2
    ctxs = (np.random.default_rng(2024).integers(8192, S, size=B, endpoint=True) if args.ragged
            else np.full(B, S, dtype=np.int64))
    max_ctx = int(ctxs.max()) + total_steps + 64
    # request r's rows follow r-1's: its context plus room for the decode steps
    span = ctxs + total_steps + 64
    starts = 1 + np.concatenate([[0], np.cumsum(span)[:-1]])
    rows = int(span.sum())

    t_setup = time.perf_counter()
    rtp = ReqToTokenPool(B, max_ctx, dev)
    kvp = MHATokenToKVPool(rows, L, KV, D, torch.bfloat16, dev)
    gen = torch.Generator(device=dev).manual_seed(1234)
    for layer in range(L):
        kvp.k_all[layer].normal_(generator=gen)
        kvp.v_all[layer].normal_(generator=gen)
    base = torch.tensor(starts, device=dev, dtype=torch.int64)
    rtp.req_to_token.copy_((base[:, None] + torch.arange(max_ctx, device=dev)[None]).clamp(max=rows).to(torch.int32))
    be = QuestOnlyBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P})
    # the prefill bounds build of requests 1 .. B-1 is timed with HIP events (request 0 warms up)
    pf0, pf1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for r in range(B):
        # prefill covers positions [0, ctx - 1); the first decode step has seq_len ctx
        be.quest.update_prefill_representations_fused(r, kvp.k_all, rtp.req_to_token[r, : int(ctxs[r]) - 1])
        be._skip_first_decode_update[r] = True
        if r == 0:
            pf0.record()
    pf1.record()
    q_all = torch.randn((L, B, H, D), generator=gen, device=dev).to(torch.bfloat16)
    k_new = torch.randn((L, B, KV, D), generator=gen, device=dev).to(torch.bfloat16)
    v_new = torch.randn((L, B, KV, D), generator=gen, device=dev).to(torch.bfloat16)
    layers = [Layer(i, D**-0.5) for i in range(L)]
    rpi = torch.arange(B, device=dev, dtype=torch.int64)
    seq_lens = torch.tensor(ctxs, device=dev, dtype=torch.int64)
    out_loc = torch.empty(B, device=dev, dtype=torch.int64)
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t_setup
    prefill = None
    if B > 1:
        pf_us = pf0.elapsed_time(pf1) * 1e3
        pf_bytes = float(sum(int(c) - 1 for c in ctxs[1:])) * L * KV * D * 2  # every prompt key read once
        prefill = {"kernel": "prefill_bounds_wave_kernel", "requests": B - 1, "layers": L,
                   "tokens_per_request": int(ctxs[1:].mean()) - 1, "us_per_request": round(pf_us / (B - 1), 1),
                   "gbs": round(pf_bytes / (pf_us * 1e-6) / 1e9, 1),
                   "hbm_frac": round(pf_bytes / (pf_us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4)}

    batch = ForwardBatch(ForwardMode.DECODE, None, None, rpi, seq_lens, out_loc, rtp, kvp, be)

    def step():
        torch.add(base, seq_lens - 1, out=out_loc)
        be.init_forward_metadata(batch)
        for layer in range(L):
            be.forward_decode(q_all[layer], k_new[layer], v_new[layer], layers[layer], batch)
        seq_lens.add_(1)

    stream = torch.cuda.current_stream()
    step()  # eager: first decode step after prefill (bounds fold skipped), allocates workspaces
    torch.cuda.synchronize()
    if args.no_graph:
        run = step
    else:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        run = graph.replay
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    us_per_layer_step = ms_per_step * 1e3 / L

    seqs_timed = [int(c) + 1 + args.warmup + args.steps // 2 for c in ctxs]
    byts = algorithmic_bytes(seqs_timed, P, TOP_K, 2 * KV * D * 2, KV * D * 2 * 2)
    step_frac = byts["headline"] / (us_per_layer_step * 1e-6) / (HBM_PEAK_GBS * 1e9)

    # per-kernel durations of the layer step's two launches (scores, selection + attention),
    # each from a graph of L launches over the L layers in turn (so that no launch finds its
    # bounds or K/V rows in a cache, as in the step), HIP events on the launch stream
    torch.add(base, seq_lens - 1, out=out_loc)
    be.quest.prepare_step(seq_lens)
    turn = {"sel": 0, "att": 0}

    def score():
        i = turn["sel"] % L
        turn["sel"] += 1
        be.forward_decode_phase(q_all[i], k_new[i], v_new[i], layers[i], batch, 1)

    def attend():
        i = turn["att"] % L
        turn["att"] += 1
        be.forward_decode_phase(q_all[i], k_new[i], v_new[i], layers[i], batch, 2)

    ms_sel = time_graph(score, L, stream)
    ms_att = time_graph(attend, L, stream)
    bw_sel = byts["bounds"] / (ms_sel * 1e-3) / 1e9
    bw_att = byts["kv"] / (ms_att * 1e-3) / 1e9
    dominant = ("quest_attend_unit_kernel", ms_att, byts["kv"], bw_att) if ms_att >= ms_sel else (
        "score_pages_fast_kernel", ms_sel, byts["bounds"], bw_sel)

    cpu = None
    if args.cpu_reps > 0:
        # the GPU's own state for layer 0 after the timed steps: run that layer once more so
        # its positions are in the backend's buffer, then the same layer-step on the host
        be.quest.prepare_step(seq_lens)
        be.forward_decode(q_all[0], k_new[0], v_new[0], layers[0], batch)
        torch.cuda.synchronize()
        c = cpu_baseline(be, q_all[0], batch, TOP_K, P, D**-0.5, reps=args.cpu_reps)
        cpu = {"value": round(c["us"], 1), "unit": "us per layer-step", "cores": c["threads"], "kind": "port",
               "cpu_model": cpu_model(), "positions_equal_gpu": c["positions_equal_gpu"],
               "sample": f"one whole layer-step (all {B} requests, layer 0 of the GPU's state: its bounds, "
                         f"queries, req_to_token and K/V pool copied to host memory), torch CPU restatement "
                         f"of the reference op sequence (scores -> masked top-k -> gather -> fp32 attention), "
                         f"{c['threads']} threads, median of {c['reps']} after {c['warmup']} warm-ups"}

    traffic, traffic_source = profiled_traffic()
    ctx_desc = (f"contexts uniform in [8192, {S}] (seeded, mean {int(ctxs.mean())})" if args.ragged
                else f"{S}-token context")
    line = {
        "metric": ("µs per Quest decode layer-step, ragged contexts, batch 16; % peak HBM BW" if args.ragged
                   else "µs per Quest decode layer-step @128K ctx, batch 16; % peak HBM BW"),
        "value": round(us_per_layer_step, 2),
        "unit": "us per layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) q/k/v, fixed seeds",
        "config": {"workload": f"quest decode, batch {B}, {ctx_desc}, {L} layers, "
                               f"32q/4kv heads x 128, page 64, top_k 2048",
                   "batch": B, "seq_len": S, "layers": L, "graph": not args.no_graph, "ragged": bool(args.ragged)},
        "hbm_frac_layer_step": round(step_frac, 4),
        "tokens_per_s": round(B / (ms_per_step * 1e-3), 1),
        "algorithmic_bytes_per_layer_step": byts,
        "kernels_us": {"score_pages_fast_kernel": round(ms_sel * 1e3, 2),
                       "quest_attend_unit_kernel": round(ms_att * 1e3, 2)},
        "roofline": {"kernel": dominant[0], "bound": "hbm", "achieved": round(dominant[3], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(dominant[3] / HBM_PEAK_GBS, 4),
                     "traffic": None if args.ragged else traffic.get(dominant[0]),
                     "traffic_source": traffic_source},
        "cpu_baseline": cpu,
        "prefill_bounds": prefill,
        "setup_s": round(setup_s, 1),
    }
    if args.hisparse_steps > 0 and not args.ragged:
        # the quest_hisparse tier, measured after and outside the headline's timed region
        del be, kvp, rtp, batch, q_all, k_new, v_new
        if not args.no_graph:
            del graph, run
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        line["hisparse"] = hisparse_measure(B, S, args.hisparse_layers, 32, args.hisparse_steps, 32)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
