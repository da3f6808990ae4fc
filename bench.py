"""Quest decode layer-step benchmark on one MI355X.

Workload (default line): batch 16, every request at 128K context (131072 tokens),
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

After the timed region, and outside it, the same line gets:
  cpu_baseline  the reference's op sequence in torch on the host cores, on the
                GPU's own layer-0 tensors;
  layouts       the same step with req_to_token laid out as the reference engine
                allocates it (prompt rows per request, decode rows bs at a time,
                interleaved) and as page runs at shuffled bases;
  configs       the path's other configurations, each with its own bytes, HBM
                fraction and CPU baseline: batch 1 x 8192; batch 8 x 32768 with
                per-page key offsets; 48 ragged layers, batch 16, contexts
                U[8192, 131072], 64 steps; batch 4 x 262144 with outlier key
                channels, 256 steps, both overlap modes, quest and quest_hisparse;
  hisparse      the quest_hisparse tier at the headline's batch and context: as
                many layers of pinned host history as the box's memory holds (up
                to 48), 128 graph-replayed decode steps, AR(1) queries, and the
                same at 4 layers.

    python bench.py [--steps K] [--warmup W] [--quick]

`--quick` measures the headline only.  `--ragged` draws each request's context
uniform in [8192, ctx] (seeded) instead.  `--layout engine|page_runs` lays out
req_to_token as above.  `--hisparse` measures the quest_hisparse tier alone
(`--hisparse-layers`, `--hisparse-route`); `--dense` the dense comparator.
"""

from __future__ import annotations

import argparse
import gc
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
# the layer step's two launches at the headline shape (KV*D = 4 x 128, bf16, GQA group 8)
SCORE_KERNEL = "score_pages_fast4_kernel"
ATTEND_KERNEL = "quest_attend_unit_kernel"


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


H, KV, D, P, TOP_K = 32, 4, 128, 64, 2048
ROW_BYTES = 2 * KV * D * 2  # K + V of one token in one layer
PAGE_BYTES = KV * D * 2 * 2  # (min, max) bounds of one page in one layer
GIB = 1 << 30


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_threads() -> int:
    """Cores this process may use: its CPU set, capped by OMP_NUM_THREADS when set."""
    return max(1, min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "0")) or 1 << 30))


def host_memory() -> dict:
    """What bounds pinned host memory here: MemTotal / MemAvailable, the memory cgroup's
    limit and RLIMIT_MEMLOCK (pinned memory needs no more: it is RAM the process holds)."""
    info = {}
    try:
        for line in open("/proc/meminfo"):
            k, v = line.split(":", 1)
            if k in ("MemTotal", "MemAvailable"):
                info[k] = int(v.split()[0]) * 1024
    except OSError:
        pass
    for f in ("/sys/fs/cgroup/memory.max", "/sys/fs/cgroup/memory/memory.limit_in_bytes"):
        try:
            v = open(f).read().strip()
            if v.isdigit():
                info["cgroup_limit"] = int(v)
                break
        except OSError:
            pass
    import resource

    soft, _ = resource.getrlimit(resource.RLIMIT_MEMLOCK)
    info["memlock_limit"] = None if soft == resource.RLIM_INFINITY else soft
    return info


def cpu_baseline(be, q, batch, reps: int = 20, warmup: int = 3, avoid: bool = False) -> dict:
    """The reference's op sequence on the host cores (oracle/torch_path.py: group_queries ->
    page_scores -> masked topk -> req_to_token gather -> fp32 decode_attention, torch CPU
    kernels), on the same tensors the GPU holds for layer 0 (copied to host memory), with
    every core of this process's CPU set; the median of `reps` timed layer-steps after
    `warmup` untimed ones.  Also reports whether its positions equal the GPU's for that
    layer (torch.topk's choice among exactly tied scores aside, they must)."""
    from oracle import torch_path as tp

    threads = host_threads()
    torch.set_num_threads(threads)
    quest = be.quest
    pool = be.token_to_kv_pool
    bounds = quest.page_k_bounds[0].cpu()
    k_buf, v_buf = pool.k_all[0].cpu(), pool.v_all[0].cpu()
    r2t = be.req_to_token.cpu()
    qc = q.cpu()
    rpi = batch.req_pool_indices.cpu()
    seq = batch.seq_lens.cpu()
    scaling = D**-0.5
    times = []
    for i in range(warmup + reps):
        t0 = time.perf_counter()
        pos, actual, _ = tp.layer_step(qc, bounds, rpi, seq, r2t, k_buf, v_buf, P, TOP_K, scaling, avoid)
        if i >= warmup:
            times.append(time.perf_counter() - t0)
    gpu_pos = be._positions[: qc.shape[0]].cpu()
    same = all(torch.equal(pos[i, : int(actual[i])], gpu_pos[i, : int(actual[i])]) for i in range(qc.shape[0]))
    return {"value": round(float(np.median(times)) * 1e6, 1), "unit": "us per layer-step", "cores": threads,
            "kind": "port", "cpu_model": cpu_model(), "positions_equal_gpu": bool(same), "reps": reps,
            "warmup": warmup}


def req_to_token_table(layout: str, ctxs: np.ndarray, max_ctx: int, total_steps: int, seed: int,
                       engine_prompt: int) -> tuple[np.ndarray, int]:
    """Pool row of every (request, position) [B, max_ctx] and the pool's row count (row 0 is
    the padding row).
      contiguous  request r's rows follow r-1's: its context plus room for the decode steps;
      engine      as the reference engine allocates them (engine.py:201-203, 232-235): each
                  request's first `engine_prompt` positions (its prompt) are one run of rows,
                  every later position was allocated by a decode step, bs rows at a time in
                  batch order, so position p >= prompt of request r sits at
                  decode_base + (p - prompt) * B + r;
      page_runs   each page's 64 positions are one run of rows, the pages of all requests at
                  shuffled page-aligned bases (seeded)."""
    B = len(ctxs)
    pos = np.arange(max_ctx, dtype=np.int64)[None, :]
    r = np.arange(B, dtype=np.int64)[:, None]
    if layout == "contiguous":
        span = ctxs.astype(np.int64) + total_steps + 64
        starts = 1 + np.concatenate([[0], np.cumsum(span)[:-1]])
        rows = int(span.sum())
        return np.minimum(starts[:, None] + pos, rows), rows
    if layout == "engine":
        prompt = int(min(engine_prompt, int(ctxs.min()) - 1))
        table = np.where(pos < prompt, 1 + r * prompt + pos, 1 + B * prompt + (pos - prompt) * B + r)
        return table, B * max_ctx
    if layout == "page_runs":
        pages = (max_ctx + P - 1) // P
        perm = np.random.default_rng(seed).permutation(B * pages).reshape(B, pages)
        table = 1 + perm[:, pos[0] // P] * P + pos % P
        return table, B * pages * P
    raise ValueError(f"unknown layout {layout!r}")


class QuestRun:
    """A quest-mode decode batch through QuestOnlyBackend (the drop-in path): pools of L
    layers with seeded N(0, 1) keys and values, the prompts' page bounds built by the prefill
    kernel, per-layer queries and new tokens, and one decode step of all L layers that
    captures in a HIP graph.

    page_offsets: keys get a per-(request, page) mean offset N(0, 0.5) (seeded per layer);
    outliers: that many channels per KV head (seeded) have their keys scaled x10."""

    def __init__(self, B: int, ctxs: np.ndarray, L: int, total_steps: int, *, layout: str = "contiguous",
                 seed: int = 1234, page_offsets: bool = False, outliers: int = 0, avoid: bool = False,
                 engine_prompt: int = 8192):
        from qwenquest_amd.attention.quest_only import QuestOnlyBackend
        from qwenquest_amd.batch import ForwardBatch, ForwardMode
        from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

        dev = torch.device("cuda", 0)
        self.B, self.L, self.avoid, self.layout = B, L, avoid, layout
        self.ctxs = np.asarray(ctxs, dtype=np.int64)
        max_ctx = int(self.ctxs.max()) + total_steps + 64
        table, rows = req_to_token_table(layout, self.ctxs, max_ctx, total_steps, seed, engine_prompt)
        t0 = time.perf_counter()
        self.rtp = ReqToTokenPool(B, max_ctx, dev)
        self.kvp = MHATokenToKVPool(rows, L, KV, D, torch.bfloat16, dev)
        self.rtp.req_to_token.copy_(torch.from_numpy(table.astype(np.int32)).to(dev))
        gen = torch.Generator(device=dev).manual_seed(seed)
        r2t = self.rtp.req_to_token
        for layer in range(L):
            if page_offsets:
                # k = N(0,1) + mu[request, page], mu ~ N(0, 0.5), rounded to bf16 once
                mu = torch.randn((B, (max_ctx + P - 1) // P), generator=gen, device=dev) * 0.5
                off = torch.zeros(rows + 1, device=dev)
                off[r2t.long().reshape(-1)] = mu[:, torch.arange(max_ctx, device=dev) // P].reshape(-1)
                k = torch.randn((rows + 1, KV, D), generator=gen, device=dev)
                self.kvp.k_all[layer].copy_((k + off[:, None, None]).to(torch.bfloat16))
                del k, off
            else:
                self.kvp.k_all[layer].normal_(generator=gen)
            if outliers:
                g2 = torch.Generator().manual_seed(seed + 7 + layer)
                for h in range(KV):
                    ch = torch.randperm(D, generator=g2)[:outliers].to(dev)
                    self.kvp.k_all[layer][:, h, ch] *= 10.0
            self.kvp.v_all[layer].normal_(generator=gen)
        cfg = {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P, "avoid_recent_overlap": avoid}
        self.be = be = QuestOnlyBackend(self.rtp, self.kvp, cfg)
        # the prefill bounds build of requests 1 .. B-1 is timed with HIP events (request 0 warms up)
        pf0, pf1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for r in range(B):
            # prefill covers positions [0, ctx - 1); the first decode step has seq_len ctx
            be.quest.update_prefill_representations_fused(r, self.kvp.k_all, r2t[r, : int(self.ctxs[r]) - 1])
            be._skip_first_decode_update[r] = True
            if r == 0:
                pf0.record()
        pf1.record()
        self.q_all = torch.randn((L, B, H, D), generator=gen, device=dev).to(torch.bfloat16)
        self.k_new = torch.randn((L, B, KV, D), generator=gen, device=dev).to(torch.bfloat16)
        self.v_new = torch.randn((L, B, KV, D), generator=gen, device=dev).to(torch.bfloat16)
        self.layers = [Layer(i, D**-0.5) for i in range(L)]
        self.rpi = torch.arange(B, device=dev, dtype=torch.int64)
        self.seq_lens = torch.tensor(self.ctxs, device=dev, dtype=torch.int64)
        self.out_loc = torch.empty(B, device=dev, dtype=torch.int64)
        # out_cache_loc = the request's first row + seq_len - 1 (one launch per step)
        self.base_m1 = torch.from_numpy(table[:, 0].astype(np.int64) - 1).to(dev)
        self.r2t_flat = r2t.view(-1)
        self.max_ctx = max_ctx
        self.batch = ForwardBatch(ForwardMode.DECODE, None, None, self.rpi, self.seq_lens, self.out_loc,
                                  self.rtp, self.kvp, be)
        torch.cuda.synchronize()
        self.setup_s = time.perf_counter() - t0
        self.prefill = None
        if B > 1:
            pf_us = pf0.elapsed_time(pf1) * 1e3
            pf_bytes = float(sum(int(c) - 1 for c in self.ctxs[1:])) * L * KV * D * 2  # every prompt key read once
            self.prefill = {"kernel": "prefill_bounds_wave_kernel", "requests": B - 1, "layers": L,
                            "tokens_per_request": int(self.ctxs[1:].mean()) - 1,
                            "us_per_request": round(pf_us / (B - 1), 1),
                            "gbs": round(pf_bytes / (pf_us * 1e-6) / 1e9, 1),
                            "hbm_frac": round(pf_bytes / (pf_us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4)}
        self.graph = None
        self.steps_done = 0

    def step(self):
        if self.layout == "contiguous":
            torch.add(self.base_m1, self.seq_lens, out=self.out_loc)
        else:  # the new token's row from the table (the engine writes it there, engine.py:232-235)
            self.out_loc.copy_(self.r2t_flat[self.rpi * self.max_ctx + self.seq_lens - 1])
        self.be.init_forward_metadata(self.batch)
        for layer in range(self.L):
            self.be.forward_decode(self.q_all[layer], self.k_new[layer], self.v_new[layer], self.layers[layer],
                                   self.batch)
        self.seq_lens.add_(1)

    def run(self, warmup: int, steps: int, graph: bool = True) -> float:
        """ms per decode step (all L layers): an eager first step (first-step skips,
        workspaces), then `warmup` and `steps` replays of the captured step, timed with the
        host clock between two synchronisations."""
        self.step()
        torch.cuda.synchronize()
        fn = self.step
        if graph:
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self.step()
            fn = self.graph.replay
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        self.steps_done = 1 + int(graph) + warmup + steps
        return (time.perf_counter() - t0) * 1e3 / steps

    def kernel_us(self) -> tuple[float, float]:
        """Average µs of the layer step's two launches (scores, selection + attention), each
        from a graph of L launches over the L layers in turn (so that no launch finds its
        bounds or K/V rows in a cache, as in the step), HIP events on the launch stream."""
        be, batch, L = self.be, self.batch, self.L
        if self.layout == "contiguous":
            torch.add(self.base_m1, self.seq_lens, out=self.out_loc)
        else:
            self.out_loc.copy_(self.r2t_flat[self.rpi * self.max_ctx + self.seq_lens - 1])
        be.quest.prepare_step(self.seq_lens)
        turn = {"sel": 0, "att": 0}

        def phase(which, ph):
            i = turn[which] % L
            turn[which] += 1
            be.forward_decode_phase(self.q_all[i], self.k_new[i], self.v_new[i], self.layers[i], batch, ph)

        stream = torch.cuda.current_stream()
        ms_sel = time_graph(lambda: phase("sel", 1), L, stream)
        ms_att = time_graph(lambda: phase("att", 2), L, stream)
        return ms_sel * 1e3, ms_att * 1e3

    def seqs_timed(self, warmup: int, steps: int) -> list[int]:
        return [int(c) + 1 + warmup + steps // 2 for c in self.ctxs]

    def cpu(self, reps: int) -> dict:
        """CPU baseline on layer 0 of the GPU's state: that layer runs once more so that its
        positions are in the backend's buffer."""
        self.be.quest.prepare_step(self.seq_lens)
        self.be.forward_decode(self.q_all[0], self.k_new[0], self.v_new[0], self.layers[0], self.batch)
        torch.cuda.synchronize()
        return cpu_baseline(self.be, self.q_all[0], self.batch, reps=reps, avoid=self.avoid)

    def close(self):
        del self.graph, self.be, self.kvp, self.rtp, self.batch, self.q_all, self.k_new, self.v_new
        gc.collect()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


def quest_config(name: str, what: str, B: int, ctxs, L: int, warmup: int, steps: int, cpu_reps: int,
                 **kw) -> dict:
    """One configuration in quest mode: µs per layer-step (graph-replayed), its own
    algorithmic bytes and HBM fraction, the two launches' times and a CPU baseline."""
    ctxs = np.asarray(ctxs, dtype=np.int64)
    run = QuestRun(B, ctxs, L, warmup + steps + 2, **kw)
    try:
        ms = run.run(warmup, steps)
        us = ms * 1e3 / L
        byts = algorithmic_bytes(run.seqs_timed(warmup, steps), P, TOP_K, ROW_BYTES, PAGE_BYTES)
        k_sel, k_att = run.kernel_us()
        res = {"what": what, "batch": B, "context": int(ctxs.max()) if len(set(ctxs.tolist())) == 1 else
               {"min": int(ctxs.min()), "mean": int(ctxs.mean()), "max": int(ctxs.max())},
               "layers": L, "steps": steps, "warmup": warmup, "us_per_layer_step": round(us, 2),
               "tokens_per_s": round(B / (ms * 1e-3), 1), "algorithmic_bytes_per_layer_step": byts["headline"],
               "hbm_frac": round(byts["headline"] / (us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4),
               "kernels_us": {SCORE_KERNEL: round(k_sel, 2), ATTEND_KERNEL: round(k_att, 2)}}
        if cpu_reps > 0:
            res["cpu_baseline"] = run.cpu(cpu_reps)
            res["cpu_baseline"]["sample"] = (f"one whole layer-step (all {B} requests, layer 0 of the GPU's state), "
                                             f"torch CPU restatement of the reference op sequence")
        print(f"[bench] config {name}: {res['us_per_layer_step']} us per layer-step", file=sys.stderr, flush=True)
        return res
    finally:
        run.close()
        del run
        torch.cuda.empty_cache()


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


def pinned_capacity(limit: int, chunk: int = 4 * GIB) -> int:
    """Pinned host memory the system hands this process: chunks pinned (qq_host_alloc, the
    host tier's allocator) until the first refusal or `limit`, then all released.  The ROCm
    driver caps pinned (GTT) memory below the RAM that is free."""
    import ctypes

    from qwenquest_amd import _lib

    lib = _lib.load()
    held = []
    try:
        while len(held) * chunk < limit:
            p = ctypes.c_void_p()
            if lib.qq_host_alloc(chunk, ctypes.byref(p)) != 0:
                break
            held.append(p.value)
    finally:
        for p in held:
            lib.qq_host_free(ctypes.c_void_p(p))
    return len(held) * chunk


def hisparse_layers_that_fit(B: int, S: int, total_steps: int, extra_slot: bool, want: int = 48,
                             reserve: int = 3 * GIB) -> tuple[int, dict]:
    """The most layers (up to `want`) whose pinned host tier fits: the pinned memory the
    system grants (pinned_capacity, probed up to what `want` layers need, and never past the
    smaller of MemAvailable and the memory cgroup's limit) less `reserve` for the other
    pinned buffers of the run, and the figures it was derived from."""
    mem = host_memory()
    R = B + int(extra_slot)
    max_ctx = S + total_steps + 64
    per_layer = 2 * (R * max_ctx + 1) * KV * D * 2
    ram = min(v for v in (mem.get("MemAvailable"), mem.get("cgroup_limit"), 1 << 62) if v)
    pinned = pinned_capacity(min(want * per_layer + reserve, ram - 32 * GIB))
    fit = max(1, min(want, (pinned - reserve) // per_layer))
    cap = {"pinned_capacity_bytes": pinned, "pinned_probe": "4 GiB chunks pinned until the first refusal",
           "mem_available_bytes": mem.get("MemAvailable"), "mem_total_bytes": mem.get("MemTotal"),
           "cgroup_limit_bytes": mem.get("cgroup_limit"), "memlock_limit_bytes": mem.get("memlock_limit"),
           "pinned_bytes_per_layer": per_layer, "reserve_bytes": reserve, "layers_that_fit": int(fit),
           "layers_of_the_full_history": 48}
    return int(fit), cap


def hisparse_measure(B: int, S: int, L: int, warmup: int, steps: int, event_steps: int, route: str = "kernel", *,
                     buf: int = 4096, rho: float = 0.9, avoid: bool = False, outliers: int = 0,
                     overlap: bool = True, cpu_reps: int = 20) -> dict:
    """quest_hisparse decode (QuestHiSparseBackend, the drop-in path) at batch B x S tokens, a
    hot buffer of buf + 1 rows per request and layer, the K/V history of L layers in pinned
    host memory, queries AR(1) with coefficient rho across steps (0: independent).  After
    `warmup` eager steps, one decode step (bounds fold + eager backup + per layer new token,
    selection, swap-in and attention) is captured in a HIP graph and replayed for `steps`
    timed steps (µs per layer-step; the backend's error poll after every replay);
    `event_steps` more steps run eagerly with HIP events around every swap-in call (plan +
    copy) on the launch stream, for the swap-in time and the missed rows.
    route "memcpy": the swap-in's copy through the copy engines (QuestHiSparseBackend
    swap_route="memcpy": a host synchronisation per swap-in, so no graph; the `steps` timed
    steps run eagerly with HIP events around each step).
    overlap: one more request slot, admitted while the batch decodes (the admission's
    overlap with decode steps)."""
    from qwenquest_amd.attention.quest_hisparse import QuestHiSparseBackend
    from qwenquest_amd.batch import ForwardBatch, ForwardMode
    from qwenquest_amd.memory import MHATokenToKVPool, ReqToTokenPool

    dev = torch.device("cuda", 0)
    total = warmup + steps + event_steps + 2
    max_ctx = S + total + 64
    t_setup = time.perf_counter()
    R = B + int(overlap)
    rtp = ReqToTokenPool(R, max_ctx, dev)
    kvp = MHATokenToKVPool(R * max_ctx, L, KV, D, torch.bfloat16, dev)
    gen = torch.Generator(device=dev).manual_seed(4321)
    for layer in range(L):
        kvp.k_all[layer].normal_(generator=gen)
        if outliers:
            g2 = torch.Generator().manual_seed(4321 + 7 + layer)
            for h in range(KV):
                kvp.k_all[layer][:, h, torch.randperm(D, generator=g2)[:outliers].to(dev)] *= 10.0
        kvp.v_all[layer].normal_(generator=gen)
    base = 1 + torch.arange(R, device=dev, dtype=torch.int64) * max_ctx
    rtp.req_to_token.copy_((base[:, None] + torch.arange(max_ctx, device=dev)[None]).to(torch.int32))
    be = QuestHiSparseBackend(rtp, kvp, {"algorithm": "quest", "top_k": TOP_K, "quest_page_size": P,
                                         "device_buffer_size": buf, "avoid_recent_overlap": avoid},
                              host_pool_size=R * max_ctx, swap_route=route, async_admission=True)
    pinned = be.coord.host_bytes()
    print(f"[bench] hisparse {B} x {S}, {L} layers: {pinned / GIB:.1f} GiB pinned host tier ready after "
          f"{time.perf_counter() - t_setup:.1f} s", file=sys.stderr, flush=True)
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
    print(f"[bench] hisparse admission {admit_ms:.0f} ms", file=sys.stderr, flush=True)

    coord = be.coord
    layers = [Layer(i, D**-0.5) for i in range(L)]
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
        be.poll_errors()  # swap-in / backup errors of the steps done so far (no synchronisation)
        e1.synchronize()
        step_ms.append(e0.elapsed_time(e1))
        seq.add_(1)
    be.poll_errors()
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
    del coord.swap_in_selected_pages  # the class's method again (no reference cycle through coord)
    overlap_rec = None
    if use_graph and overlap:
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
            be.poll_errors()
            ends.append((s0, s1))
            seq.add_(1)
        torch.cuda.synchronize()
        be.poll_errors()
        backup_ms = b0.elapsed_time(b1)
        during = [a.elapsed_time(b) for a, b in ends if b0.elapsed_time(b) <= backup_ms]
        coord.wait_admission(B)
        overlap_rec = {
            "request_tokens": prompt,
            "layers": L,
            "backup_ms": round(backup_ms, 2),
            "backup_d2h_gbs": round(prompt * L * ROW_BYTES / (backup_ms * 1e-3) / 1e9, 2),
            "decode_steps_within_backup": len(during),
            "decode_us_per_layer_step_within_backup": round(float(np.mean(during)) * 1e3 / L, 2) if during else None,
            "decode_us_per_layer_step_alone": round(float(np.mean(step_ms)) * 1e3 / L, 2),
        }
    cpu_plan = hisparse_cpu_baseline(coord, step, next_inputs, seq, B, buf, reps=cpu_reps) if cpu_reps > 0 else None
    miss_rows = float(np.mean(misses)) / L if misses else 0.0
    swap_us = float(np.mean(swap_ms)) * 1e3 / L if swap_ms else 0.0
    h2d = miss_rows * ROW_BYTES / (swap_us * 1e-6) / 1e9 if swap_us > 0 else 0.0
    peak = pinned_h2d_peak()
    d2h_peak = pinned_h2d_peak(d2h=True)
    admit_bytes = B * prompt * L * ROW_BYTES
    admit_gbs = admit_bytes / (admit_ms * 1e-3) / 1e9
    st = coord.stats
    res = {
        "layers": L,
        "steps": steps,
        "warmup": warmup,
        "pinned_host_bytes": pinned,
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
            "overlap": overlap_rec,
        },
        "workload": f"quest_hisparse decode, batch {B}, {S}-token context, hot buffer {buf}+1 rows, {L} layers' "
                    f"history in pinned host memory ({pinned / GIB:.1f} GiB), "
                    + (f"AR(1) queries rho {rho}" if rho else "independent N(0,1) queries per step")
                    + (f", {outliers} key channels per KV head x10" if outliers else "")
                    + f", avoid_recent_overlap {avoid}; {warmup} warm-up steps, {steps} "
                    f"{'graph-replayed' if use_graph else 'eager'} timed steps, {event_steps} eager steps with events "
                    f"around the swap-in; swap-in copy: "
                    f"{'copy kernel reading pinned host memory' if use_graph else 'hipMemcpyAsync per run of host rows on a side stream + scatter'}",
        "setup_s": round(setup_s, 1),
    }
    del be, coord, kvp, rtp, graph, batch, pre
    gc.collect()  # the pinned host tier is released here, not at some later collection
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def hisparse_cpu_baseline(coord, step, next_inputs, seq, B: int, buf: int, reps: int = 20) -> dict:
    """The reference's swap-in on the host cores (coordinator.py:232-304) for one layer-step:
    the B requests of layer 0 in one decode step, from the state the GPU's swap-in started
    from (buffer_tokens, lru_slots, req_to_host_pool, the selected positions) - the reference's
    op sequence batched over the requests (oracle/torch_path.swap_in_batch: unique, isin,
    sort, searchsorted as batch-wide torch CPU ops on every core of this process's CPU set;
    requests at or under the buffer take the fast path), then the misses' K and V rows copied
    host tier -> hot buffer; the median of `reps` after 3 warm-ups.  The planned rows are
    checked against the GPU's."""
    from oracle import torch_path as tp

    cap = {}
    swap = coord.swap_in_selected_pages

    def capture(reqs, seqs, positions, layer_id, **kw):
        if layer_id == 0 and not cap:
            cap["tokens"] = coord.buffer_tokens[0].cpu()
            cap["lru"] = coord.lru_slots[0].cpu()
            cap["r2h"] = coord.req_to_host_pool.cpu()
            cap["pos"] = positions.cpu().to(torch.int64)
            cap["seq"] = seqs.cpu().to(torch.int64)
            cap["reqs"] = reqs.cpu().to(torch.int64)
            rows = swap(reqs, seqs, positions, layer_id, **kw)
            cap["rows"] = rows.cpu()
            return rows
        return swap(reqs, seqs, positions, layer_id, **kw)

    coord.swap_in_selected_pages = capture
    next_inputs()
    step()
    torch.cuda.synchronize()
    seq.add_(1)
    del coord.swap_in_selected_pages
    threads = host_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    host_k, host_v = coord.host_k_all[0], coord.host_v_all[0]
    hot_k = torch.empty((coord.max_reqs * (buf + 1),) + tuple(host_k.shape[1:]), dtype=host_k.dtype)
    hot_v = torch.empty_like(hot_k)
    reqs, seqs, pos = cap["reqs"], cap["seq"], cap["pos"]
    top_k = pos.shape[1]
    n = seqs.clamp(max=top_k)
    long_b = seqs > buf

    def plan_and_copy() -> torch.Tensor:
        rows = torch.full((B, top_k), -1, dtype=torch.int64)
        base = reqs * (buf + 1)
        short = ~long_b
        if bool(short.any()):  # fast path, coordinator.py:252-255
            rows[short] = base[short].unsqueeze(1) + pos[short]
        if bool(long_b.any()):
            lr = reqs[long_b]
            tokens, lru = cap["tokens"][lr].clone(), cap["lru"][lr].clone()
            slots, mreq, victims, hidx = tp.swap_in_batch(tokens, lru, pos[long_b], seqs[long_b], cap["r2h"][lr])
            rows[long_b] = base[long_b].unsqueeze(1) + slots
            if victims.numel():
                dst = base[long_b][mreq] + victims
                hot_k.index_copy_(0, dst, host_k.index_select(0, hidx))
                hot_v.index_copy_(0, dst, host_v.index_select(0, hidx))
        keep = torch.arange(top_k).unsqueeze(0) < n.unsqueeze(1)
        return torch.where(keep, rows, torch.full_like(rows, -1))

    try:
        for _ in range(3):
            rows = plan_and_copy()
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            plan_and_copy()
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev)
    return {"value": round(float(np.median(times)) * 1e6, 1), "unit": f"us per layer-step ({B} requests' swap-in)",
            "cores": threads, "kind": "port", "cpu_model": cpu_model(),
            "rows_equal_gpu": bool(torch.equal(rows, cap["rows"])),
            "sample": "one layer-step: the reference's swap-in op sequence (fast path or _swap_in_long: unique, "
                      "isin, sort, searchsorted) batched over all requests of layer 0 in one decode step, torch CPU "
                      f"kernels on {threads} threads, plus the misses' K/V row copies, from the GPU's state before "
                      f"its swap-in; median of {reps} after 3 warm-ups"}


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


def measure_configs(cpu_reps: int) -> dict:
    """The path's configurations other than the headline, each after the previous one's
    memory is freed: µs per layer-step (graph-replayed, each step's layers cycled so that no
    layer-step finds its data in the 256 MB Infinity Cache), its own algorithmic bytes, HBM
    fraction and CPU baseline."""
    out = {}
    out["c1_b1_8k"] = quest_config(
        "c1", "batch 1 x 8192 tokens, q/k/v N(0,1); one layer's shape, 48 independent layers cycled",
        1, [8192], 48, 8, 64, cpu_reps)
    out["c2_b8_32k_page_offsets"] = quest_config(
        "c2", "batch 8 x 32768 tokens, keys N(0,1) + a per-(request, page) mean offset N(0, 0.5), v/q N(0,1); "
              "48 independent layers cycled", 8, [32768] * 8, 48, 8, 64, cpu_reps, page_offsets=True)
    ctxs = np.random.default_rng(2024).integers(8192, 131072, size=16, endpoint=True)
    out["c3_ragged_48_layers"] = quest_config(
        "c3", "48 layers, batch 16, contexts uniform in [8192, 131072] (seeded), 64 decode steps, "
              "pages completing and finalized during the run; CPU baseline: one layer (layer 0) of one step",
        16, ctxs, 48, 4, 64, cpu_reps)
    for avoid in (False, True):
        out[f"c5_b4_262k_outliers_quest_avoid_{str(avoid).lower()}"] = quest_config(
            "c5", f"batch 4 x 262144 tokens, keys N(0,1) with 4 channels per KV head x10, avoid_recent_overlap "
                  f"{avoid}, 256 decode steps; 8 independent layers cycled", 4, [262144] * 4, 8, 8, 256, cpu_reps,
            outliers=4, avoid=avoid)
    for avoid in (False, True):
        r = hisparse_measure(4, 262144, 8, 16, 256, 16, buf=4096, rho=0.9, avoid=avoid, outliers=4, overlap=False,
                             cpu_reps=cpu_reps)
        print(f"[bench] config c5 hisparse avoid={avoid}: {r['us_per_layer_step']} us per layer-step",
              file=sys.stderr, flush=True)
        out[f"c5_b4_262k_outliers_quest_hisparse_avoid_{str(avoid).lower()}"] = {
            k: r[k] for k in ("workload", "layers", "steps", "us_per_layer_step", "swap_in_rows_per_layer_step",
                              "swap_in_us_per_layer_step", "h2d_gbs", "h2d_frac_of_memcpy_peak", "hit_rate",
                              "cpu_baseline_swap_in", "pinned_host_bytes")}
    return out


def measure_layouts(headline_us: float, B: int, S: int, L: int, warmup: int, steps: int) -> dict:
    """The headline step with req_to_token laid out as the reference engine allocates rows and
    as page runs at shuffled bases (req_to_token_table); the delta against the contiguous
    headline."""
    out = {}
    for layout, what in (("engine", "prompt rows contiguous per request (8192-token prompts), every later position "
                                    "allocated by a decode step, 16 rows at a time in batch order (engine.py:232-235)"),
                         ("page_runs", "each page's 64 positions one run of rows, all pages at shuffled bases")):
        run = QuestRun(B, np.full(B, S), L, warmup + steps + 2, layout=layout)
        try:
            ms = run.run(warmup, steps)
            us = ms * 1e3 / L
            k_sel, k_att = run.kernel_us()
            out[layout] = {"what": what, "us_per_layer_step": round(us, 2),
                           "delta_us_vs_contiguous": round(us - headline_us, 2),
                           "kernels_us": {SCORE_KERNEL: round(k_sel, 2),
                                          ATTEND_KERNEL: round(k_att, 2)}}
            print(f"[bench] layout {layout}: {out[layout]['us_per_layer_step']} us per layer-step", file=sys.stderr,
                  flush=True)
        finally:
            run.close()
            del run
            torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--ctx", type=int, default=131072)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--quick", action="store_true", help="the headline only (no layouts, configs or hisparse)")
    ap.add_argument("--cpu-reps", type=int, default=20, help="timed CPU-baseline layer-steps (0 = skip)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB three times (scale for the HBM byte counters)")
    ap.add_argument("--ragged", action="store_true",
                    help="contexts drawn uniform in [8192, ctx] per request (seeded) instead of all ctx")
    ap.add_argument("--layout", choices=("contiguous", "engine", "page_runs"), default="contiguous",
                    help="req_to_token layout of the headline (see req_to_token_table)")
    ap.add_argument("--hisparse", action="store_true", help="measure the quest_hisparse tier instead")
    ap.add_argument("--hisparse-layers", type=int, default=4)
    ap.add_argument("--hisparse-route", choices=("kernel", "memcpy"), default="kernel",
                    help="--hisparse: the swap-in's host -> device copy (memcpy: hipMemcpyAsync per run on a side stream)")
    ap.add_argument("--hisparse-steps", type=int, default=128,
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

    _lib.load()
    torch.cuda.set_device(0)
    B, S, L = args.batch, args.ctx, args.layers
    ctxs = (np.random.default_rng(2024).integers(8192, S, size=B, endpoint=True) if args.ragged
            else np.full(B, S, dtype=np.int64))
    run = QuestRun(B, ctxs, L, args.warmup + args.steps + 2, layout=args.layout)
    ms_per_step = run.run(args.warmup, args.steps, graph=not args.no_graph)
    us_per_layer_step = ms_per_step * 1e3 / L
    byts = algorithmic_bytes(run.seqs_timed(args.warmup, args.steps), P, TOP_K, ROW_BYTES, PAGE_BYTES)
    step_frac = byts["headline"] / (us_per_layer_step * 1e-6) / (HBM_PEAK_GBS * 1e9)
    us_sel, us_att = run.kernel_us()
    bw_sel = byts["bounds"] / (us_sel * 1e-6) / 1e9
    bw_att = byts["kv"] / (us_att * 1e-6) / 1e9
    dominant = (ATTEND_KERNEL, us_att, byts["kv"], bw_att) if us_att >= us_sel else (
        SCORE_KERNEL, us_sel, byts["bounds"], bw_sel)
    cpu = None
    if args.cpu_reps > 0:
        cpu = run.cpu(args.cpu_reps)
        cpu["sample"] = (f"one whole layer-step (all {B} requests, layer 0 of the GPU's state: its bounds, queries, "
                         f"req_to_token and K/V pool copied to host memory), torch CPU restatement of the reference "
                         f"op sequence (scores -> masked top-k -> gather -> fp32 attention), {cpu['cores']} threads, "
                         f"median of {cpu['reps']} after {cpu['warmup']} warm-ups")
    prefill, setup_s = run.prefill, run.setup_s
    run.close()
    del run
    torch.cuda.empty_cache()

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
                               f"32q/4kv heads x 128, page 64, top_k 2048, req_to_token {args.layout}",
                   "batch": B, "seq_len": S, "layers": L, "graph": not args.no_graph, "ragged": bool(args.ragged),
                   "layout": args.layout},
        "hbm_frac_layer_step": round(step_frac, 4),
        "tokens_per_s": round(B / (ms_per_step * 1e-3), 1),
        "algorithmic_bytes_per_layer_step": byts,
        "kernels_us": {SCORE_KERNEL: round(us_sel, 2), ATTEND_KERNEL: round(us_att, 2)},
        "roofline": {"kernel": dominant[0], "bound": "hbm", "achieved": round(dominant[3], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(dominant[3] / HBM_PEAK_GBS, 4),
                     "traffic": None if (args.ragged or args.layout != "contiguous") else traffic.get(dominant[0]),
                     "traffic_source": traffic_source},
        "cpu_baseline": cpu,
        "prefill_bounds": prefill,
        "setup_s": round(setup_s, 1),
    }
    print(f"[bench] headline: {line['value']} us per layer-step", file=sys.stderr, flush=True)
    if not args.quick and not args.ragged and args.layout == "contiguous" and not args.no_graph:
        # measured after and outside the headline's timed region
        line["layouts"] = measure_layouts(us_per_layer_step, B, S, L, args.warmup, args.steps)
        line["configs"] = measure_configs(args.cpu_reps)
        if args.hisparse_steps > 0:
            fit, cap = hisparse_layers_that_fit(B, S, 32 + args.hisparse_steps + 32 + 16 + 2, True)
            while True:
                try:
                    his = hisparse_measure(B, S, fit, 32, args.hisparse_steps, 32, cpu_reps=args.cpu_reps)
                    break
                except RuntimeError as e:  # the system would not pin that much: half the layers
                    if fit <= 4 or "hipHostMalloc" not in str(e):
                        raise
                    cap.setdefault("pin_failures", []).append({"layers": fit, "error": str(e)[:200]})
                    gc.collect()
                    torch.cuda.empty_cache()
                    fit //= 2
            his["pinned_capacity"] = cap
            print(f"[bench] hisparse {fit} layers: {his['us_per_layer_step']} us per layer-step", file=sys.stderr,
                  flush=True)
            if fit != 4:
                small = hisparse_measure(B, S, 4, 32, args.hisparse_steps, 32, overlap=False, cpu_reps=0)
                his["layers_sweep_us_per_layer_step"] = {"4": small["us_per_layer_step"],
                                                         str(fit): his["us_per_layer_step"]}
            line["hisparse"] = his
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
