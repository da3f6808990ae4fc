"""HiSparse hierarchical KV cache, Quest mode (reference ``src/qwenquest/hisparse/coordinator.py``).

Two tiers, the reference's layout and bookkeeping:

* host: every request's full KV history in **pinned host memory**
  (``host_k/v[layer]``, rows handed out by ``host_allocator``), addressed by
  ``req_to_host_pool[req, position]``;
* device: per request ``device_buffer_size`` LRU slots + 1 reserved newest-token
  slot (``device_k/v[layer]``, ``buffer_tokens``, ``lru_slots``).

All copies, the swap-in planning and the eager backup's bookkeeping (skip flags,
host-row allocation from a free list kept on the device) run in HIP kernels on the
current stream; the kernels read and write the pinned host tier directly over
PCIe, so a decode step needs no host synchronisation and can be captured in a
HIP graph.  The reference's error conditions (too few victims, a position without
host backup, an exhausted host pool) are detected on the device: the affected
request's swap-in rows become -1, which makes its attention output NaN, and the
kernels set a device error word plus a mirror of it in pinned host memory.
:meth:`check_errors` raises what the reference raises; ``prepare_decode_step``
runs it on the mirror (no synchronisation, so an error surfaces one step late),
``stats`` and ``sync_errors=True`` (after every swap-in) on the device word.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from qwenquest_amd import _lib
from qwenquest_amd.memory import MHATokenToKVPool, kv_pair_zeros
from qwenquest_amd.quest import QuestAlgorithm

__all__ = ["DeviceRowAllocator", "HiSparseCoordinator", "SwapInStats", "pinned_zeros"]

_ERR_VICTIMS, _ERR_HOST_ROW, _ERR_HOST_OOM = 1, 2, 4


class _PinnedBlock:
    """One block of pinned host memory from qq_host_alloc, released when the last tensor
    viewing it is gone."""

    def __init__(self, nbytes: int):
        self.ptr = 0
        ptr = ctypes.c_void_p()
        _lib.call("qq_host_alloc", nbytes, ctypes.byref(ptr))
        self.ptr, self.nbytes = int(ptr.value), nbytes
        self._free = _lib.load().qq_host_free

    def __del__(self):
        if self.ptr:
            self._free(ctypes.c_void_p(self.ptr))
            self.ptr = 0


def pinned_zeros(shape: tuple[int, ...], dtype: torch.dtype) -> torch.Tensor:
    """A zeroed host tensor in pinned memory of exactly its size.  torch's pinned allocator
    rounds every allocation up to a power of two, so a 48-layer host tier of 2 x 102 GiB
    (batch 16 x 128K) would pin 2 x 128 GiB; this one pins what the tier holds."""
    elems = 1
    for d in shape:
        elems *= int(d)
    nbytes = elems * torch.tensor([], dtype=dtype).element_size()
    block = _PinnedBlock(max(nbytes, 1))
    arr = (ctypes.c_uint8 * block.nbytes).from_address(block.ptr)
    arr._block = block  # the memory lives as long as any tensor viewing arr
    t = torch.frombuffer(arr, dtype=torch.uint8)[:nbytes].view(dtype).view(shape)
    t.zero_()
    return t


class DeviceRowAllocator:
    """The host tier's free list (``TokenToKVPoolAllocator``, reference memory.py:47-72) kept on
    the device: ``ring[(head + i) % size]`` for ``i < count`` are the free rows in order, alloc
    takes from the head, free appends at the tail - the reference's order of rows.  The decode
    step's backups allocate from it inside a kernel; ``alloc``/``free`` serve admission and
    release, ``available_size`` reads the count (a synchronisation, for introspection)."""

    def __init__(self, size: int, device: torch.device, err: torch.Tensor, err_mirror_dev: int):
        self.size = size
        self.device = device
        self.ring = torch.arange(1, size + 1, dtype=torch.int64, device=device)
        self.state = torch.tensor([0, size], dtype=torch.int64, device=device)  # head, count
        self._err, self._err_mirror_dev = err, err_mirror_dev

    def available_size(self) -> int:
        return int(self.state[1].item())

    def alloc(self, n: int) -> torch.Tensor:
        if n > self.available_size():
            raise RuntimeError(f"KV pool out of memory: need {n} token slots, {self.available_size()} free")
        out = torch.empty(n, dtype=torch.int64, device=self.device)
        _lib.call("qq_hisparse_ring_alloc", _lib.ptr(self.ring), _lib.ptr(self.state), self.size, n, _lib.ptr(out),
                  _lib.ptr(self._err), self._err_mirror_dev, _lib.stream(self.device))
        return out

    def free(self, indices: torch.Tensor) -> None:
        idx = indices.to(device=self.device, dtype=torch.int64).flatten().contiguous()
        _lib.call("qq_hisparse_ring_free", _lib.ptr(self.ring), _lib.ptr(self.state), self.size, _lib.ptr(idx),
                  int(idx.numel()), _lib.stream(self.device))


@dataclass
class SwapInStats:
    """Hit/miss accounting of the LRU hot buffer (coordinator.py:48-59)."""

    hits: int = 0
    misses: int = 0
    fast_path_calls: int = 0

    @property
    def hit_rate(self) -> float:
        total = self.hits + self.misses
        return self.hits / total if total else float("nan")


class HiSparseCoordinator:
    def __init__(
        self,
        *,
        quest: QuestAlgorithm,
        num_layers: int,
        kv_heads: int,
        head_dim: int,
        max_reqs: int,
        max_context_len: int,
        top_k: int,
        device_buffer_size: int,
        host_pool_size: int,
        dtype: torch.dtype,
        device: torch.device | str,
        host_device: torch.device | str = "cpu",
        sync_errors: bool = False,
        swap_route: str = "kernel",
        async_admission: bool = False,
    ):
        # coordinator.py:91-94
        if device_buffer_size < top_k:
            raise ValueError("device_buffer_size must be >= top_k")
        if quest.top_k != top_k:
            raise ValueError(f"QuestAlgorithm.top_k ({quest.top_k}) != top_k ({top_k})")
        self.device = torch.device(device)
        self.host_device = torch.device(host_device)
        if self.device.type != "cuda":
            raise RuntimeError("qwenquest_amd.HiSparseCoordinator needs a GPU device (no CPU path)")
        if self.host_device.type != "cpu":
            raise ValueError("the host tier lives in pinned CPU memory: host_device must be 'cpu'")
        self.quest = quest
        self.num_layers = num_layers
        self.kv_heads, self.head_dim = kv_heads, head_dim
        self.max_reqs, self.max_context_len = max_reqs, max_context_len
        self.top_k = top_k
        self.device_buffer_size = buf = device_buffer_size
        self.dtype = dtype
        self.sync_errors = sync_errors
        # the swap-in's host -> device copy: "kernel" = the plan kernel's misses read by a copy
        # kernel straight from pinned host memory (no host synchronisation, graph-capturable);
        # "memcpy" = the misses' runs of consecutive host rows as hipMemcpyAsync on a side
        # stream into a staging buffer, then a scatter (the upstream route of
        # coordinator.py:282-291; the copy list is on the device, so each swap-in synchronises)
        if swap_route not in ("kernel", "memcpy"):
            raise ValueError(f"swap_route must be 'kernel' or 'memcpy', got {swap_route!r}")
        self.swap_route = swap_route
        self.row_elems = kv_heads * head_dim
        self.row_bytes = self.row_elems * torch.tensor([], dtype=dtype).element_size()

        # ---- host tier (pinned), full history of every request (rows from host_allocator)
        hshape = (num_layers, host_pool_size + 1, kv_heads, head_dim)
        self.host_k_all = pinned_zeros(hshape, dtype)
        self.host_v_all = pinned_zeros(hshape, dtype)
        self.host_k = list(self.host_k_all.unbind(0))
        self.host_v = list(self.host_v_all.unbind(0))
        self._host_k_dev = self._device_address(self.host_k_all)
        self._host_v_dev = self._device_address(self.host_v_all)
        self.req_to_host_pool = torch.full((max_reqs, max_context_len), -1, dtype=torch.int64, device=self.device)

        # ---- device tier: per request buf LRU slots + 1 newest-token slot
        dshape = (num_layers, max_reqs * (buf + 1), kv_heads, head_dim)
        self.device_k_all, self.device_v_all = kv_pair_zeros(dshape, dtype, self.device)
        self.device_k = list(self.device_k_all.unbind(0))
        self.device_v = list(self.device_v_all.unbind(0))
        self.req_to_device_buffer = torch.arange(max_reqs * (buf + 1), dtype=torch.int64,
                                                 device=self.device).view(max_reqs, buf + 1)
        self.buffer_tokens = torch.full((num_layers, max_reqs, buf), -1, dtype=torch.int64, device=self.device)
        self._lru_init = torch.arange(buf, dtype=torch.int64, device=self.device)
        self.lru_slots = self._lru_init.repeat(num_layers, max_reqs, 1)

        # swap-in workspaces + device counters (hits, misses, fast path) + error word, and the
        # error word's mirror in pinned host memory (read by the host without a synchronisation)
        self._rows = torch.empty((max_reqs, top_k), dtype=torch.int64, device=self.device)
        self._copy_dst = torch.empty((max_reqs, top_k), dtype=torch.int64, device=self.device)
        self._copy_src = torch.empty((max_reqs, top_k), dtype=torch.int64, device=self.device)
        self._copy_count = torch.zeros(max_reqs, dtype=torch.int32, device=self.device)
        self._stats = torch.zeros(3, dtype=torch.int64, device=self.device)
        self._err = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._err_host = torch.zeros(4, dtype=torch.int32, pin_memory=True)
        self._err_host_dev = self._device_address(self._err_host)
        if swap_route == "memcpy":
            self._side = torch.cuda.Stream(self.device)
            self._stage_k = torch.empty((max_reqs * top_k, kv_heads, head_dim), dtype=dtype, device=self.device)
            self._stage_v = torch.empty_like(self._stage_k)
        # admission's host backup (every prompt row's K and V to the pinned host tier: 2 KiB per
        # token and layer over PCIe, the bulk of an admission) on a side stream when
        # async_admission: the caller's stream goes on while it runs and waits for a request's
        # backup (an event) only before a decode step of that request, before its release or
        # before the request slot is admitted again.  The backup then goes through the copy
        # engines (hipMemcpyAsync per run of rows consecutive in the pool and in the host
        # tier): with a swap-in's copy kernel reading host memory at the same time, that
        # kernel keeps its full host -> device rate (57 GB/s measured) and the backup gets
        # ~30 GB/s; a backup by copy kernel took both to ~43 GB/s
        self.async_admission = async_admission
        self._adm_stream = torch.cuda.Stream(self.device) if async_admission else None
        self._adm_pending: dict[int, torch.cuda.Event] = {}
        # the eager backup's per-step state, on the device: first-step skip flags and the
        # host-row free list; persistent step buffers (graph capture)
        self._skip_first_backup = torch.zeros(max_reqs, dtype=torch.uint8, device=self.device)
        self.host_allocator = DeviceRowAllocator(host_pool_size, self.device, self._err, self._err_host_dev)
        self._step_host_idx = torch.empty(max_reqs, dtype=torch.int64, device=self.device)
        self._step_dev_rows = torch.empty(max_reqs, dtype=torch.int64, device=self.device)

    @staticmethod
    def _device_address(t: torch.Tensor) -> int:
        out = ctypes.c_void_p()
        _lib.call("qq_host_device_pointer", t.data_ptr(), ctypes.byref(out))
        return int(out.value)

    def _host_layer(self, base: int, layer: int) -> int:
        return base + layer * (self.host_k_all.shape[1]) * self.row_bytes

    # -------------------------------------------------- errors / stats

    def check_errors(self, sync: bool = True) -> None:
        """Raise what the reference raises (coordinator.py:278-279, 285-286; memory.py:62-66) for
        an error the kernels detected.  ``sync``: read the device error word (a synchronisation);
        otherwise its mirror in pinned host memory, which the kernels write as they detect an
        error (visible to the host once that kernel has finished)."""
        if sync:
            err = int(self._err.item())
        else:
            m = self._err_host.tolist()
            err = (_ERR_VICTIMS if m[0] else 0) | (_ERR_HOST_ROW if m[1] else 0) | (_ERR_HOST_OOM if m[2] else 0)
        if err:
            self._err.zero_()
            self._err_host.zero_()
            if err & _ERR_HOST_OOM:
                raise RuntimeError("KV pool out of memory: the host tier has no free rows for the eager backup")
            if err & _ERR_VICTIMS:
                raise RuntimeError("device_buffer_size too small for this top-k")
            raise AssertionError("positions without host backup were selected")

    @property
    def stats(self) -> SwapInStats:
        self.check_errors()
        h, m, f = self._stats.tolist()
        return SwapInStats(hits=h, misses=m, fast_path_calls=f)

    # -------------------------------------------------- [H1] admission

    def admission_done(self, req_pool_idx: int) -> bool:
        """Whether request ``req_pool_idx``'s admission backup has finished (no synchronisation;
        always true without async_admission).  Its prompt rows in the token pool may be reused
        only then."""
        ev = self._adm_pending.get(int(req_pool_idx))
        return ev is None or ev.query()

    def wait_admission(self, req_pool_idx: int | None = None) -> None:
        """Order the current stream after the admission backup of one request (all pending ones
        for None); the host does not wait."""
        reqs = list(self._adm_pending) if req_pool_idx is None else [int(req_pool_idx)]
        cur = torch.cuda.current_stream(self.device)
        for r in reqs:
            ev = self._adm_pending.pop(r, None)
            if ev is not None:
                cur.wait_event(ev)

    _MAX_BACKUP_RUNS = 64

    def _row_runs(self, idx: torch.Tensor, host_idx: torch.Tensor, pool_rows: int) -> list | None:
        """The prompt's rows as runs (pool row, host row, length) consecutive on both sides, for
        copy-engine copies; None (the copy kernel) past _MAX_BACKUP_RUNS runs or for rows
        outside the buffers.  Reads both index lists on the host (a synchronisation)."""
        src, dst = idx.cpu(), host_idx.cpu()
        n = src.numel()
        if n == 0:
            return []
        if int(src.min()) < 0 or int(src.max()) >= pool_rows or int(dst.min()) < 0 \
                or int(dst.max()) >= self.host_k_all.shape[1]:
            return None
        cut = (torch.nonzero((src[1:] != src[:-1] + 1) | (dst[1:] != dst[:-1] + 1)).flatten() + 1).tolist()
        if len(cut) + 1 > self._MAX_BACKUP_RUNS:
            return None
        starts, ends = [0] + cut, cut + [n]
        return [(int(src[a]), int(dst[a]), e - a) for a, e in zip(starts, ends)]

    def _wait_admissions_of(self, req_pool_indices: torch.Tensor) -> None:
        """Before a step that reads the host tier of these requests: wait for their pending
        admission backups (every pending one when the indices live on the device)."""
        if req_pool_indices.device.type == "cpu":
            reqs = [r for r in req_pool_indices.tolist() if r in self._adm_pending]
        else:
            reqs = list(self._adm_pending)
        if reqs and torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                "an admission backup of this batch is still pending: call wait_admission() and run the "
                "stream past it before capturing a decode step"
            )
        for r in reqs:
            self.wait_admission(r)

    def admit_request(
        self,
        req_pool_idx: int,
        prefill_len: int,
        token_to_kv_pool: MHATokenToKVPool,
        prefill_indices: torch.Tensor,
    ) -> None:
        """[H1] Back up the prefill to host, keep positions [0, buf) hot, build the bounds
        (coordinator.py:138-174)."""
        req = int(req_pool_idx)
        n = int(prefill_len)
        buf = self.device_buffer_size
        stream = _lib.stream(self.device)
        self.wait_admission(req)  # the slot's previous backup, if it is still running
        idx = prefill_indices.to(device=self.device, dtype=torch.int64).contiguous()
        host_idx = self.host_allocator.alloc(n)
        pool = token_to_kv_pool
        _lib.call("qq_hisparse_request_state", _lib.ptr(self.buffer_tokens), _lib.ptr(self.lru_slots),
                  self.num_layers, self.max_reqs, buf, _lib.ptr(self.req_to_host_pool),
                  self.max_context_len, req, _lib.ptr(host_idx), n, 0, stream)
        backup_stream = stream
        runs = None
        if self.async_admission:
            side = self._adm_stream
            side.wait_stream(torch.cuda.current_stream(self.device))  # prompt rows and host rows ready
            idx.record_stream(side)
            host_idx.record_stream(side)
            backup_stream = side.cuda_stream
            runs = self._row_runs(idx, host_idx, pool.k_all.shape[1])
        if runs is not None:
            # the copy engines: decode steps' swap-in kernels on the other stream keep their
            # host -> device rate while this device -> host backup runs
            with torch.cuda.stream(self._adm_stream):
                for s0, h0, m in runs:
                    for layer in range(self.num_layers):
                        self.host_k_all[layer, h0 : h0 + m].copy_(pool.k_all[layer, s0 : s0 + m], non_blocking=True)
                        self.host_v_all[layer, h0 : h0 + m].copy_(pool.v_all[layer, s0 : s0 + m], non_blocking=True)
        else:
            for src_all, host_base in ((pool.k_all, self._host_k_dev), (pool.v_all, self._host_v_dev)):
                _lib.call("qq_copy_rows", _lib.ptr(src_all), src_all.stride(0) * src_all.element_size(),
                          src_all.shape[1], _lib.ptr(idx), host_base,
                          self.host_k_all.stride(0) * self.host_k_all.element_size(), self.host_k_all.shape[1],
                          _lib.ptr(host_idx), n, self.num_layers, self.row_bytes, backup_stream)
        if self.async_admission:
            ev = torch.cuda.Event()
            ev.record(self._adm_stream)
            self._adm_pending[req] = ev
        n_dev = min(n, buf)
        dev_rows = self.req_to_device_buffer[req, :n_dev].contiguous()
        for src_all, dst_all in ((pool.k_all, self.device_k_all), (pool.v_all, self.device_v_all)):
            _lib.call("qq_copy_rows", _lib.ptr(src_all), src_all.stride(0) * src_all.element_size(),
                      src_all.shape[1], _lib.ptr(idx), _lib.ptr(dst_all),
                      dst_all.stride(0) * dst_all.element_size(), dst_all.shape[1], _lib.ptr(dev_rows),
                      n_dev, self.num_layers, self.row_bytes, stream)
        self.quest.update_prefill_representations_fused(req, pool.k_all, idx)
        self._skip_first_backup[req] = 1

    # -------------------------------------------------- [H2] per decode step

    def newest_slot(self, seq_lens: torch.Tensor) -> torch.Tensor:
        return (seq_lens.long() - 1).clamp(max=self.device_buffer_size)

    def prepare_decode_step(self, req_pool_indices: torch.Tensor, seq_lens: torch.Tensor) -> None:
        """[H2] Fold the previous token into the bounds and back it up to host
        (coordinator.py:183-215), all on the device: the first step after admission is skipped
        per request by a device flag, host rows come from the device free list in batch order,
        and the fold and the copies skip the entries left at -1."""
        if not self.sync_errors:
            self.check_errors(sync=False)
        bs = int(req_pool_indices.shape[0])
        if bs == 0:
            return
        if bs > self.max_reqs:
            raise ValueError(f"batch {bs} exceeds max_reqs {self.max_reqs}")
        if self._adm_pending:
            self._wait_admissions_of(req_pool_indices)
        stream = _lib.stream(self.device)
        rpi = req_pool_indices.to(device=self.device, dtype=torch.int64).contiguous()
        seq = seq_lens.to(device=self.device, dtype=torch.int64).contiguous()
        host_idx = self._step_host_idx[:bs]
        dev_rows = self._step_dev_rows[:bs]
        ha = self.host_allocator
        _lib.call("qq_hisparse_backup_step", _lib.ptr(rpi), _lib.ptr(seq), bs, _lib.ptr(self._skip_first_backup),
                  self.device_buffer_size, self.max_reqs, _lib.ptr(self.req_to_host_pool), self.max_context_len,
                  _lib.ptr(ha.ring), _lib.ptr(ha.state), ha.size, _lib.ptr(host_idx), _lib.ptr(dev_rows),
                  _lib.ptr(self._err), self._err_host_dev, stream)
        self.quest.update_decode_representations_fused(rpi, self.device_k_all, dev_rows)
        for src_all, host_base in ((self.device_k_all, self._host_k_dev), (self.device_v_all, self._host_v_dev)):
            _lib.call("qq_copy_rows", _lib.ptr(src_all), src_all.stride(0) * src_all.element_size(),
                      src_all.shape[1], _lib.ptr(dev_rows), host_base,
                      self.host_k_all.stride(0) * self.host_k_all.element_size(), self.host_k_all.shape[1],
                      _lib.ptr(host_idx), bs, self.num_layers, self.row_bytes, stream)
        if self.sync_errors:
            self.check_errors()

    def write_new_token(self, layer_id: int, req_pool_indices: torch.Tensor, seq_lens: torch.Tensor,
                        k: torch.Tensor, v: torch.Tensor) -> None:
        """set_kv_buffer redirected into the hot buffer's newest slot (coordinator.py:217-228)."""
        bs = int(req_pool_indices.shape[0])
        rpi = req_pool_indices.to(device=self.device, dtype=torch.int64).contiguous()
        seq = seq_lens.to(device=self.device, dtype=torch.int64).contiguous()
        kk = k.reshape(bs, self.row_elems).contiguous()
        vv = v.reshape(bs, self.row_elems).to(kk.dtype).contiguous()
        _lib.call("qq_hisparse_write_new_token", _lib.ptr(self.device_k[layer_id]),
                  _lib.ptr(self.device_v[layer_id]), _lib.dtype_code(self.dtype), _lib.ptr(kk), _lib.ptr(vv),
                  _lib.dtype_code(kk.dtype), _lib.ptr(rpi), _lib.ptr(seq), bs, self.device_buffer_size,
                  self.max_reqs, self.row_elems, _lib.stream(self.device))

    # -------------------------------------------------- [H3] swap-in

    def swap_in_selected_pages(
        self,
        req_pool_indices: torch.Tensor,
        seq_lens: torch.Tensor,
        top_k_result: torch.Tensor,
        layer_id: int,
        *,
        actual_lens: torch.Tensor | None = None,
        out: torch.Tensor | None = None,
        new_k: torch.Tensor | None = None,
        new_v: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """[H3] Make the selected positions device-resident; ``[bs, top_k]`` int64 rows of
        ``device_k/v[layer_id]``, -1 past each request's ``min(seq_len, top_k)``
        (coordinator.py:232-304).  ``new_k``/``new_v`` (``[bs, kv_heads, head_dim]`` in the
        hot buffer's dtype, swap_route "kernel" only): the step's new token, written to each
        request's newest slot by the same launch (what write_new_token does,
        coordinator.py:217-228)."""
        bs = int(req_pool_indices.shape[0])
        if bs > self.max_reqs:
            raise ValueError(f"batch {bs} exceeds max_reqs {self.max_reqs}")
        if self._adm_pending:
            self._wait_admissions_of(req_pool_indices)
        rpi = req_pool_indices.to(device=self.device, dtype=torch.int64).contiguous()
        seq = seq_lens.to(device=self.device, dtype=torch.int64).contiguous()
        new_ptrs = (None, None)
        if new_k is not None or new_v is not None:
            if self.swap_route != "kernel":
                raise ValueError("the new token rides with the swap-in only on swap_route='kernel'")
            nk = new_k.reshape(bs, self.row_elems)
            nv = new_v.reshape(bs, self.row_elems)
            if nk.dtype != self.dtype or nv.dtype != self.dtype:
                raise ValueError(f"new K/V dtype {nk.dtype}/{nv.dtype} != hot buffer dtype {self.dtype}")
            nk, nv = nk.contiguous(), nv.contiguous()
            new_ptrs = (_lib.ptr(nk), _lib.ptr(nv))
        pos = top_k_result.to(device=self.device, dtype=torch.int32)
        if pos.shape[1] < self.top_k:
            pos = torch.nn.functional.pad(pos, (0, self.top_k - pos.shape[1]))
        pos = pos.contiguous()
        actual = actual_lens if actual_lens is not None else seq.clamp(max=self.top_k).to(torch.int32)
        actual = actual.to(device=self.device, dtype=torch.int32).contiguous()
        rows = out if out is not None else torch.empty((bs, self.top_k), dtype=torch.int64, device=self.device)
        if self.swap_route == "memcpy":
            _lib.call(
                "qq_hisparse_swap_plan", _lib.ptr(pos), pos.stride(0), _lib.ptr(actual), _lib.ptr(seq),
                _lib.ptr(rpi), bs, self.max_reqs, self.device_buffer_size, self.top_k,
                _lib.ptr(self.buffer_tokens[layer_id]), _lib.ptr(self.lru_slots[layer_id]),
                _lib.ptr(self.req_to_host_pool), self.max_context_len, _lib.ptr(rows), _lib.ptr(self._copy_dst),
                _lib.ptr(self._copy_src), _lib.ptr(self._copy_count), _lib.ptr(self._stats), _lib.ptr(self._err),
                self._err_host_dev, _lib.stream(self.device),
            )
            self._copy_misses_memcpy(bs, layer_id)
            if self.sync_errors:
                self.check_errors()
            return rows
        _lib.call(
            "qq_hisparse_swap_in", _lib.ptr(pos), pos.stride(0), _lib.ptr(actual), _lib.ptr(seq), _lib.ptr(rpi),
            bs, self.max_reqs, self.device_buffer_size, self.top_k, _lib.ptr(self.buffer_tokens[layer_id]),
            _lib.ptr(self.lru_slots[layer_id]), _lib.ptr(self.req_to_host_pool), self.max_context_len,
            _lib.ptr(self.device_k[layer_id]), _lib.ptr(self.device_v[layer_id]),
            self._host_layer(self._host_k_dev, layer_id), self._host_layer(self._host_v_dev, layer_id),
            self.row_bytes, self.host_k_all.shape[1], _lib.ptr(rows), _lib.ptr(self._copy_dst),
            _lib.ptr(self._copy_src), _lib.ptr(self._copy_count), _lib.ptr(self._stats), _lib.ptr(self._err),
            self._err_host_dev, new_ptrs[0], new_ptrs[1], _lib.stream(self.device),
        )
        if self.sync_errors:
            self.check_errors()
        return rows

    def _copy_misses_memcpy(self, bs: int, layer_id: int) -> None:
        """The planned misses of one layer through the copy engines: runs of consecutive host
        rows as hipMemcpyAsync (pinned host -> staging) on a side stream, then one scatter of
        the staged rows into their hot-buffer slots on the current stream."""
        counts = self._copy_count[:bs].tolist()  # synchronises: the copy list is on the device
        total = int(sum(counts))
        if total == 0:
            return
        src = torch.cat([self._copy_src[b, :c] for b, c in enumerate(counts) if c > 0]).cpu()
        dst = torch.cat([self._copy_dst[b, :c] for b, c in enumerate(counts) if c > 0])
        cut = (torch.nonzero(src[1:] != src[:-1] + 1).flatten() + 1).tolist()
        starts = [0] + cut
        ends = cut + [total]
        main = torch.cuda.current_stream(self.device)
        self._side.wait_stream(main)  # the staging buffers' previous scatter has run
        hk, hv = self.host_k_all[layer_id], self.host_v_all[layer_id]
        with torch.cuda.stream(self._side):
            for a, e in zip(starts, ends):
                s0 = int(src[a])
                self._stage_k[a:e].copy_(hk[s0 : s0 + e - a], non_blocking=True)
                self._stage_v[a:e].copy_(hv[s0 : s0 + e - a], non_blocking=True)
        main.wait_stream(self._side)
        idx = torch.arange(total, dtype=torch.int64, device=self.device)
        rows_dev = self.device_k[layer_id].shape[0]
        for stage, dev in ((self._stage_k, self.device_k[layer_id]), (self._stage_v, self.device_v[layer_id])):
            _lib.call("qq_copy_rows", _lib.ptr(stage), 0, total, _lib.ptr(idx), _lib.ptr(dev), 0, rows_dev,
                      _lib.ptr(dst), total, 1, self.row_bytes, _lib.stream(self.device))

    # -------------------------------------------------- [H4] release

    def request_finished(self, req_pool_idx: int) -> None:
        """[H4] Free the host rows, reset the request's state and bounds (coordinator.py:308-316)."""
        req = int(req_pool_idx)
        self.wait_admission(req)  # its host rows are not freed under a running backup
        self.host_allocator.free(self.req_to_host_pool[req])  # its rows >= 0, in position order
        _lib.call("qq_hisparse_request_state", _lib.ptr(self.buffer_tokens), _lib.ptr(self.lru_slots),
                  self.num_layers, self.max_reqs, self.device_buffer_size, _lib.ptr(self.req_to_host_pool),
                  self.max_context_len, req, None, 0, 1, _lib.stream(self.device))
        self._skip_first_backup[req] = 0
        self.quest.invalidate_request(req)

    # -------------------------------------------------- introspection

    def device_bytes(self) -> int:
        return 2 * self.device_k_all.numel() * self.device_k_all.element_size()

    def host_bytes(self) -> int:
        return 2 * self.host_k_all.numel() * self.host_k_all.element_size()
