"""ctypes binding of ``libqwenquest_amd.so`` (the C ABI in ``include/qwenquest_amd.h``).

The library is loaded on first use.  There is no fallback: if the shared
library is missing or a GPU is absent, calls raise instead of computing on the
CPU.  Status codes map to the exception types the reference raises:
``QQ_EINVAL`` -> ValueError, ``QQ_ERUNTIME`` / ``QQ_EHIP`` -> RuntimeError.
"""

from __future__ import annotations

import ctypes
import os

import torch

QQ_OK, QQ_EINVAL, QQ_ERUNTIME, QQ_EHIP = 0, -1, -2, -3
DTYPE_BF16, DTYPE_F32 = 0, 1

LIB_NAME = "libqwenquest_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float

# name -> (restype, argtypes); must match include/qwenquest_amd.h
SIGNATURES: dict[str, tuple] = {
    "qq_version": (_I, []),
    "qq_last_error": (ctypes.c_char_p, []),
    "qq_quest_reset": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "qq_quest_prefill_bounds": (
        _I,
        [_P, _L, _I, _L, _P, _I, _L, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    ),
    "qq_quest_decode_update": (
        _I,
        [_P, _L, _I, _L, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P],
    ),
    "qq_quest_decode_finalize": (_I, [_P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "qq_quest_prepare_step": (_I, [_P, _I, _I, _I, _I, _P, _P, _P]),
    "qq_quest_decode_step_locs": (_I, [_P, _P, _I, _P, _P, _L, _L, _L, _P, _P]),
    "qq_quest_decode_step_sync_bytes": (_L, [_I]),
    "qq_quest_decode_step": (
        _I,
        [_P, _P, _I, _P, _P, _L, _L, _L, _P, _P, _L, _I, _L, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
         _P, _P, _P, _L, _P],
    ),
    "qq_quest_retrieve_topk": (
        _I,
        [_P, _I, _L, _I, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P],
    ),
    "qq_quest_group_queries": (_I, [_P, _I, _L, _I, _I, _I, _I, _P, _P]),
    "qq_quest_page_scores": (_I, [_P, _I, _L, _P, _I, _P, _I, _I, _I, _I, _I, _P, _P]),
    "qq_decode_attention_workspace_bytes": (_L, [_I, _I, _I, _I]),
    "qq_quest_decode_attention": (
        _I,
        [_P, _I, _L, _I, _P, _P, _I, _L, _I, _I, _P, _L, _L, _P, _P, _L, _P, _I, _F, _P, _P, _L, _P],
    ),
    "qq_decode_attention_rows": (
        _I,
        [_P, _I, _L, _I, _P, _P, _I, _L, _I, _I, _P, _L, _P, _I, _F, _P, _P, _L, _P, _L, _P],
    ),
    "qq_quest_fused_step": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _I]),
    "qq_quest_forward_decode": (
        _I,
        [_P, _I, _L, _I, _P, _P, _I, _P, _P, _P, _I, _L, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I,
         _I, _I, _I, _P, _L, _L, _F, _P, _P, _P, _P, _L, _P, _L, _P],
    ),
    "qq_quest_forward_decode_phase": (
        _I,
        [_P, _I, _L, _I, _P, _P, _I, _P, _P, _P, _I, _L, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I,
         _I, _I, _I, _P, _L, _L, _F, _P, _P, _P, _P, _L, _P, _L, _I, _P],
    ),
    "qq_quest_forward_decode_noalloc": (
        _I,
        [_P, _I, _L, _I, _P, _P, _I, _P, _P, _P, _I, _L, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I,
         _I, _I, _I, _P, _L, _L, _F, _P, _P, _P],
    ),
    "qq_quest_forward_decode_noalloc_max_bytes": (_L, []),
    "qq_quest_layer_step_sync_bytes": (_L, [_I, _I]),
    "qq_dense_forward_decode": (
        _I,
        [_P, _I, _L, _I, _P, _P, _I, _P, _P, _P, _I, _L, _I, _I, _P, _P, _I, _P, _L, _L, _F, _P, _P, _L,
         _P, _L, _P],
    ),
    "qq_dense_decode_workspace_bytes": (_L, [_I, _L, _I, _I]),
    "qq_kv_scatter": (_I, [_P, _P, _I, _L, _P, _P, _I, _P, _I, _L, _P]),
    "qq_hisparse_swap_in": (
        _I,
        [_P, _L, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _L, _P, _P, _P, _P, _L, _L, _P, _P, _P,
         _P, _P, _P, _P, _P, _P, _P],
    ),
    "qq_hisparse_swap_plan": (
        _I,
        [_P, _L, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _P],
    ),
    "qq_copy_rows": (_I, [_P, _L, _L, _P, _P, _L, _L, _P, _I, _I, _L, _P]),
    "qq_hisparse_request_state": (_I, [_P, _P, _I, _I, _I, _P, _L, _I, _P, _L, _I, _P]),
    "qq_hisparse_backup_step": (_I, [_P, _P, _I, _P, _I, _I, _P, _L, _P, _P, _L, _P, _P, _P, _P, _P]),
    "qq_hisparse_ring_alloc": (_I, [_P, _P, _L, _L, _P, _P, _P, _P]),
    "qq_hisparse_ring_free": (_I, [_P, _P, _L, _P, _L, _P]),
    "qq_hisparse_write_new_token": (_I, [_P, _P, _I, _P, _P, _I, _P, _P, _I, _I, _I, _L, _P]),
    "qq_host_device_pointer": (_I, [_P, ctypes.POINTER(ctypes.c_void_p)]),
    "qq_host_alloc": (_I, [_L, ctypes.POINTER(ctypes.c_void_p)]),
    "qq_host_free": (_I, [_P]),
}

_lib: ctypes.CDLL | None = None


class LibraryNotBuilt(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load the library (once) and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryNotBuilt(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def check(status: int) -> None:
    if status == QQ_OK:
        return
    msg = load().qq_last_error().decode(errors="replace")
    if status == QQ_EINVAL:
        raise ValueError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


def ptr(t: torch.Tensor | None) -> int | None:
    """Device pointer of a CUDA (HIP) tensor; the product path never takes CPU tensors."""
    if t is None:
        return None
    if not t.is_cuda:
        raise RuntimeError(
            "qwenquest_amd runs on the GPU only: got a CPU tensor (there is no CPU fallback)"
        )
    return t.data_ptr()


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float32:
        return DTYPE_F32
    raise ValueError(f"unsupported dtype {dt}; the kernels take bfloat16 or float32")


def stream(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream
