"""The C-ABI library loads, exports every symbol the header declares with the
argument count the ctypes binding uses, and reports argument errors - all
without a GPU (no kernel is launched)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "qwenquest_amd.h")


def _declarations() -> dict[str, int]:
    """name -> number of parameters, parsed from include/qwenquest_amd.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int|int64_t|const char\*)\s+(qq_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        decls[m.group(1)] = len(params)
    return decls


@pytest.fixture(scope="module")
def lib():
    from qwenquest_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        from qwenquest_amd import build

        build.build()
    return _lib.load()


def test_header_declares_the_entry_points():
    decls = _declarations()
    assert len(decls) >= 12
    for name in ("qq_quest_retrieve_topk", "qq_quest_decode_attention", "qq_quest_prefill_bounds"):
        assert name in decls


def test_every_declared_symbol_is_exported_with_matching_arity(lib):
    from qwenquest_amd import _lib

    decls = _declarations()
    for name, nargs in decls.items():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _lib.SIGNATURES, f"{name} missing from the ctypes binding"
        assert len(_lib.SIGNATURES[name][1]) == nargs, f"{name}: binding arity != header"
    assert set(_lib.SIGNATURES) == set(decls)


def test_version_and_error_mapping_without_gpu(lib):
    from qwenquest_amd import _lib

    assert lib.qq_version() == 100
    # argument validation happens before any HIP call: page_size 0 -> QQ_EINVAL
    st = lib.qq_quest_prepare_step(None, 1, 0, 64, 0, None, None, None)
    assert st == _lib.QQ_EINVAL
    assert b"bad arguments" in lib.qq_last_error()
    with pytest.raises(ValueError):
        _lib.check(st)
    st = lib.qq_quest_retrieve_topk(None, 0, 0, 32, None, 0, None, None, None, 1, 1, 1, 4, 128,
                                    64, 100, None, None, None, None)
    assert st == _lib.QQ_EINVAL and b"multiple" in lib.qq_last_error()
    assert lib.qq_decode_attention_workspace_bytes(16, 2048, 32, 128) == 16 * 32 * 32 * 130 * 4


def test_cpu_tensors_are_refused():
    import torch

    from qwenquest_amd import _lib

    with pytest.raises(RuntimeError, match="GPU only"):
        _lib.ptr(torch.zeros(4))


def test_library_has_no_host_fallback_symbols(lib):
    """Every exported qq_ symbol is one the header declares (nothing undocumented)."""
    out = os.popen(f"nm -D --defined-only {lib._name}").read()
    exported = set(re.findall(r"\b(qq_\w+)\b", out))
    assert exported == set(_declarations())
    assert ctypes.sizeof(ctypes.c_void_p) == 8


def test_forward_decode_phase_is_validated_without_gpu(lib):
    """A phase other than 1, 2 or 3 is refused (QQ_EINVAL) before any HIP call; the
    fused layer step's sync buffer holds one 128-byte counter line per (request, KV head)."""
    from qwenquest_amd import _lib

    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    args = [fake, 0, 4096, 32, None, None, 0, None, fake, fake, 0, 100, fake, 0, fake, fake, fake, fake,
            2, 4, 64, 4, 128, 64, 2048, fake, 64, 4, 0.088, fake, fake, fake, fake, 1 << 20, None, 0]
    for phase in (0, 4, -1):
        st = lib.qq_quest_forward_decode_phase(*args, phase, None)
        assert st == _lib.QQ_EINVAL and b"phase" in lib.qq_last_error()
    assert lib.qq_quest_layer_step_sync_bytes(16, 4) == 16 * 4 * 128
    assert lib.qq_quest_layer_step_sync_bytes(0, 4) == 0


def test_fused_step_predicate_without_gpu(lib):
    """qq_quest_fused_step: the shapes the fused layer step takes (no HIP call)."""
    from qwenquest_amd import _lib

    bf, f32 = _lib.DTYPE_BF16, _lib.DTYPE_F32
    # the benchmark shape: 32 q / 4 KV heads x 128, page 64, top_k 2048, 2049 pages
    assert lib.qq_quest_fused_step(bf, bf, bf, 32, 4, 128, 64, 2048, 2049) == 1
    assert lib.qq_quest_fused_step(bf, bf, -1, 32, 4, 128, 64, 2048, 8192) == 1  # no new token; 8192 pages
    assert lib.qq_quest_fused_step(bf, bf, bf, 32, 4, 128, 64, 2048, 8193) == 0  # too many pages
    assert lib.qq_quest_fused_step(bf, bf, bf, 32, 4, 128, 16, 2048, 2049) == 0  # page 16
    assert lib.qq_quest_fused_step(bf, bf, bf, 32, 4, 128, 64, 4224, 2049) == 0  # 65 selected pages
    assert lib.qq_quest_fused_step(bf, bf, f32, 32, 4, 128, 64, 2048, 2049) == 0  # fp32 new token
    assert lib.qq_quest_fused_step(f32, bf, bf, 32, 4, 128, 64, 2048, 2049) == 0  # fp32 queries
    assert lib.qq_quest_fused_step(bf, bf, bf, 16, 2, 128, 64, 2048, 2049) == 0  # 2 KV heads
    assert lib.qq_quest_fused_step(bf, bf, bf, 128, 4, 128, 64, 2048, 2049) == 0  # G = 32
