"""C-ABI checks that need no GPU: libc3hip.so loads, exports every function
include/c3hip.h declares, and the ctypes mirrors match the C struct layout."""

from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "c3hip.h"


def _declared_functions() -> list:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(c3h_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_families():
    names = set(_declared_functions())
    for fam in ("c3h_init", "c3h_last_error", "c3h_malloc", "c3h_memcpy_h2d_async", "c3h_stream_create",
                "c3h_event_record", "c3h_gemm", "c3h_conv2d", "c3h_qgemm", "c3h_flash_attention",
                "c3h_layernorm", "c3h_softmax", "c3h_ew", "c3h_gather", "c3h_argmax", "c3h_maxpool2d",
                "c3h_quantize", "c3h_dequantize", "c3h_program_run", "c3h_program_capture", "c3h_abi_sizes"):
        assert fam in names, fam


def test_library_exports_every_declared_symbol():
    from hackathon_amd import _lib

    lib = _lib.lib()  # also verifies struct sizes against c3h_abi_sizes
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert missing == []
    raw = C.CDLL(str(_lib.LIB_PATH))
    for n in _declared_functions():
        getattr(raw, n)


def test_ctypes_struct_sizes_match_c():
    from hackathon_amd import _lib

    _lib.lib()
    _lib.check_abi()
    assert C.sizeof(_lib.EwInst) == 24
    assert C.sizeof(_lib.Op) == 48


def test_every_kernel_family_has_an_args_struct_and_op_kind():
    from hackathon_amd import _lib

    lib = _lib.lib()
    for name, args in _lib.KERNELS.items():
        assert hasattr(lib, name)
        assert args in _lib.OP_KIND
    assert len(set(_lib.OP_KIND.values())) == len(_lib.OP_KIND)


def test_invalid_arguments_fail_before_any_launch():
    """Host-side validation returns C3H_EINVAL with a message, without touching a device."""
    from hackathon_amd import _lib

    lib = _lib.lib()
    g = _lib.GemmArgs()
    g.m, g.n, g.k, g.batch = 4, 4, 4, 0  # batch 0 is invalid
    assert lib.c3h_gemm(C.byref(g), None) == -1
    assert "bad sizes" in _lib.last_error()
    q = _lib.QGemmArgs()
    q.m, q.n, q.k, q.mode = 4, 4, 16, 7
    assert lib.c3h_qgemm(C.byref(q), None) == -1
    assert "mode" in _lib.last_error()
    with pytest.raises(_lib.C3HError):
        _lib.check(lib.c3h_gemm(C.byref(g), None), "c3h_gemm")
