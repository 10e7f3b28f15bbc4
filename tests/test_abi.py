"""The C-ABI library loads and exports every entry point include/ttlhip.h
declares (no compute calls: this runs without a GPU)."""

import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ttlhip.h")


def declared_symbols():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ttlh_\w+)\s*\(", src, flags=re.M)))


def test_header_declares_the_expected_entry_points():
    syms = declared_symbols()
    for s in ("ttlh_eltwise", "ttlh_matmul", "ttlh_matmul_bfp8w", "ttlh_matmul_bfp8w_ws",
              "ttlh_bfp4_pack_host", "ttlh_bfp4_unpack_host", "ttlh_bfp4_unpack", "ttlh_matmul_bfp4w_ws",
              "ttlh_matmul_bfp8w_workspace_bytes", "ttlh_bfp8_pack_host",
              "ttlh_bfp8_unpack_host", "ttlh_bfp8_unpack", "ttlh_sdpa_fwd", "ttlh_transpose_bf16",
              "ttlh_last_error",
              "ttlh_version"):
        assert s in syms, s


def test_library_exports_every_declared_symbol():
    from ttlhip import _lib
    lib = _lib.load()
    for s in declared_symbols():
        assert hasattr(lib, s), f"{s} declared in ttlhip.h but not exported"
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"
    assert lib.ttlh_version() == 2


def test_validation_errors_need_no_gpu():
    from ttlhip import _lib
    lib = _lib.load()
    # a matmul with K not a multiple of 32 is rejected before any device call
    st = lib.ttlh_matmul(1, 0, 40, 1, 0, 64, 1, 0, 64, 64, 64, 40, 0, None)
    assert st == _lib.TTLH_EINVAL
    assert b"multiples of 32" in lib.ttlh_last_error()
    st = lib.ttlh_sdpa_fwd(16, 16, 16, 16, 1, 1, 100, 128, 0.1, 0, None)
    assert st == _lib.TTLH_EUNSUPPORTED


def test_bfp8_two_pass_workspace_is_checked_before_any_device_call():
    from ttlhip import _lib
    lib = _lib.load()
    need = lib.ttlh_matmul_bfp8w_workspace_bytes(4096, 11008, 4096)
    assert need == 4096 * 11008 * 2
    st = lib.ttlh_matmul_bfp8w_ws(16, 4096, 16, 16, 11008, 4096, 11008, 4096, 16, need - 1, None)
    assert st == _lib.TTLH_EINVAL
    assert b"workspace" in lib.ttlh_last_error()
    st = lib.ttlh_matmul_bfp8w_ws(16, 4096, 16, 16, 11008, 4096, 11008, 4096, None, need, None)
    assert st == _lib.TTLH_EINVAL
