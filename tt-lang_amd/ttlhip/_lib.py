"""ctypes binding of libttlhip.so (declarations: include/ttlhip.h).

The library is built in-tree by tt-lang_amd/csrc/build.py and loaded from
this directory.  torch is imported first on purpose: torch ships its own HIP
runtime with the same SONAME (libamdhip64.so.7), and loading torch first makes
the dynamic linker bind libttlhip.so to that one runtime, so device pointers
and streams are shared.  There is no CPU fallback: a missing library or a
missing GPU raises.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the library load, see module docstring)

LIB_PATH = Path(os.environ.get("TTLH_LIBRARY", Path(__file__).resolve().parent / "libttlhip.so"))

TTLH_OK = 0
TTLH_EINVAL = 1
TTLH_EUNSUPPORTED = 2
TTLH_EHIP = 3

TTLH_BF16 = 0
TTLH_F32 = 1

TTLH_MAX_INSTR = 12
TTLH_MAX_STACK = 3
TTLH_BFP8_TILE_BYTES = 1088
TTLH_BFP4_TILE_BYTES = 576

# opcodes (enum ttlh_opcode)
OP = {
    "add": 1, "sub": 2, "mul": 3, "div": 4, "max": 5, "min": 6, "pow": 7,
    "floordiv": 8, "mod": 9,
    "exp": 16, "log": 17, "sqrt": 18, "rsqrt": 19, "tanh": 20, "abs": 21,
    "neg": 22, "relu": 23, "sigmoid": 24, "recip": 25, "powi": 26,
    "exp2": 27, "expm1": 28, "logp1": 29, "sin": 30, "cos": 31, "tan": 32, "asin": 33,
    "acos": 34, "atan": 35, "asinh": 36, "acosh": 37, "atanh": 38, "gelu": 39, "silu": 40,
    "softsign": 41, "hardsigmoid": 42, "elu": 43, "celu": 44, "selu": 45, "softplus": 46,
}
BINARY_OPS = {k for k, v in OP.items() if 1 <= v <= 9}
UNARY_OPS = {k for k, v in OP.items() if 16 <= v <= 46}
# unary ops with parameters (imm, imm2)
PARAM_UNARY_OPS = {"powi", "elu", "celu", "selu", "softplus"}

# forms (enum ttlh_form)
FORM_LOAD, FORM_PUSH, FORM_CONST, FORM_PUSH_CONST, FORM_UNARY = 0, 1, 2, 3, 4
FORM_BIN, FORM_BIN_REV, FORM_BIN_IMM, FORM_BIN_IMM_REV, FORM_BIN_POP = 5, 6, 7, 8, 9


class Instr(C.Structure):
    _fields_ = [
        ("op", C.c_uint8), ("form", C.c_uint8), ("rnd", C.c_uint8), ("pad", C.c_uint8),
        ("imm", C.c_float), ("imm2", C.c_float),
    ]


# ttlh_reduce kinds and dimension bits
REDUCE_SUM, REDUCE_MAX = 0, 1
REDUCE_DIM0, REDUCE_DIM1 = 1, 2


class Operand(C.Structure):
    _fields_ = [
        ("ptr", C.c_void_p), ("dtype", C.c_int32), ("pad", C.c_int32),
        ("row_stride", C.c_int64), ("col_stride", C.c_int64),
        ("row_mask", C.c_int64), ("col_mask", C.c_int64),
        ("row_off", C.c_int64), ("col_off", C.c_int64),
    ]


class RowReduce(C.Structure):
    _fields_ = [
        ("prog", C.POINTER(Instr)), ("in_", C.POINTER(Operand)), ("n_instr", C.c_int32),
        ("kind", C.c_int32), ("scaler", C.c_void_p), ("scaler_dtype", C.c_int32),
        ("scale_imm", C.c_float), ("out", C.c_void_p), ("out_dtype", C.c_int32),
        ("out_pad", C.c_int32), ("out_ld", C.c_int64),
    ]


# every symbol include/ttlhip.h declares, with its ctypes signature
_i64, _vp, _int = C.c_int64, C.c_void_p, C.c_int
SIGNATURES = {
    "ttlh_eltwise": (_int, [C.POINTER(Instr), C.POINTER(Operand), _int, _vp, _int, _i64, _i64,
                            _i64, _i64, _i64, _vp]),
    "ttlh_tilize": (_int, [_vp, _i64, _vp, _i64, _i64, _int, _vp]),
    "ttlh_untilize": (_int, [_vp, _vp, _i64, _i64, _i64, _int, _vp]),
    "ttlh_transpose_bf16": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _vp]),
    "ttlh_reduce_workspace_bytes": (_i64, [_int, _i64, _i64]),
    "ttlh_reduce": (_int, [C.POINTER(Instr), C.POINTER(Operand), _int, _int, _int, _vp, _int,
                           C.c_float, _vp, _int, _i64, _int, _i64, _i64, _i64, _i64, _vp, _i64,
                           _vp]),
    "ttlh_reduce_noalloc": (_int, [C.POINTER(Instr), C.POINTER(Operand), _int, _int, _int, _vp,
                                   _int, C.c_float, _vp, _int, _i64, _int, _i64, _i64, _i64, _i64,
                                   _vp]),
    "ttlh_reduce_rows_eltwise": (_int, [C.POINTER(RowReduce), _int, C.POINTER(Instr),
                                        C.POINTER(Operand), _int, _vp, _int, _i64, _i64, _i64,
                                        _i64, _i64, _vp]),
    "ttlh_matmul": (_int, [_vp, _int, _i64, _vp, _int, _i64, _vp, _int, _i64, _i64, _i64, _i64,
                           _int, _vp]),
    "ttlh_matmul_eltwise": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _i64, C.POINTER(Instr),
                                   C.POINTER(Operand), _int, _int, _vp, _int, _i64, _i64, _i64,
                                   _vp]),
    "ttlh_bfp8_pack_host": (_int, [_vp, _vp, _i64, _i64]),
    "ttlh_bfp8_unpack_host": (_int, [_vp, _vp, _i64, _i64]),
    "ttlh_bfp8_unpack": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "ttlh_matmul_bfp8w": (_int, [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "ttlh_matmul_bfp8w_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "ttlh_bfp4_pack_host": (_int, [_vp, _vp, _i64, _i64]),
    "ttlh_bfp4_unpack_host": (_int, [_vp, _vp, _i64, _i64]),
    "ttlh_bfp4_unpack": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "ttlh_matmul_bfp4w_ws": (_int, [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp]),
    "ttlh_matmul_bfp8w_ws": (_int, [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp]),
    "ttlh_sdpa_fwd": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, C.c_float, _int, _vp]),
    "ttlh_last_error": (C.c_char_p, []),
    "ttlh_version": (_int, []),
}

_lib = None


class TTLHError(RuntimeError):
    """A libttlhip.so entry point returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed (status {code}): {msg}")
        self.code = code


def load() -> C.CDLL:
    """Loads libttlhip.so (once) and binds every declared entry point."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python tt-lang_amd/csrc/build.py` "
            "(or __graft_entry__.build()); there is no CPU fallback"
        )
    lib = C.CDLL(os.fspath(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(fn: str, status: int) -> None:
    if status != TTLH_OK:
        msg = load().ttlh_last_error().decode(errors="replace")
        if status == TTLH_EINVAL:
            raise ValueError(f"{fn}: {msg}")
        raise TTLHError(fn, status, msg)


def call(fn: str, *args) -> None:
    """Calls entry point `fn` and raises on a non-zero status."""
    check(fn, getattr(load(), fn)(*args))


def require_device() -> None:
    if not torch.cuda.is_available():
        raise RuntimeError(
            "tt-lang_amd executes on an AMD GPU (MI355X, gfx950); no HIP device is visible "
            "and there is no CPU fallback"
        )


def stream_ptr(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return TTLH_BF16
    if dt == torch.float32:
        return TTLH_F32
    raise TypeError(f"tt-lang_amd kernels take bfloat16 or float32 tensors, got {dt}")
