"""bfloat8_b and bfloat4_b oracles: the C restatements (bfp8_ref.c) via
ctypes plus independent numpy restatements (TEST INFRASTRUCTURE ONLY).

Formats: see bfp8_ref.c.  decode_table() / decode4_table() are the exact
float64 values of every (exponent, element) pair, the closed forms the codecs
must reproduce.
"""

import ctypes as C
from pathlib import Path

import numpy as np
import torch

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        from . import build_ref
        path = build_ref.LIB
        if not path.exists():
            build_ref.build()
        _LIB = C.CDLL(str(path))
        _LIB.oracle_bfp8_pack.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int64]
        _LIB.oracle_bfp8_unpack.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int64]
        _LIB.oracle_bfp8_decode.argtypes = [C.c_uint8, C.c_uint8]
        _LIB.oracle_bfp8_decode.restype = C.c_uint16
        _LIB.oracle_bfp4_pack.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int64]
        _LIB.oracle_bfp4_unpack.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int64]
        _LIB.oracle_bfp4_decode.argtypes = [C.c_uint8, C.c_uint8]
        _LIB.oracle_bfp4_decode.restype = C.c_uint16
    return _LIB


def pack_c(x: torch.Tensor) -> torch.Tensor:
    x = x.detach().float().contiguous()
    rows, cols = x.shape
    out = torch.empty((rows // 32) * (cols // 32) * 1088, dtype=torch.uint8)
    lib().oracle_bfp8_pack(x.data_ptr(), out.data_ptr(), rows, cols)
    return out


def unpack_c(q: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    q = q.contiguous()
    out = torch.empty((rows, cols), dtype=torch.bfloat16)
    lib().oracle_bfp8_unpack(q.data_ptr(), out.data_ptr(), rows, cols)
    return out


def decode_table() -> np.ndarray:
    """[256 exponents, 256 bytes] -> exact float64 value (-1)^s m 2^(e-133)."""
    e = np.arange(256, dtype=np.float64)[:, None]
    b = np.arange(256)[None, :]
    m = (b & 0x7F).astype(np.float64)
    s = np.where(b & 0x80, -1.0, 1.0)
    v = s * m * np.exp2(e - 133.0)
    return np.where(np.abs(v) >= 2.0 ** 128, s * np.inf, v)  # overflow (e = 255 only)


def _faces(rows, cols):
    """numpy index maps: element (r, c) -> (tile, face, face row, face col)."""
    r = np.arange(rows)[:, None]
    c = np.arange(cols)[None, :]
    tile = (r // 32) * (cols // 32) + (c // 32)
    rr, cc = r % 32, c % 32
    face = (rr // 16) * 2 + (cc // 16)
    return tile, face, rr % 16, cc % 16


def pack_np(x: np.ndarray) -> np.ndarray:
    """numpy restatement of the packer (float64 arithmetic, RNE)."""
    x = np.asarray(x, dtype=np.float32)
    rows, cols = x.shape
    tile, face, fr, fc = _faces(rows, cols)
    ex = ((x.view(np.uint32) >> 23) & 0xFF).astype(np.int64)
    # shared exponent per (tile, face, face row): max over the 16 columns
    key = (tile * 4 + face) * 16 + fr
    nkey = (rows // 32) * (cols // 32) * 64
    e = np.zeros(nkey, dtype=np.int64)
    np.maximum.at(e, key.ravel(), ex.ravel())
    scaled = np.abs(x.astype(np.float64)) * np.exp2(133.0 - e[key])
    m = np.minimum(np.round(scaled), 127).astype(np.int64)  # np.round is half-to-even
    sign = (x.view(np.uint32) >> 31).astype(np.int64)
    out = np.zeros((rows // 32) * (cols // 32) * 1088, dtype=np.uint8)
    base = tile * 1088
    out[(base + 16 * face + fr).ravel()] = e[key].ravel().astype(np.uint8)
    out[(base + 64 + 256 * face + 16 * fr + fc).ravel()] = ((sign << 7) | m).ravel().astype(np.uint8)
    return out


def unpack_np(q: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Exact float64 values of a packed matrix."""
    q = np.asarray(q, dtype=np.uint8)
    tile, face, fr, fc = _faces(rows, cols)
    base = tile * 1088
    e = q[base + 16 * face + fr].astype(np.int64)
    b = q[base + 64 + 256 * face + 16 * fr + fc].astype(np.int64)
    return decode_table()[e, b]


# ---------------------------------------------------------------------------
# bfloat4_b: 576-byte tiles (python/ttl/dtype_utils.py:176-177)


def pack4_c(x: torch.Tensor) -> torch.Tensor:
    x = x.detach().float().contiguous()
    rows, cols = x.shape
    out = torch.empty((rows // 32) * (cols // 32) * 576, dtype=torch.uint8)
    lib().oracle_bfp4_pack(x.data_ptr(), out.data_ptr(), rows, cols)
    return out


def unpack4_c(q: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    q = q.contiguous()
    out = torch.empty((rows, cols), dtype=torch.bfloat16)
    lib().oracle_bfp4_unpack(q.data_ptr(), out.data_ptr(), rows, cols)
    return out


def decode4_table() -> np.ndarray:
    """[256 exponents, 16 nibbles] -> exact float64 value (-1)^s m 2^(e-129)."""
    e = np.arange(256, dtype=np.float64)[:, None]
    n = np.arange(16)[None, :]
    m = (n & 7).astype(np.float64)
    s = np.where(n & 8, -1.0, 1.0)
    v = s * m * np.exp2(e - 129.0)
    return np.where(np.abs(v) >= 2.0 ** 128, s * np.inf, v)


def pack4_np(x: np.ndarray) -> np.ndarray:
    """numpy restatement of the bfloat4_b packer (float64 arithmetic, RNE)."""
    x = np.asarray(x, dtype=np.float32)
    rows, cols = x.shape
    tile, face, fr, fc = _faces(rows, cols)
    ex = ((x.view(np.uint32) >> 23) & 0xFF).astype(np.int64)
    key = (tile * 4 + face) * 16 + fr
    e = np.zeros((rows // 32) * (cols // 32) * 64, dtype=np.int64)
    np.maximum.at(e, key.ravel(), ex.ravel())
    m = np.minimum(np.round(np.abs(x.astype(np.float64)) * np.exp2(129.0 - e[key])), 7)
    nib = (((x.view(np.uint32) >> 31).astype(np.int64) << 3) | m.astype(np.int64))
    out = np.zeros((rows // 32) * (cols // 32) * 576, dtype=np.int64)
    base = tile * 576
    out[(base + 16 * face + fr).ravel()] = e[key].ravel()
    byte = (base + 64 + 128 * face + 8 * fr + fc // 2).ravel()
    np.add.at(out, byte, (nib << (4 * (fc & 1))).ravel())
    return out.astype(np.uint8)


def unpack4_np(q: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Exact float64 values of a packed bfloat4_b matrix."""
    q = np.asarray(q, dtype=np.uint8)
    tile, face, fr, fc = _faces(rows, cols)
    base = tile * 576
    e = q[base + 16 * face + fr].astype(np.int64)
    nib = (q[base + 64 + 128 * face + 8 * fr + fc // 2].astype(np.int64) >> (4 * (fc & 1))) & 15
    return decode4_table()[e, nib]
