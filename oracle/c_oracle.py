"""ctypes wrapper of the C oracle (``oracle/c/oracle.c``) -- test infrastructure only.

Operates on numpy arrays; builds the library on first use if it is missing.
"""

from __future__ import annotations

import ctypes

import numpy as np

from oracle import build_c

_LIB = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not build_c.OUT.exists():
            build_c.build()
        _LIB = ctypes.CDLL(str(build_c.OUT))
        _LIB.oracle_f32_to_f16.restype = ctypes.c_uint16
        _LIB.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        _LIB.oracle_f16_to_f32.restype = ctypes.c_float
        _LIB.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    return _LIB


def _p(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


def slot_scatter(pool: np.ndarray, source: np.ndarray, blocks: list[int], start: int) -> None:
    """In-place: pool (H, NB, BS, D), source (H, T, D) of the same dtype."""
    H, NB, BS, D = pool.shape
    assert pool.flags.c_contiguous and source.dtype == pool.dtype
    src = np.ascontiguousarray(source)
    tbl = np.asarray(blocks, dtype=np.int32)
    rc = lib().oracle_slot_scatter(
        _p(pool), pool.itemsize, H, NB, BS, D, _p(src), src.shape[1], _p(tbl), tbl.size, start
    )
    if rc:
        raise IndexError(f"oracle_slot_scatter: {rc}")


def gather(pool: np.ndarray, blocks: list[int], seq_len: int) -> np.ndarray:
    H, NB, BS, D = pool.shape
    out = np.empty((H, seq_len, D), dtype=pool.dtype)
    tbl = np.asarray(blocks, dtype=np.int32)
    rc = lib().oracle_gather(
        _p(np.ascontiguousarray(pool)), pool.itemsize, H, NB, BS, D, _p(tbl), tbl.size, seq_len,
        _p(out),
    )
    if rc:
        raise IndexError(f"oracle_gather: {rc}")
    return out


def quantize(w: np.ndarray, group_size: int, bits: int) -> tuple[np.ndarray, np.ndarray]:
    """``(codes int8 (n, k), scales float16 (n, k/g))``."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    codes = np.empty((n, k), dtype=np.int8)
    scales = np.empty((n, k // group_size), dtype=np.uint16)
    rc = lib().oracle_quantize(_p(w), n, k, group_size, bits, _p(codes), _p(scales))
    if rc:
        raise ValueError("ragged group")
    return codes, scales.view(np.float16)


def pack_int4(codes: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    n, k = codes.shape
    out = np.empty((n, k // 2), dtype=np.uint8)
    lib().oracle_pack_int4(_p(codes), n, k, _p(out))
    return out


def unpack_int4(packed: np.ndarray, k: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    n = packed.shape[0]
    out = np.empty((n, k), dtype=np.int8)
    lib().oracle_unpack_int4(_p(packed), n, k, _p(out))
    return out


def dequantize(codes: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    sc = np.ascontiguousarray(scales, dtype=np.float16).view(np.uint16)
    n, k = codes.shape
    out = np.empty((n, k), dtype=np.uint16)
    lib().oracle_dequantize(_p(codes), _p(sc), n, k, group_size, _p(out))
    return out.view(np.float16)


def f32_to_f16(x: float) -> np.float16:
    return np.array([lib().oracle_f32_to_f16(x)], dtype=np.uint16).view(np.float16)[0]
