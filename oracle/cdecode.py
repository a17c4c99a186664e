"""ctypes binding of the C restatement in mxfp4_ref.c (test infrastructure)."""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, '_lib', 'liborc.so')
_lib = None


def build() -> str:
    """Compile mxfp4_ref.c with gcc into oracle/_lib/liborc.so and return its path."""
    subprocess.run(['make', '-s', '-B', '-C', _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        _lib.orc_mxfp4_decode.argtypes = [p, p, ctypes.c_int64, p]
        _lib.orc_topk_sorted.argtypes = [p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, p]
        _lib.orc_group.argtypes = [p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, p, p, p, p]
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def mxfp4_decode_bits(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """uint8 [..., n, 16] + uint8 [..., n] -> uint32 FP32 bit patterns [..., n*32]."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    if blocks.shape[:-1] != scales.shape or blocks.shape[-1] != 16:
        raise ValueError('invalid MXFP4 block/scale geometry')
    n = scales.size
    out = np.empty(n*32, dtype=np.uint32)
    lib().orc_mxfp4_decode(_ptr(blocks), _ptr(scales), n, _ptr(out))
    return out.reshape(*scales.shape[:-1], scales.shape[-1]*32) if scales.ndim else out


def topk_sorted(values: np.ndarray, k: int) -> np.ndarray:
    """float32 [rows, n] -> int64 [rows, k]: the k best (NaN first, lowest index on ties), ascending."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    rows, n = values.shape
    out = np.empty((rows, k), dtype=np.int64)
    lib().orc_topk_sorted(_ptr(values), rows, n, k, _ptr(out))
    return out


def group(ids: np.ndarray, experts: int):
    """int64 [rows, k] -> (counts [E], offsets [E+1], pair_row [rows*k], pair_slot [rows*k])."""
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    rows, k = ids.shape
    counts = np.empty(experts, dtype=np.int32)
    offsets = np.empty(experts + 1, dtype=np.int32)
    pair_row = np.empty(rows*k, dtype=np.int32)
    pair_slot = np.empty(rows*k, dtype=np.int32)
    lib().orc_group(_ptr(ids), rows, k, experts, _ptr(counts), _ptr(offsets), _ptr(pair_row), _ptr(pair_slot))
    return counts, offsets, pair_row, pair_slot
