"""GGUF expert-block formats: type ids, block geometry, row sizes and host quantisers.

Block geometry follows hot/kt_gguf_hot.py:76-91 (BLOCK_INFO, _row_bytes); the four
types with kernels here are the ones the hot path's configurations use.
"""
from __future__ import annotations

import numpy as np

from . import _lib

GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_Q6_K = 14
GGML_IQ3_S = 21
TYPE_NAMES = {GGML_Q8_0: "Q8_0", GGML_Q4_K: "Q4_K", GGML_Q6_K: "Q6_K", GGML_IQ3_S: "IQ3_S"}
NAME_TYPES = {v: k for k, v in TYPE_NAMES.items()}

# ggml type -> (values per block, bytes per block); the reference's table (kt_gguf_hot.py:76-80)
BLOCK_INFO = {
    8: (32, 34), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
    16: (256, 66), 19: (256, 74), 20: (32, 18), 21: (256, 110), 22: (256, 82), 23: (256, 136),
    18: (256, 98), 42: (64, 18),
}
# types with kernels in libktmi (the rest of BLOCK_INFO are sizes only)
KERNEL_TYPES = frozenset(TYPE_NAMES)


def row_bytes(cols: int, t: int) -> int:
    """Bytes of a row of `cols` values of ggml type t (hot/kt_gguf_hot.py:88-91)."""
    blck, ts = BLOCK_INFO[t]
    assert cols % blck == 0, (cols, t)
    return cols // blck * ts


def quantize_rows(x: np.ndarray, t: int, threads: int = 0) -> np.ndarray:
    """fp32 [rows, cols] -> uint8 [rows, row_bytes(cols, t)] on the host CPU."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    out = np.empty((rows, row_bytes(cols, t)), dtype=np.uint8)
    rc = _lib.lib().ktmi_quantize_rows_host(x.ctypes.data, rows, cols, t, out.ctypes.data, threads)
    _lib.check(rc, "quantize_rows_host")
    return out
