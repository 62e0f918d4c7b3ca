"""GGUF expert blocks -> bf16 rows on the GPU (drop-in for kt_gguf_dequant.py, P:11284-11498).

`dequant_experts(raw, raw_stride, type_id, n, rows, cols, out)` keeps the reference's
contract (P:11471-11498): raw is an expert-major uint8 device tensor with raw_stride bytes
per expert, out is [n, rows, cols] bf16 with contiguous rows and out.stride(0) elements
between experts; it runs on the current stream. Every value is the exact fp32
dequantisation rounded once to bf16. Types: Q8_0, Q4_K, Q6_K, IQ3_S (the reference's
Triton file covers IQ3_S among its i-quants; Q8_0 / Q4_K / Q6_K have no GPU dequantizer
there).
"""
from __future__ import annotations

import torch

from . import _lib
from .gguf import BLOCK_INFO, KERNEL_TYPES

GGML_Q8_0, GGML_Q4_K, GGML_Q6_K, GGML_IQ3_S = 8, 12, 14, 21


def dequant_experts(raw: torch.Tensor, raw_stride: int, type_id: int, n: int, rows: int, cols: int,
                    out: torch.Tensor) -> None:
    if type_id not in KERNEL_TYPES:
        raise ValueError(f"no GPU dequantizer for ggml type {type_id}")
    blck, _ = BLOCK_INFO[type_id]
    assert cols % blck == 0, (type_id, cols, blck)
    assert out.dtype == torch.bfloat16 and out.stride(-1) == 1 and out.stride(-2) == cols, out.stride()
    rc = _lib.lib().ktmi_dequant_experts(raw.data_ptr(), raw_stride, type_id, n, rows, cols, out.data_ptr(),
                                         out.stride(0) if out.dim() == 3 else rows * cols,
                                         _lib.stream_ptr(out.device))
    _lib.check(rc, "dequant_experts")
