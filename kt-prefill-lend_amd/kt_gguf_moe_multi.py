"""The GGUF MoE GEMV for decode windows (drop-in for hot/kt_gguf_moe_multi.py).

`moe_a8_vec_multi(X, W, ids, top_k, type, rows, tokens, table=False)` keeps the
reference's contract (hot/kt_gguf_moe_multi.py:81-82, kernel kt_gguf_moe_multi.cu:653):
Y [tokens*top_k, rows] in X's dtype, route p = t*top_k + k uses token t and expert
ids[p], ids < 0 (experts on the CPU) give zero rows, and the routes of one expert share
one read of its weights. Unlike the reference's window build it is correct at any token
count (an expert with more than 4 routes runs them 4 at a time), so `moe_a8_vec_routes`
(the per-route build, :85-87) gives the same sums and is kept for the callers that ask
for it. With table=True, W is an int64 device table of per-slot weight addresses.

It runs on the current HIP stream, allocates its q8_1 scratch from torch's caching
allocator, never synchronises and is graph-capturable.
"""
from __future__ import annotations

import os

import torch

from . import _lib
from .gguf import KERNEL_TYPES

MAX_TOKENS = int(os.environ.get("KT_GGUF_MOE_MAXM", "4"))
ROUTES = os.environ.get("KT_GGUF_MOE_ROUTES", "1") == "1"
DENSE = os.environ.get("KT_GGUF_DENSE_MULTI", "1") == "1"
DENSE_MIN_ROWS = 513
DENSE_TYPES = set(KERNEL_TYPES)
_zero_ids = {}


def enabled() -> bool:
    return os.environ.get("KT_GGUF_MOE_MULTI", "1") == "1"


def _run(X, W, ids, top_k, qtype, rows, tokens, table, per_route):
    if ids.dtype != torch.int32:
        # the reference reads the ids as int32 unchecked (hot/kt_gguf_hot.py:286-292); refuse instead
        raise TypeError(f"moe_a8_vec: ids must be int32, got {ids.dtype}")
    X = X.contiguous()
    ids = ids.contiguous()
    cols = X.shape[1]
    Y = torch.empty((tokens * top_k, rows), dtype=X.dtype, device=X.device)
    L = _lib.lib()
    ws_bytes = L.ktmi_moe_a8_vec_workspace(cols, tokens)
    ws = torch.empty((max(ws_bytes, 16),), dtype=torch.uint8, device=X.device)
    rc = L.ktmi_moe_a8_vec(X.data_ptr(), _lib.dtype_code(X.dtype), cols, W.data_ptr(), int(bool(table)),
                           ids.data_ptr(), top_k, qtype, rows, tokens, int(per_route), Y.data_ptr(),
                           ws.data_ptr(), ws_bytes, _lib.stream_ptr(X.device))
    _lib.check(rc, "moe_a8_vec")
    return Y


def moe_a8_vec_multi(X, W, ids, top_k, qtype, rows, tokens, table=False):
    return _run(X, W, ids, top_k, qtype, rows, tokens, table, per_route=False)


def moe_a8_vec_routes(X, W, ids, top_k, qtype, rows, tokens, table=False):
    """Route p's rows from expert ids[p], each route on its own; zeros for ids < 0."""
    return _run(X, W, ids, top_k, qtype, rows, tokens, table, per_route=True)


def reads_table(tokens: int) -> bool:
    """Whether the kernel for a window of this many tokens can read slot weights through
    the pointer table (hot/kt_gguf_moe_multi.py:90-95). Every ktmi kernel can."""
    return enabled()


def dense_ok(x, qweight, qtype) -> bool:
    return (DENSE and 2 <= x.shape[0] <= MAX_TOKENS and qtype in DENSE_TYPES and qweight.dim() == 2
            and qweight.shape[0] >= DENSE_MIN_ROWS and qweight.dtype == torch.uint8 and qweight.is_contiguous())


def dense_a8_vec(x, qweight, qtype):
    """y = x @ W^T for a dense GGUF weight [rows, row_bytes], each row read once for all tokens
    (a one-expert MoE, hot/kt_gguf_moe_multi.py:98-112)."""
    T = x.shape[0]
    rows = qweight.shape[0]
    key = (x.device, T)
    ids = _zero_ids.get(key)
    if ids is None:
        ids = _zero_ids[key] = torch.zeros(T, dtype=torch.int32, device=x.device)
    y = moe_a8_vec_multi(x, qweight.view(1, rows, qweight.shape[1]), ids, 1, qtype, rows, T)
    return y.view(T, rows)
