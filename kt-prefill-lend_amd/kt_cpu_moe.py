"""CPU cold experts and the GPU <-> CPU handoff (the other half of every hybrid layer).

`KTCPUExperts` is the CPU side of the KT wrapper for one layer, over libktmi's native engine
(ktmi_cpu_moe_*): kt-kernel's LLAMAFILE MoE forward_many numerics (K:2571-2800) on the host
cores, its weights a bank of every expert of the layer (the streamer's / hot cache's pinned
bank, [E, part bytes] per projection). `submit(x, ids, w)` stages the inputs from the device
on the current stream and returns at once; the engine's worker thread computes while the
stream runs the GPU's hot experts; `sync_add(out)` waits and adds the CPU output into the GPU
output on the stream (BaseMoEWrapper.submit_forward / sync_forward around the GPU method,
P:10590-10602; kt_uva_handoff.submit / sync_add, P:41025-41301). `forward` is the synchronous
host call.

Environment: KTMI_CPU_ISA=scalar (at creation) selects the portable int8 kernels instead of
AVX-512 VNNI.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import _lib


class KTCPUExperts:
    def __init__(self, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor, hidden: int, inter: int,
                 types: Sequence[int], threads: int = 0, max_tokens: int = 0, max_top_k: int = 0):
        for t in (gate, up, down):
            if t.device.type != "cpu" or t.dtype != torch.uint8 or t.dim() != 2 or not t.is_contiguous():
                raise RuntimeError("bank parts must be contiguous uint8 [E, part bytes] host tensors")
        if types[0] != types[1]:
            raise RuntimeError(f"gate/up types differ ({types[0]}, {types[1]})")
        self.K, self.N, self.types = hidden, inter, tuple(types)
        self._keep = (gate, up, down)  # the engine reads them in place
        self.E = gate.shape[0]
        b = _lib.ktmi_bank(gate.data_ptr(), up.data_ptr(), down.data_ptr(), gate.shape[1], up.shape[1],
                           down.shape[1], gate.shape[0])
        L = _lib.lib()
        h = L.ktmi_cpu_moe_create(hidden, inter, types[0], types[2], b, threads, max_tokens, max_top_k)
        if not h:
            raise RuntimeError(f"cpu_moe_create: {L.ktmi_last_error().decode()}")
        self._h = h
        self.max_tokens, self.max_top_k = max_tokens, max_top_k

    @classmethod
    def from_bank(cls, bank, hidden: int, inter: int, **kw) -> "KTCPUExperts":
        """From a streamer Bank or a [gate, up, down] list with its types given as types=."""
        if isinstance(bank, (list, tuple)):
            return cls(bank[0], bank[1], bank[2], hidden, inter, kw.pop("types"), **kw)
        return cls(bank.gate, bank.up, bank.down, hidden, inter, bank.types, **kw)

    @property
    def threads(self) -> int:
        return _lib.lib().ktmi_cpu_moe_threads(self._h)

    @property
    def isa(self) -> str:
        return _lib.lib().ktmi_cpu_moe_isa(self._h).decode()

    def set_add_wait(self, microseconds: int) -> None:
        """Bound on how long the add that sync_add enqueues ahead of a decode window's CPU side
        waits for it (default 10 s); past it the layer's rows become NaN and sync_add raises."""
        _lib.check(_lib.lib().ktmi_cpu_moe_set_add_wait(self._h, int(microseconds)), "cpu_moe_set_add_wait")

    def close(self):
        if getattr(self, "_h", None):
            _lib.lib().ktmi_cpu_moe_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass

    def forward(self, x: torch.Tensor, expert_ids: torch.Tensor, weights: torch.Tensor,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Host tensors: x bf16 [T, K], expert_ids int32 [T, k] (-1 / out of range: not on the
        CPU), weights fp32 [T, k] -> bf16 [T, K]."""
        x = x.contiguous()
        ids = expert_ids.to(torch.int32).contiguous()
        w = weights.to(torch.float32).contiguous()
        T, k = ids.shape
        if out is None:
            out = torch.empty((T, self.K), dtype=torch.bfloat16)
        rc = _lib.lib().ktmi_cpu_moe_forward(self._h, T, k, ids.data_ptr(), w.data_ptr(), x.data_ptr(), out.data_ptr())
        _lib.check(rc, "cpu_moe_forward")
        return out

    def submit(self, x: torch.Tensor, expert_ids: torch.Tensor, weights: torch.Tensor) -> None:
        """Device tensors on the current stream; at most max_tokens x max_top_k."""
        x = x.contiguous()
        ids = expert_ids.to(torch.int32).contiguous()
        w = weights.to(torch.float32).contiguous()
        self._inputs = (x, ids, w)  # alive until the stream has copied them
        T, k = ids.shape
        rc = _lib.lib().ktmi_cpu_moe_submit(self._h, x.data_ptr(), ids.data_ptr(), w.data_ptr(), T, k,
                                            _lib.stream_ptr(x.device))
        _lib.check(rc, "cpu_moe_submit")

    def sync_add(self, out: torch.Tensor) -> torch.Tensor:
        """out (device bf16 [T, K], contiguous) += the submitted layer's CPU output, on the
        current stream; returns out."""
        if out.dtype != torch.bfloat16 or not out.is_contiguous():
            raise RuntimeError("sync_add: out must be a contiguous bf16 tensor")
        rc = _lib.lib().ktmi_cpu_moe_sync_add(self._h, out.data_ptr(), _lib.stream_ptr(out.device))
        _lib.check(rc, "cpu_moe_sync_add")
        return out
