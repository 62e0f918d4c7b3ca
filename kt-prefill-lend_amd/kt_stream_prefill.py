"""Streamed GGUF prefill: the layer-weight streamer (drop-in for the reference's
kt_stream_prefill_gguf module, P:40470-41050).

Experts' raw GGUF bytes live in pinned host banks, one per layer (`Bank`: gate, up and down
parts, [E, part bytes] each, the reference's _bank, P:40700-40752). A prefill chunk runs a
layer's experts in groups of GROUP_SIZE: while the grouped layer kernels work on group g in
one device slot, group g+1 is copied into the other slot on a copy stream of its own
(`ktmi_streamer_*`, the reference's _Slot / _stage / run, P:40543-40550, 40773-40787,
40928-40992). Each group's partial output is added to the layer's bf16 accumulator
(acc.add_(out), P:40819).

Differences from the reference, on purpose:
  * the slots hold the raw blocks in the layout the grouped kernels read, so there is no
    bf16 copy of each group's weights (the reference dequantises into w13_bf16 / w2_bf16,
    P:40789-40798) and no CUTLASS workspace;
  * banks are built lazily per layer from an expert reader (`reader=`: a GGUFExperts over
    the GGUF file, or any source with banks(layer, N, rank, p2l)), as the reference's
    _bank does (P:40712-40752), or handed in as pinned tensors (`set_bank`);
  * `run` takes plain tensors (x, topk weights, expert ids); `run_layers` pipelines whole
    layers, so layer l+1's weights stream in while layer l computes.

Environment (same names as the reference): KT_GPU_STREAM_PREFILL (token threshold, 0 =
off), KT_GPU_STREAM_GROUP (experts per group, 8), KT_GPU_STREAM_TIMING=1 (log per layer).
"""
from __future__ import annotations

import ctypes as C
import os
import time
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import _lib
from .gguf import row_bytes

STREAM_THRESHOLD = int(os.environ.get("KT_GPU_STREAM_PREFILL", "0") or 0)
GROUP_SIZE = int(os.environ.get("KT_GPU_STREAM_GROUP", "8") or 8)
TIMING = os.environ.get("KT_GPU_STREAM_TIMING") == "1"


def _log(msg: str):
    print(f"[kt-stream-gguf {time.strftime('%H:%M:%S')}] {msg}", flush=True)


def part_bytes(types: Tuple[int, int, int], N: int, K: int) -> Tuple[int, int, int]:
    """Bytes of one expert's gate, up and down parts (P:40583)."""
    return N * row_bytes(K, types[0]), N * row_bytes(K, types[1]), K * row_bytes(N, types[2])


@dataclass
class Bank:
    """One layer's pinned host bank: gate, up, down uint8 [E, part bytes] (physical order)."""

    gate: torch.Tensor
    up: torch.Tensor
    down: torch.Tensor
    types: Tuple[int, int, int]

    def __post_init__(self):
        E = self.gate.shape[0]
        for t in (self.gate, self.up, self.down):
            if t.dtype != torch.uint8 or t.dim() != 2 or t.shape[0] != E or not t.is_contiguous():
                raise RuntimeError("bank parts must be contiguous uint8 [E, part bytes] tensors")
            if t.device.type != "cpu":
                raise RuntimeError("bank parts live in host memory")
        if self.gate.shape[1] != self.up.shape[1]:
            raise RuntimeError("gate and up parts must have the same size")
        if self.types[0] != self.types[1]:
            # hot/kt_gguf_hot.py:176-178: gate and up share a type
            raise RuntimeError(f"gate/up types differ ({self.types[0]}, {self.types[1]})")

    @property
    def n_experts(self) -> int:
        return self.gate.shape[0]

    def c_struct(self) -> _lib.ktmi_bank:
        return _lib.ktmi_bank(self.gate.data_ptr(), self.up.data_ptr(), self.down.data_ptr(), self.gate.shape[1],
                              self.up.shape[1], self.down.shape[1], self.gate.shape[0])

    @classmethod
    def pinned(cls, E: int, parts: Tuple[int, int, int], types: Tuple[int, int, int]) -> "Bank":
        """An empty pinned bank (torch's pinned allocator: hipHostMalloc)."""
        mk = lambda n: torch.empty((E, n), dtype=torch.uint8, pin_memory=True)  # noqa: E731
        return cls(mk(parts[0]), mk(parts[1]), mk(parts[2]), types)

    @classmethod
    def from_slot_rows(cls, w13: torch.Tensor, w2: torch.Tensor, N: int, types: Tuple[int, int, int]) -> "Bank":
        """A pinned bank from slot-layout host tensors w13 [E, 2N, rb13] ([gate; up]) and
        w2 [E, K, rb2]."""
        E = w13.shape[0]
        b = cls.pinned(E, (N * w13.shape[2], N * w13.shape[2], w2.shape[1] * w2.shape[2]), types)
        b.gate.copy_(w13[:, :N].reshape(E, -1))
        b.up.copy_(w13[:, N:].reshape(E, -1))
        b.down.copy_(w2.reshape(E, -1))
        return b


class KTStreamPrefillGGUF:
    """Process-wide (per device) streaming state shared by every MoE layer (P:40641)."""

    def __init__(self, N: int, K: int, top_k: int, types: Tuple[int, int, int], group_size: int = GROUP_SIZE,
                 device=None, n_slots: int = 2, reader=None, rank: int = 0, p2l=None):
        self.N, self.K, self.top_k, self.G = N, K, top_k, group_size
        self.reader, self.rank = reader, rank
        self._p2l = p2l  # layer -> physical_to_logical list, or None
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.types = tuple(types)
        pg, pu, pd = part_bytes(self.types, N, K)
        self.n_slots = n_slots
        self._banks: Dict[int, Bank] = {}
        L = _lib.lib()
        with torch.cuda.device(self.device):
            h = L.ktmi_streamer_create(self.G, pg + pu, pd, n_slots)
        if not h:
            raise RuntimeError(f"streamer_create failed: {L.ktmi_last_error().decode()}")
        self._h = C.c_void_p(h)
        self.slots = []
        for i in range(n_slots):
            a, b = C.c_void_p(), C.c_void_p()
            _lib.check(L.ktmi_streamer_slot(self._h, i, C.byref(a), C.byref(b)), "streamer_slot")
            self.slots.append((a.value, b.value))
        self._ws: Optional[torch.Tensor] = None
        self.calls = 0

    def close(self):
        if getattr(self, "_h", None):
            _lib.lib().ktmi_streamer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass

    # -- banks ---------------------------------------------------------------

    def set_bank(self, layer_idx: int, bank: Bank):
        if bank.types != self.types:
            raise RuntimeError(f"layer {layer_idx}: bank types {bank.types} != streamer types {self.types}")
        if (bank.gate.shape[1], bank.up.shape[1], bank.down.shape[1]) != part_bytes(self.types, self.N, self.K):
            raise RuntimeError(f"layer {layer_idx}: bank part bytes do not match N={self.N}, K={self.K}")
        self._banks[layer_idx] = bank

    def bank(self, layer_idx: int) -> Bank:
        """The layer's bank: set_bank's, or built on first use from the reader (this rank's
        part of every expert, physical order under a placement map)."""
        b = self._banks.get(layer_idx)
        if b is None:
            if self.reader is None:
                raise RuntimeError(f"no bank for layer {layer_idx} (set_bank, or a reader)")
            t0 = time.time()
            types = tuple(self.reader.types(layer_idx))
            p2l = self._p2l.get(layer_idx) if isinstance(self._p2l, dict) else None
            gate, up, down = self.reader.banks(layer_idx, self.N, self.rank, p2l)
            b = Bank(gate, up, down, types)
            self.set_bank(layer_idx, b)
            if TIMING or len(self._banks) == 1:
                _log(f"rank {self.rank}: layer {layer_idx} bank {sum(t.numel() for t in (gate, up, down)) / 1e9:.2f} GB "
                     f"pinned in {time.time() - t0:.1f} s (types {types}{', placement map' if p2l is not None else ''})")
        return b

    def _bank(self, layer_idx: int):
        """[gate, up, down] of the layer's bank (the hot cache fills its slots from these)."""
        b = self.bank(layer_idx)
        return [b.gate, b.up, b.down]

    def build_all_banks(self, layers: Sequence[int]):
        for li in layers:
            self.bank(li)

    # -- staging and one group --------------------------------------------------

    def _stage(self, slot: int, layer_idx: int, base: int, n: int):
        cb = self.bank(layer_idx).c_struct()
        _lib.check(_lib.lib().ktmi_streamer_stage(self._h, slot, C.byref(cb), base, n), "streamer_stage")

    def _workspace(self, T: int, n: int) -> torch.Tensor:
        desc = self._desc(0, n)
        need = _lib.lib().ktmi_moe_layer_workspace(desc, T, self.top_k, _lib.MODE_AUTO)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty((max(need, 256),), dtype=torch.uint8, device=self.device)
        return self._ws

    def _desc(self, slot: int, n: int) -> _lib.ktmi_layer:
        w13, w2 = self.slots[slot]
        return _lib.ktmi_layer(self.K, self.N, n, self.types[0], self.types[2], w13, w2, 0, 0)

    def _group_body(self, slot: int, base: int, n: int, g: dict):
        L = _lib.lib()
        stream = _lib.stream_ptr(self.device)
        x, w, ids, acc, out, local = g["x"], g["w"], g["ids"], g["acc"], g["out"], g["local"]
        T = x.shape[0]
        _lib.check(L.ktmi_remap_ids(ids.data_ptr(), ids.numel(), base, n, local.data_ptr(), stream), "remap_ids")
        ws = self._workspace(T, n)
        desc = self._desc(slot, n)
        _lib.check(L.ktmi_moe_layer(desc, x.data_ptr(), w.data_ptr(), local.data_ptr(), T, self.top_k, out.data_ptr(),
                                    ws.data_ptr(), ws.numel(), _lib.MODE_AUTO, stream), "moe_layer")
        _lib.check(L.ktmi_add_bf16(acc.data_ptr(), out.data_ptr(), acc.numel(), stream), "add_bf16")

    def _inputs(self, x, topk_weights, physical_ids):
        if x.dtype != torch.bfloat16 or physical_ids.dtype != torch.int32:
            raise TypeError("x must be bf16 and the expert ids int32")
        T = x.shape[0]
        return {
            "x": x.contiguous(),
            "w": topk_weights.to(torch.float32).contiguous(),
            "ids": physical_ids.contiguous(),
            "acc": torch.zeros((T, self.K), dtype=torch.bfloat16, device=self.device),
            "out": torch.empty((T, self.K), dtype=torch.bfloat16, device=self.device),
            "local": torch.empty_like(physical_ids, memory_format=torch.contiguous_format),
        }

    # -- the pipeline -------------------------------------------------------------

    def _pipeline(self, units: Sequence[Tuple[int, int, int, dict]]):
        """units: (layer_idx, first expert, n, inputs). Group u+1 is staged while group u
        computes, slots used round robin."""
        L = _lib.lib()
        cur = _lib.stream_ptr(self.device)
        if not units:
            return
        self._stage(0, *units[0][:3])
        for ui, (layer_idx, base, n, g) in enumerate(units):
            slot = ui % self.n_slots
            _lib.check(L.ktmi_streamer_acquire(self._h, slot, cur), "streamer_acquire")
            self._group_body(slot, base, n, g)
            _lib.check(L.ktmi_streamer_release(self._h, slot, cur), "streamer_release")
            if ui + 1 < len(units):
                self._stage((ui + 1) % self.n_slots, *units[ui + 1][:3])

    def groups(self, layer_idx: int, first: int = 0) -> List[Tuple[int, int]]:
        E = self.bank(layer_idx).n_experts
        return [(b, min(self.G, E - b)) for b in range(first, E, self.G)]

    def run(self, layer_idx: int, x: torch.Tensor, topk_weights: torch.Tensor, physical_ids: torch.Tensor,
            first: int = 0) -> torch.Tensor:
        """Sum over the streamed experts [first, E) of their outputs for this layer,
        [tokens, hidden] bf16 (P:40928-40992). physical_ids are bank indices; other ids
        (CPU experts, -1) contribute nothing."""
        t0 = time.perf_counter()
        g = self._inputs(x, topk_weights, physical_ids)
        self._pipeline([(layer_idx, b, n, g) for b, n in self.groups(layer_idx, first)])
        self.calls += 1
        if TIMING:
            torch.cuda.current_stream(self.device).synchronize()
            _log(f"layer{layer_idx} tokens={x.shape[0]} groups={len(self.groups(layer_idx, first))} "
                 f"total={(time.perf_counter() - t0) * 1e3:.1f}ms")
        return g["acc"]

    def run_layers(self, items: Sequence[Tuple[int, torch.Tensor, torch.Tensor, torch.Tensor]],
                   first: int = 0) -> List[torch.Tensor]:
        """Several layers back to back, [(layer_idx, x, topk_weights, ids)], streamed as one
        pipeline: the next group (of this layer or the next) is copied while the current one
        computes. The layers' inputs are given up front (a benchmark or replay of recorded
        routing); returns each layer's output."""
        units, outs = [], []
        for layer_idx, x, w, ids in items:
            g = self._inputs(x, w, ids)
            outs.append(g["acc"])
            units += [(layer_idx, b, n, g) for b, n in self.groups(layer_idx, first)]
        self._pipeline(units)
        self.calls += len(items)
        return outs

    def copy_stream(self) -> int:
        """The copy stream's handle (hipStream_t as an int)."""
        return _lib.lib().ktmi_streamer_copy_stream(self._h) or 0

    def sync_copies(self):
        _lib.check(_lib.lib().ktmi_streamer_sync(self._h), "streamer_sync")


_instance: Optional[KTStreamPrefillGGUF] = None


def preallocate(N: int, K: int, top_k: int, types, device=None, reader=None, rank: int = 0) -> Optional[KTStreamPrefillGGUF]:
    """Create the process-wide streamer early (its slots count toward the memory budget
    before the KV pool is sized, P:40607-40636); a no-op when streaming is off."""
    global _instance
    if STREAM_THRESHOLD <= 0:
        return None
    if _instance is None:
        _instance = KTStreamPrefillGGUF(N, K, top_k, types, GROUP_SIZE, device, reader=reader, rank=rank)
    return _instance


def stream_prefill_for(N: int, K: int, top_k: int, types, num_tokens: int) -> Optional[KTStreamPrefillGGUF]:
    """The streamer for a chunk of num_tokens tokens, or None below KT_GPU_STREAM_PREFILL
    or under graph capture (P:41004-41024)."""
    if STREAM_THRESHOLD <= 0 or num_tokens < STREAM_THRESHOLD:
        return None
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        return None
    return preallocate(N, K, top_k, types)
