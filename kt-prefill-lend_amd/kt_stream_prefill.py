"""Streamed GGUF prefill: the layer-weight streamer (drop-in for the reference's
kt_stream_prefill module, P:40470-41050).

The reference's KT wrapper calls four entry points, with these signatures here too:
  * `stream_prefill_init_early(method, layer)` once the last layer has loaded (P:10515):
    builds the streamer and every layer's bank at load time when KT_GPU_STREAM_EARLY_INIT=1
    (P:40995-41002);
  * `stream_prefill_for(method, layer, num_tokens)` per MoE forward (P:10581): the
    process-wide streamer for a chunk of at least KT_GPU_STREAM_PREFILL tokens, else None
    (also under graph capture), created on the first qualifying call (P:41004-41024);
  * `KTStreamPrefillGGUF.run(method, layer, dispatch_output, physical_ids)` (P:10629): the
    sum over the streamed experts of their outputs for this layer, [tokens, hidden] bf16
    (P:40928-40992). Experts [first, E) are streamed, first = 0 when the GPU method
    streams its hot experts too (streams_hot_experts), else num_gpu_experts;
  * `preallocate(layer)` (P:40607-40636): the device slots and, for the server's chunk
    size, the layer workspace, made before SGLang sizes its KV pool.

Experts' raw GGUF bytes live in pinned host banks, one per layer (`Bank`: gate, up and down
parts, [E, part bytes] each, physical order under a placement map; the reference's _bank,
P:40712-40752). A chunk runs a layer's experts in groups of GROUP_SIZE: while the grouped
layer kernels work on group g in one device slot, group g+1 is copied into the other slot
on a copy stream of its own (`ktmi_streamer_*`: the reference's _Slot / _stage / run,
P:40543-40550, 40773-40787). Each group's partial output is added to the layer's bf16
accumulator (acc.add_(out), P:40819).

Differences from the reference, on purpose:
  * the slots hold raw blocks in the layout the grouped kernels read: no bf16 copy of each
    group's weights (the reference dequantises into w13_bf16 / w2_bf16, P:40789-40798), no
    CUTLASS workspace and no graph per group (a group is four native launches);
  * banks can also be handed in as pinned tensors (`set_bank`), and `run_tensors` /
    `run_layers` take plain tensors; `run_layers` streams several layers as one pipeline,
    so layer l+1's weights arrive while layer l computes.

Environment (the reference's names): KT_GPU_STREAM_PREFILL (token threshold, 0 = off),
KT_GPU_STREAM_GROUP (experts per group, 8), KT_GPU_STREAM_TIMING=1 (log per layer),
KT_GPU_STREAM_EARLY_INIT=1, KT_GPU_STREAM_SELFTEST=2 (checks the first streamed layer
against an fp32 torch FFN of the bank's dequantised experts and logs the agreement).
"""
from __future__ import annotations

import ctypes as C
import os
import time
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import _lib, sglang_env
from .gguf import row_bytes

STREAM_THRESHOLD = int(os.environ.get("KT_GPU_STREAM_PREFILL", "0") or 0)
GROUP_SIZE = int(os.environ.get("KT_GPU_STREAM_GROUP", "8") or 8)
TIMING = os.environ.get("KT_GPU_STREAM_TIMING") == "1"
EARLY_INIT = os.environ.get("KT_GPU_STREAM_EARLY_INIT", "0") == "1"
SELFTEST = os.environ.get("KT_GPU_STREAM_SELFTEST", "0")


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


class _Geometry:
    """Per layer the (gate, up, down) ggml types and this rank's part bytes of one expert,
    and the slot capacity every layer fits in (the reference's _Geometry, P:40547-40590)."""

    def __init__(self, N: int, K: int, types_by_layer: Dict[int, Tuple[int, int, int]]):
        if not types_by_layer:
            raise RuntimeError("the streamer needs at least one expert layer")
        self.N, self.K = N, K
        self.types = dict(types_by_layer)
        self.parts = {li: part_bytes(t, N, K) for li, t in self.types.items()}
        self.cap13 = max(p[0] + p[1] for p in self.parts.values())
        self.cap2 = max(p[2] for p in self.parts.values())

    @classmethod
    def of_reader(cls, reader, N: int, K: int, world: int) -> "_Geometry":
        from .gguf import BLOCK_INFO, KERNEL_TYPES

        if N * world != reader.inter or K != reader.K:
            raise RuntimeError(f"streamed experts {reader.inter} x {reader.K} vs layer {N} per rank x {world} / {K}")
        layers = reader.layers() if hasattr(reader, "layers") else list(range(reader.num_layers))
        types = {}
        for li in layers:
            t = tuple(int(v) for v in reader.types(li))
            bad = [v for v in t if v not in KERNEL_TYPES]
            if bad or t[0] != t[1]:
                raise RuntimeError(f"layer {li}: expert types {t} cannot be streamed (gate and up must agree and "
                                   f"have kernels: {sorted(KERNEL_TYPES)})")
            if K % BLOCK_INFO[t[0]][0] or N % BLOCK_INFO[t[2]][0]:
                raise RuntimeError(f"layer {li}: K={K} / N={N} are not whole blocks of types {t}")
            types[li] = t
        return cls(N, K, types)


class _DeviceSlots:
    """The device half of the streamer on one GPU: the native double-buffered slots
    (ktmi_streamer_create: raw gate/up and down bytes of up to G experts each, a copy
    stream, loaded / released events) and the layer workspace."""

    def __init__(self, device: torch.device, G: int, cap13: int, cap2: int, n_slots: int = 2):
        L = _lib.lib()
        self.device, self.G, self.n_slots = device, G, n_slots
        with torch.cuda.device(device):
            h = L.ktmi_streamer_create(G, cap13, cap2, n_slots)
        if not h:
            raise RuntimeError(f"streamer_create failed: {L.ktmi_last_error().decode()}")
        self.handle = C.c_void_p(h)
        self.slots = []
        for i in range(n_slots):
            a, b = C.c_void_p(), C.c_void_p()
            _lib.check(L.ktmi_streamer_slot(self.handle, i, C.byref(a), C.byref(b)), "streamer_slot")
            self.slots.append((a.value, b.value))
        self.cap13, self.cap2 = cap13, cap2
        self.ws: Optional[torch.Tensor] = None

    def workspace(self, need: int) -> torch.Tensor:
        if self.ws is None or self.ws.numel() < need:
            self.ws = torch.empty((max(need, 256),), dtype=torch.uint8, device=self.device)
        return self.ws

    def close(self):
        if getattr(self, "handle", None):
            _lib.lib().ktmi_streamer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass


# device index -> _DeviceSlots made by preallocate() before the KV pool is sized
_prealloc: Dict[int, _DeviceSlots] = {}


def _current_device() -> torch.device:
    return torch.device("cuda", torch.cuda.current_device())


class KTStreamPrefillGGUF:
    """Process-wide (per device) streaming state shared by every MoE layer (P:40641-40700)."""

    def __init__(self, method, layer):
        rank, world = sglang_env.tp_rank_world()
        from . import kt_gguf_hot

        reader = kt_gguf_hot._reader(method.kt_config.weight_path)  # one reader per path
        N, K = layer.intermediate_size_per_partition, layer.hidden_size
        self._setup(N, K, layer.top_k, _Geometry.of_reader(reader, N, K, world), GROUP_SIZE, None, reader, rank, 2)
        _log(f"rank {rank}: streamed GGUF prefill above {STREAM_THRESHOLD} tokens, G={self.G}, N={N} K={K}, "
             f"{len(self.geometry.types)} layers, slots {2 * self.G * (self.dev.cap13 + self.dev.cap2) / 1e6:.0f} MB")

    @classmethod
    def standalone(cls, N: int, K: int, top_k: int, types: Tuple[int, int, int], group_size: int = GROUP_SIZE,
                   device=None, reader=None, rank: int = 0, world: int = 1, n_slots: int = 2,
                   layers: Optional[Sequence[int]] = None) -> "KTStreamPrefillGGUF":
        """A streamer without a method/layer pair (benchmarks, tests): one set of expert types
        for every layer (banks from set_bank, or from `reader` when given)."""
        obj = cls.__new__(cls)
        if reader is not None and layers is None:
            geo = _Geometry.of_reader(reader, N, K, world)
        else:
            geo = _Geometry(N, K, {li: tuple(types) for li in (layers if layers is not None else [0])})
        geo.default = tuple(types)
        obj._setup(N, K, top_k, geo, group_size, device, reader, rank, n_slots)
        return obj

    def _setup(self, N, K, top_k, geometry, G, device, reader, rank, n_slots):
        self.N, self.K, self.top_k, self.G = N, K, top_k, G
        self.geometry, self.reader, self.rank = geometry, reader, rank
        self.device = torch.device(device) if device is not None else _current_device()
        pre = _prealloc.get(self.device.index)
        if (pre is not None and pre.G >= G and pre.cap13 >= geometry.cap13 and pre.cap2 >= geometry.cap2
                and pre.n_slots == n_slots):
            self.dev = pre
        else:
            self.dev = _DeviceSlots(self.device, G, geometry.cap13, geometry.cap2, n_slots)
        self.n_slots = n_slots
        self._banks: Dict[int, Bank] = {}
        self.calls = 0
        self._checked = False

    # -- geometry and banks ------------------------------------------------------

    def types(self, layer_idx: int) -> Tuple[int, int, int]:
        t = self.geometry.types.get(layer_idx)
        if t is None:
            t = getattr(self.geometry, "default", None)
            if t is None:
                raise RuntimeError(f"layer {layer_idx} has no routed experts in the streamed GGUF")
        return t

    def set_bank(self, layer_idx: int, bank: Bank):
        types = self.types(layer_idx)
        if bank.types != types:
            raise RuntimeError(f"layer {layer_idx}: bank types {bank.types} != the layer's {types}")
        want = part_bytes(types, self.N, self.K)
        if (bank.gate.shape[1], bank.up.shape[1], bank.down.shape[1]) != want:
            raise RuntimeError(f"layer {layer_idx}: bank part bytes do not match N={self.N}, K={self.K}")
        self._banks[layer_idx] = bank

    def bank(self, layer_idx: int) -> Bank:
        """The layer's bank: set_bank's, or built on first use from the reader (this rank's
        part of every expert, physical order under SGLang's placement map)."""
        b = self._banks.get(layer_idx)
        if b is None:
            if self.reader is None:
                raise RuntimeError(f"no bank for layer {layer_idx} (set_bank, or a reader)")
            t0 = time.time()
            p2l = sglang_env.physical_to_logical(layer_idx)
            p2l = None if sglang_env.is_identity(p2l) else p2l
            gate, up, down = self.reader.banks(layer_idx, self.N, self.rank, p2l)
            b = Bank(gate, up, down, self.types(layer_idx))
            self.set_bank(layer_idx, b)
            if TIMING or len(self._banks) == 1:
                _log(f"rank {self.rank}: layer {layer_idx} bank {sum(t.numel() for t in (gate, up, down)) / 1e9:.2f} GB "
                     f"pinned in {time.time() - t0:.1f} s (types {b.types}{', placement map' if p2l is not None else ''})")
        return b

    def _bank(self, layer_idx: int):
        """[gate, up, down] of the layer's bank (the hot cache fills its slots from these)."""
        b = self.bank(layer_idx)
        return [b.gate, b.up, b.down]

    def build_all_banks(self, layers: Optional[Sequence[int]] = None):
        t0 = time.time()
        for li in (layers if layers is not None else sorted(self.geometry.types)):
            self.bank(li)
        gb = sum(sum(t.numel() for t in (b.gate, b.up, b.down)) for b in self._banks.values()) / 1e9
        _log(f"rank {self.rank}: {len(self._banks)} layer banks, {gb:.1f} GB pinned, in {time.time() - t0:.0f} s")

    # -- staging and one group --------------------------------------------------

    def _stage(self, slot: int, layer_idx: int, base: int, n: int):
        cb = self.bank(layer_idx).c_struct()
        _lib.check(_lib.lib().ktmi_streamer_stage(self.dev.handle, slot, C.byref(cb), base, n), "streamer_stage")

    def _desc(self, slot: int, n: int, layer_idx: int) -> _lib.ktmi_layer:
        w13, w2 = self.dev.slots[slot]
        t = self.types(layer_idx)
        return _lib.ktmi_layer(self.K, self.N, n, t[0], t[2], w13, w2, 0, 0)

    def _group_body(self, slot: int, layer_idx: int, base: int, n: int, g: dict):
        L = _lib.lib()
        stream = _lib.stream_ptr(self.device)
        x, w, ids, acc, out, local = g["x"], g["w"], g["ids"], g["acc"], g["out"], g["local"]
        T = x.shape[0]
        _lib.check(L.ktmi_remap_ids(ids.data_ptr(), ids.numel(), base, n, local.data_ptr(), stream), "remap_ids")
        desc = self._desc(slot, n, layer_idx)
        ws = self.dev.workspace(L.ktmi_moe_layer_workspace(desc, T, self.top_k, _lib.MODE_AUTO))
        _lib.check(L.ktmi_moe_layer(desc, x.data_ptr(), w.data_ptr(), local.data_ptr(), T, self.top_k, out.data_ptr(),
                                    ws.data_ptr(), ws.numel(), _lib.MODE_AUTO, stream), "moe_layer")
        _lib.check(L.ktmi_add_bf16(acc.data_ptr(), out.data_ptr(), acc.numel(), stream), "add_bf16")

    def _inputs(self, x, topk_weights, physical_ids):
        if x.dtype != torch.bfloat16:
            raise TypeError(f"x must be bf16, got {x.dtype}")
        if physical_ids.shape != topk_weights.shape or physical_ids.shape[0] != x.shape[0]:
            raise ValueError(f"ids {tuple(physical_ids.shape)} / weights {tuple(topk_weights.shape)} vs x "
                             f"{tuple(x.shape)}")
        if physical_ids.shape[1] != self.top_k:
            raise ValueError(f"top_k {physical_ids.shape[1]} != the streamer's {self.top_k}")
        T = x.shape[0]
        return {
            "x": x.contiguous(),
            "w": topk_weights.to(torch.float32).contiguous(),
            "ids": physical_ids.to(torch.int32).contiguous(),
            "acc": torch.zeros((T, self.K), dtype=torch.bfloat16, device=self.device),
            "out": torch.empty((T, self.K), dtype=torch.bfloat16, device=self.device),
            "local": torch.empty(physical_ids.shape, dtype=torch.int32, device=self.device),
        }

    # -- the pipeline -------------------------------------------------------------

    def _pipeline(self, units: Sequence[Tuple[int, int, int, dict]]):
        """units: (layer_idx, first expert, n, inputs). Group u+1 is staged while group u
        computes, slots used round robin."""
        L = _lib.lib()
        cur = _lib.stream_ptr(self.device)
        if not units:
            return
        h = self.dev.handle
        self._stage(0, *units[0][:3])
        for ui, (layer_idx, base, n, g) in enumerate(units):
            slot = ui % self.n_slots
            _lib.check(L.ktmi_streamer_acquire(h, slot, cur), "streamer_acquire")
            self._group_body(slot, layer_idx, base, n, g)
            _lib.check(L.ktmi_streamer_release(h, slot, cur), "streamer_release")
            if ui + 1 < len(units):
                self._stage((ui + 1) % self.n_slots, *units[ui + 1][:3])

    def groups(self, layer_idx: int, first: int = 0) -> List[Tuple[int, int]]:
        E = self.bank(layer_idx).n_experts
        return [(b, min(self.G, E - b)) for b in range(first, E, self.G)]

    def run(self, method, layer, dispatch_output, physical_ids: torch.Tensor) -> torch.Tensor:
        """Sum of the streamed experts' outputs for this layer, [tokens, hidden] bf16
        (P:40928-40992): layer method.kt_config.layer_idx, x = dispatch_output.hidden_states,
        route weights from its topk_output, physical_ids the routed experts' bank rows (other
        ids, -1 included, contribute nothing)."""
        layer_idx = method.kt_config.layer_idx
        gpu_method = getattr(method, "gpu_method", None)
        first = 0 if getattr(gpu_method, "streams_hot_experts", False) else int(getattr(method, "num_gpu_experts", 0))
        x = dispatch_output.hidden_states
        acc = self.run_tensors(layer_idx, x, dispatch_output.topk_output.topk_weights, physical_ids, first)
        if SELFTEST == "2" and not self._checked and layer_idx == min(self.geometry.types, default=layer_idx):
            self._checked = True
            self._reference_check(layer_idx, x, physical_ids, dispatch_output.topk_output.topk_weights, acc, first)
        return acc

    def run_tensors(self, layer_idx: int, x: torch.Tensor, topk_weights: torch.Tensor, physical_ids: torch.Tensor,
                    first: int = 0) -> torch.Tensor:
        """`run` on plain tensors: the sum over the streamed experts [first, E)."""
        t0 = time.perf_counter()
        g = self._inputs(x, topk_weights, physical_ids)
        groups = self.groups(layer_idx, first)
        self._pipeline([(layer_idx, b, n, g) for b, n in groups])
        self.calls += 1
        if TIMING:
            torch.cuda.current_stream(self.device).synchronize()
            _log(f"layer{layer_idx} tokens={x.shape[0]} groups={len(groups)} "
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

    def _reference_check(self, layer_idx, x, ids, w, acc, first):
        """KT_GPU_STREAM_SELFTEST=2 (the reference's self-check, P:40821-40853): recomputes the
        streamed experts' share of this layer in fp32 from their bf16-dequantised bank bytes,
        one routed expert at a time, and logs how far `acc` is from it (relative L2, cosine,
        largest difference). A diagnostic: `acc` is returned unchanged either way."""
        from . import kt_gguf_dequant as DQ

        torch.cuda.current_stream(self.device).synchronize()
        bank, types = self.bank(layer_idx), self.types(layer_idx)
        N, K = self.N, self.K
        routed = ids.to(device=self.device, dtype=torch.int64)
        coef_all = w.to(device=self.device, dtype=torch.float32)
        experts = [e for e in torch.unique(routed).tolist() if first <= e < bank.n_experts]
        proj = (("gate", bank.gate, types[0], (N, K)), ("up", bank.up, types[1], (N, K)),
                ("down", bank.down, types[2], (K, N)))
        expected = torch.zeros(acc.shape, dtype=torch.float32, device=self.device)
        xf = x.to(torch.float32)
        for e in experts:
            wt = {}
            for name, part, t, (rows, cols) in proj:
                dq = torch.empty((1, rows, cols), dtype=torch.bfloat16, device=self.device)
                src = part[e].view(1, -1).to(self.device)
                DQ.dequant_experts(src, src.shape[1], t, 1, rows, cols, dq)
                wt[name] = dq[0].to(torch.float32)
            hit = routed == e  # a token routes to an expert at most once
            rows_e = hit.any(dim=1).nonzero().squeeze(1)
            scale = (coef_all * hit).sum(dim=1)[rows_e]
            xe = xf[rows_e]
            g = torch.matmul(xe, wt["gate"].t())
            act = g * torch.sigmoid(g) * torch.matmul(xe, wt["up"].t())
            expected[rows_e] += torch.matmul(act, wt["down"].t()) * scale[:, None]
        got = acc.to(torch.float32)
        rel = ((got - expected).norm() / expected.norm().clamp_min(1e-30)).item()
        cos = (torch.dot(got.flatten(), expected.flatten())
               / (got.norm() * expected.norm()).clamp_min(1e-30)).item()
        worst = (got - expected).abs().max().item() if got.numel() else 0.0
        _log(f"rank {self.rank}: self-check of layer {layer_idx} over {x.shape[0]} tokens and {len(experts)} "
             f"streamed experts: rel L2 {rel:.2e}, cos {cos:.6f}, max |diff| {worst:.4g}")
        return rel, cos

    def copy_stream(self) -> int:
        """The copy stream's handle (hipStream_t as an int)."""
        return _lib.lib().ktmi_streamer_copy_stream(self.dev.handle) or 0

    def sync_copies(self):
        _lib.check(_lib.lib().ktmi_streamer_sync(self.dev.handle), "streamer_sync")

    def close(self):
        if self.dev is not _prealloc.get(self.device.index):
            self.dev.close()


_instance: Optional[KTStreamPrefillGGUF] = None
_failed = False


def preallocate(layer) -> None:
    """The device slots (and, given the server's chunk size, the layer workspace) for the
    current device, made early so they count before the KV pool is sized (P:40607-40636).
    A no-op when streaming is off or already done for this device."""
    if STREAM_THRESHOLD <= 0:
        return
    device = _current_device()
    if device.index in _prealloc:
        return
    from . import kt_gguf_hot

    path = sglang_env.server_weight_path()
    if not path:
        raise RuntimeError("streamer preallocate: no GGUF path (server kt_weight_path or KT_WEIGHT_PATH)")
    _, world = sglang_env.tp_rank_world()
    N, K = layer.intermediate_size_per_partition, layer.hidden_size
    geo = _Geometry.of_reader(kt_gguf_hot._reader(path), N, K, world)
    dev = _prealloc[device.index] = _DeviceSlots(device, GROUP_SIZE, geo.cap13, geo.cap2)
    T = sglang_env.chunk_rows()
    if T > 0:
        t = next(iter(geo.types.values()))
        desc = _lib.ktmi_layer(K, N, GROUP_SIZE, t[0], t[2], dev.slots[0][0], dev.slots[0][1], 0, 0)
        dev.workspace(_lib.lib().ktmi_moe_layer_workspace(desc, T, layer.top_k, _lib.MODE_AUTO))
    mb = (2 * GROUP_SIZE * (geo.cap13 + geo.cap2) + (dev.ws.numel() if dev.ws is not None else 0)) / 1e6
    _log(f"preallocated 2 slots of {GROUP_SIZE} experts and the workspace for {T} rows ({mb:.0f} MB) on {device}")


def _streaming_enabled() -> bool:
    """Streaming is on (KT_GPU_STREAM_PREFILL > 0) and no attempt to build the streamer has
    failed in this process."""
    return STREAM_THRESHOLD > 0 and not _failed


def _build_streamer(method, layer, occasion: str) -> KTStreamPrefillGGUF:
    """Makes the process's streamer. Fail-closed: if building it raises, streaming stays off
    for the rest of the process (the entry points return None from then on) and the error
    propagates to the caller."""
    global _instance, _failed
    try:
        _instance = KTStreamPrefillGGUF(method, layer)
    except Exception as exc:
        _failed = True
        _log(f"streaming disabled for this process: building the streamer {occasion} raised "
             f"{type(exc).__name__}: {exc}")
        raise
    return _instance


def stream_prefill_init_early(method, layer) -> None:
    """With KT_GPU_STREAM_EARLY_INIT=1, builds the streamer and the pinned bank of every
    streamed layer while the model loads (the reference's entry point, P:10515), instead of
    at the first long chunk. Idempotent; a failure disables streaming and propagates."""
    global _failed
    if not EARLY_INIT or not _streaming_enabled() or _instance is not None:
        return
    started = time.time()
    st = _build_streamer(method, layer, "at load time")
    try:
        st.build_all_banks()
    except Exception as exc:
        _failed = True
        _log(f"streaming disabled for this process: the load-time banks raised {type(exc).__name__}: {exc}")
        raise
    _log(f"rank {st.rank}: streamer and banks ready at load time ({time.time() - started:.0f} s)")


def stream_prefill_for(method, layer, num_tokens: int) -> Optional[KTStreamPrefillGGUF]:
    """The streamer that runs a chunk of `num_tokens` tokens (the reference's per-forward
    entry point, P:10581), or None: streaming off or disabled, a chunk below
    KT_GPU_STREAM_PREFILL, or a stream under graph capture. The first qualifying chunk
    builds the streamer."""
    if not _streaming_enabled() or num_tokens < STREAM_THRESHOLD:
        return None
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        return None
    if _instance is not None:
        return _instance
    _log(f"building the streamer for a {num_tokens}-token chunk of layer {method.kt_config.layer_idx}")
    return _build_streamer(method, layer, f"for a {num_tokens}-token chunk")
