"""Hot-expert registry and dynamic cache (drop-in for hot/kt_hot_cache.py).

Per layer the GPU holds two int32 tables over the logical experts: log2slot (slot or -1)
and log2cpu (-1 for a resident expert, else the logical id), plus fp32 route counts.
`route(layer, ids)` is one native kernel for any number of routes (ktmi_hot_route): the
two lookups and the count update, graph-capturable (the reference's fused Triton kernel
covers <= 64 routes and falls back to torch gathers above, :62-75, :121-143).

Residency is carried by the ids alone: an expert is in log2slot xor in log2cpu
(`check_tables`, :293-316). Between steps `before_forward` runs the swap policy every
KT_HOT_INTERVAL decode steps (:376-432): counts read one round late through a pinned
buffer, decayed by KT_HOT_DECAY; per layer the coldest residents give way to the hottest
non-residents when candidate > KT_HOT_MARGIN * resident, at most KT_HOT_SWAPS per layer;
a swap copies the expert's bytes from the pinned bank into the slot (`fill`, :245-271).
"""
from __future__ import annotations

import json
import os
import time
from typing import Dict, List, Optional

import torch

from . import _lib

ENABLED = os.environ.get("KT_HOT_DYNAMIC") == "1"
INTERVAL = int(os.environ.get("KT_HOT_INTERVAL", "32"))
MAX_SWAPS = int(os.environ.get("KT_HOT_SWAPS", "8"))
DECAY = float(os.environ.get("KT_HOT_DECAY", "0.9"))
MARGIN = float(os.environ.get("KT_HOT_MARGIN", "1.5"))
SEED = os.environ.get("KT_HOT_SEED")
EMPTY, ABSENT = -1, -2


def _log(msg):
    print(f"[kt-hot {time.strftime('%H:%M:%S')}] {msg}", flush=True)


def route_native(ids: torch.Tensor, log2slot: torch.Tensor, log2cpu: torch.Tensor, counts: Optional[torch.Tensor]):
    """slot_ids = log2slot[ids], cpu_ids = log2cpu[ids], counts[ids] += 1 (one kernel)."""
    if ids.dtype != torch.int32:
        raise TypeError(f"route: ids must be int32, got {ids.dtype}")
    flat = ids.contiguous().view(-1)
    slot_ids = torch.empty_like(flat)
    cpu_ids = torch.empty_like(flat)
    rc = _lib.lib().ktmi_hot_route(flat.data_ptr(), flat.numel(), log2slot.data_ptr(), log2cpu.data_ptr(),
                                   counts.data_ptr() if counts is not None else 0, slot_ids.data_ptr(),
                                   cpu_ids.data_ptr(), _lib.stream_ptr(ids.device))
    _lib.check(rc, "hot_route")
    return slot_ids.view_as(ids), cpu_ids.view_as(ids)


class HotCache:
    def __init__(self, num_layers: int, num_experts: int, slots: int, device, rank: int = 0):
        self.L, self.E, self.N, self.device, self.rank = num_layers, num_experts, slots, torch.device(device), rank
        self.log2slot_cpu = torch.full((num_layers, num_experts), -1, dtype=torch.int32)
        self.log2cpu_cpu = torch.arange(num_experts, dtype=torch.int32).repeat(num_layers, 1)
        self.log2slot = self.log2slot_cpu.to(self.device)
        self.log2cpu = self.log2cpu_cpu.to(self.device)
        self.counts = torch.zeros((num_layers, num_experts), dtype=torch.float32, device=self.device)
        self.S = slots
        self.slot2log: List[List[int]] = [[EMPTY] * slots for _ in range(num_layers)]
        self.layers: Dict[int, tuple] = {}  # layer_idx -> (hot method, layer)
        self.banks: Dict[int, list] = {}    # layer_idx -> [gate, up, down] pinned uint8 [E, part_bytes]
        pin = self.device.type == "cuda"
        self._counts_host = torch.zeros((num_layers, num_experts), dtype=torch.float32, pin_memory=pin)
        self._counts_event = None
        self.ready = False
        self.step = self.rounds = self.swaps = 0
        self.bytes = 0
        self.swap_s = 0.0

    # -- graph side -----------------------------------------------------------------

    def route(self, layer_idx: int, ids: torch.Tensor):
        """ids: logical [T, k] int32 (>= 0). Returns (slot ids, -1 for CPU experts; logical
        ids, -1 for resident ones)."""
        return route_native(ids, self.log2slot[layer_idx], self.log2cpu[layer_idx], self.counts[layer_idx])

    def push_tables(self) -> None:
        self.log2slot.copy_(self.log2slot_cpu, non_blocking=True)
        self.log2cpu.copy_(self.log2cpu_cpu, non_blocking=True)

    # -- residency ------------------------------------------------------------------

    def _set(self, layer_idx: int, slot: int, logical: int) -> None:
        """Slot <- logical (>= 0) or EMPTY; host tables only."""
        old = self.slot2log[layer_idx][slot]
        if old >= 0:
            self.log2slot_cpu[layer_idx, old] = -1
            self.log2cpu_cpu[layer_idx, old] = old
        self.slot2log[layer_idx][slot] = logical
        if logical >= 0:
            self.log2slot_cpu[layer_idx, logical] = slot
            self.log2cpu_cpu[layer_idx, logical] = -1

    def fill(self, layer_idx: int, slot: int, logical: int) -> None:
        """Copy an expert's bytes from the layer's pinned bank into a slot (async H2D)."""
        method, layer = self.layers[layer_idx]
        gate, up, down = self.banks[layer_idx]
        N = method.N
        w13, w2 = layer.w13_qweight.data, layer.w2_qweight.data
        g = gate[logical].view(N, -1)
        u = up[logical].view(N, -1)
        d = down[logical].view(w2.shape[1], -1)
        w13[slot, :N].copy_(g, non_blocking=True)
        w13[slot, N:].copy_(u, non_blocking=True)
        w2[slot].copy_(d, non_blocking=True)
        self.bytes += g.numel() + u.numel() + d.numel()

    def check_tables(self) -> str:
        """'' when every expert of every layer is on exactly one side (a slot that holds it,
        or the CPU) and the device tables equal the host's; else the first violation."""
        s_cpu, c_cpu = self.log2slot_cpu, self.log2cpu_cpu
        if not torch.equal(self.log2slot.cpu(), s_cpu) or not torch.equal(self.log2cpu.cpu(), c_cpu):
            return "device tables differ from the host's"
        if not bool(((s_cpu >= 0) ^ (c_cpu >= 0)).all()):
            return "an expert both or neither on a slot and on the CPU"
        if not bool(((c_cpu < 0) | (c_cpu == torch.arange(self.E, dtype=torch.int32))).all()):
            return "CPU id is not the logical id"
        for li in range(self.L):
            for e in (s_cpu[li] >= 0).nonzero().flatten().tolist():
                sl = int(s_cpu[li, e])
                if self.slot2log[li][sl] != e:
                    return f"layer {li} expert {e} -> slot {sl} holding {self.slot2log[li][sl]}"
            for sl, e in enumerate(self.slot2log[li]):
                if e >= 0 and int(s_cpu[li, e]) != sl:
                    return f"layer {li} slot {sl} holds {e} but the table says {int(s_cpu[li, e])}"
        return ""

    def seed(self, placement: Optional[str] = None, p2l=None) -> None:
        """Initial residents: the placement map's first N per layer (filled from the banks)
        or logical 0..N-1 (what the loader put in the slots)."""
        if placement:
            p2l = json.load(open(placement))["physical_to_logical_map"]
        for li in sorted(self.layers) if self.layers else range(self.L):
            for s in range(self.N):
                e = int(p2l[li][s]) if p2l is not None else s
                self._set(li, s, e)
                if p2l is not None and e != s and li in self.banks:
                    self.fill(li, s, e)
        self.push_tables()
        self.ready = True

    # -- policy, between steps --------------------------------------------------------

    def plan_swaps(self, counts: torch.Tensor):
        """[(layer, slot, candidate)] for host counts [L, E]: per layer the coldest residents
        against the hottest non-residents, margin test, at most MAX_SWAPS, in order."""
        res = torch.tensor(self.slot2log)  # [L, S]
        score_res = counts.gather(1, res.clamp(min=0))
        score_res = torch.where(res == EMPTY, torch.full_like(score_res, -1.0), score_res)
        # resident mask: empty slots scatter into a dummy column E that is dropped
        resident = torch.zeros((counts.shape[0], counts.shape[1] + 1), dtype=torch.bool)
        resident.scatter_(1, torch.where(res >= 0, res, torch.full_like(res, counts.shape[1])), True)
        resident = resident[:, :-1]
        k = min(MAX_SWAPS, self.S, self.E)
        cand_score, cand_idx = torch.topk(torch.where(resident, torch.full_like(counts, -1.0), counts), k, dim=1)
        order = torch.argsort(score_res, dim=1, stable=True)[:, :k]
        rs = score_res.gather(1, order)
        do = ((cand_score > 0) & (cand_score > MARGIN * rs)).to(torch.int64).cumprod(1).bool()
        return [(li, int(order[li, j]), int(cand_idx[li, j])) for li, j in do.nonzero().tolist()]

    def before_forward(self, is_decode: bool = True) -> None:
        if not self.ready or not is_decode:
            return
        self.step += 1
        if self.step % INTERVAL:
            return
        t0 = time.time()
        if self._counts_event is not None and not self._counts_event.query():
            return
        counts = self._counts_host.clone() if self._counts_event is not None else None
        self._counts_host.copy_(self.counts, non_blocking=True)
        self.counts.mul_(DECAY)
        if self._counts_event is None:
            self._counts_event = torch.cuda.Event()
        self._counts_event.record(torch.cuda.current_stream(self.device))
        if counts is None:
            return
        swaps = 0
        for li, s_, c in self.plan_swaps(counts):
            if li not in self.layers:
                continue
            self._set(li, s_, c)
            if li in self.banks:
                self.fill(li, s_, c)
            swaps += 1
        if swaps:
            self.push_tables()
        self.rounds += 1
        self.swaps += swaps
        self.swap_s += time.time() - t0


_cache: Optional[HotCache] = None


def register(method, layer, num_layers: int, num_experts: int) -> Optional[HotCache]:
    """Called per layer; the cache is built on the first call and seeded once every layer
    is known (hot/kt_hot_cache.py:438-455)."""
    global _cache
    if not ENABLED:
        return None
    kt = method.kt_config
    if _cache is None:
        if kt.num_gpu_experts <= 0:
            raise RuntimeError("KT_HOT_DYNAMIC=1 needs num_gpu_experts > 0")
        _cache = HotCache(num_layers, num_experts, kt.num_gpu_experts, layer.w13_qweight.device)
    c = _cache
    if kt.layer_idx not in c.layers:
        c.layers[kt.layer_idx] = (method, layer)
        if len(c.layers) == num_layers:
            c.seed(SEED)
    return c if c.ready else None


def before_forward(is_decode: bool = True) -> None:
    if _cache is not None:
        _cache.before_forward(is_decode)
