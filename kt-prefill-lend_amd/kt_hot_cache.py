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
The banks are the streamer's when one is loaded (one pinned copy serves both), else the
cache's own, built from the hot method's expert reader (`_bank`, :157-214;
KT_HOT_BANKS=own forces these).

Out of scope here: the KV-lending slots (lend_slot / take_back_slot, the base tables) and
the Q2_0 -> Q8_0 down repack.
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
OWN_BANKS = os.environ.get("KT_HOT_BANKS", "")
LOG_EVERY = int(os.environ.get("KT_HOT_LOG_EVERY", "0") or 0)
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
        self.banks: Dict[int, list] = {}    # own banks: layer_idx -> [gate, up, down] pinned uint8 [E, part]
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

    def _bank(self, layer_idx: int):
        """[gate, up, down] uint8 [E, part bytes] in pinned host memory, physical order:
        the streamer's bank when it is loaded, else the cache's own from the hot method's
        reader (hot/kt_hot_cache.py:157-214)."""
        b = self.banks.get(layer_idx)
        if b is not None:
            return b
        if OWN_BANKS != "own":
            from . import kt_stream_prefill as SP

            inst = SP._instance
            if inst is not None and (inst.reader is not None or layer_idx in inst._banks):
                return inst._bank(layer_idx)
        t0 = time.time()
        method, _layer = self.layers[layer_idx]
        b = method.reader.banks(layer_idx, method.N, getattr(method, "rank", 0), None)
        self.banks[layer_idx] = b
        if layer_idx == min(self.layers):
            _log(f"rank {self.rank}: layer {layer_idx} own bank {sum(t.numel() for t in b) / 1e9:.2f} GB pinned in "
                 f"{time.time() - t0:.1f} s (no streamer)")
        return b

    def fill(self, layer_idx: int, slot: int, logical: int) -> None:
        """Copy an expert's bytes from the layer's pinned bank into a slot (async H2D)."""
        method, layer = self.layers[layer_idx]
        gate, up, down = self._bank(layer_idx)
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

    def fill_empty(self, counts: torch.Tensor, seed_rank: Optional[torch.Tensor] = None) -> int:
        """Fill every EMPTY slot with the hottest non-residents of its layer (counts [L, E]
        on the host; ties broken by the seed map's order, seed_rank[l, e] = rank of e).
        Host tables only; the caller pushes them (hot/kt_hot_cache.py:334-353)."""
        n = 0
        for li in sorted(self.layers) if self.layers else range(self.L):
            empty = [s_ for s_, e in enumerate(self.slot2log[li]) if e == EMPTY]
            if not empty:
                continue
            score = counts[li].double().clone()
            if seed_rank is not None:
                score = score + (self.E - seed_rank[li].double()) / (self.E + 1) * 1e-3
            res = [e for e in self.slot2log[li] if e >= 0]
            if res:
                score[torch.tensor(res)] = float("-inf")
            for s_, c in zip(empty, torch.topk(score, len(empty)).indices.tolist()):
                self._set(li, s_, c)
                if li in self.layers:
                    self.fill(li, s_, c)
                n += 1
        return n

    def seed(self, placement: Optional[str] = None, p2l=None) -> None:
        """Initial residents: the placement map's first N per layer (filled from the banks)
        or logical 0..N-1 (what the loader put in the slots)."""
        t0 = time.time()
        if placement:
            p2l = json.load(open(placement))["physical_to_logical_map"]
        for li in sorted(self.layers) if self.layers else range(self.L):
            for s in range(self.N):
                e = int(p2l[li][s]) if p2l is not None else s
                self._set(li, s, e)
                if p2l is not None and e != s and li in self.layers:
                    self.fill(li, s, e)
        self.push_tables()
        self.ready = True
        if self.layers:
            _log(f"rank {self.rank}: {len(self.layers)} layers x {self.N} slots seeded from "
                 f"{placement or ('a placement map' if p2l is not None else 'logical order')} in {time.time() - t0:.1f} s "
                 f"({self.bytes / 1e9:.2f} GB copied); interval {INTERVAL}, max {MAX_SWAPS} swaps/layer, "
                 f"decay {DECAY}, margin {MARGIN}")
        self.bytes = 0

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

    def before_forward(self, forward_batch=True) -> None:
        """Between steps: the swap policy every INTERVAL decode steps (and, under MTP, the
        target's verify steps). forward_batch: SGLang's ForwardBatch (its forward_mode), or a
        bool meaning "this is a decode step"."""
        mode = getattr(forward_batch, "forward_mode", None)
        if mode is not None:
            is_decode = mode.is_decode() or (hasattr(mode, "is_target_verify") and mode.is_target_verify())
        else:
            is_decode = bool(forward_batch)
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
            self.fill(li, s_, c)
            swaps += 1
        if swaps:
            self.push_tables()
        self.rounds += 1
        self.swaps += swaps
        self.swap_s += time.time() - t0
        if self.rounds == 1 or (LOG_EVERY and self.rounds % LOG_EVERY == 0) or self.rounds % 64 == 0:
            _log(f"rank {self.rank}: round {self.rounds} (step {self.step}): {swaps} swaps this round, "
                 f"{self.swaps} total, {self.bytes / 1e9:.2f} GB, {self.swap_s * 1e3 / self.rounds:.1f} ms/round; "
                 f"GPU share of recent routes {self.gpu_share(counts):.3f}")

    def gpu_share(self, counts: torch.Tensor) -> float:
        """Fraction of the counted routes whose expert is resident now (host counts [L, E])."""
        res = torch.tensor(self.slot2log)
        hit = counts.gather(1, res.clamp(min=0)) * (res >= 0)
        return float(hit.sum()) / max(float(counts.sum()), 1.0)


_cache: Optional[HotCache] = None


def register(method, layer, num_layers: Optional[int] = None, num_experts: Optional[int] = None) -> Optional[HotCache]:
    """Called by the KT wrapper on its first decode apply of each layer; the cache is built
    on the first call and seeded once every layer is known (hot/kt_hot_cache.py:438-455).
    method: the KT wrapper method (kt_config, global_num_experts, tp_rank, gpu_method) or
    the hot GPU method itself with num_layers / num_experts given."""
    global _cache
    if not ENABLED:
        return None
    kt = method.kt_config
    gpu = getattr(method, "gpu_method", method)
    L = getattr(kt, "num_layers", None) or num_layers
    E = getattr(method, "global_num_experts", None) or num_experts
    if L is None or E is None:
        raise RuntimeError("hot cache register: the number of layers and experts is unknown")
    if _cache is None:
        if kt.num_gpu_experts <= 0:
            raise RuntimeError("KT_HOT_DYNAMIC=1 needs num_gpu_experts > 0")
        _cache = HotCache(L, E, kt.num_gpu_experts, layer.w13_qweight.device, getattr(method, "tp_rank", 0))
    c = _cache
    if kt.layer_idx not in c.layers:
        c.layers[kt.layer_idx] = (gpu, layer)
        if len(c.layers) == L:
            c.seed(SEED)
    return c if c.ready else None


def before_forward(forward_batch=True) -> None:
    if _cache is not None:
        _cache.before_forward(forward_batch)
