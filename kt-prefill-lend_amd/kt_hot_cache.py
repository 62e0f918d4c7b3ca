"""Decode-adaptive hot experts: which experts of each layer sit in the GPU slots
(drop-in for hot/kt_hot_cache.py: `register`, `HotCache.route / push_tables /
check_tables / before_forward`, `_cache`, `ENABLED`, the KT_HOT_* knobs).

State. Per layer, `resident[layer]` lists the logical expert held by every slot (EMPTY for
none). Everything else is derived from it: the two int32 lookup tables the forward pass
reads, log2slot[layer, e] (the slot holding e, or -1) and log2cpu[layer, e] (-1 when e is
resident, else e itself), kept on the host and pushed to the GPU between steps. Because the
tables are recomputed from the residency list, an expert is always on exactly one side.

Forward side. `route(layer, ids)` is one native kernel (ktmi_hot_route): both lookups and
a +1 on fp32 route counts per expert, graph-capturable and for any number of routes.

Policy side, between steps (`before_forward`): every KT_HOT_INTERVAL decode (or MTP
verify) steps the counts are snapshotted to pinned host memory without waiting for the
forward stream (the policy acts on the previous snapshot, so it runs one round behind),
then decayed by KT_HOT_DECAY on the GPU. Per layer the policy pairs the coldest slots with
the hottest non-resident experts and swaps a pair while the candidate's count exceeds
KT_HOT_MARGIN times the slot's (an empty slot counts -1), at most KT_HOT_SWAPS per layer,
stopping at the first pair that fails. A swap copies the expert's bytes from the layer's
pinned bank into the slot (the GGUF streamer's banks when it is loaded, else banks built
from the hot method's expert reader; KT_HOT_BANKS=own forces the latter).

Out of scope: the KV-lent slots of the reference (lend_slot / take_back_slot and the base
tables) and the Q2_0 down repack.
"""
from __future__ import annotations

import json
import os
import time
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from . import _lib, sglang_env

ENABLED = os.environ.get("KT_HOT_DYNAMIC") == "1"
INTERVAL = int(os.environ.get("KT_HOT_INTERVAL", "32"))
MAX_SWAPS = int(os.environ.get("KT_HOT_SWAPS", "8"))
DECAY = float(os.environ.get("KT_HOT_DECAY", "0.9"))
MARGIN = float(os.environ.get("KT_HOT_MARGIN", "1.5"))
SEED = os.environ.get("KT_HOT_SEED")
LOG_EVERY = int(os.environ.get("KT_HOT_LOG", "0") or 0)
OWN_BANKS = os.environ.get("KT_HOT_BANKS", "auto")
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


def pair_swaps(resident: np.ndarray, counts: np.ndarray, margin: float, limit: int) -> List[Tuple[int, int]]:
    """One layer's swaps [(slot, expert)]: slots from coldest (empty first, then by count,
    then by slot index) against non-resident experts from hottest (by count, then by id);
    the k-th pair is taken while the expert's count is positive and exceeds margin times
    the slot's count, and the first pair that fails ends the list."""
    E = counts.shape[0]
    slot_score = np.where(resident >= 0, counts[np.clip(resident, 0, E - 1)], -1.0)
    slots = sorted(range(len(resident)), key=lambda s: (slot_score[s], s))
    held = set(int(e) for e in resident if e >= 0)
    experts = sorted((e for e in range(E) if e not in held), key=lambda e: (-counts[e], e))
    out = []
    for s, e in zip(slots[:limit], experts[:limit]):
        c = float(counts[e])
        if not (c > 0 and c > margin * float(slot_score[s])):
            break
        out.append((s, e))
    return out


class HotCache:
    def __init__(self, num_layers: int, num_experts: int, slots: int, device, rank: int = 0):
        self.L, self.E, self.N, self.S = num_layers, num_experts, slots, slots
        self.device, self.rank = torch.device(device), rank
        self.resident = np.full((num_layers, slots), EMPTY, dtype=np.int64)
        self.log2slot_cpu = torch.empty((num_layers, num_experts), dtype=torch.int32)
        self.log2cpu_cpu = torch.empty((num_layers, num_experts), dtype=torch.int32)
        for li in range(num_layers):
            self._derive(li)
        self.log2slot = self.log2slot_cpu.to(self.device)
        self.log2cpu = self.log2cpu_cpu.to(self.device)
        self.counts = torch.zeros((num_layers, num_experts), dtype=torch.float32, device=self.device)
        self.layers: Dict[int, tuple] = {}  # layer_idx -> (hot method, layer module)
        self.banks: Dict[int, list] = {}    # own banks: layer_idx -> [gate, up, down] pinned uint8 [E, part]
        self._snapshot = torch.zeros((num_layers, num_experts), dtype=torch.float32,
                                     pin_memory=self.device.type == "cuda")
        self._snapshot_done: Optional[torch.cuda.Event] = None
        self.ready = False
        self.step = self.rounds = self.swaps = 0
        self.bytes = 0
        self.swap_s = 0.0

    # -- forward side ---------------------------------------------------------------

    def route(self, layer_idx: int, ids: torch.Tensor):
        """ids: logical [T, k] int32 (>= 0). Returns (slot ids, -1 for CPU experts; logical
        ids, -1 for resident ones)."""
        return route_native(ids, self.log2slot[layer_idx], self.log2cpu[layer_idx], self.counts[layer_idx])

    def push_tables(self) -> None:
        """The host tables to the GPU, ordered on the current stream."""
        self.log2slot.copy_(self.log2slot_cpu, non_blocking=True)
        self.log2cpu.copy_(self.log2cpu_cpu, non_blocking=True)

    # -- residency ------------------------------------------------------------------

    def _derive(self, li: int) -> None:
        """Recompute layer li's host tables from its residency list."""
        res = self.resident[li]
        held = res >= 0
        slot_of = torch.full((self.E,), -1, dtype=torch.int32)
        slot_of[torch.from_numpy(res[held])] = torch.from_numpy(np.nonzero(held)[0].astype(np.int32))
        self.log2slot_cpu[li] = slot_of
        self.log2cpu_cpu[li] = torch.where(slot_of >= 0, torch.tensor(-1, dtype=torch.int32),
                                           torch.arange(self.E, dtype=torch.int32))

    def assign(self, li: int, slot: int, expert: int) -> None:
        """Slot `slot` of layer li now holds `expert` (or EMPTY); host tables only."""
        if expert >= 0 and expert in self.resident[li] and self.resident[li][slot] != expert:
            raise ValueError(f"layer {li}: expert {expert} already sits in another slot")
        self.resident[li][slot] = expert
        self._derive(li)

    def _banks_of(self, li: int):
        """[gate, up, down] uint8 [E, part bytes] of layer li in pinned host memory, physical
        order: the streamer's when it is loaded (one pinned copy for both), else the
        cache's own from the hot method's reader."""
        if li in self.banks:
            return self.banks[li]
        if OWN_BANKS != "own":
            from . import kt_stream_prefill as SP

            inst = SP._instance
            if inst is not None and (inst.reader is not None or li in inst._banks):
                return inst._bank(li)
        t0 = time.time()
        method, _ = self.layers[li]
        p2l = sglang_env.physical_to_logical(li)
        p2l = None if sglang_env.is_identity(p2l) else p2l
        b = self.banks[li] = method.reader.banks(li, method.N, getattr(method, "rank", 0), p2l)
        if li == min(self.layers):
            _log(f"rank {self.rank}: built a {sum(t.numel() for t in b) / 1e9:.2f} GB pinned bank for layer {li} in "
                 f"{time.time() - t0:.1f} s (no streamer bank to share)")
        return b

    def load_slot(self, li: int, slot: int, expert: int) -> None:
        """Copy an expert's gate, up and down bytes from the layer's bank into a slot
        (asynchronous host-to-device copies on the current stream)."""
        method, layer = self.layers[li]
        gate, up, down = self._banks_of(li)
        N = method.N
        w13, w2 = layer.w13_qweight.data, layer.w2_qweight.data
        pieces = ((w13[slot, :N], gate[expert]), (w13[slot, N:], up[expert]), (w2[slot], down[expert]))
        for dst, src in pieces:
            dst.copy_(src.view(dst.shape), non_blocking=True)
            self.bytes += src.numel()


    def place(self, li: int, slot: int, expert: int) -> None:
        self.assign(li, slot, expert)
        if li in self.layers:
            self.load_slot(li, slot, expert)

    def check_tables(self) -> str:
        """'' when the tables on both sides agree with the residency lists, else a
        description of the first problem found."""
        if not torch.equal(self.log2slot.cpu(), self.log2slot_cpu):
            return "GPU slot table is stale (push_tables not run)"
        if not torch.equal(self.log2cpu.cpu(), self.log2cpu_cpu):
            return "GPU CPU-id table is stale (push_tables not run)"
        ids = torch.arange(self.E, dtype=torch.int32)
        for li in range(self.L):
            res = self.resident[li]
            held = [int(e) for e in res if e >= 0]
            if len(set(held)) != len(held):
                return f"layer {li}: an expert occupies two slots ({sorted(held)})"
            s_row, c_row = self.log2slot_cpu[li], self.log2cpu_cpu[li]
            on_gpu, on_cpu = s_row >= 0, c_row >= 0
            if bool((on_gpu == on_cpu).any()):
                e = int(torch.nonzero(on_gpu == on_cpu)[0])
                return f"layer {li}: expert {e} is on {'both sides' if on_gpu[e] else 'neither side'}"
            if bool((c_row[on_cpu] != ids[on_cpu]).any()):
                return f"layer {li}: a CPU id is not the expert's own id"
            for s, e in enumerate(res):
                if e >= 0 and int(s_row[e]) != s:
                    return f"layer {li}: slot {s} holds expert {e} but the table points at {int(s_row[e])}"
            if int(on_gpu.sum()) != len(held):
                return f"layer {li}: the table lists {int(on_gpu.sum())} resident experts, the slots hold {len(held)}"
        return ""

    def fill_empty(self, counts: torch.Tensor, seed_rank: Optional[torch.Tensor] = None) -> int:
        """Every EMPTY slot takes the hottest non-resident expert of its layer (host counts
        [L, E]; equal counts go to the lower seed rank, then the lower id); host tables and
        slot bytes. Returns the number of slots filled."""
        n = 0
        for li in (sorted(self.layers) if self.layers else range(self.L)):
            free = [s for s in range(self.S) if self.resident[li][s] == EMPTY]
            if not free:
                continue
            c = counts[li].double().numpy()
            rank = seed_rank[li].numpy() if seed_rank is not None else np.zeros(self.E)
            held = set(int(e) for e in self.resident[li] if e >= 0)
            order = sorted((e for e in range(self.E) if e not in held), key=lambda e: (-c[e], rank[e], e))
            for s, e in zip(free, order):
                self.place(li, s, e)
                n += 1
        return n

    def seed(self, placement: Optional[str] = None, p2l=None) -> None:
        """Initial residents per layer: the first N entries of a placement map's
        physical_to_logical_map (a JSON file, or `p2l` given as [L][>= N]), copied from the
        banks where they differ from what the loader put in the slots; without a map the
        slots keep logical experts 0..N-1."""
        t0 = time.time()
        if placement:
            with open(placement) as f:
                p2l = json.load(f)["physical_to_logical_map"]
        for li in (sorted(self.layers) if self.layers else range(self.L)):
            want = [int(p2l[li][s]) for s in range(self.N)] if p2l is not None else list(range(self.N))
            self.resident[li] = EMPTY
            self.resident[li][:] = want
            self._derive(li)
            if li in self.layers:
                for s, e in enumerate(want):
                    if e != s:
                        self.load_slot(li, s, e)
        self.push_tables()
        self.ready = True
        if self.layers:
            source = placement or ("the given map" if p2l is not None else "logical order")
            _log(f"rank {self.rank}: {self.N} slots x {len(self.layers)} layers start from {source} "
                 f"({self.bytes / 1e9:.2f} GB copied, {time.time() - t0:.1f} s); every {INTERVAL} steps up to "
                 f"{MAX_SWAPS} swaps a layer, decay {DECAY}, margin {MARGIN}")
        self.bytes = 0

    # -- policy, between steps --------------------------------------------------------

    def plan_swaps(self, counts: torch.Tensor) -> List[Tuple[int, int, int]]:
        """[(layer, slot, expert)] for host counts [L, E] (pair_swaps per layer)."""
        c = counts.double().numpy()
        limit = min(MAX_SWAPS, self.S, self.E)
        return [(li, s, e) for li in range(self.L) for s, e in pair_swaps(self.resident[li], c[li], MARGIN, limit)]

    def _take_snapshot(self) -> Optional[torch.Tensor]:
        """The previous round's counts if their copy has landed (else None and no new
        snapshot); starts the next copy and decays the live counts."""
        prev = None
        if self._snapshot_done is not None:
            if not self._snapshot_done.query():
                return None
            prev = self._snapshot.clone()
        self._snapshot.copy_(self.counts, non_blocking=True)
        self.counts.mul_(DECAY)
        if self._snapshot_done is None:
            self._snapshot_done = torch.cuda.Event()
        self._snapshot_done.record(torch.cuda.current_stream(self.device))
        return prev

    def before_forward(self, forward_batch=True) -> None:
        """Runs the policy on every INTERVAL-th decode step. forward_batch: SGLang's
        ForwardBatch (decode and MTP target-verify steps count), or a bool "decode step"."""
        mode = getattr(forward_batch, "forward_mode", None)
        if mode is None:
            decode = bool(forward_batch)
        else:
            decode = mode.is_decode() or bool(getattr(mode, "is_target_verify", lambda: False)())
        if not (self.ready and decode):
            return
        self.step += 1
        if self.step % INTERVAL:
            return
        t0 = time.time()
        counts = self._take_snapshot()
        if counts is None:
            return
        done = 0
        for li, s, e in self.plan_swaps(counts):
            if li in self.layers:
                self.place(li, s, e)
                done += 1
        if done:
            self.push_tables()
        self.rounds += 1
        self.swaps += done
        self.swap_s += time.time() - t0
        if self.rounds == 1 or (LOG_EVERY and self.rounds % LOG_EVERY == 0) or self.rounds % 64 == 0:
            _log(f"rank {self.rank}: policy round {self.rounds} at step {self.step}: {done} swaps ({self.swaps} in all, "
                 f"{self.bytes / 1e9:.2f} GB moved, {1e3 * self.swap_s / self.rounds:.1f} ms a round); "
                 f"resident experts took {100 * self.gpu_share(counts):.1f}% of the counted routes")

    def gpu_share(self, counts: torch.Tensor) -> float:
        """Fraction of the counted routes (host counts [L, E]) whose expert is resident now."""
        c = counts.double().numpy()
        hit = sum(float(c[li][self.resident[li][self.resident[li] >= 0]].sum()) for li in range(self.L))
        return hit / max(float(c.sum()), 1.0)


_cache: Optional[HotCache] = None


def register(method, layer, num_layers: Optional[int] = None, num_experts: Optional[int] = None) -> Optional[HotCache]:
    """Called by the KT wrapper for each layer after loading (P:10522); the cache is created
    by the first call and seeded (KT_HOT_SEED) when the last layer has registered. Returns
    the cache once it is ready. method: the KT wrapper method (kt_config, global_num_experts,
    tp_rank, gpu_method), or the hot GPU method itself with num_layers / num_experts."""
    global _cache
    if not ENABLED:
        return None
    kt = method.kt_config
    hot = getattr(method, "gpu_method", method)
    n_layers = getattr(kt, "num_layers", None) or num_layers
    n_experts = getattr(method, "global_num_experts", None) or num_experts
    if n_layers is None or n_experts is None:
        raise RuntimeError("hot cache: the layer and expert counts are unknown (pass num_layers / num_experts)")
    if _cache is None:
        if kt.num_gpu_experts <= 0:
            raise RuntimeError("KT_HOT_DYNAMIC=1 needs GPU expert slots (num_gpu_experts > 0)")
        _cache = HotCache(n_layers, n_experts, kt.num_gpu_experts, layer.w13_qweight.device, getattr(method, "tp_rank", 0))
    if kt.layer_idx not in _cache.layers:
        _cache.layers[kt.layer_idx] = (hot, layer)
        if len(_cache.layers) == n_layers:
            _cache.seed(SEED)
    return _cache if _cache.ready else None


def before_forward(forward_batch=True) -> None:
    if _cache is not None:
        _cache.before_forward(forward_batch)
