"""Seeded synthetic hot-expert MoE workloads (the layer shapes the hot path is measured on).

Recipe (one numpy PCG64 stream per workload, seed 20261201 + index):
  * activations x ~ N(0, 1), fp32 rounded to bf16 (RNE), [T, hidden];
  * expert popularity p_r ~ r^-s over ranks r = 1..E, given to experts by a seeded
    permutation; router logits log p_e + Gumbel(0, 1); top-k distinct experts by logit
    (descending); route weights = softmax over the k selected logits (fp32);
  * the H most popular experts are hot, slot s <-> the s-th most popular; routes to the
    other experts get slot id -1 (they belong to the CPU);
  * hot expert weights W_gate, W_up [N, hidden], W_down [hidden, N] ~ N(0, 0.02), quantised
    row-wise to the workload's GGUF types (host quantisers), one seed per slot.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Tuple

import numpy as np

from .gguf import GGML_IQ3_S, GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, quantize_rows, row_bytes

SEED_BASE = 20261201


@dataclass(frozen=True)
class Workload:
    index: int
    name: str
    hidden: int
    inter: int
    experts: int
    top_k: int
    hot: int
    types: Tuple[int, int, int]  # gate, up, down
    zipf: float
    tokens: Tuple[int, ...]
    layers: int = 1

    @property
    def seed(self) -> int:
        return SEED_BASE + self.index


WORKLOADS: Dict[str, Workload] = {
    w.name: w
    for w in (
        Workload(0, "q8_0-h2048-n768-e128-k8-hot16", 2048, 768, 128, 8, 16, (GGML_Q8_0,) * 3, 1.1, (512,)),
        Workload(1, "q4_k-h2048-n512-e256-k8-hot32-decode", 2048, 512, 256, 8, 32, (GGML_Q4_K,) * 3, 1.1,
                 (1, 4, 8, 16)),
        Workload(2, "q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", 2048, 512, 256, 8, 40,
                 (GGML_Q4_K, GGML_Q4_K, GGML_Q6_K), 1.1, (2048, 16384, 32768)),
        Workload(3, "iq3_s-h2048-n512-e512-k10-hot48", 2048, 512, 512, 10, 48, (GGML_IQ3_S,) * 3, 1.2, (16384,)),
        Workload(4, "q4_k+q6_k-h7168-n2048-e256-k8-hot24-stream4", 7168, 2048, 256, 8, 24,
                 (GGML_Q4_K, GGML_Q4_K, GGML_Q6_K), 1.1, (6144,), layers=4),
    )
}


def bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def popularity(w: Workload):
    """(p [E] normalised, perm: rank -> expert id)."""
    rng = np.random.Generator(np.random.PCG64([w.seed, 0]))
    ranks = np.arange(1, w.experts + 1, dtype=np.float64)
    p_rank = ranks ** (-w.zipf)
    p_rank /= p_rank.sum()
    perm = rng.permutation(w.experts)
    p = np.empty(w.experts)
    p[perm] = p_rank
    return p, perm


def routing(w: Workload, tokens: int):
    """(topk_ids int32 [T, k] logical, topk_weights fp32 [T, k], slot_ids int32 [T, k], hot [H])."""
    p, perm = popularity(w)
    rng = np.random.Generator(np.random.PCG64([w.seed, 1, tokens]))
    logits = (np.log(p)[None, :] + rng.gumbel(size=(tokens, w.experts))).astype(np.float32)
    part = np.argpartition(-logits, w.top_k - 1, axis=1)[:, : w.top_k]
    sel = np.take_along_axis(logits, part, axis=1)
    order = np.argsort(-sel, axis=1, kind="stable")
    ids = np.take_along_axis(part, order, axis=1).astype(np.int32)
    sl = np.take_along_axis(sel, order, axis=1).astype(np.float64)
    e = np.exp(sl - sl.max(axis=1, keepdims=True))
    weights = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    hot = perm[: w.hot].astype(np.int32)
    log2slot = np.full(w.experts, -1, np.int32)
    log2slot[hot] = np.arange(w.hot, dtype=np.int32)
    return ids, weights, log2slot[ids], hot


def activations(w: Workload, tokens: int) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64([w.seed, 2, tokens]))
    return bf16_bits(rng.standard_normal((tokens, w.hidden), dtype=np.float32))


def expert_weights(w: Workload, slot: int, layer: int = 0, threads: int = 0):
    """(w13 uint8 [2N, rb(hidden, gate)] rows [gate; up], w2 uint8 [hidden, rb(N, down)])."""
    rng = np.random.Generator(np.random.PCG64([w.seed, 3, layer, slot]))
    N, K = w.inter, w.hidden
    gate = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    up = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    down = (rng.standard_normal((K, N), dtype=np.float32) * np.float32(0.02))
    w13 = np.concatenate([quantize_rows(gate, w.types[0], threads), quantize_rows(up, w.types[1], threads)])
    return w13, quantize_rows(down, w.types[2], threads)


def slot_tensors(w: Workload, layer: int = 0, threads: int = 0):
    """All hot slots: (w13 uint8 [H, 2N, rb13], w2 uint8 [H, hidden, rb2])."""
    rb13 = row_bytes(w.hidden, w.types[0])
    rb2 = row_bytes(w.inter, w.types[2])
    w13 = np.empty((w.hot, 2 * w.inter, rb13), np.uint8)
    w2 = np.empty((w.hot, w.hidden, rb2), np.uint8)
    for s in range(w.hot):
        w13[s], w2[s] = expert_weights(w, s, layer, threads)
    return w13, w2


def small(w: Workload, hot: int = None, experts: int = None, **kw) -> Workload:
    """The same recipe at a reduced size (for parity tests)."""
    from dataclasses import replace

    return replace(w, hot=hot or w.hot, experts=experts or w.experts, **kw)
