"""GPU hot experts straight from GGUF blocks (drop-in for hot/kt_gguf_hot.py).

Slot layout per layer (E_gpu = num_gpu_experts, N = intermediate per rank, K = hidden),
as the reference keeps it (hot/kt_gguf_hot.py:17-21):
    w13_qweight  uint8 [E_gpu, 2N, row_bytes(K, gate/up type)]   rows [gate; up]
    w2_qweight   uint8 [E_gpu, K,  row_bytes(N, down type)]
Gate and up must share a type.

`KTGGUFHotExpertsMethod.apply(layer, dispatch_output)` computes this rank's GPU half of a
MoE layer in one native call (ktmi_moe_layer): decode-sized route counts take the int8
GEMV over raw blocks (the reference's window kernel), larger ones sort the routes by slot
and run the dequant-in-LDS bf16 MFMA grouped GEMMs; the weighted top-k combine is the
reference's _combine order in both. Routes with slot id -1 (experts on the CPU) add
nothing. KT_HOT_LAYER_MODE=auto|gemv|grouped overrides the choice.

Weights come from an expert source: an object with E, inter, K, types(layer_idx) and
slice(layer_idx, proj, N, rank, experts) -> uint8 [n, rows, part_row_bytes] (the
reference's _GGUFExperts, :109-160). `register_source(path, source)` binds one to the
kt_config.weight_path the method is built with.
"""
from __future__ import annotations

import os
import time
from collections import namedtuple
from typing import Dict

import torch

from . import _lib
from .gguf import BLOCK_INFO, KERNEL_TYPES, row_bytes as _row_bytes

try:  # inside SGLang the real combine input type is used
    from sglang.srt.layers.moe.token_dispatcher import StandardCombineInput  # type: ignore
except Exception:  # noqa: BLE001
    StandardCombineInput = namedtuple("StandardCombineInput", ["hidden_states"])

DispatchOutput = namedtuple("DispatchOutput", ["hidden_states", "topk_output"])
TopKOutput = namedtuple("TopKOutput", ["topk_weights", "topk_ids", "router_logits"])

GGML_Q8_0 = 8
_MODES = {"auto": _lib.MODE_AUTO, "gemv": _lib.MODE_GEMV, "grouped": _lib.MODE_GROUPED}


def _log(msg):
    print(f"[kt-gguf-hot {time.strftime('%H:%M:%S')}] {msg}", flush=True)


_sources: Dict[str, object] = {}


def register_source(path: str, source) -> None:
    """Bind an expert source to a weight path (what the reference opens as a GGUF)."""
    _sources[path] = source


def _reader(path: str):
    src = _sources.get(path)
    if src is None:
        raise RuntimeError(f"no expert source registered for {path!r} (register_source)")
    return src


def layer_desc(w13: torch.Tensor, w2: torch.Tensor, hidden: int, inter: int, type13: int, type2: int,
               table: bool = False) -> _lib.ktmi_layer:
    """The C descriptor of a layer's slot tensors. It holds raw device pointers: the caller
    keeps w13 and w2 alive for as long as the descriptor is used."""
    L = _lib.ktmi_layer()
    L.hidden, L.inter = hidden, inter
    L.n_slots = w13.shape[0]
    L.type13, L.type2 = type13, type2
    L.w13, L.w2 = w13.data_ptr(), w2.data_ptr()
    L.w_is_table = int(table)
    return L


def moe_layer(desc: _lib.ktmi_layer, x: torch.Tensor, topk_weights: torch.Tensor, slot_ids: torch.Tensor,
              mode: int = _lib.MODE_AUTO, out: torch.Tensor = None, workspace: torch.Tensor = None) -> torch.Tensor:
    """One hot-expert MoE layer on the GPU: y [T, K] bf16 from x [T, K] bf16, fp32 route
    weights [T, k] and int32 slot ids [T, k] (-1 = not on the GPU)."""
    if x.dtype != torch.bfloat16:
        raise TypeError(f"moe_layer: x must be bf16, got {x.dtype}")
    if slot_ids.dtype != torch.int32:
        raise TypeError(f"moe_layer: slot ids must be int32, got {slot_ids.dtype}")
    T, top_k = slot_ids.shape
    x = x.contiguous()
    w = topk_weights.to(torch.float32).contiguous()
    ids = slot_ids.contiguous()
    L = _lib.lib()
    if out is None:
        out = torch.empty((T, desc.hidden), dtype=torch.bfloat16, device=x.device)
    need = L.ktmi_moe_layer_workspace(desc, T, top_k, mode)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty((max(need, 256),), dtype=torch.uint8, device=x.device)
    rc = L.ktmi_moe_layer(desc, x.data_ptr(), w.data_ptr(), ids.data_ptr(), T, top_k, out.data_ptr(),
                          workspace.data_ptr(), workspace.numel(), mode, _lib.stream_ptr(x.device))
    _lib.check(rc, "moe_layer")
    return out


def _combine(out: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """out [T, top_k, K] (the routes' rows), w [T, top_k]: sum_k bf16(out * bf16(w)) in fp32,
    rounded once (hot/kt_gguf_hot.py:62-71)."""
    T, top_k, K = out.shape
    out = out.contiguous()
    w = w.to(torch.float32).contiguous()
    res = torch.empty((T, K), dtype=out.dtype, device=out.device)
    rc = _lib.lib().ktmi_combine(out.data_ptr(), _lib.dtype_code(out.dtype), w.data_ptr(), T, top_k, K,
                                 res.data_ptr(), _lib.stream_ptr(out.device))
    _lib.check(rc, "combine")
    return res


def silu_and_mul(h: torch.Tensor) -> torch.Tensor:
    """[R, 2N] -> [R, N] = silu(h[:, :N]) * h[:, N:] (the sgl_kernel op the reference calls)."""
    R, N2 = h.shape
    h = h.contiguous()
    out = torch.empty((R, N2 // 2), dtype=h.dtype, device=h.device)
    rc = _lib.lib().ktmi_silu_and_mul(h.data_ptr(), _lib.dtype_code(h.dtype), R, N2 // 2, out.data_ptr(),
                                      _lib.stream_ptr(h.device))
    _lib.check(rc, "silu_and_mul")
    return out


class KTGGUFHotExpertsMethod:
    """GPU-expert method the KT wrapper wraps when the experts are GGUF blocks
    (hot/kt_gguf_hot.py:163-304)."""

    # the streamer's banks cover the hot slots at streamed-prefill sizes (P:10615-10623)
    streams_hot_experts = True

    def __init__(self, kt_config, layer):
        self.kt_config = kt_config
        self.num_gpu_experts = kt_config.num_gpu_experts
        self.reader = _reader(kt_config.weight_path)
        self.rank = getattr(layer, "moe_tp_rank", 0)
        self.world = getattr(layer, "moe_tp_size", 1)
        self.types = tuple(self.reader.types(kt_config.layer_idx))
        if self.types[0] != self.types[1]:
            raise RuntimeError(f"layer {kt_config.layer_idx}: gate {self.types[0]} and up {self.types[1]} differ")
        self.type13, self.type2 = self.types[0], self.types[2]
        for t in (self.type13, self.type2):
            if t not in KERNEL_TYPES:
                raise RuntimeError(f"layer {kt_config.layer_idx}: ggml type {t} has no ktmi kernel")
        self.moe_runner_config = None
        self.mode = _MODES[os.environ.get("KT_HOT_LAYER_MODE", "auto")]
        self._desc = None
        self._ws = None

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition, params_dtype,
                       **extra_weight_attrs):
        E, N, K = num_experts, intermediate_size_per_partition, hidden_size
        self.N, self.K = N, K
        if N * self.world != self.reader.inter or K != self.reader.K:
            raise RuntimeError(f"GGUF experts {self.reader.inter}x{self.reader.K} vs layer {N}x{self.world} / {K}")
        if E == 0:
            return
        dev = torch.device("cuda", torch.cuda.current_device())
        w13 = torch.nn.Parameter(torch.empty((E, 2 * N, _row_bytes(K, self.type13)), dtype=torch.uint8, device=dev),
                                 requires_grad=False)
        w2 = torch.nn.Parameter(torch.empty((E, K, _row_bytes(N, self.type2)), dtype=torch.uint8, device=dev),
                                requires_grad=False)
        w13.weight_loader = w2.weight_loader = self._refuse_loader
        layer.register_parameter("w13_qweight", w13)
        layer.register_parameter("w2_qweight", w2)

    @staticmethod
    def _refuse_loader(param, loaded_weight, *a, **k):
        raise RuntimeError("GGUF hot experts take no checkpoint expert tensors")

    def process_weights_after_loading(self, layer, physical_to_logical=None) -> None:
        """Fill the slots with this rank's TP slice of logical experts p2l[:E] (identity
        without a placement map), hot/kt_gguf_hot.py:213-234."""
        E = self.num_gpu_experts
        if E == 0:
            return
        p2l = (torch.as_tensor(physical_to_logical[:E], dtype=torch.int64) if physical_to_logical is not None
               else torch.arange(E))
        li, N = self.kt_config.layer_idx, self.N
        gate = self.reader.slice(li, "gate", N, self.rank, p2l)
        up = self.reader.slice(li, "up", N, self.rank, p2l)
        layer.w13_qweight.data[:, :N].copy_(torch.as_tensor(gate))
        layer.w13_qweight.data[:, N:].copy_(torch.as_tensor(up))
        down = torch.as_tensor(self.reader.slice(li, "down", N, self.rank, p2l))
        assert tuple(down.shape) == tuple(layer.w2_qweight.shape), (down.shape, layer.w2_qweight.shape)
        layer.w2_qweight.data.copy_(down)
        self._desc = None

    def create_moe_runner(self, layer, moe_runner_config):
        self.moe_runner_config = moe_runner_config

    def _layer_desc(self, layer):
        p13 = getattr(layer, "kt_kv_ptr13", None)
        tbl = p13 is not None
        w13 = p13 if tbl else layer.w13_qweight
        w2 = layer.kt_kv_ptr2 if tbl else layer.w2_qweight
        key = (w13.data_ptr(), w2.data_ptr(), tbl)
        if self._desc is None or self._desc[0] != key:
            d = layer_desc(w13, w2, self.K, self.N, self.type13, self.type2, tbl)
            if tbl:
                d.n_slots = w13.shape[0]
            self._desc = (key, d)
        return self._desc[1]

    def apply(self, layer, dispatch_output):
        x = dispatch_output.hidden_states
        topk_weights, topk_ids, _ = dispatch_output.topk_output
        ids = topk_ids if topk_ids.dtype == torch.int32 else topk_ids.to(torch.int32)
        y = moe_layer(self._layer_desc(layer), x, topk_weights, ids, self.mode)
        return StandardCombineInput(hidden_states=y)
