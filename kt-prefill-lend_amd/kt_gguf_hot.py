"""GPU hot experts straight from GGUF blocks (drop-in for hot/kt_gguf_hot.py).

Slot layout per layer (E_gpu = num_gpu_experts, N = intermediate per rank, K = hidden),
as the reference keeps it (hot/kt_gguf_hot.py:17-21):
    w13_qweight  uint8 [E_gpu, 2N, row_bytes(K, gate/up type)]   rows [gate; up]
    w2_qweight   uint8 [E_gpu, K,  row_bytes(N, down type)]
Gate and up must share a type.

`KTGGUFHotExpertsMethod.apply(layer, dispatch_output)` computes this rank's GPU half of a
MoE layer in one native call (ktmi_moe_layer): decode-sized route counts take the int8
GEMV over raw blocks (the reference's window kernel), larger ones sort the routes by slot
and run the bf16 MFMA grouped GEMMs (GGUF blocks dequantised in registers); the weighted top-k combine is the
reference's _combine order in both. Routes with slot id -1 (experts on the CPU) add
nothing. KT_HOT_LAYER_MODE=auto|gemv|grouped overrides the choice.

Weights come from an expert source: an object with E, inter, K, types(layer_idx) and
slice(layer_idx, proj, N, rank, experts) -> uint8 [n, rows, part_row_bytes] (the
reference's _GGUFExperts, :109-160). `GGUFExperts` is that source over a GGUF file (one
reader per path, shared by all layers); `register_source(path, source)` binds any other
source to the kt_config.weight_path the method is built with.
"""
from __future__ import annotations

import os
import time
from collections import namedtuple
from typing import Dict

import torch


from . import _lib
from .gguf import BLOCK_INFO, KERNEL_TYPES, GGUFFile, row_bytes as _row_bytes

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


class GGUFExperts:
    """The routed experts of a GGUF file (hot/kt_gguf_hot.py:109-160): per layer the
    tensors blk.{l}.ffn_{gate,up,down}_exps.weight, shapes [E, inter, K] (gate, up) and
    [E, K, inter] (down), read as views over the file mapping."""

    def __init__(self, path: str):
        self.file = GGUFFile(path)
        cfg = self.file.model_config()
        self.E = cfg["num_experts"]
        self.inter = cfg["moe_intermediate_size"]
        self.K = cfg["hidden_size"]
        self.num_layers = cfg["num_layers"]

    def _raw(self, name: str):
        """(uint8 torch view of the tensor's bytes over the mapping, ggml type)."""
        import warnings

        data = self.file.raw(name)
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")  # read-only buffer, only copied out
            return torch.from_numpy(data), self.file.ggml_type(name)

    def types(self, layer_idx: int):
        return tuple(self.file.ggml_type(f"blk.{layer_idx}.ffn_{p}_exps.weight") for p in ("gate", "up", "down"))

    def _view(self, layer_idx: int, proj: str, N: int, rank: int) -> torch.Tensor:
        """This rank's TP part of every expert: rows [N*rank, N*(rank+1)) of gate/up, the
        matching block-aligned columns of down; uint8 [E, rows, part_row_bytes]."""
        data, t = self._raw(f"blk.{layer_idx}.ffn_{proj}_exps.weight")
        blck, ts = BLOCK_INFO[t]
        if proj != "down":
            if self.K % blck:
                raise ValueError(f"layer {layer_idx} {proj}: hidden {self.K} is not whole blocks of {blck}")
            return data.view(self.E, self.inter, (self.K // blck) * ts)[:, N * rank:N * (rank + 1), :]
        if self.inter % blck or (N * rank) % blck or N % blck:
            raise ValueError(f"layer {layer_idx} down: slice [{N * rank}, {N * (rank + 1)}) of {self.inter} is not "
                             f"block-aligned ({blck})")
        v = data.view(self.E, self.K, self.inter // blck, ts)[:, :, (N * rank) // blck:(N * (rank + 1)) // blck, :]
        return v.reshape(self.E, self.K, -1)

    def slice(self, layer_idx: int, proj: str, N: int, rank: int, experts) -> torch.Tensor:
        """Raw bytes of this rank's part of the given logical experts: uint8
        [len(experts), rows, part_row_bytes] (a copy)."""
        ids = torch.as_tensor(experts, dtype=torch.int64)
        return self._view(layer_idx, proj, N, rank)[ids].contiguous()

    def banks(self, layer_idx: int, N: int, rank: int = 0, p2l=None, pin: bool = True):
        """[gate, up, down]: this rank's part of every expert of the layer as uint8
        [E, part_bytes] in host memory (pinned when a GPU is present), physical order
        p2l[physical] = logical when a placement map is given (P:40712-40752)."""
        out = []
        pin = pin and torch.cuda.is_available()
        for proj in ("gate", "up", "down"):
            v = self._view(layer_idx, proj, N, rank).reshape(self.E, -1)
            if p2l is not None:
                v = v[torch.as_tensor(p2l, dtype=torch.int64)]
            h = torch.empty(v.shape, dtype=torch.uint8, pin_memory=pin)
            h.copy_(v)
            out.append(h)
        return out


_sources: Dict[str, object] = {}


def register_source(path: str, source) -> None:
    """Bind an expert source to a weight path (instead of opening it as a GGUF file)."""
    _sources[path] = source


def _reader(path: str):
    """The registered source for the path, else the (cached) GGUF reader of the file."""
    src = _sources.get(path)
    if src is None:
        if not path or not os.path.isfile(path):
            raise RuntimeError(f"no expert source registered for {path!r} and no GGUF file there")
        src = _sources[path] = GGUFExperts(path)
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
