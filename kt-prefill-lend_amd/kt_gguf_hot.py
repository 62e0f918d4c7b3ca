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


from . import _lib, sglang_env
from .gguf import BLOCK_INFO, KERNEL_TYPES, GGUFFile, row_bytes as _row_bytes

try:  # inside SGLang the real combine input type is used
    from sglang.srt.layers.moe.token_dispatcher import StandardCombineInput  # type: ignore
except Exception:  # noqa: BLE001
    StandardCombineInput = namedtuple("StandardCombineInput", ["hidden_states"])

DispatchOutput = namedtuple("DispatchOutput", ["hidden_states", "topk_output"])
TopKOutput = namedtuple("TopKOutput", ["topk_weights", "topk_ids", "router_logits"])

GGML_Q8_0 = 8
_MODES = {"auto": _lib.MODE_AUTO, "gemv": _lib.MODE_GEMV, "grouped": _lib.MODE_GROUPED, "decode": _lib.MODE_DECODE}


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
        """(uint8 torch view of the tensor's bytes over the file's private mapping, ggml type)."""
        return torch.from_numpy(self.file.raw(name)), self.file.ggml_type(name)

    def types(self, layer_idx: int):
        return tuple(self.file.ggml_type(f"blk.{layer_idx}.ffn_{p}_exps.weight") for p in ("gate", "up", "down"))

    def layers(self):
        """The layers that hold routed-expert tensors (blk.{l}.ffn_gate_exps.weight), in order;
        dense leading layers are skipped."""
        return [li for li in range(self.num_layers) if self.file.has_tensor(f"blk.{li}.ffn_gate_exps.weight")]

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


def _slot_types(layer_idx: int, types) -> tuple:
    """(type13, type2) of a layer's slots from the GGUF's (gate, up, down) types: the slot
    rows hold gate and up back to back, so those two must agree, and each type needs a
    kernel here."""
    gate, up, down = types
    if gate != up:
        raise RuntimeError(f"layer {layer_idx}: the slots keep gate and up rows in one tensor, but the GGUF "
                           f"stores them as ggml types {gate} and {up}")
    missing = sorted({t for t in (gate, down) if t not in KERNEL_TYPES})
    if missing:
        raise RuntimeError(f"layer {layer_idx}: ggml type(s) {missing} have no kernel in libktmi "
                           f"(supported: {sorted(KERNEL_TYPES)})")
    return gate, down


def _no_checkpoint_tensors(param, loaded_weight, *args, **kwargs):
    """weight_loader of the slot tensors: they are filled from the GGUF after loading
    (process_weights_after_loading), so a checkpoint tensor routed here is a wiring error."""
    raise RuntimeError("GGUF hot-expert slots are filled from the GGUF file, not from checkpoint tensors")


class KTGGUFHotExpertsMethod:
    """GPU-expert method the KT wrapper wraps when the experts are GGUF blocks
    (hot/kt_gguf_hot.py:163-304): the same constructor, create_weights /
    process_weights_after_loading / create_moe_runner / apply signatures and attributes."""

    # the streamer's banks cover the hot slots at streamed-prefill sizes (P:10615-10623)
    streams_hot_experts = True

    def __init__(self, kt_config, layer):
        li = kt_config.layer_idx
        self.kt_config = kt_config
        self.num_gpu_experts = kt_config.num_gpu_experts
        self.reader = _reader(kt_config.weight_path)
        self.rank, self.world = getattr(layer, "moe_tp_rank", 0), getattr(layer, "moe_tp_size", 1)
        self.types = tuple(self.reader.types(li))
        self.type13, self.type2 = _slot_types(li, self.types)
        self.moe_runner_config = None
        self.mode = _MODES[os.environ.get("KT_HOT_LAYER_MODE", "auto")]
        self._desc = None
        self._ws = None

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition, params_dtype,
                       **extra_weight_attrs):
        """Registers w13_qweight uint8 [E, 2N, rb(K)] and w2_qweight uint8 [E, K, rb(N)]
        (E = num_experts slots, N = this rank's intermediate rows) on the current device."""
        self.N, self.K = intermediate_size_per_partition, hidden_size
        gguf_shape = (self.reader.inter, self.reader.K)
        if (self.N * self.world, self.K) != gguf_shape:
            raise RuntimeError(f"the GGUF's experts are {gguf_shape[0]} intermediate x {gguf_shape[1]} hidden; this "
                               f"layer asks for {self.N} per rank x {self.world} ranks and hidden {self.K}")
        if num_experts == 0:
            return
        dev = torch.device("cuda", torch.cuda.current_device())
        shapes = {"w13_qweight": (num_experts, 2 * self.N, _row_bytes(self.K, self.type13)),
                  "w2_qweight": (num_experts, self.K, _row_bytes(self.N, self.type2))}
        for name, shape in shapes.items():
            param = torch.nn.Parameter(torch.empty(shape, dtype=torch.uint8, device=dev), requires_grad=False)
            param.weight_loader = _no_checkpoint_tensors
            layer.register_parameter(name, param)

    def process_weights_after_loading(self, layer, physical_to_logical=None) -> None:
        """Copies this rank's TP part of the slots' experts out of the GGUF. Slot s holds
        logical expert p2l[s]: the map given here, else SGLang's expert-location map for
        this layer (hot/kt_gguf_hot.py:213-220), else the identity."""
        n = self.num_gpu_experts
        if n == 0:
            return
        li, N = self.kt_config.layer_idx, self.N
        p2l = physical_to_logical if physical_to_logical is not None else sglang_env.physical_to_logical(li)
        experts = torch.arange(n) if p2l is None else torch.as_tensor(p2l, dtype=torch.int64)[:n]
        w13, w2 = layer.w13_qweight.data, layer.w2_qweight.data
        for proj, dst in (("gate", w13[:, :N]), ("up", w13[:, N:]), ("down", w2)):
            src = torch.as_tensor(self.reader.slice(li, proj, N, self.rank, experts))
            if tuple(src.shape) != tuple(dst.shape):
                raise RuntimeError(f"layer {li} {proj}: GGUF slice {tuple(src.shape)} does not fit the slots "
                                   f"{tuple(dst.shape)}")
            dst.copy_(src)
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
