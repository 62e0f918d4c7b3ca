"""The KT wrapper's hot-expert pieces: the CPU-mask hook and the GPU/CPU route split.

`_prefix_gpu_experts_mask` is the inference-ABI mask for kt-kernel (P:10389-10400);
`cpu_experts_mask` applies the CPU-mask hook (hot/sglang-kt-hot-cpu-mask.py:21-35, landed
at P:10465-10476): under the dynamic hot cache the mask is empty, so the CPU computes
exactly the logical ids it is given (residents arrive as -1); KT_HOT_CPU_PREFIX_MASK=1
restores the prefix mask (for comparison only).

`hot_split_apply` is the hot-cache branch of KTEPWrapperMethod.apply (P:10590-10602):
route once, hand the CPU its ids, run the GPU method on the slot ids, then add the CPU
partial. The CPU side is a `kt_cpu_moe.KTCPUExperts` (libktmi's CPU expert engine:
submit stages the inputs and returns, sync_add adds the output on the stream), or any
submit / sync callables of the caller's own engine.
"""
from __future__ import annotations

import os

import torch

from . import kt_hot_cache


def _prefix_gpu_experts_mask(num_experts: int, num_gpu_experts: int) -> torch.Tensor:
    """bool [num_experts] on the CPU, True for ids 0..num_gpu_experts-1."""
    if not 0 <= num_gpu_experts <= num_experts:
        raise ValueError(f"num_gpu_experts must be in [0, {num_experts}], got {num_gpu_experts}")
    mask = torch.zeros(num_experts, dtype=torch.bool, device="cpu")
    mask[:num_gpu_experts] = True
    return mask


def cpu_experts_mask(num_experts: int, num_gpu_experts: int, hot_enabled: bool = None) -> torch.Tensor:
    """The gpu_experts_mask kt-kernel is built with (the CPU-mask hook)."""
    if hot_enabled is None:
        hot_enabled = kt_hot_cache.ENABLED
    prefix = os.environ.get("KT_HOT_CPU_PREFIX_MASK", "0") == "1"
    return _prefix_gpu_experts_mask(num_experts, 0 if (hot_enabled and not prefix) else num_gpu_experts)


def mask_cpu_expert_ids(topk_ids: torch.Tensor, num_gpu_experts: int) -> torch.Tensor:
    """Static placement: GPU experts are physical 0..num_gpu_experts-1, the rest -1 (in place)."""
    topk_ids[topk_ids >= num_gpu_experts] = -1
    return topk_ids


def hot_split_apply(cache, layer_idx: int, gpu_method, layer, dispatch_output, cpu_submit=None, cpu_sync=None,
                    cpu=None):
    """GPU half on the resident slots + CPU half on the rest; returns hidden [T, K].
    cpu: a KTCPUExperts for this layer (its bank indexed by logical expert id); or
    cpu_submit(layer, dispatch_output) / cpu_sync(x) -> the CPU partial."""
    x = dispatch_output.hidden_states
    tk = dispatch_output.topk_output
    slot_ids, cpu_ids = cache.route(layer_idx, tk.topk_ids)
    if cpu is not None:
        cpu.submit(x, cpu_ids, tk.topk_weights)
    elif cpu_submit is not None:
        cpu_submit(layer, dispatch_output._replace(topk_output=tk._replace(topk_ids=cpu_ids)))
    out = gpu_method.apply(layer, dispatch_output._replace(topk_output=tk._replace(topk_ids=slot_ids))).hidden_states
    if cpu is not None:
        out = cpu.sync_add(out.contiguous())
    elif cpu_sync is not None:
        out = out + cpu_sync(x)
    return out
