"""What the hot-expert path reads from the SGLang process it runs in.

The reference modules import these straight from SGLang; here each lives behind one
function that asks SGLang when it is importable and otherwise returns what a caller
without a server (a benchmark, the tests, a stand-alone script) gets:

* `tp_rank_world()`: the tensor-parallel rank and size (the reference's
  get_tensor_model_parallel_rank / _world_size, P:40489-40492); (0, 1) alone.
* `server_weight_path()`: the GGUF path the server was started with (server args'
  kt_weight_path, read by the streamer's preallocate, P:40607-40615); the environment
  variable KT_WEIGHT_PATH alone.
* `chunk_rows()`: the server's chunked-prefill size (P:40506-40512); 0 alone.
* `physical_to_logical(layer_idx)`: the expert-location map of a layer, int64 [E_phys]
  (physical slot -> logical expert), or None when there is no map
  (get_global_expert_location_metadata().physical_to_logical_map_cpu, read by
  hot/kt_gguf_hot.py:213-220 and the streamer's _physical_to_logical, P:40701-40710).
"""
from __future__ import annotations

import os
from typing import Optional, Tuple

import torch


def tp_rank_world() -> Tuple[int, int]:
    try:
        from sglang.srt.distributed import get_tensor_model_parallel_rank, get_tensor_model_parallel_world_size
    except ImportError:
        return 0, 1
    return int(get_tensor_model_parallel_rank()), int(get_tensor_model_parallel_world_size())


def _server_args():
    try:
        from sglang.srt.server_args import get_global_server_args
    except ImportError:
        return None
    try:
        return get_global_server_args()
    except Exception:  # noqa: BLE001 - no server configured in this process
        return None


def server_weight_path() -> Optional[str]:
    args = _server_args()
    path = getattr(args, "kt_weight_path", None) if args is not None else None
    return path or os.environ.get("KT_WEIGHT_PATH") or None


def chunk_rows() -> int:
    args = _server_args()
    return int(getattr(args, "chunked_prefill_size", 0) or 0) if args is not None else 0


def physical_to_logical(layer_idx: int) -> Optional[torch.Tensor]:
    try:
        from sglang.srt.eplb.expert_location_dispatch import get_global_expert_location_metadata
    except ImportError:
        return None
    meta = get_global_expert_location_metadata()
    if meta is None:
        return None
    return torch.as_tensor(meta.physical_to_logical_map_cpu[layer_idx]).to(torch.int64)


def is_identity(p2l: Optional[torch.Tensor]) -> bool:
    """True for no map or the identity placement."""
    return p2l is None or torch.equal(p2l, torch.arange(p2l.numel(), dtype=torch.int64))
