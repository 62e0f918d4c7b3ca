"""ktmi: the hot-expert MoE path of a KTransformers + SGLang hybrid on one MI355X (gfx950).

Host-side mirror of the reference's plugin modules (kt_gguf_hot, kt_gguf_moe_multi,
kt_hot_cache, kt_gguf_dequant, the KT wrapper's CPU-mask hook) over the C ABI of
lib/libktmi.so (include/ktmi.h): hand-written HIP kernels for the dequant, the route
lookup and sort, the int8 decode GEMV, the bf16 MFMA grouped GEMMs that dequantise in registers, with
fused SiLU*mul, and the deterministic weighted combine.

The directory name is not a Python identifier; load it as `kt_prefill_lend_amd` with
`load_package()` below (tests, bench.py and __graft_entry__.py do).
"""
from __future__ import annotations

__all__ = ["gguf", "kt_gguf_moe_multi", "kt_gguf_dequant", "kt_gguf_hot", "kt_hot_cache", "kt_ep_wrapper", "synth"]


def load_package(name: str = "kt_prefill_lend_amd"):
    """Import this directory as a package named `name` (idempotent)."""
    import importlib.util
    import sys
    from pathlib import Path

    if name in sys.modules:
        return sys.modules[name]
    root = Path(__file__).resolve().parent
    spec = importlib.util.spec_from_file_location(name, root / "__init__.py", submodule_search_locations=[str(root)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod
