"""ktmi_moe_layer_noalloc (the layer with the library's own per-GPU scratch array in place of
a caller workspace) against ktmi_moe_layer with a workspace, through the C ABI: two calls in
a row, the second smaller (a 512-token grouped chunk, then an 8-token decode window), each
bit for bit; a layer whose workspace exceeds the array is refused before any device work."""
import ctypes as C

import numpy as np
import pytest

from conftest import bf16_bits_of, bf16_tensor, to_dev

pytestmark = pytest.mark.gpu


def _layer(dev, name, T):
    import kt_prefill_lend_amd.kt_gguf_hot as H
    import kt_prefill_lend_amd.synth as S

    w = S.WORKLOADS[name]
    _, tw, slot, _ = S.routing(w, T)
    w13, w2 = S.slot_tensors(w)
    W13, W2 = to_dev(w13, dev), to_dev(w2, dev)
    desc = H.layer_desc(W13, W2, w.hidden, w.inter, w.types[0], w.types[2])
    x = bf16_tensor(S.activations(w, T), dev)
    return w, desc, (W13, W2), x, to_dev(tw, dev), to_dev(slot, dev)


def _with_workspace(dev, desc, x, tw, slot):
    import torch

    import kt_prefill_lend_amd._lib as L

    T, k = slot.shape
    lib = L.lib()
    y = torch.empty((T, desc.hidden), dtype=torch.bfloat16, device=dev)
    need = lib.ktmi_moe_layer_workspace(C.byref(desc), T, k, L.MODE_AUTO)
    ws = torch.empty((max(need, 256),), dtype=torch.uint8, device=dev)
    L.check(lib.ktmi_moe_layer(C.byref(desc), x.data_ptr(), tw.data_ptr(), slot.data_ptr(), T, k, y.data_ptr(),
                               ws.data_ptr(), ws.numel(), L.MODE_AUTO, L.stream_ptr(dev)), "moe_layer")
    return y


def _noalloc(dev, desc, x, tw, slot):
    import torch

    import kt_prefill_lend_amd._lib as L

    T, k = slot.shape
    y = torch.full((T, desc.hidden), float("nan"), dtype=torch.bfloat16, device=dev)
    L.check(L.lib().ktmi_moe_layer_noalloc(C.byref(desc), x.data_ptr(), tw.data_ptr(), slot.data_ptr(), T, k,
                                           y.data_ptr(), L.MODE_AUTO, L.stream_ptr(dev)), "moe_layer_noalloc")
    return y


def test_noalloc_layer_matches_the_workspace_layer(dev):
    import torch

    import kt_prefill_lend_amd._lib as L

    lib = L.lib()
    cases = [("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", 512), ("q4_k-h2048-n512-e256-k8-hot32-decode", 8)]
    for i, (name, T) in enumerate(cases):
        w, desc, keep, x, tw, slot = _layer(dev, name, T)
        mode = lib.ktmi_moe_layer_mode(C.byref(desc), T, w.top_k)
        need = lib.ktmi_moe_layer_workspace(C.byref(desc), T, w.top_k, L.MODE_AUTO)
        print(f"noalloc call {i}: {name} T={T} mode {mode} scratch {need} bytes", flush=True)
        assert need <= L.NOALLOC_SCRATCH_BYTES
        y_ws = _with_workspace(dev, desc, x, tw, slot)
        y_na = _noalloc(dev, desc, x, tw, slot)
        torch.cuda.synchronize()
        a, b = bf16_bits_of(y_ws), bf16_bits_of(y_na)
        assert np.array_equal(a, b), (name, T, int((a != b).sum()))
        assert (slot.cpu().numpy() >= 0).any() and np.any(a != 0)
        del keep


def test_noalloc_refuses_a_layer_past_its_scratch(dev):
    import kt_prefill_lend_amd._lib as L

    name, T = "q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", 4096
    w, desc, keep, x, tw, slot = _layer(dev, name, T)
    lib = L.lib()
    assert lib.ktmi_moe_layer_workspace(C.byref(desc), T, w.top_k, L.MODE_AUTO) > L.NOALLOC_SCRATCH_BYTES
    rc = lib.ktmi_moe_layer_noalloc(C.byref(desc), x.data_ptr(), tw.data_ptr(), slot.data_ptr(), T, w.top_k,
                                    x.data_ptr(), L.MODE_AUTO, L.stream_ptr(dev))
    assert rc != 0 and b"scratch" in lib.ktmi_last_error()
    del keep
