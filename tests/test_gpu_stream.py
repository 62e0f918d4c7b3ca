"""The layer-weight streamer through the C ABI: groups of experts staged from pinned host
banks into double-buffered device slots while the grouped layer runs on the other slot."""
from dataclasses import replace

import numpy as np
import pytest

from conftest import bf16_bits_of, bf16_tensor, to_dev
from helpers import dequant_w
from oracle import gguf_ref as R

pytestmark = pytest.mark.gpu


def _pkg():
    import kt_prefill_lend_amd._lib as L
    import kt_prefill_lend_amd.kt_gguf_hot as H
    import kt_prefill_lend_amd.kt_stream_prefill as SP
    import kt_prefill_lend_amd.synth as S

    return L, H, SP, S


def _layers(n_layers, T, E=6):
    """Per layer: workload, x bits, weights, ids (expert index in [0, E) or -1), w13, w2."""
    _, _, _, S = _pkg()
    base = S.WORKLOADS["q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill"]
    w = replace(base, hidden=512, inter=256, hot=E, experts=24)
    out = []
    for layer in range(n_layers):
        wl = replace(w, index=w.index + 100 * layer)  # another seed per layer
        _, tw, slot, _ = S.routing(wl, T)
        xb = S.activations(wl, T)
        w13, w2 = S.slot_tensors(wl, layer=layer)
        out.append((wl, xb, tw, slot, w13, w2))
    return out


def _resident(dev, wl, xb, tw, slot, w13, w2):
    import torch

    L, H, _, _ = _pkg()
    W13, W2 = to_dev(w13, dev), to_dev(w2, dev)  # the descriptor holds raw pointers: keep these alive
    desc = H.layer_desc(W13, W2, wl.hidden, wl.inter, wl.types[0], wl.types[2])
    y = H.moe_layer(desc, bf16_tensor(xb, dev), to_dev(tw, dev), to_dev(slot, dev), L.MODE_AUTO)
    torch.cuda.synchronize()
    return bf16_bits_of(y)


def _d2h(ptr, nbytes):
    """bytes of device memory at ptr (hipMemcpy through libamdhip64)."""
    import ctypes as C

    h = C.CDLL("libamdhip64.so")
    h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    out = np.empty(nbytes, np.uint8)
    assert h.hipDeviceSynchronize() == 0
    assert h.hipMemcpy(out.ctypes.data, ptr, nbytes, 2) == 0  # hipMemcpyDeviceToHost
    return out


def test_staged_slot_layout(dev):
    """A staged group is the slot layout the layer reads: w13 [n, 2N, rb] with expert i's
    gate rows then up rows, w2 [n, K, rb2], for experts [first, first + n) of the bank."""
    import torch

    _, _, SP, _ = _pkg()
    (wl, xb, tw, slot, w13, w2), = _layers(1, 8)
    st = SP.KTStreamPrefillGGUF.standalone(wl.inter, wl.hidden, wl.top_k, wl.types, group_size=4, device=dev)
    st.set_bank(0, SP.Bank.from_slot_rows(torch.from_numpy(w13), torch.from_numpy(w2), wl.inter, wl.types))
    for sl, first, n in ((0, 0, 4), (1, 4, 2), (0, 1, 3)):
        st._stage(sl, 0, first, n)
        st.sync_copies()
        p13, p2 = st.dev.slots[sl]
        got13 = _d2h(p13, n * w13[0].nbytes).reshape(n, *w13.shape[1:])
        got2 = _d2h(p2, n * w2[0].nbytes).reshape(n, *w2.shape[1:])
        assert np.array_equal(got13, w13[first:first + n]), (sl, first, n)
        assert np.array_equal(got2, w2[first:first + n]), (sl, first, n)
    st.close()


@pytest.mark.parametrize("T", [40, 8], ids=["grouped", "decode"])
def test_one_group_equals_resident_layer(dev, T):
    """All experts in one group: the streamed layer is the resident layer, bit for bit."""
    import torch

    _, _, SP, _ = _pkg()
    (wl, xb, tw, slot, w13, w2), = _layers(1, T)
    st = SP.KTStreamPrefillGGUF.standalone(wl.inter, wl.hidden, wl.top_k, wl.types, group_size=wl.hot, device=dev)
    st.set_bank(0, SP.Bank.from_slot_rows(torch.from_numpy(w13), torch.from_numpy(w2), wl.inter, wl.types))
    y = st.run_tensors(0, bf16_tensor(xb, dev), to_dev(tw, dev), to_dev(slot, dev))
    torch.cuda.synchronize()
    got, res = bf16_bits_of(y), _resident(dev, wl, xb, tw, slot, w13, w2)
    g, d = dequant_w(w13, w2, wl.types, wl.hidden, wl.inter)
    ref = R.ffn_reference(xb, slot, tw, g, d)
    e_got = R.rel_errors(R.bf16_to_f32(got), ref)
    e_res = R.rel_errors(R.bf16_to_f32(res), ref)
    diff_rows = np.nonzero((got != res).any(axis=1))[0]
    assert diff_rows.size == 0, (e_got, e_res, diff_rows[:20])
    assert e_got[0] < 2e-2 and e_res[0] < 2e-2
    assert np.array_equal(got, res)
    st.close()


def test_groups_and_layers_pipeline(dev):
    """Groups of 4 of 6 experts (two slots in turn) over three layers: each layer's sum of
    group outputs against the fp64 FFN, run_layers (one pipeline over all layers) equal to
    per-layer runs bit for bit, and a streamer slot reused after its release."""
    import torch

    _, _, SP, _ = _pkg()
    layers = _layers(3, 40)
    wl0 = layers[0][0]
    st = SP.KTStreamPrefillGGUF.standalone(wl0.inter, wl0.hidden, wl0.top_k, wl0.types, group_size=4, device=dev)
    for i, (wl, xb, tw, slot, w13, w2) in enumerate(layers):
        st.set_bank(i, SP.Bank.from_slot_rows(torch.from_numpy(w13), torch.from_numpy(w2), wl.inter, wl.types))
    singles = []
    for i, (wl, xb, tw, slot, w13, w2) in enumerate(layers):
        y = st.run_tensors(i, bf16_tensor(xb, dev), to_dev(tw, dev), to_dev(slot, dev))
        torch.cuda.synchronize()
        got = bf16_bits_of(y)
        singles.append(got)
        g, d = dequant_w(w13, w2, wl.types, wl.hidden, wl.inter)
        ref = R.ffn_reference(xb, slot, tw, g, d)
        l2, _, cos = R.rel_errors(R.bf16_to_f32(got), ref)
        assert l2 < 2e-2 and cos > 0.999, (i, l2, cos)
    items = [(i, bf16_tensor(xb, dev), to_dev(tw, dev), to_dev(slot, dev)) for i, (wl, xb, tw, slot, _, _) in
             enumerate(layers)]
    outs = st.run_layers(items)
    torch.cuda.synchronize()
    for i, y in enumerate(outs):
        assert np.array_equal(bf16_bits_of(y), singles[i]), i
    st.close()


def test_streamer_rejects_bad_groups(dev):
    import torch

    L, _, SP, _ = _pkg()
    (wl, xb, tw, slot, w13, w2), = _layers(1, 8)
    st = SP.KTStreamPrefillGGUF.standalone(wl.inter, wl.hidden, wl.top_k, wl.types, group_size=4, device=dev)
    st.set_bank(0, SP.Bank.from_slot_rows(torch.from_numpy(w13), torch.from_numpy(w2), wl.inter, wl.types))
    with pytest.raises(RuntimeError, match="group of at most"):
        st._stage(0, 0, 0, 5)
    with pytest.raises(RuntimeError, match="experts"):
        st._stage(0, 0, 4, 4)
    st.close()


def test_selftest_logs_agreement(dev, monkeypatch, capsys):
    """KT_GPU_STREAM_SELFTEST=2 (P:40821-40853, called at P:40986-40987): the first streamed
    layer's run() recomputes the streamed experts' share in fp32 and logs the agreement;
    the logged relative L2 is below the 2e-2 bar, and the same check on a damaged output
    reports the damage (it is not vacuous)."""
    import re
    from types import SimpleNamespace as NS

    import torch

    L, H, SP, _ = _pkg()
    (wl, xb, tw, slot, w13, w2), = _layers(1, 40)
    monkeypatch.setattr(SP, "SELFTEST", "2")
    st = SP.KTStreamPrefillGGUF.standalone(wl.inter, wl.hidden, wl.top_k, wl.types, group_size=4, device=dev)
    st.set_bank(0, SP.Bank.from_slot_rows(torch.from_numpy(w13), torch.from_numpy(w2), wl.inter, wl.types))
    x, tw_d, ids_d = bf16_tensor(xb, dev), to_dev(tw, dev), to_dev(slot, dev)
    method = NS(kt_config=NS(layer_idx=0), num_gpu_experts=0, gpu_method=NS(streams_hot_experts=True))
    do = H.DispatchOutput(x, H.TopKOutput(tw_d, ids_d, None))
    acc = st.run(method, None, do, ids_d)
    torch.cuda.synchronize()
    log = capsys.readouterr().out
    m = re.search(r"self-check of layer 0 .*rel L2 ([0-9.eE+-]+), cos ([0-9.eE+-]+)", log)
    assert m, log
    rel, cos = float(m.group(1)), float(m.group(2))
    assert rel < 2e-2 and cos > 0.999, log
    # once per process: a second run does not check again
    st.run(method, None, do, ids_d)
    torch.cuda.synchronize()
    assert "self-check" not in capsys.readouterr().out
    rel_bad, _ = st._reference_check(0, x, ids_d, tw_d, acc * 0.5, 0)
    assert 0.45 < rel_bad < 0.55, rel_bad
    st.close()
