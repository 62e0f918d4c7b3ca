"""The hot-expert registry end to end on the GPU: slots filled from a GGUF file through the
hot method, routing, the layer against the oracle's FFN over the residents, swap rounds that
copy experts from the pinned banks, and the streamer reading its banks from the same GGUF."""
from types import SimpleNamespace

import numpy as np
import pytest

from conftest import bf16_bits_of, bf16_tensor, to_dev
from helpers import dequant_w, make_expert_gguf
from oracle import gguf_ref as R

pytestmark = pytest.mark.gpu

TOL_REL_L2 = 2e-2
E, N, K, L, S, TOPK = 16, 256, 512, 2, 6, 4
TYPES = (R.GGML_Q4_K, R.GGML_Q4_K, R.GGML_Q6_K)


def _routing(T, seed, hot_bias=None):
    rng = np.random.default_rng(seed)
    logits = rng.gumbel(size=(T, E)) + (np.log(np.arange(1, E + 1) ** -1.1) if hot_bias is None else hot_bias)
    ids = np.argsort(-logits, axis=1)[:, :TOPK].astype(np.int32)
    sel = np.take_along_axis(logits, ids, axis=1)
    w = np.exp(sel - sel.max(axis=1, keepdims=True))
    return ids, (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


def _layer_check(dev, method, layer, x_bits, ids, tw, slot_np):
    import torch

    import kt_prefill_lend_amd.kt_gguf_hot as H

    y = method.apply(layer, H.DispatchOutput(bf16_tensor(x_bits, dev), H.TopKOutput(
        to_dev(tw, dev), torch.from_numpy(slot_np).to(dev), None))).hidden_states
    torch.cuda.synchronize()
    got = R.bf16_to_f32(bf16_bits_of(y))
    g, d = dequant_w(layer.w13_qweight.cpu().numpy(), layer.w2_qweight.cpu().numpy(), TYPES, K, N)
    ref = R.ffn_reference(x_bits, slot_np, tw, g, d)
    l2, _, cos = R.rel_errors(got, ref)
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, cos)


def test_gguf_slots_route_and_swaps(dev, tmp_path, monkeypatch):
    import torch

    import kt_prefill_lend_amd.kt_gguf_hot as H
    import kt_prefill_lend_amd.kt_hot_cache as C

    p = tmp_path / "experts.gguf"
    raw = make_expert_gguf(p, L, E, N, K, TYPES)
    monkeypatch.setattr(C, "ENABLED", True)
    monkeypatch.setattr(C, "INTERVAL", 1)
    monkeypatch.setattr(C, "OWN_BANKS", "own")
    monkeypatch.setattr(C, "_cache", None)
    methods, layers = [], []
    cache = None
    for li in range(L):
        kt = SimpleNamespace(weight_path=str(p), num_gpu_experts=S, layer_idx=li, num_layers=L)
        layer = SimpleNamespace()
        layer.register_parameter = lambda name, prm, _l=layer: setattr(_l, name, prm)
        m = H.KTGGUFHotExpertsMethod(kt, layer)
        m.create_weights(layer, S, K, N, torch.bfloat16)
        m.process_weights_after_loading(layer)  # logical experts 0..S-1 from the GGUF
        methods.append(m)
        layers.append(layer)
        cache = C.register(m, layer, num_layers=L, num_experts=E)
    assert cache is not None and cache.check_tables() == ""
    assert np.array_equal(layers[1].w13_qweight[3, :N].cpu().numpy(), raw[(1, "gate")][3])

    T = 48
    xb = R.bf16_bits(np.random.default_rng(5).standard_normal((T, K)).astype(np.float32))
    for li in range(L):
        ids, tw = _routing(T, 10 + li)
        slot_ids, cpu_ids = cache.route(li, to_dev(ids, dev))
        slot_np = slot_ids.cpu().numpy()
        assert np.array_equal(slot_np, np.where(ids < S, ids, -1))
        assert np.array_equal(cpu_ids.cpu().numpy(), np.where(ids < S, -1, ids))
        _layer_check(dev, methods[li], layers[li], xb, ids, tw, slot_np)

    # routes that favour experts 10..15: two policy rounds (counts are read one round late)
    bias = np.full(E, -3.0)
    bias[10:] = 2.0
    for rnd in range(3):
        for li in range(L):
            cache.route(li, to_dev(_routing(256, 100 + rnd * 7 + li, bias)[0], dev))
        torch.cuda.synchronize()
        cache.before_forward(True)
        torch.cuda.synchronize()
    assert cache.swaps > 0 and cache.check_tables() == ""
    for li in range(L):
        res = cache.resident[li].tolist()
        assert sum(e >= 10 for e in res) >= 3, res
        for s_, e in enumerate(res):
            assert np.array_equal(layers[li].w13_qweight[s_, N:].cpu().numpy(), raw[(li, "up")][e])
            assert np.array_equal(layers[li].w2_qweight[s_].cpu().numpy(), raw[(li, "down")][e])
        ids, tw = _routing(T, 30 + li, bias)
        slot_np = cache.route(li, to_dev(ids, dev))[0].cpu().numpy()
        log2slot = cache.log2slot_cpu[li].numpy()
        assert np.array_equal(slot_np, log2slot[ids])
        _layer_check(dev, methods[li], layers[li], xb, ids, tw, slot_np)
    monkeypatch.setattr(C, "_cache", None)


def test_streamer_banks_from_gguf(dev, tmp_path, monkeypatch):
    """A streamed layer over every expert with the banks read from the GGUF (TP rank 1 of
    2), through the reference's entry points (stream_prefill_for, run with the wrapper's
    method/layer/dispatch_output), against the oracle's FFN over the same slices."""
    import torch

    import kt_prefill_lend_amd.kt_gguf_hot as H
    import kt_prefill_lend_amd.kt_stream_prefill as SP

    from types import SimpleNamespace as NS

    import kt_prefill_lend_amd.sglang_env as SE

    p = tmp_path / "tp.gguf"
    make_expert_gguf(p, 1, E, N, K, TYPES, world=2)
    rd = H._reader(str(p))
    # the reference wrapper's objects: TP rank 1 of 2, the GPU method streams its hot experts
    monkeypatch.setattr(SE, "tp_rank_world", lambda: (1, 2))
    monkeypatch.setattr(SP, "STREAM_THRESHOLD", 32)
    monkeypatch.setattr(SP, "GROUP_SIZE", 4)
    monkeypatch.setattr(SP, "_instance", None)
    monkeypatch.setattr(SP, "_failed", False)
    kt = NS(layer_idx=0, weight_path=str(p), num_gpu_experts=2, num_layers=1)
    method = NS(kt_config=kt, num_gpu_experts=2, gpu_method=NS(streams_hot_experts=True))
    fl = NS(intermediate_size_per_partition=N, hidden_size=K, top_k=TOPK)
    T = 64
    st = SP.stream_prefill_for(method, fl, T)
    assert st is not None and st.rank == 1
    ids, tw = _routing(T, 3)
    xb = R.bf16_bits(np.random.default_rng(9).standard_normal((T, K)).astype(np.float32))
    x, ids_d = bf16_tensor(xb, dev), to_dev(ids, dev)
    y = st.run(method, fl, H.DispatchOutput(x, H.TopKOutput(to_dev(tw, dev), ids_d, None)), ids_d)
    torch.cuda.synchronize()
    got = R.bf16_to_f32(bf16_bits_of(y))
    all_e = list(range(E))
    w13 = torch.cat([rd.slice(0, "gate", N, 1, all_e), rd.slice(0, "up", N, 1, all_e)], dim=1).numpy()
    w2 = rd.slice(0, "down", N, 1, all_e).numpy()
    g, d = dequant_w(w13, w2, TYPES, K, N)
    ref = R.ffn_reference(xb, ids, tw, g, d)
    l2, _, cos = R.rel_errors(got, ref)
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, cos)
    st.close()
