"""The hybrid layer on the GPU: hot experts in GPU slots, the rest on the CPU engine through
the handoff (submit before the GPU method, sync_add after), against the composition of the
two halves (bit-exact) and the oracle's FFN over every route."""
from types import SimpleNamespace

import numpy as np
import pytest

from conftest import bf16_bits_of, bf16_tensor, to_dev
from helpers import dequant_w
from oracle import gguf_ref as R

pytestmark = pytest.mark.gpu

TOL_REL_L2 = 2e-2
E, S, N, K, TOPK = 24, 8, 256, 512, 4
TYPES = (R.GGML_Q4_K, R.GGML_Q4_K, R.GGML_Q6_K)


def _setup(dev):
    import torch

    from kt_prefill_lend_amd import gguf as G
    import kt_prefill_lend_amd.kt_cpu_moe as CM
    import kt_prefill_lend_amd.kt_gguf_hot as H

    rng = np.random.default_rng(11)
    w13 = np.stack([G.quantize_rows(rng.standard_normal((2 * N, K), dtype=np.float32) * 0.02, TYPES[0])
                    for _ in range(E)])
    w2 = np.stack([G.quantize_rows(rng.standard_normal((K, N), dtype=np.float32) * 0.02, TYPES[2]) for _ in range(E)])
    bank = [torch.from_numpy(np.ascontiguousarray(w13[:, :N].reshape(E, -1))).pin_memory(),
            torch.from_numpy(np.ascontiguousarray(w13[:, N:].reshape(E, -1))).pin_memory(),
            torch.from_numpy(np.ascontiguousarray(w2.reshape(E, -1))).pin_memory()]
    cpu = CM.KTCPUExperts(*bank, K, N, TYPES, threads=8, max_tokens=320, max_top_k=TOPK)
    W13, W2 = to_dev(w13[:S], dev), to_dev(w2[:S], dev)  # logical experts 0..S-1 resident
    desc = H.layer_desc(W13, W2, K, N, TYPES[0], TYPES[2])
    return w13, w2, cpu, (W13, W2, desc)


def _routes(T, seed):
    rng = np.random.default_rng(seed)
    logits = rng.gumbel(size=(T, E)) + np.log(np.arange(1, E + 1) ** -1.1)
    ids = np.argsort(-logits, axis=1)[:, :TOPK].astype(np.int32)
    w = rng.random((T, TOPK)).astype(np.float32)
    return ids, w / w.sum(axis=1, keepdims=True)


def test_hybrid_layer(dev):
    import torch

    import kt_prefill_lend_amd.kt_gguf_hot as H

    w13, w2, cpu, (W13, W2, desc) = _setup(dev)
    g, d = dequant_w(w13, w2, TYPES, K, N)
    # back-to-back layers, an empty one; up to 256 tokens sync_add enqueues its add before the
    # CPU side ends (it waits on the worker's completion word), the 300-token layer adds after
    for rep, T in enumerate((40, 3, 0, 300, 96, 1)):
        ids, w = _routes(T, 20 + rep)
        slot = np.where(ids < S, ids, -1).astype(np.int32)
        cold = np.where(ids < S, -1, ids).astype(np.int32)
        xb = R.bf16_bits(np.random.default_rng(rep).standard_normal((T, K)).astype(np.float32))
        x, wd = bf16_tensor(xb, dev), to_dev(w, dev)
        cpu.submit(x, to_dev(cold, dev), wd)
        y = H.moe_layer(desc, x, wd, to_dev(slot, dev))
        cpu.sync_add(y)
        torch.cuda.synchronize()
        got = bf16_bits_of(y)
        # the composition of the halves: GPU-only layer + the engine's host forward, one bf16 add
        y_gpu = R.bf16_to_f32(bf16_bits_of(H.moe_layer(desc, x, wd, to_dev(slot, dev))))
        y_cpu = R.bf16_to_f32(bf16_bits_of(cpu.forward(torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16),
                                                        torch.from_numpy(cold), torch.from_numpy(w))))
        assert np.array_equal(got, R.bf16_bits(y_gpu + y_cpu)), T
        if T:
            ref = R.ffn_reference(xb, ids, w, g, d)
            l2, _, cos = R.rel_errors(R.bf16_to_f32(got), ref)
            assert l2 < TOL_REL_L2 and cos > 0.999, (T, l2, cos)
    with pytest.raises(RuntimeError):
        cpu.sync_add(y)  # nothing submitted
    cpu.close()


def test_hot_split_apply_with_cpu_engine(dev):
    """The wrapper's hot-cache branch with the CPU engine as its CPU side."""
    import torch

    import kt_prefill_lend_amd.kt_ep_wrapper as W
    import kt_prefill_lend_amd.kt_gguf_hot as H

    w13, w2, cpu, (W13, W2, desc) = _setup(dev)
    log2slot = torch.tensor([s if s < S else -1 for s in range(E)], dtype=torch.int32, device=dev)
    log2cpu = torch.tensor([-1 if s < S else s for s in range(E)], dtype=torch.int32, device=dev)
    cache = SimpleNamespace(route=lambda li, ids: (log2slot[ids.long()], log2cpu[ids.long()]))
    gpu = SimpleNamespace(apply=lambda layer, do: H.StandardCombineInput(
        hidden_states=H.moe_layer(desc, do.hidden_states, do.topk_output.topk_weights, do.topk_output.topk_ids)))
    T = 32
    ids, w = _routes(T, 5)
    xb = R.bf16_bits(np.random.default_rng(9).standard_normal((T, K)).astype(np.float32))
    do = H.DispatchOutput(bf16_tensor(xb, dev), H.TopKOutput(to_dev(w, dev), to_dev(ids, dev), None))
    y = W.hot_split_apply(cache, 0, gpu, None, do, cpu=cpu)
    torch.cuda.synchronize()
    g, d = dequant_w(w13, w2, TYPES, K, N)
    l2, _, cos = R.rel_errors(R.bf16_to_f32(bf16_bits_of(y)), R.ffn_reference(xb, ids, w, g, d))
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, cos)
    cpu.close()


def test_add_gives_up_past_its_bound(dev):
    """A decode window whose CPU side takes longer than the add's wait bound (forced from the
    host: a 200 us bound, one CPU thread, 256 tokens of cold routes): every block of the add
    stops waiting and exits normally, the layer's rows become NaN, sync_add raises, and the
    engine serves the next layer correctly with the default bound."""
    import torch

    import kt_prefill_lend_amd.kt_cpu_moe as CM

    w13, w2, cpu8, _ = _setup(dev)
    cpu8.close()
    bank = [torch.from_numpy(np.ascontiguousarray(w13[:, :N].reshape(E, -1))).pin_memory(),
            torch.from_numpy(np.ascontiguousarray(w13[:, N:].reshape(E, -1))).pin_memory(),
            torch.from_numpy(np.ascontiguousarray(w2.reshape(E, -1))).pin_memory()]
    cpu = CM.KTCPUExperts(*bank, K, N, TYPES, threads=1, max_tokens=256, max_top_k=TOPK)
    T = 256
    ids, w = _routes(T, 77)
    xb = R.bf16_bits(np.random.default_rng(77).standard_normal((T, K)).astype(np.float32))
    x, wd, ids_d = bf16_tensor(xb, dev), to_dev(w, dev), to_dev(ids, dev)
    t0 = __import__("time").perf_counter()
    cpu.forward(torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16), torch.from_numpy(ids), torch.from_numpy(w))
    cpu_ms = (__import__("time").perf_counter() - t0) * 1e3
    assert cpu_ms > 1.0, cpu_ms  # the CPU side outlasts the bound by a wide margin
    cpu.set_add_wait(200)
    y = torch.zeros((T, K), dtype=torch.bfloat16, device=dev)
    cpu.submit(x, ids_d, wd)
    with pytest.raises(RuntimeError, match="stopped waiting"):
        cpu.sync_add(y)
    torch.cuda.synchronize()
    assert torch.isnan(y.float()).all()
    cpu.set_add_wait(10_000_000)
    y = torch.zeros((T, K), dtype=torch.bfloat16, device=dev)
    cpu.submit(x, ids_d, wd)
    cpu.sync_add(y)
    torch.cuda.synchronize()
    y_cpu = cpu.forward(torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16), torch.from_numpy(ids),
                        torch.from_numpy(w))
    # out starts at zero: the add gives bf16(0 + cpu) (+0 where the CPU side gave -0)
    assert np.array_equal(bf16_bits_of(y), R.bf16_bits(R.bf16_to_f32(bf16_bits_of(y_cpu)) + np.float32(0)))
    with pytest.raises(RuntimeError):
        cpu.set_add_wait(0)
    cpu.close()
