"""Each workload of the layer at its real shape on the GPU (grouped MFMA mode for the
prefill chunks, the GEMV and the MFMA decode modes for decode windows): a token sample against the oracle's
fp64 FFN over the exactly dequantised weights (relative L2 < 2e-2, cosine > 0.999), plus
tokens with no hot route exactly zero."""
import numpy as np
import pytest

from conftest import bf16_bits_of, bf16_tensor, to_dev
from helpers import dequant_w, scale_f16_fields
from oracle import gguf_ref as R

pytestmark = pytest.mark.gpu

TOL_REL_L2 = 2e-2


def _pkg():
    import kt_prefill_lend_amd._lib as L
    import kt_prefill_lend_amd.kt_gguf_hot as H
    import kt_prefill_lend_amd.synth as S

    return L, H, S


_weights = {}


def _slots(name):
    """Quantised hot slots and their dequantised fp32 values, once per workload."""
    _, _, S = _pkg()
    if name not in _weights:
        w = S.WORKLOADS[name]
        w13, w2 = S.slot_tensors(w, threads=16)
        g, d = dequant_w(w13, w2, w.types, w.hidden, w.inter)
        _weights.clear()
        _weights[name] = (w13, w2, g, d)
    return _weights[name]


def _check(dev, name, T, mode, sample_every):
    import torch

    L, H, S = _pkg()
    w = S.WORKLOADS[name]
    w13, w2, g, d = _slots(name)
    _, tw, slot, _ = S.routing(w, T)
    xb = S.activations(w, T)
    W13, W2 = to_dev(w13, dev), to_dev(w2, dev)
    desc = H.layer_desc(W13, W2, w.hidden, w.inter, w.types[0], w.types[2])
    y = H.moe_layer(desc, bf16_tensor(xb, dev), to_dev(tw, dev), to_dev(slot, dev), mode)
    torch.cuda.synchronize()
    got = R.bf16_to_f32(bf16_bits_of(y))
    sample = np.arange(0, T, sample_every)
    ref = R.ffn_reference(xb[sample], slot[sample], tw[sample], g, d)
    l2, l1, cos = R.rel_errors(got[sample], ref)
    print(f"{name} T={T}: rel L2 {l2:.2e} rel L1 {l1:.2e} cos {cos:.6f}")
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, l1, cos)
    cold = (slot < 0).all(axis=1)
    assert np.all(got[cold] == 0)


def test_q8_0_512_tokens(dev):
    L, _, _ = _pkg()
    _check(dev, "q8_0-h2048-n768-e128-k8-hot16", 512, L.MODE_AUTO, 1)


@pytest.mark.parametrize("mode", ["decode", "gemv"])
@pytest.mark.parametrize("T", [1, 4, 8, 16, 32])
def test_q4_k_decode_windows(dev, T, mode):
    L, _, _ = _pkg()
    _check(dev, "q4_k-h2048-n512-e256-k8-hot32-decode", T, L.MODE_DECODE if mode == "decode" else L.MODE_GEMV, 1)


@pytest.mark.parametrize("T", [8, 16, 25])
def test_iq3_s_decode_mode_windows(dev, T):
    """The decode mode on the IQ3_S workload at its real shape (hidden 2048, top-10: 80 / 160 /
    250 routes), where its staged rows fit; the Q8_0 and Q6_K rows of hidden 2048 do not
    (decode_mfma_fits) and those layers take the GEMV mode."""
    L, _, _ = _pkg()
    _check(dev, "iq3_s-h2048-n512-e512-k10-hot48", T, L.MODE_DECODE, 1)


@pytest.mark.parametrize("T", [2048, 32768])
def test_prefill_chunks(dev, T):
    L, _, _ = _pkg()
    _check(dev, "q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", T, L.MODE_GROUPED, max(1, T // 256))


@pytest.mark.parametrize("name,T", [("q8_0-h2048-n768-e128-k8-hot16", 4096),
                                    ("q4_k-h2048-n512-e256-k8-hot32-decode", 8192)])
def test_256_route_tiles_other_types(dev, name, T):
    """Chunks long enough for 256-route tiles (per-wave epilogue staging) with the Q8_0 GEMMs
    and with Q4_K in the down GEMM, which the headline shapes do not reach."""
    L, _, _ = _pkg()
    _check(dev, name, T, L.MODE_GROUPED, max(1, T // 96))


def test_iq3_s_16k_chunk(dev):
    L, _, _ = _pkg()
    _check(dev, "iq3_s-h2048-n512-e512-k10-hot48", 16384, L.MODE_GROUPED, 64)


class _MemExperts:
    """An expert source over pinned host banks (the streamer's reader interface: E, inter, K,
    layers(), types(l), banks(l, N, rank, p2l)). Bank row e of layer l is distinct expert
    (e + l) % D with a signature of its own: the fp16 scales of its gate rows and of its
    down rows multiplied by 2^(e // D) (an exact scaling of their dequantised values), so no
    two rows of a layer hold the same bytes and a slot or row read from the wrong place
    changes the output."""

    def __init__(self, w, D, layers):
        import torch

        import kt_prefill_lend_amd.synth as S

        self.E, self.inter, self.K, self.num_layers = w.hot, w.inter, w.hidden, layers
        self.w = w
        self.parts = [S.expert_weights(w, s, 0, 16) for s in range(D)]
        self.D = D
        N = w.inter
        self._banks = {}
        for li in range(layers):
            gate, up, down = [], [], []
            for e in range(self.E):
                w13, w2 = self.parts[self.base(li, e)]
                f = self.factor(e)
                gate.append(scale_f16_fields(w13[:N], w.types[0], f).reshape(-1))
                up.append(w13[N:].reshape(-1))
                down.append(scale_f16_fields(w2, w.types[2], f).reshape(-1))
            self._banks[li] = [torch.from_numpy(np.stack(p)).pin_memory() for p in (gate, up, down)]

    def base(self, layer_idx, e):
        return (e + layer_idx) % self.D

    def factor(self, e):
        return float(2 ** (e // self.D))

    def reference(self, layer_idx, xb, slot, tw, g, d):
        """The oracle's FFN over bank rows: row e's weights are its base expert's dequantised
        values with the gate rows and the down rows times factor(e), one row at a time."""
        N = self.inter
        ref = np.zeros((xb.shape[0], self.K), np.float64)
        for e in np.unique(slot[slot >= 0]):
            b, f = self.base(layer_idx, int(e)), np.float32(self.factor(int(e)))
            ge = g[b].copy()
            ge[:N] *= f
            ids = np.where(slot == e, 0, -1).astype(np.int32)
            ref += R.ffn_reference(xb, ids, tw, ge[None], (d[b] * f)[None])
        return ref

    def layers(self):
        return list(range(self.num_layers))

    def types(self, layer_idx):
        return self.w.types

    def banks(self, layer_idx, N, rank=0, p2l=None):
        assert N == self.inter and rank == 0 and p2l is None
        return self._banks[layer_idx]


@pytest.mark.timeout(600)
def test_streamed_large_expert_layers(dev, monkeypatch):
    """Large-expert layers (hidden 7168, intermediate 2048, 24 hot Q4_K/Q6_K experts, 6144
    tokens, 4 layers) through the reference's streamer entry points: stream_prefill_for
    (method, layer, T) and run(method, layer, dispatch_output, physical_ids), groups of 8
    experts in the two slots. Each layer against the oracle's FFN on a token sample; the
    4-layer pipeline (run_layers) equal to the per-layer runs bit for bit; one group of all
    24 experts equal to the resident layer bit for bit. Every bank row carries its own
    signature (_MemExperts), so each slot's bytes are checked where they land."""
    from types import SimpleNamespace as NS

    import torch

    import kt_prefill_lend_amd.kt_stream_prefill as SP

    L, H, S = _pkg()
    w = S.WORKLOADS["q4_k+q6_k-h7168-n2048-e256-k8-hot24-stream4"]
    T, D, nl = w.tokens[0], 3, w.layers
    print(f"config 5: quantising {D} experts, pinning {nl} banks", flush=True)
    src = _MemExperts(w, D, nl)
    H.register_source("mem://large-experts", src)
    g, d = dequant_w(np.stack([p[0] for p in src.parts]), np.stack([p[1] for p in src.parts]), w.types, w.hidden,
                     w.inter)
    print("config 5: oracle weights ready", flush=True)
    monkeypatch.setattr(SP, "STREAM_THRESHOLD", 4096)
    monkeypatch.setattr(SP, "GROUP_SIZE", 8)
    monkeypatch.setattr(SP, "_instance", None)
    monkeypatch.setattr(SP, "_failed", False)
    fl = NS(intermediate_size_per_partition=w.inter, hidden_size=w.hidden, top_k=w.top_k)

    def method(li):
        kt = NS(layer_idx=li, weight_path="mem://large-experts", num_gpu_experts=w.hot, num_layers=nl)
        return NS(kt_config=kt, num_gpu_experts=w.hot, gpu_method=NS(streams_hot_experts=True))

    assert SP.stream_prefill_for(method(0), fl, 2048) is None  # below the threshold
    st = SP.stream_prefill_for(method(0), fl, T)
    assert st is not None and st.G == 8
    inputs, outs = [], []
    sample = np.arange(0, T, 192)
    for li in range(nl):
        wl = S.small(w, index=w.index + 100 * li)  # other routing and activations per layer
        _, tw, slot, _ = S.routing(wl, T)
        xb = S.activations(wl, T)
        x, tw_d, ids_d = bf16_tensor(xb, dev), to_dev(tw, dev), to_dev(slot, dev)
        inputs.append((li, x, tw_d, ids_d))
        do = H.DispatchOutput(x, H.TopKOutput(tw_d, ids_d, None))
        y = st.run(method(li), fl, do, ids_d)
        torch.cuda.synchronize()
        got = R.bf16_to_f32(bf16_bits_of(y))
        outs.append(bf16_bits_of(y))
        ref = src.reference(li, xb[sample], slot[sample], tw[sample], g, d)
        l2, l1, cos = R.rel_errors(got[sample], ref)
        print(f"config 5 layer {li}: rel L2 {l2:.2e} rel L1 {l1:.2e} cos {cos:.6f}", flush=True)
        assert l2 < TOL_REL_L2 and cos > 0.999, (li, l2, l1, cos)
        assert np.all(got[(slot < 0).all(axis=1)] == 0)
    piped = st.run_layers(inputs)
    torch.cuda.synchronize()
    for li, y in enumerate(piped):
        assert np.array_equal(bf16_bits_of(y), outs[li]), f"pipelined layer {li} differs from its single run"
    # one group of all 24 experts == the resident layer on the same 24 slots
    one = SP.KTStreamPrefillGGUF.standalone(w.inter, w.hidden, w.top_k, w.types, group_size=w.hot, device=dev,
                                            reader=src)
    li, x, tw_d, ids_d = inputs[0]
    y1 = bf16_bits_of(one.run_tensors(0, x, tw_d, ids_d))
    gate, up, down = src._banks[0]
    W13 = torch.cat([gate.view(w.hot, w.inter, -1), up.view(w.hot, w.inter, -1)], dim=1).to(dev)
    W2 = down.view(w.hot, w.hidden, -1).to(dev)
    desc = H.layer_desc(W13, W2, w.hidden, w.inter, w.types[0], w.types[2])
    yr = bf16_bits_of(H.moe_layer(desc, x, tw_d, ids_d, L.MODE_AUTO))
    torch.cuda.synchronize()
    assert np.array_equal(y1, yr), "streamed (one group) and resident layers differ"
    one.close()
    st.close()
