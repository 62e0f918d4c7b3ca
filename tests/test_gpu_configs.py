"""Each workload of the layer at its real shape on the GPU (grouped MFMA mode for the
prefill chunks, fused GEMV mode for decode windows): a token sample against the oracle's
fp64 FFN over the exactly dequantised weights (relative L2 < 2e-2, cosine > 0.999), plus
tokens with no hot route exactly zero."""
import numpy as np
import pytest

from conftest import bf16_bits_of, bf16_tensor, to_dev
from helpers import dequant_w
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


@pytest.mark.parametrize("T", [1, 4, 8, 16])
def test_q4_k_decode_windows(dev, T):
    L, _, _ = _pkg()
    _check(dev, "q4_k-h2048-n512-e256-k8-hot32-decode", T, L.MODE_AUTO, 1)


@pytest.mark.parametrize("T", [2048, 32768])
def test_prefill_chunks(dev, T):
    L, _, _ = _pkg()
    _check(dev, "q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", T, L.MODE_GROUPED, max(1, T // 256))


def test_iq3_s_16k_chunk(dev):
    L, _, _ = _pkg()
    _check(dev, "iq3_s-h2048-n512-e512-k10-hot48", 16384, L.MODE_GROUPED, 64)
