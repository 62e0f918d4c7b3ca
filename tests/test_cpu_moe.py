"""The product CPU expert engine (libktmi ktmi_cpu_moe_*) against the oracle's C
restatement of kt-kernel's forward_many: bit-identical bf16 outputs for every weight type,
both integer kernels (AVX-512 VNNI and portable) and any thread count; cold ids ignored;
and against the fp64 FFN within the layer tolerance."""
import numpy as np
import pytest
import torch

from helpers import dequant_w
from oracle import cpu_moe as O
from oracle import gguf_ref as R

TOL_REL_L2 = 2e-2
CASES = [  # (gate/up type, down type, hidden, inter)
    (R.GGML_Q8_0, R.GGML_Q8_0, 512, 256),
    (R.GGML_Q4_K, R.GGML_Q6_K, 512, 256),
    (R.GGML_Q4_K, R.GGML_Q4_K, 768, 512),
    (R.GGML_IQ3_S, R.GGML_IQ3_S, 512, 256),
]


def _experts(t13, t2, K, N, E, seed):
    from kt_prefill_lend_amd import gguf as G

    rng = np.random.default_rng(seed)
    w13 = np.stack([np.concatenate([G.quantize_rows(rng.standard_normal((N, K), dtype=np.float32) * 0.02, t13),
                                    G.quantize_rows(rng.standard_normal((N, K), dtype=np.float32) * 0.02, t13)])
                    for _ in range(E)])
    w2 = np.stack([G.quantize_rows(rng.standard_normal((K, N), dtype=np.float32) * 0.02, t2) for _ in range(E)])
    return w13, w2


def _engine(w13, w2, K, N, types, **kw):
    import kt_prefill_lend_amd.kt_cpu_moe as CM

    E = w13.shape[0]
    gate = torch.from_numpy(np.ascontiguousarray(w13[:, :N].reshape(E, -1)))
    up = torch.from_numpy(np.ascontiguousarray(w13[:, N:].reshape(E, -1)))
    down = torch.from_numpy(np.ascontiguousarray(w2.reshape(E, -1)))
    return CM.KTCPUExperts(gate, up, down, K, N, types, **kw)


def _inputs(T, k, E, K, seed):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    ids[rng.random((T, k)) < 0.3] = -1   # residents (on the GPU)
    ids[0, :] = -1                       # a token with nothing on the CPU
    ids[1, 0] = E + 3                    # outside the bank
    w = rng.random((T, k)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    x = R.bf16_bits(rng.standard_normal((T, K)).astype(np.float32))
    return ids, w, x


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1]}")
def test_engine_matches_oracle_bitwise(case, monkeypatch):
    t13, t2, K, N = case
    E, T, k = 6, 9, 4
    w13, w2 = _experts(t13, t2, K, N, E, seed=t13 * 100 + t2)
    ids, w, x = _inputs(T, k, E, K, seed=t2)
    ref = O.forward(x, ids, w, w13, w2, t13, t2, N, threads=2)
    ref_bits = R.bf16_bits(ref)
    outs = {}
    for isa in ("native", "scalar"):
        if isa == "scalar":
            monkeypatch.setenv("KTMI_CPU_ISA", "scalar")
        for threads in (1, 5):
            eng = _engine(w13, w2, K, N, (t13, t13, t2), threads=threads)
            if isa == "scalar":
                assert eng.isa == "scalar"
            got = eng.forward(torch.from_numpy(x.view(np.int16)).view(torch.bfloat16), torch.from_numpy(ids),
                              torch.from_numpy(w))
            bits = got.view(torch.int16).numpy().view(np.uint16)
            assert np.array_equal(bits, ref_bits), (isa, threads, np.argwhere(bits != ref_bits)[:5])
            outs[(isa, threads)] = bits
            eng.close()
    assert np.all(outs[("native", 1)][0] == 0)  # no CPU route: zero row
    # against the fp64 FFN over the same experts (CPU routes only)
    g, d = dequant_w(w13, w2, (t13, t13, t2), K, N)
    cpu_ids = np.where((ids >= 0) & (ids < E), ids, -1)
    l2, _, cos = R.rel_errors(R.bf16_to_f32(ref_bits), R.ffn_reference(x, cpu_ids, w, g, d))
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, cos)


def test_engine_rejects_bad_setup():
    import kt_prefill_lend_amd.kt_cpu_moe as CM

    z = torch.zeros((2, 16), dtype=torch.uint8)
    with pytest.raises(RuntimeError):
        CM.KTCPUExperts(z, z, z, 512, 256, (R.GGML_Q4_K, R.GGML_Q4_K, 3))  # type without a CPU kernel
    with pytest.raises(RuntimeError):
        CM.KTCPUExperts(z, z, z, 512, 256, (R.GGML_Q4_K, R.GGML_Q4_K, R.GGML_Q6_K))  # part bytes
    with pytest.raises(RuntimeError):
        CM.KTCPUExperts(z, z, z, 512, 256, (R.GGML_Q4_K, R.GGML_Q8_0, R.GGML_Q6_K))  # gate/up types
