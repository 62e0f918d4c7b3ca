"""Host-side tests (no GPU): the C-ABI library loads and exports every declared symbol,
host quantisers round-trip through the oracle, the synthetic workloads, the hot cache's
host logic and the CPU-mask hook."""
import re
from pathlib import Path

import numpy as np
import pytest

from helpers import TYPES
from oracle import gguf_ref as R

ROOT = Path(__file__).resolve().parent.parent


def _declared_symbols():
    txt = (ROOT / "include" / "ktmi.h").read_text()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(ktmi_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    from kt_prefill_lend_amd import _lib

    L = _lib.lib()
    decl = _declared_symbols()
    assert len(decl) >= 15
    for name in decl:
        assert hasattr(L, name), name
    assert set(decl) == set(_lib.SIGNATURES), set(decl) ^ set(_lib.SIGNATURES)


def test_pure_host_entry_points():
    from kt_prefill_lend_amd import _lib

    L = _lib.lib()
    assert L.ktmi_version() >= 100
    for t in TYPES:
        assert L.ktmi_type_supported(t) == 1
        assert L.ktmi_row_bytes(2048, t) == R.row_bytes(2048, t)
    assert L.ktmi_type_supported(23) == 0
    assert L.ktmi_row_bytes(100, 12) == 0
    assert L.ktmi_q8_1_row_bytes(700) == 1024 // 32 * 36
    assert L.ktmi_moe_a8_vec_workspace(2048, 3) == 3 * 2048 // 32 * 36
    # argument errors are reported before any device work
    rc = L.ktmi_dequant_experts(0, 0, 23, 1, 1, 256, 0, 0, 0)
    assert rc == -2 and b"23" in L.ktmi_last_error()
    rc = L.ktmi_moe_a8_vec(0, 2, 100, 0, 0, 0, 1, 12, 1, 1, 0, 0, 0, 0, 0)
    assert rc == -1 and b"block size" in L.ktmi_last_error()


def test_layer_workspace_sizes():
    from kt_prefill_lend_amd import _lib

    L = _lib.lib()
    d = _lib.ktmi_layer(hidden=2048, inter=512, n_slots=40, type13=12, type2=14)
    assert L.ktmi_moe_layer_mode(d, 4, 8) == _lib.MODE_GEMV
    assert L.ktmi_moe_layer_mode(d, 16384, 8) == _lib.MODE_GROUPED
    g = L.ktmi_moe_layer_workspace(d, 16384, 8, _lib.MODE_GROUPED)
    R_ = 16384 * 8
    assert g >= R_ * (512 + 2048) * 2 + R_ * 4
    assert L.ktmi_moe_layer(d, 0, 0, 0, 1, 8, 0, 0, 0, 0, 0) == -1  # null weights


@pytest.mark.parametrize("t", TYPES)
def test_host_quantiser_round_trip(t):
    from kt_prefill_lend_amd import gguf

    rng = np.random.default_rng(30 + t)
    x = (rng.standard_normal((8, 512)) * 0.02).astype(np.float32)
    q = gguf.quantize_rows(x, t, threads=2)
    assert q.shape == (8, R.row_bytes(512, t))
    y = R.dequant_rows(q, t, 512)
    rel = np.linalg.norm(y - x) / np.linalg.norm(x)
    bound = {R.GGML_Q8_0: 0.01, R.GGML_Q4_K: 0.12, R.GGML_Q6_K: 0.04, R.GGML_IQ3_S: 0.25}[t]
    assert rel < bound, rel
    # deterministic and thread-count independent
    assert np.array_equal(q, gguf.quantize_rows(x, t, threads=1))


def test_iq3s_quantiser_picks_nearest_codebook_point():
    from kt_prefill_lend_amd import gguf

    grid = R.iq3s_grid().view(np.uint8).reshape(512, 4).astype(np.float64)
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((1, 256)) * 0.02).astype(np.float32)
    q = gguf.quantize_rows(x, R.GGML_IQ3_S, threads=1)
    d, nib, g, neg = R._iq3_s_fields(q.reshape(1, 110))
    db = d[0].astype(np.float64) * (1 + 2 * nib[0])
    v = np.abs(x[0]).astype(np.float64) / db
    for grp in range(64):
        vv = v[4 * grp:4 * grp + 4]
        best = ((grid - vv) ** 2).sum(axis=1).min()
        got = ((g[0, 4 * grp:4 * grp + 4] - vv) ** 2).sum()
        assert got <= best * (1 + 1e-5) + 1e-9
    assert np.array_equal(neg[0] == 1, x[0] < 0)


def test_synthetic_workload_recipe():
    import kt_prefill_lend_amd.synth as S

    w = S.WORKLOADS["q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill"]
    ids, tw, slot, hot = S.routing(w, 2048)
    assert ids.shape == (2048, 8) and ids.dtype == np.int32
    assert all(len(set(r)) == 8 for r in ids.tolist())  # distinct experts per token
    assert np.allclose(tw.sum(axis=1), 1.0, atol=1e-5) and np.all(tw > 0)
    assert np.all(np.diff(tw, axis=1) <= 1e-7)  # descending logits -> descending weights
    p, perm = S.popularity(w)
    assert np.array_equal(hot, perm[:40]) and np.all(p[hot].min() >= np.delete(p, hot).max())
    hot_frac = (slot >= 0).mean()
    assert 0.6 < hot_frac < 0.8  # ~0.70 at this Zipf exponent
    assert np.array_equal(slot >= 0, np.isin(ids, hot))
    a, b = S.routing(w, 64)[0], S.routing(w, 64)[0]
    assert np.array_equal(a, b)
    x = S.activations(w, 4)
    assert x.dtype == np.uint16 and x.shape == (4, 2048)


def test_hot_cache_host_logic():
    import torch

    import kt_prefill_lend_amd.kt_hot_cache as C

    c = C.HotCache(2, 10, 3, "cpu")
    c.seed()
    assert c.check_tables() == ""
    assert c.log2slot_cpu[0, :3].tolist() == [0, 1, 2] and c.log2cpu_cpu[0, :4].tolist() == [-1, -1, -1, 3]
    c._set(1, 0, 7)
    c.push_tables()
    assert c.check_tables() == ""
    assert c.log2slot_cpu[1, 7] == 0 and c.log2cpu_cpu[1, 0] == 0
    counts = torch.zeros(2, 10)
    counts[0, 5] = 10.0  # hot non-resident
    counts[0, 1] = 1.0   # cold resident
    counts[0, 0] = 9.0
    counts[0, 2] = 9.5
    plan = c.plan_swaps(counts)
    assert plan[0] == (0, 1, 5)
    assert all(li == 0 for li, _, _ in plan)
    # the margin test: 5 replaces 1 (10 > 1.5*1) but nothing replaces 0 (9) with a weaker candidate
    assert len(plan) == 1
    # a broken table is reported
    c.log2cpu_cpu[0, 5] = -1
    assert c.check_tables() != ""


def test_cpu_mask_hook(monkeypatch):
    import kt_prefill_lend_amd.kt_ep_wrapper as W

    m = W._prefix_gpu_experts_mask(8, 3)
    assert m.tolist() == [True] * 3 + [False] * 5
    assert not W.cpu_experts_mask(8, 3, hot_enabled=True).any()
    assert W.cpu_experts_mask(8, 3, hot_enabled=False).sum() == 3
    monkeypatch.setenv("KT_HOT_CPU_PREFIX_MASK", "1")
    assert W.cpu_experts_mask(8, 3, hot_enabled=True).sum() == 3
    with pytest.raises(ValueError):
        W._prefix_gpu_experts_mask(4, 5)
    import torch

    ids = torch.tensor([[0, 5], [2, 3]])
    assert W.mask_cpu_expert_ids(ids, 3).tolist() == [[0, -1], [2, -1]]


def test_stream_bank_validation_and_threshold(monkeypatch):
    import torch

    import kt_prefill_lend_amd.kt_stream_prefill as SP

    N, K = 256, 512
    types = (12, 12, 14)
    pg, pu, pd = SP.part_bytes(types, N, K)
    assert (pg, pu, pd) == (N * (K // 256) * 144, N * (K // 256) * 144, K * (N // 256) * 210)
    ok = SP.Bank(torch.zeros((3, pg), dtype=torch.uint8), torch.zeros((3, pu), dtype=torch.uint8),
                 torch.zeros((3, pd), dtype=torch.uint8), types)
    assert ok.n_experts == 3
    with pytest.raises(RuntimeError):
        SP.Bank(torch.zeros((3, pg), dtype=torch.int16), torch.zeros((3, pu), dtype=torch.uint8),
                torch.zeros((3, pd), dtype=torch.uint8), types)
    with pytest.raises(RuntimeError):
        SP.Bank(torch.zeros((3, pg), dtype=torch.uint8), torch.zeros((2, pu), dtype=torch.uint8),
                torch.zeros((3, pd), dtype=torch.uint8), types)
    with pytest.raises(RuntimeError, match="gate/up types"):
        SP.Bank(torch.zeros((3, pg), dtype=torch.uint8), torch.zeros((3, pu), dtype=torch.uint8),
                torch.zeros((3, pd), dtype=torch.uint8), (12, 14, 14))
    monkeypatch.setattr(SP, "STREAM_THRESHOLD", 0)
    assert SP.stream_prefill_for(N, K, 8, types, 100000) is None
    monkeypatch.setattr(SP, "STREAM_THRESHOLD", 4096)
    monkeypatch.setattr(SP, "preallocate", lambda *a, **k: "streamer")
    assert SP.stream_prefill_for(N, K, 8, types, 1024) is None
    assert SP.stream_prefill_for(N, K, 8, types, 8192) == "streamer"


def test_layer_argument_errors_before_device_work():
    """The layer entry point rejects bad arguments with a status and a message before it
    touches the device (the pointers below are never dereferenced): a short workspace,
    misaligned activations, a forced GEMV mode past its route limit, a chunk past the
    activations' 4 GiB buffer range."""
    from kt_prefill_lend_amd import _lib

    L = _lib.lib()
    d = _lib.ktmi_layer(hidden=2048, inter=512, n_slots=40, type13=12, type2=14, w13=1 << 20, w2=2 << 20)
    p, big = 1 << 24, 1 << 62
    need = L.ktmi_moe_layer_workspace(d, 4096, 8, _lib.MODE_GROUPED)
    rc = L.ktmi_moe_layer(d, p, p, p, 4096, 8, p, p, need - 1, _lib.MODE_GROUPED, 0)
    assert rc == -4 and b"workspace" in L.ktmi_last_error()
    rc = L.ktmi_moe_layer(d, p + 8, p, p, 4096, 8, p, p, big, _lib.MODE_GROUPED, 0)
    assert rc == -1 and b"aligned" in L.ktmi_last_error()
    rc = L.ktmi_moe_layer(d, p, p, p, 10000, 8, p, p, big, _lib.MODE_GEMV, 0)
    assert rc == -1 and b"65535" in L.ktmi_last_error()
    rc = L.ktmi_moe_layer(d, p, p, p, 1 << 20, 8, p, p, big, _lib.MODE_GROUPED, 0)
    assert rc == -1 and b"4 GiB" in L.ktmi_last_error()
