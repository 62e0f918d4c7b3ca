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
    assert L.ktmi_moe_layer_mode(d, 4, 8) == _lib.MODE_GEMV  # 32 routes: below the decode mode's 64
    assert L.ktmi_moe_layer_mode(d, 8, 8) == _lib.MODE_DECODE
    assert L.ktmi_moe_layer_mode(d, 16384, 8) == _lib.MODE_GROUPED
    # the decode mode's workspace: h [R, inter] bf16 and the routes' outputs [R, hidden] bf16
    assert L.ktmi_moe_layer_workspace(d, 4, 8, _lib.MODE_DECODE) == 4 * 8 * 512 * 2 + 4 * 8 * 2048 * 2
    assert L.ktmi_moe_layer_workspace(d, 65, 2, _lib.MODE_DECODE) == 0  # past its 64 tokens
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
    c.assign(1, 0, 7)
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
    assert "neither side" in c.check_tables()
    with pytest.raises(ValueError, match="another slot"):
        c.assign(1, 1, 7)  # expert 7 already sits in slot 0 of layer 1


def test_swap_pairing_rules():
    """pair_swaps: coldest slots (empty first) against the hottest non-residents, the
    margin test per pair, the first failing pair ends the list, ties by index, at most
    `limit` swaps; brute-forced against an explicit enumeration of the rule."""
    import kt_prefill_lend_amd.kt_hot_cache as C

    res = np.array([3, C.EMPTY, 0, 5])
    counts = np.array([4.0, 9.0, 9.0, 1.0, 0.0, 2.0, 7.0, 0.0])
    # slots by (score, index): slot 1 (empty, -1), slot 3 (expert 5: 2), slot 0 (expert 3: 1)...
    # scores: slot0=1 (e3), slot1=-1, slot2=4 (e0), slot3=2 (e5) -> order 1, 0, 3, 2
    # candidates by (-count, id): 1 (9), 2 (9), 6 (7), 4 (0), 7 (0)
    assert C.pair_swaps(res, counts, 1.5, 8) == [(1, 1), (0, 2), (3, 6)]  # 9 > -1.5, 9 > 1.5, 7 > 3; 0 fails
    assert C.pair_swaps(res, counts, 1.5, 2) == [(1, 1), (0, 2)]
    assert C.pair_swaps(res, counts, 5.0, 8) == [(1, 1), (0, 2)]  # 7 > 5*2 fails, ends the list
    assert C.pair_swaps(res, np.zeros(8), 1.5, 8) == []  # a candidate needs a positive count
    rng = np.random.default_rng(3)
    for _ in range(200):
        E, S = 12, 4
        res = rng.permutation(E)[:S].astype(np.int64)
        res[rng.random(S) < 0.2] = C.EMPTY
        counts = rng.integers(0, 5, E).astype(float)
        margin = float(rng.choice([1.0, 1.5, 2.0]))
        got = C.pair_swaps(res, counts, margin, 3)
        score = [counts[e] if e >= 0 else -1.0 for e in res]
        slots = sorted(range(S), key=lambda s: (score[s], s))
        cands = sorted(set(range(E)) - set(int(e) for e in res if e >= 0), key=lambda e: (-counts[e], e))
        want = []
        for k in range(min(3, len(cands))):
            if counts[cands[k]] > 0 and counts[cands[k]] > margin * score[slots[k]]:
                want.append((slots[k], cands[k]))
            else:
                break
        assert got == want


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


def _stand_ins(layer_idx=3, streams_hot=True, num_gpu_experts=4, path="/nonexistent.gguf"):
    """A KT wrapper method and a FusedMoE layer as the reference's wrapper hands them over
    (only the attributes the streamer and the hot method read)."""
    from types import SimpleNamespace as NS

    kt = NS(layer_idx=layer_idx, weight_path=path, num_gpu_experts=num_gpu_experts, num_layers=4)
    method = NS(kt_config=kt, num_gpu_experts=num_gpu_experts, gpu_method=NS(streams_hot_experts=streams_hot))
    layer = NS(intermediate_size_per_partition=256, hidden_size=512, top_k=8, moe_tp_rank=0, moe_tp_size=1)
    return method, layer


def test_stream_prefill_entry_points(monkeypatch):
    """stream_prefill_for / stream_prefill_init_early / preallocate with the reference's
    signatures (P:10515, 10581, 40607, 40995-41024): threshold, capture and failure
    handling, one process-wide instance built from (method, layer)."""
    import kt_prefill_lend_amd.kt_stream_prefill as SP

    made = []

    class Fake:
        def __init__(self, method, layer):
            made.append((method, layer))
            self.banks_built, self.rank = False, 0

        def build_all_banks(self):
            self.banks_built = True

    method, layer = _stand_ins()
    monkeypatch.setattr(SP, "KTStreamPrefillGGUF", Fake)
    monkeypatch.setattr(SP, "_instance", None)
    monkeypatch.setattr(SP, "_failed", False)
    monkeypatch.setattr(SP, "STREAM_THRESHOLD", 0)
    assert SP.stream_prefill_for(method, layer, 100000) is None
    assert SP.preallocate(layer) is None  # streaming off: nothing is made
    SP.stream_prefill_init_early(method, layer)
    assert not made
    monkeypatch.setattr(SP, "STREAM_THRESHOLD", 4096)
    assert SP.stream_prefill_for(method, layer, 1024) is None and not made
    st = SP.stream_prefill_for(method, layer, 8192)
    assert isinstance(st, Fake) and made == [(method, layer)]
    assert SP.stream_prefill_for(method, layer, 4096) is st and len(made) == 1  # one instance per process
    # early init: only with KT_GPU_STREAM_EARLY_INIT=1, and it builds every bank
    monkeypatch.setattr(SP, "_instance", None)
    monkeypatch.setattr(SP, "EARLY_INIT", False)
    SP.stream_prefill_init_early(method, layer)
    assert SP._instance is None
    monkeypatch.setattr(SP, "EARLY_INIT", True)
    SP.stream_prefill_init_early(method, layer)
    assert SP._instance is not None and SP._instance.banks_built
    # a failed init is remembered: later calls return None instead of retrying
    monkeypatch.setattr(SP, "_instance", None)

    def broken(method, layer):
        raise RuntimeError("no GGUF")

    monkeypatch.setattr(SP, "KTStreamPrefillGGUF", broken)
    with pytest.raises(RuntimeError, match="no GGUF"):
        SP.stream_prefill_for(method, layer, 8192)
    assert SP._failed and SP.stream_prefill_for(method, layer, 8192) is None


def test_stream_run_takes_the_reference_arguments(monkeypatch):
    """run(method, layer, dispatch_output, physical_ids): the layer index comes from
    method.kt_config, x and the route weights from dispatch_output, and the first streamed
    expert is 0 when the GPU method streams its hot experts, else num_gpu_experts."""
    import torch

    import kt_prefill_lend_amd.kt_gguf_hot as H
    import kt_prefill_lend_amd.kt_stream_prefill as SP

    seen = []
    st = SP.KTStreamPrefillGGUF.__new__(SP.KTStreamPrefillGGUF)
    st.geometry = SP._Geometry(256, 512, {3: (12, 12, 14)})
    st._checked = True
    st.run_tensors = lambda li, x, w, ids, first=0: seen.append((li, x, w, ids, first)) or "acc"
    x, w, ids = torch.zeros((2, 512)), torch.ones((2, 8)), torch.zeros((2, 8), dtype=torch.int32)
    d = H.DispatchOutput(x, H.TopKOutput(w, ids, None))
    for streams_hot, first in ((True, 0), (False, 4)):
        method, layer = _stand_ins(streams_hot=streams_hot)
        assert st.run(method, layer, d, ids) == "acc"
        li, xs, ws, i2, f = seen[-1]
        assert (li, f) == (3, first) and xs is x and ws is w and i2 is ids


def test_sglang_expert_location_map_places_the_slots(monkeypatch):
    """process_weights_after_loading(layer) reads SGLang's expert-location map for its layer
    when SGLang is there (hot/kt_gguf_hot.py:213-220): slot s gets logical expert p2l[s];
    without SGLang or with no metadata the slots hold experts 0..n-1."""
    import sys
    import types as T

    import torch

    import kt_prefill_lend_amd.kt_gguf_hot as H

    E, N, K, n, li = 8, 256, 256, 3, 1

    class Source:  # expert e's bytes are all e (gate), e + 64 (up), e + 128 (down)
        inter, K_, types_ = N, K, (12, 12, 14)

        def types(self, layer_idx):
            return self.types_

        def slice(self, layer_idx, proj, N_, rank, experts):
            rows, rb = (N_, H._row_bytes(K, 12)) if proj != "down" else (K, H._row_bytes(N_, 14))
            base = {"gate": 0, "up": 64, "down": 128}[proj]
            ex = torch.as_tensor(experts, dtype=torch.int64)
            return (ex.to(torch.uint8) + base).view(-1, 1, 1).expand(len(ex), rows, rb).contiguous()

    src = Source()
    src.K = K
    H.register_source("mem://experts", src)
    method, layer = _stand_ins(layer_idx=li, num_gpu_experts=n, path="mem://experts")
    m = H.KTGGUFHotExpertsMethod(method.kt_config, layer)
    m.N, m.K = N, K
    mod = torch.nn.Module()
    mod.register_parameter("w13_qweight", torch.nn.Parameter(torch.zeros((n, 2 * N, H._row_bytes(K, 12)),
                                                                         dtype=torch.uint8), requires_grad=False))
    mod.register_parameter("w2_qweight", torch.nn.Parameter(torch.zeros((n, K, H._row_bytes(N, 14)),
                                                                        dtype=torch.uint8), requires_grad=False))

    def slots():
        return ([int(mod.w13_qweight[s, 0, 0]) for s in range(n)], [int(mod.w13_qweight[s, N, 0]) - 64 for s in range(n)],
                [int(mod.w2_qweight[s, 0, 0]) - 128 for s in range(n)])

    for name in ("sglang", "sglang.srt", "sglang.srt.eplb", "sglang.srt.eplb.expert_location_dispatch"):
        monkeypatch.delitem(sys.modules, name, raising=False)
    m.process_weights_after_loading(mod)  # no SGLang: identity
    assert slots() == ([0, 1, 2],) * 3
    p2l = torch.tensor([[0, 1, 2, 3, 4, 5, 6, 7], [5, 2, 7, 0, 1, 3, 4, 6]])
    meta = T.SimpleNamespace(physical_to_logical_map_cpu=p2l)
    fake = T.ModuleType("sglang.srt.eplb.expert_location_dispatch")
    fake.get_global_expert_location_metadata = lambda: meta
    for name in ("sglang", "sglang.srt", "sglang.srt.eplb"):
        monkeypatch.setitem(sys.modules, name, T.ModuleType(name))
    monkeypatch.setitem(sys.modules, "sglang.srt.eplb.expert_location_dispatch", fake)
    m.process_weights_after_loading(mod)  # layer 1's map
    assert slots() == ([5, 2, 7],) * 3
    fake.get_global_expert_location_metadata = lambda: None
    m.process_weights_after_loading(mod)  # SGLang without a map: identity
    assert slots() == ([0, 1, 2],) * 3
    m.process_weights_after_loading(mod, physical_to_logical=[6, 4, 1])  # an explicit map wins
    assert slots() == ([6, 4, 1],) * 3


def test_layer_argument_errors_before_device_work():
    """The layer entry point rejects bad arguments with a status and a message before it
    touches the device (the pointers below are never dereferenced): a short workspace,
    misaligned activations, a forced GEMV mode past its route limit."""
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
    rc = L.ktmi_moe_layer(d, p, p, p, 40, 8, p, p, big, _lib.MODE_DECODE, 0)  # 320 routes
    assert rc == -1 and b"decode mode" in L.ktmi_last_error()
    assert L.ktmi_moe_layer_mode(d, 16, 8) == _lib.MODE_DECODE
    assert L.ktmi_moe_layer_mode(d, 33, 8) == _lib.MODE_GROUPED
    assert L.ktmi_moe_layer_mode(d, 128, 2) == _lib.MODE_GEMV  # 128 tokens: past the decode mode's 64


@pytest.mark.parametrize("hidden,inter,top_k,pass_tokens", [(7168, 2048, 8, 37376), (2048, 512, 8, 130816),
                                                             (512, 4096, 10, 52224), (256, 256, 1, 8388352)])
def test_grouped_pass_plan(hidden, inter, top_k, pass_tokens):
    """The grouped mode's token passes: the largest multiple of 256 tokens whose x [T, hidden],
    H [T top_k, inter] and Y [T top_k, hidden] bf16 buffers all stay under 4 GiB - 64 KiB (its
    kernels' 32-bit buffer offsets, 0xFFFFFFF0 marking a dropped store); the workspace covers
    one pass, so it grows with the tokens up to a pass and stays there."""
    from kt_prefill_lend_amd import _lib

    L = _lib.lib()
    d = _lib.ktmi_layer(hidden=hidden, inter=inter, n_slots=24, type13=12, type2=14, w13=1 << 20, w2=2 << 20)
    got = L.ktmi_moe_layer_pass_tokens(d, top_k)
    assert got == pass_tokens
    limit = 0xFFFF0000
    assert 2 * got * hidden <= limit and 2 * got * top_k * inter <= limit and 2 * got * top_k * hidden <= limit
    nxt = got + 256
    assert max(2 * nxt * top_k * inter, 2 * nxt * top_k * hidden) > limit
    ws = lambda t: L.ktmi_moe_layer_workspace(d, t, top_k, _lib.MODE_GROUPED)  # noqa: E731
    assert ws(got - 1) < ws(got) == ws(got + 1) == ws(3 * got + 17)
    # the Y buffer of one pass alone is R * hidden * 2 bytes
    assert ws(got) >= 2 * got * top_k * hidden


def test_dense_ok_and_reads_table(monkeypatch):
    """dense_ok / reads_table (hot/kt_gguf_moe_multi.py:90-100): the dense GEMV takes 2 to
    KT_GGUF_MOE_MAXM tokens of a contiguous uint8 weight with more than 512 rows of a type with
    kernels, unless KT_GGUF_DENSE_MULTI=0; every ktmi kernel reads slot weights through the
    pointer table, so reads_table only follows KT_GGUF_MOE_MULTI."""
    import torch

    import kt_prefill_lend_amd.kt_gguf_moe_multi as M

    x = lambda t: torch.zeros((t, 512), dtype=torch.bfloat16)  # noqa: E731
    w = lambda r: torch.zeros((r, 288), dtype=torch.uint8)  # noqa: E731
    assert M.MAX_TOKENS == 4 and M.DENSE_MIN_ROWS == 513
    assert M.dense_ok(x(2), w(513), 12) and M.dense_ok(x(4), w(4096), 14)
    assert not M.dense_ok(x(1), w(513), 12)   # one token: the plain GEMV
    assert not M.dense_ok(x(5), w(513), 12)   # past the window
    assert not M.dense_ok(x(2), w(512), 12)   # small matrices stay on the plain path
    assert not M.dense_ok(x(2), w(513), 13)   # Q5_K: no kernel here
    assert not M.dense_ok(x(2), w(600)[:, :144].contiguous().t(), 12)  # not [rows, bytes] contiguous
    assert not M.dense_ok(x(2), w(1024)[::2], 12)
    assert not M.dense_ok(x(2), torch.zeros((513, 72), dtype=torch.int32), 12)
    monkeypatch.setattr(M, "DENSE", False)
    assert not M.dense_ok(x(2), w(513), 12)
    for t in (1, 4, 5, 64):
        assert M.reads_table(t)
    monkeypatch.setenv("KT_GGUF_MOE_MULTI", "0")
    assert not M.reads_table(1)


def test_scale_f16_fields_scales_dequant_exactly():
    """The test helper that signs bank rows: fp16 scales times a power of two give exactly
    that multiple of every dequantised value (so the oracle can scale its arrays instead of
    decoding the signed rows)."""
    from helpers import TYPES, random_blocks, scale_f16_fields
    from oracle import gguf_ref as R

    rng = np.random.default_rng(4)
    for t in TYPES:
        cols = 512
        rows = random_blocks(t, 6, cols, rng)
        for f in (2.0, 128.0):
            got = R.dequant_rows(scale_f16_fields(rows, t, f), t, cols)
            assert np.array_equal(got, R.dequant_rows(rows, t, cols) * np.float32(f)), (t, f)
