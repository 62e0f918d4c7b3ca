"""GPU parity of the whole hot-expert layer (GEMV and grouped MFMA modes) against the
oracle's `_reference_check` FFN, through the C ABI."""
from dataclasses import replace

import numpy as np
import pytest

from conftest import bf16_bits_of, bf16_tensor, to_dev
from helpers import dequant_w, gemv_layer_oracle
from oracle import gguf_ref as R

pytestmark = pytest.mark.gpu

TOL_REL_L2 = 2e-2  # layer outputs vs the fp64 FFN on the bf16-dequantised weights


def _pkg():
    import kt_prefill_lend_amd._lib as L
    import kt_prefill_lend_amd.kt_gguf_hot as H
    import kt_prefill_lend_amd.synth as S

    return L, H, S


def _case(name, tokens, hidden=None, inter=None, hot=None, experts=None):
    _, _, S = _pkg()
    w = S.WORKLOADS[name]
    w = replace(w, hidden=hidden or w.hidden, inter=inter or w.inter, hot=hot or w.hot, experts=experts or w.experts)
    ids, tw, slot, _ = S.routing(w, tokens)
    xb = S.activations(w, tokens)
    w13, w2 = S.slot_tensors(w)
    return w, xb, tw, slot, w13, w2


def _run(dev, w, xb, tw, slot, w13, w2, mode):
    import torch

    L, H, _ = _pkg()
    W13, W2 = to_dev(w13, dev), to_dev(w2, dev)
    desc = H.layer_desc(W13, W2, w.hidden, w.inter, w.types[0], w.types[2])
    y = H.moe_layer(desc, bf16_tensor(xb, dev), to_dev(tw, dev), to_dev(slot, dev), mode)
    torch.cuda.synchronize()
    return bf16_bits_of(y)


CASES = [
    # (workload, tokens, hidden, inter, hot, experts)
    ("q8_0-h2048-n768-e128-k8-hot16", 40, 512, 256, 6, 24),
    ("q4_k-h2048-n512-e256-k8-hot32-decode", 16, 512, 256, 8, 32),
    ("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", 48, 512, 256, 8, 32),
    ("iq3_s-h2048-n512-e512-k10-hot48", 40, 512, 256, 8, 40),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0].split("-")[0] for c in CASES])
@pytest.mark.parametrize("mode", ["gemv", "decode", "grouped"])
def test_layer_vs_ffn_reference(dev, case, mode):
    L, _, S = _pkg()
    if mode == "decode":  # at most 256 routes
        case = (case[0], min(case[1], 256 // S.WORKLOADS[case[0]].top_k)) + tuple(case[2:])
    w, xb, tw, slot, w13, w2 = _case(*case)
    m = {"gemv": L.MODE_GEMV, "decode": L.MODE_DECODE, "grouped": L.MODE_GROUPED}[mode]
    got = R.bf16_to_f32(_run(dev, w, xb, tw, slot, w13, w2, m))
    g, d = dequant_w(w13, w2, w.types, w.hidden, w.inter)
    ref = R.ffn_reference(xb, slot, tw, g, d)
    l2, l1, cos = R.rel_errors(got, ref)
    print(f"{case[0]} {mode}: rel L2 {l2:.2e} rel L1 {l1:.2e} cos {cos:.6f}")
    assert l2 < TOL_REL_L2 and l1 < 0.025 and cos > 0.999, (l2, l1, cos)
    # tokens with no hot route are exactly zero
    cold_tok = (slot < 0).all(axis=1)
    assert np.all(got[cold_tok] == 0)


def test_gemv_mode_matches_reference_kernel_numerics(dev):
    """The decode path reproduces the reference kernels' own sequence (q8_1 GEMV, bf16,
    SiLU*mul, q8_1 GEMV, combine) to bf16 rounding."""
    L, _, _ = _pkg()
    w, xb, tw, slot, w13, w2 = _case("q4_k-h2048-n512-e256-k8-hot32-decode", 4, 512, 256, 8, 32)
    got = R.bf16_to_f32(_run(dev, w, xb, tw, slot, w13, w2, L.MODE_GEMV))
    exp = R.bf16_to_f32(gemv_layer_oracle(xb, tw, slot, w13, w2, w.types, w.hidden, w.inter))
    l2, _, _ = R.rel_errors(got, exp)
    assert l2 < 4e-3, l2


FUSED = [
    # (workload, tokens, top slot must exceed one 16-route pass): at most 256 routes, so GEMV
    # mode runs the two fused decode launches; 3 tokens stage every h row in LDS, the larger
    # windows (240 routes, 138 KB of h) read h from HBM and split the busiest slot's routes
    # over passes of the gate/up block
    ("q8_0-h2048-n768-e128-k8-hot16", 3, False),
    ("q8_0-h2048-n768-e128-k8-hot16", 30, True),
    ("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", 3, False),
    ("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", 30, True),
    ("iq3_s-h2048-n512-e512-k10-hot48", 3, False),
    ("iq3_s-h2048-n512-e512-k10-hot48", 24, True),
]


@pytest.mark.parametrize("case", FUSED, ids=[f"{c[0].split('-')[0]}-T{c[1]}" for c in FUSED])
def test_fused_decode_every_type(dev, case):
    """The fused decode launches for every weight type (gate/up and down), against the
    oracle's step-by-step restatement of the reference kernels' numerics."""
    L, _, _ = _pkg()
    name, T, multi_pass = case
    w, xb, tw, slot, w13, w2 = _case(name, T, 512, 256, 8, 32)
    assert slot.size <= 256
    per_slot = np.bincount(slot[slot >= 0], minlength=8)
    assert (per_slot.max() > 16) == multi_pass, per_slot
    got = R.bf16_to_f32(_run(dev, w, xb, tw, slot, w13, w2, L.MODE_GEMV))
    exp = R.bf16_to_f32(gemv_layer_oracle(xb, tw, slot, w13, w2, w.types, w.hidden, w.inter))
    l2, _, _ = R.rel_errors(got, exp)
    print(f"{name} T={T}: rel L2 vs the reference-kernel sequence {l2:.2e}")
    assert l2 < 4e-3, l2
    assert np.all(got[(slot < 0).all(axis=1)] == 0)


@pytest.mark.parametrize("T", [32, 33])
def test_decode_at_the_fused_route_limit(dev, T):
    """GEMV mode at 256 routes (32 tokens x 8: the most the fused decode launches take) and at
    264 (33 tokens: the stage-by-stage GEMV sequence), against the oracle's restatement of
    the reference kernels' sequence."""
    L, _, _ = _pkg()
    w, xb, tw, slot, w13, w2 = _case("q4_k-h2048-n512-e256-k8-hot32-decode", T, 512, 256, 8, 32)
    got = R.bf16_to_f32(_run(dev, w, xb, tw, slot, w13, w2, L.MODE_GEMV))
    exp = R.bf16_to_f32(gemv_layer_oracle(xb, tw, slot, w13, w2, w.types, w.hidden, w.inter))
    l2, _, _ = R.rel_errors(got, exp)
    assert l2 < 4e-3, l2
    assert np.all(got[(slot < 0).all(axis=1)] == 0)


@pytest.mark.parametrize("mode", ["gemv", "decode", "grouped"])
def test_layer_deterministic(dev, mode):
    L, _, _ = _pkg()
    T = 24 if mode == "decode" else 300  # the decode mode takes at most 256 routes
    w, xb, tw, slot, w13, w2 = _case("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", T, 512, 256, 8, 32)
    m = {"gemv": L.MODE_GEMV, "decode": L.MODE_DECODE, "grouped": L.MODE_GROUPED}[mode]
    a = _run(dev, w, xb, tw, slot, w13, w2, m)
    b = _run(dev, w, xb, tw, slot, w13, w2, m)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("t13,t2", [(R.GGML_Q4_K, R.GGML_Q6_K), (R.GGML_Q8_0, R.GGML_Q8_0), (R.GGML_IQ3_S, R.GGML_IQ3_S)])
def test_decode_mode_column_groups(dev, t13, t2):
    """The decode mode with slots of 64, 33, 17 and 1 routes (4, 3, 2 and 1 groups of 16 MFMA
    columns), 64 tokens x top-4 = 256 routes: against the fp64 FFN, and within the layer
    tolerance of the GEMV mode."""
    L, H, S = _pkg()
    base = S.WORKLOADS["q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill"]
    w = replace(base, hidden=512, inter=256, hot=8, experts=32, top_k=4, types=(t13, t13, t2))
    T = 64
    rng = np.random.default_rng(21)
    slot = np.full((T, 4), -1, np.int32)
    slot[:, 0] = 0                      # slot 0: every token
    slot[:33, 1] = 1                    # slot 1: 33 tokens
    slot[5:22, 2] = 2                   # slot 2: 17 tokens
    slot[40, 2] = 3                     # slot 3: one token
    others = rng.integers(4, w.hot, size=(T, 1))
    slot[:, 3:] = np.where(rng.random((T, 1)) < 0.5, others, -1)
    tw = rng.random((T, 4)).astype(np.float32)
    tw /= tw.sum(axis=1, keepdims=True)
    xb = S.activations(w, T)
    w13, w2 = S.slot_tensors(w)
    got = R.bf16_to_f32(_run(dev, w, xb, tw, slot, w13, w2, L.MODE_DECODE))
    g, d = dequant_w(w13, w2, w.types, w.hidden, w.inter)
    ref = R.ffn_reference(xb, slot, tw, g, d)
    l2, l1, cos = R.rel_errors(got, ref)
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, l1, cos)
    gemv = R.bf16_to_f32(_run(dev, w, xb, tw, slot, w13, w2, L.MODE_GEMV))
    assert R.rel_errors(got, gemv)[0] < TOL_REL_L2


def test_decode_mode_repeated_slot(dev):
    """A slot listed two or three times by a token (168 routes of 64 tokens on slot 0, 11
    groups of 16 MFMA columns, past the 64 a slot can hold without repeats): every route is
    computed, against the fp64 FFN (which sums the repeats) and the GEMV mode."""
    L, H, S = _pkg()
    base = S.WORKLOADS["q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill"]
    w = replace(base, hidden=512, inter=256, hot=8, experts=32, top_k=4)
    T = 64
    rng = np.random.default_rng(22)
    slot = np.full((T, 4), -1, np.int32)
    slot[:, 0] = 0
    slot[:, 1] = 0
    slot[:40, 2] = 0
    slot[40:, 2] = rng.integers(1, w.hot, size=T - 40)
    slot[:, 3] = np.where(rng.random(T) < 0.5, rng.integers(1, w.hot, size=T), -1)
    assert (slot == 0).sum() == 168
    tw = rng.random((T, 4)).astype(np.float32)
    tw /= tw.sum(axis=1, keepdims=True)
    xb = S.activations(w, T)
    w13, w2 = S.slot_tensors(w)
    got = R.bf16_to_f32(_run(dev, w, xb, tw, slot, w13, w2, L.MODE_DECODE))
    g, d = dequant_w(w13, w2, w.types, w.hidden, w.inter)
    ref = R.ffn_reference(xb, slot, tw, g, d)
    l2, l1, cos = R.rel_errors(got, ref)
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, l1, cos)
    gemv = R.bf16_to_f32(_run(dev, w, xb, tw, slot, w13, w2, L.MODE_GEMV))
    assert R.rel_errors(got, gemv)[0] < TOL_REL_L2


@pytest.mark.parametrize("seed", range(6))
def test_decode_mode_random_windows(dev, seed):
    """The decode mode on random windows: 1 to 64 tokens, top-1 to top-8 (at most 256 routes),
    slot ids mixing hot slots, -1 and ids past the table, some tokens naming a slot twice;
    against the fp64 FFN."""
    L, H, S = _pkg()
    rng = np.random.default_rng(100 + seed)
    top_k = int(rng.integers(1, 9))
    T = int(rng.integers(1, min(64, 256 // top_k) + 1))
    base = S.WORKLOADS["q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill"]
    w = replace(base, hidden=512, inter=256, hot=8, experts=32, top_k=top_k)
    slot = rng.integers(-2, w.hot + 3, size=(T, top_k)).astype(np.int32)
    slot[slot == -2] = -1
    if T > 2:
        slot[1, :] = slot[1, 0]  # one token naming one slot top_k times
    tw = rng.random((T, top_k)).astype(np.float32)
    tw /= tw.sum(axis=1, keepdims=True)
    xb = S.activations(w, T)
    w13, w2 = S.slot_tensors(w)
    got = R.bf16_to_f32(_run(dev, w, xb, tw, slot, w13, w2, L.MODE_DECODE))
    g, d = dequant_w(w13, w2, w.types, w.hidden, w.inter)
    hot = np.where((slot >= 0) & (slot < w.hot), slot, -1)
    ref = R.ffn_reference(xb, hot, tw, g, d)
    print(f"seed {seed}: T {T} top-{top_k}")
    cold = (hot < 0).all(axis=1)
    assert np.all(got[cold] == 0)
    if (~cold).any():
        l2, l1, cos = R.rel_errors(got[~cold], ref[~cold])
        assert l2 < TOL_REL_L2 and cos > 0.999, (l2, l1, cos)


@pytest.mark.parametrize("top_k", [1, 3, 6, 9, 12, 17])
def test_grouped_mode_any_top_k(dev, top_k):
    """The grouped mode at top-k that are not 8 (the combine reads k's in groups of 8, then of
    2, a group's k's past top_k and its cold routes reading zeros): slot ids mixing hot slots,
    -1 and ids past the table, one token naming one slot top_k times; against the fp64 FFN."""
    L, H, S = _pkg()
    rng = np.random.default_rng(200 + top_k)
    T = 97
    base = S.WORKLOADS["q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill"]
    w = replace(base, hidden=512, inter=256, hot=8, experts=32, top_k=top_k)
    slot = rng.integers(-2, w.hot + 3, size=(T, top_k)).astype(np.int32)
    slot[slot == -2] = -1
    slot[1, :] = slot[1, 0] if slot[1, 0] >= 0 else 0
    tw = rng.random((T, top_k)).astype(np.float32)
    tw /= tw.sum(axis=1, keepdims=True)
    xb = S.activations(w, T)
    w13, w2 = S.slot_tensors(w)
    got = R.bf16_to_f32(_run(dev, w, xb, tw, slot, w13, w2, L.MODE_GROUPED))
    g, d = dequant_w(w13, w2, w.types, w.hidden, w.inter)
    hot = np.where((slot >= 0) & (slot < w.hot), slot, -1)
    ref = R.ffn_reference(xb, hot, tw, g, d)
    cold = (hot < 0).all(axis=1)
    assert np.all(got[cold] == 0)
    l2, l1, cos = R.rel_errors(got[~cold], ref[~cold])
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, l1, cos)


def test_grouped_edge_cases(dev):
    """Empty slots, a single token, all-cold tokens, slots with one route."""
    L, _, _ = _pkg()
    w, xb, tw, slot, w13, w2 = _case("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", 5, 512, 256, 8, 32)
    slot = slot.copy()
    slot[0, :] = -1          # a token with no hot route
    slot[1, :] = -1
    slot[1, 3] = 7           # slot 7 with exactly one route
    for T in (1, 5):
        got = R.bf16_to_f32(_run(dev, w, xb[:T], tw[:T], slot[:T], w13, w2, L.MODE_GROUPED))
        g, d = dequant_w(w13, w2, w.types, w.hidden, w.inter)
        ref = R.ffn_reference(xb[:T], slot[:T], tw[:T], g, d)
        assert np.all(got[0] == 0)
        if T > 1:
            l2, _, _ = R.rel_errors(got, ref)
            assert l2 < TOL_REL_L2


@pytest.mark.parametrize("hot", [400, 512])
def test_grouped_sorts_agree_many_slots(dev, hot):
    """Chunks of up to 4096 routes are sorted by one block (sort_small), longer ones by three
    launches: the first 500 tokens of a 600-token chunk (4800 routes, three launches) equal the
    same 500 tokens alone (4000 routes: one block with 400 slots; three launches with 512,
    whose chunk counts exceed the one block's LDS) bit for bit, at hundreds of slots; both
    against the fp64 FFN."""
    L, _, _ = _pkg()
    w, xb, tw, slot, w13, w2 = _case("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", 600, 256, 256, hot, 1024)
    assert len(np.unique(slot[slot >= 0])) > hot // 2
    a = _run(dev, w, xb[:500], tw[:500], slot[:500], w13, w2, L.MODE_GROUPED)
    b = _run(dev, w, xb, tw, slot, w13, w2, L.MODE_GROUPED)
    assert np.array_equal(a, b[:500])
    g, d = dequant_w(w13, w2, w.types, w.hidden, w.inter)
    l2, _, cos = R.rel_errors(R.bf16_to_f32(b), R.ffn_reference(xb, slot, tw, g, d))
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, cos)


def test_grouped_past_the_combine_grid_limit(dev):
    """70000 tokens (560k routes, hidden 256): the combine runs in slices of 65535 tokens (the
    grid's y limit). Tokens past the first slice equal a call on those tokens alone, bit for
    bit (a token's output depends only on its own routes), and a token sample from both
    slices matches the fp64 FFN."""
    L, _, _ = _pkg()
    T, cut = 70000, 65535
    w, xb, tw, slot, w13, w2 = _case("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", T, 256, 256, 8, 32)
    y = _run(dev, w, xb, tw, slot, w13, w2, L.MODE_GROUPED)
    tail = _run(dev, w, xb[cut:], tw[cut:], slot[cut:], w13, w2, L.MODE_GROUPED)
    assert np.array_equal(y[cut:], tail)
    g, d = dequant_w(w13, w2, w.types, w.hidden, w.inter)
    sample = np.concatenate([np.arange(0, cut, 2049), np.arange(cut - 3, T, 157)])
    ref = R.ffn_reference(xb[sample], slot[sample], tw[sample], g, d)
    l2, l1, cos = R.rel_errors(R.bf16_to_f32(y[sample]), ref)
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, l1, cos)


@pytest.mark.timeout(300)
def test_grouped_past_one_pass(dev):
    """Hidden 7168, top-8: a grouped pass holds 37376 tokens (its Y buffer [R, hidden] bf16
    stays under the kernels' 32-bit offsets), so 37676 tokens run as two passes. The tokens
    of the second pass equal a call on those tokens alone, bit for bit, and a token sample
    from both passes, around the boundary included, matches the fp64 FFN."""
    L, H, _ = _pkg()
    w, xb, tw, slot, w13, w2 = _case("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", 37676, 7168, 256, 4, 32)
    desc = L.ktmi_layer(hidden=w.hidden, inter=w.inter, n_slots=w.hot, type13=w.types[0], type2=w.types[2],
                        w13=1 << 20, w2=1 << 21)
    cut = L.lib().ktmi_moe_layer_pass_tokens(desc, w.top_k)
    T = xb.shape[0]
    assert cut == 37376 and T > cut
    print(f"past one pass: {T} tokens, {(slot >= 0).sum()} hot routes", flush=True)
    y = _run(dev, w, xb, tw, slot, w13, w2, L.MODE_GROUPED)
    tail = _run(dev, w, xb[cut:], tw[cut:], slot[cut:], w13, w2, L.MODE_GROUPED)
    assert np.array_equal(y[cut:], tail)
    g, d = dequant_w(w13, w2, w.types, w.hidden, w.inter)
    sample = np.concatenate([np.arange(0, cut - 8, 997), np.arange(cut - 8, T, 31)])
    ref = R.ffn_reference(xb[sample], slot[sample], tw[sample], g, d)
    l2, l1, cos = R.rel_errors(R.bf16_to_f32(y[sample]), ref)
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, l1, cos)


def test_grouped_at_full_shape(dev):
    """The prefill workload's real layer shape (hidden 2048, inter 512, 40 slots, Q4_K/Q6_K)
    at 1024 tokens, against the fp64 FFN on a sample of tokens."""
    L, _, _ = _pkg()
    w, xb, tw, slot, w13, w2 = _case("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", 1024)
    got = R.bf16_to_f32(_run(dev, w, xb, tw, slot, w13, w2, L.MODE_GROUPED))
    g, d = dequant_w(w13, w2, w.types, w.hidden, w.inter)
    sample = np.arange(0, 1024, 8)
    ref = R.ffn_reference(xb[sample], slot[sample], tw[sample], g, d)
    l2, l1, cos = R.rel_errors(got[sample], ref)
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, l1, cos)


@pytest.mark.parametrize("mode", ["gemv", "decode", "grouped"])
def test_layer_empty_input_and_foreign_ids(dev, mode):
    """T = 0 is a no-op; slot ids >= S or < -1 (experts owned by no slot here) behave exactly
    like -1."""
    import torch

    L, H, _ = _pkg()
    m = {"gemv": L.MODE_GEMV, "decode": L.MODE_DECODE, "grouped": L.MODE_GROUPED}[mode]
    w, xb, tw, slot, w13, w2 = _case("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", 24, 512, 256, 8, 32)
    W13, W2 = to_dev(w13, dev), to_dev(w2, dev)
    desc = H.layer_desc(W13, W2, w.hidden, w.inter, w.types[0], w.types[2])
    y0 = H.moe_layer(desc, bf16_tensor(xb[:0], dev), to_dev(tw[:0], dev), to_dev(slot[:0], dev), m)
    torch.cuda.synchronize()
    assert tuple(y0.shape) == (0, w.hidden)
    rng = np.random.default_rng(11)
    pick = rng.random(slot.shape) < 0.3
    foreign = slot.copy()
    foreign[pick] = np.where(rng.random(int(pick.sum())) < 0.5, w.hot + 5, -7).astype(np.int32)
    cold = slot.copy()
    cold[pick] = -1
    a = _run(dev, w, xb, tw, foreign, w13, w2, m)
    b = _run(dev, w, xb, tw, cold, w13, w2, m)
    assert np.array_equal(a, b)


def test_grouped_headline_chunk_properties(dev):
    """The 16384-token prefill chunk at its real shape: a token sample against the fp64 FFN,
    and two size-independent identities that hold bit-exactly because every route's output
    depends only on its own row: permuting the tokens permutes the output, and doubling the
    route weights doubles it."""
    L, _, _ = _pkg()
    T = 16384
    w, xb, tw, slot, w13, w2 = _case("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", T)
    y = _run(dev, w, xb, tw, slot, w13, w2, L.MODE_GROUPED)
    g, d = dequant_w(w13, w2, w.types, w.hidden, w.inter)
    sample = np.arange(0, T, 97)
    ref = R.ffn_reference(xb[sample], slot[sample], tw[sample], g, d)
    l2, l1, cos = R.rel_errors(R.bf16_to_f32(y[sample]), ref)
    assert l2 < TOL_REL_L2 and cos > 0.999, (l2, l1, cos)
    perm = np.random.default_rng(12).permutation(T)
    yp = _run(dev, w, xb[perm], tw[perm], slot[perm], w13, w2, L.MODE_GROUPED)
    assert np.array_equal(yp, y[perm])
    y2 = _run(dev, w, xb, tw * np.float32(2), slot, w13, w2, L.MODE_GROUPED)
    assert np.array_equal(R.bf16_to_f32(y2), 2 * R.bf16_to_f32(y))


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["gemv", "decode", "grouped"])
def test_layer_in_hip_graph(dev, mode):
    """The layer call captured in a HIP graph (no memsets, no host sync inside): every replay,
    with eager layer calls on other inputs between the replays, reproduces the eager output
    bit for bit."""
    import torch

    L, H, _ = _pkg()
    m = {"gemv": L.MODE_GEMV, "decode": L.MODE_DECODE, "grouped": L.MODE_GROUPED}[mode]
    w, xb, tw, slot, w13, w2 = _case("q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill", 12 if mode != "grouped" else 300,
                                     512, 256, 8, 32)
    W13, W2 = to_dev(w13, dev), to_dev(w2, dev)
    desc = H.layer_desc(W13, W2, w.hidden, w.inter, w.types[0], w.types[2])
    T, k = slot.shape
    x, twd, sd = bf16_tensor(xb, dev), to_dev(tw, dev), to_dev(slot, dev)
    lib = L.lib()
    out = torch.empty((T, w.hidden), dtype=torch.bfloat16, device=dev)
    ws = torch.empty((lib.ktmi_moe_layer_workspace(desc, T, k, m),), dtype=torch.uint8, device=dev)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        H.moe_layer(desc, x, twd, sd, m, out, ws)
    torch.cuda.synchronize()
    ref = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        H.moe_layer(desc, x, twd, sd, m, out, ws)
    x2 = bf16_tensor(xb[::-1].copy(), dev)
    for r in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {r}"
        H.moe_layer(desc, x2, twd, sd, m)  # eager work between the replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("mode,T", [("grouped", 48), ("grouped", 4096), ("gemv", 8), ("gemv", 64), ("decode", 8),
                                    ("decode", 32)])
def test_slot_address_table_matches_contiguous_slots(dev, mode, T):
    """Slots given as a device table of per-slot addresses (w_is_table, each slot its own
    allocation, in reverse order) give the same bits as the contiguous slot tensors: 128- and
    256-route grouped tiles, the fused decode layer and the stage-by-stage GEMV layer."""
    import torch

    L, H, S = _pkg()
    w = S.WORKLOADS["q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill"]
    _, tw, slot, _ = S.routing(w, T)
    xb = S.activations(w, T)
    w13, w2 = S.slot_tensors(w)
    W13, W2 = to_dev(w13, dev), to_dev(w2, dev)
    m = {"gemv": L.MODE_GEMV, "decode": L.MODE_DECODE, "grouped": L.MODE_GROUPED}[mode]
    x, twd, sd = bf16_tensor(xb, dev), to_dev(tw, dev), to_dev(slot, dev)
    ref = H.moe_layer(H.layer_desc(W13, W2, w.hidden, w.inter, w.types[0], w.types[2]), x, twd, sd, m)
    n = W13.shape[0]
    p13 = [None] * n
    p2 = [None] * n
    for s in reversed(range(n)):
        p13[s], p2[s] = W13[s].clone(), W2[s].clone()
    t13 = torch.tensor([p.data_ptr() for p in p13], dtype=torch.int64, device=dev)
    t2 = torch.tensor([p.data_ptr() for p in p2], dtype=torch.int64, device=dev)
    got = H.moe_layer(H.layer_desc(t13, t2, w.hidden, w.inter, w.types[0], w.types[2], table=True), x, twd, sd, m)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits_of(got), bf16_bits_of(ref))
