"""Pins of the CPU oracle (no GPU): golden blocks, the reference's integer vec_dot,
closed forms, brute force and invariants. See oracle/gguf_ref.py's header."""
import hashlib
from pathlib import Path

import numpy as np
import pytest

from helpers import TYPES, random_blocks
from oracle import gguf_ref as R

GOLDEN = Path(__file__).resolve().parent / "golden" / "dequant_golden.npz"


def test_iq3s_grid_pinned():
    g = R.iq3s_grid()
    assert g.size == 512
    assert hashlib.sha256(g.astype("<u4").tobytes()).hexdigest() == R.IQ3S_GRID_SHA256
    assert np.all(np.diff(g.astype(np.int64)) > 0)
    b = g.view(np.uint8)
    assert set(np.unique(b).tolist()) == {1, 3, 5, 7, 9, 11, 13, 15}


@pytest.mark.parametrize("t", TYPES)
def test_dequant_matches_golden_loops(t):
    d = np.load(GOLDEN)
    raw, val = d[f"raw_{t}"], d[f"val_{t}"]
    blck, _ = R.BLOCK_INFO[t]
    got = R.dequant_rows(raw.reshape(1, -1), t, raw.shape[0] * blck).reshape(val.shape)
    assert np.array_equal(got.view(np.uint32), val.view(np.uint32))
    assert np.all(got[0] == 0)


def test_exactness_facts():
    """Q8_0 and IQ3_S values, and Q4_K's d*sc*q, are exact in fp32 (so no op order matters)."""
    rng = np.random.default_rng(0)
    for t in (R.GGML_Q8_0, R.GGML_IQ3_S):
        raw = random_blocks(t, 4, 512, rng)
        y32 = R.dequant_rows(raw, t, 512).astype(np.float64)
        # recompute in fp64 from the same fields: must agree exactly
        if t == R.GGML_Q8_0:
            b = raw.reshape(-1, 34)
            d = R.f16_bits_to_f32(b[:, :2].copy().view(np.uint16)[:, 0]).astype(np.float64)
            ref = d[:, None] * b[:, 2:].view(np.int8).astype(np.float64)
        else:
            d, nib, g, neg = R._iq3_s_fields(raw.reshape(-1, 110))
            ref = d.astype(np.float64)[:, None] * (1 + 2 * nib) * g * np.where(neg == 1, -1, 1)
        assert np.array_equal(y32.reshape(-1), ref.reshape(-1))


@pytest.mark.parametrize("t", TYPES)
def test_literal_vec_dot_equals_dequant_dot(t):
    """The reference's int8 vec_dot (its own index arithmetic) equals the dot product of the
    oracle's dequantised weights with the dequantised q8_1 activations: pins every
    nibble/scale/sign/grid mapping of dequant_rows against vecdotq.cuh."""
    rng = np.random.default_rng(10 + t)
    blck, ts = R.BLOCK_INFO[t]
    nblk = 6
    raw = random_blocks(t, 1, blck * nblk, rng).reshape(nblk, ts)
    x = rng.standard_normal((1, blck * nblk)).astype(np.float32)
    qs, d8, s8, _ = R.quantize_q8_1(x)
    q8 = R.q8_1_pack(qs, d8, s8).reshape(-1, 36)
    w = R.dequant_rows(raw.reshape(1, -1), t, blck * nblk).astype(np.float64).reshape(-1)
    xd = (np.repeat(d8[0], 32)[: blck * nblk].astype(np.float64) * qs[0, : blck * nblk].astype(np.float64))
    for b in range(nblk):
        lit = R.vec_dot_block_literal(t, raw[b], q8[b * blck // 32:(b + 1) * blck // 32])
        deq = float(w[b * blck:(b + 1) * blck] @ xd[b * blck:(b + 1) * blck])
        assert abs(lit - deq) <= 1e-5 * (abs(deq) + np.abs(w[b * blck:(b + 1) * blck]).sum() * np.abs(xd).max()), (b, lit, deq)


@pytest.mark.parametrize("t", TYPES)
def test_vectorised_row_sums_equal_literal(t):
    rng = np.random.default_rng(20 + t)
    blck, ts = R.BLOCK_INFO[t]
    cols = 512
    rows, T = 3, 2
    W = random_blocks(t, rows, cols, rng)
    x = rng.standard_normal((T, cols)).astype(np.float32)
    qs, d8, s8, _ = R.quantize_q8_1(x)
    got = R._row_sums_int(t, W, cols, qs, d8)  # [rows, T]
    q8 = R.q8_1_pack(qs, d8, s8).reshape(T, -1, 36)
    for r in range(rows):
        blocks = W[r].reshape(-1, ts)
        for tk in range(T):
            lit = sum(R.vec_dot_block_literal(t, blocks[b], q8[tk, b * blck // 32:(b + 1) * blck // 32])
                      for b in range(cols // blck))
            assert abs(got[r, tk] - lit) <= 1e-9 * max(1.0, abs(lit))


def test_quantize_q8_1_closed_form():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 96)).astype(np.float32) * 5
    x[2, 32:64] = 0.0
    qs, d, s, draw = R.quantize_q8_1(x)
    assert qs.shape == (3, 512) and d.shape == (3, 16)
    blk = x.reshape(3, 3, 32)
    amax = np.abs(blk).max(axis=2)
    assert np.array_equal(draw[:, :3], (amax / np.float32(127)).astype(np.float32))
    q = qs[:, :96].reshape(3, 3, 32).astype(np.float32)
    assert np.all(np.abs(blk - draw[:, :3, None] * q) <= draw[:, :3, None] * 0.5 * (1 + 1e-6) + 1e-30)
    assert np.all(np.abs(q).max(axis=2)[amax > 0] == 127)
    assert np.all(qs[2, 32:64] == 0) and d[2, 1] == 0
    assert np.all(qs[:, 96:] == 0)  # padding
    # ties round away from zero (roundf), not to even
    t = np.zeros((1, 32), np.float32)
    t[0, 0] = 127.0
    t[0, 1] = 2.5
    t[0, 2] = -0.5
    q2, _, _, _ = R.quantize_q8_1(t)
    assert q2[0, 1] == 3 and q2[0, 2] == -1


def test_combine_brute_force():
    rng = np.random.default_rng(2)
    T, k, K = 3, 5, 7
    ob = R.bf16_bits(rng.standard_normal((T, k, K)).astype(np.float32))
    w = rng.random((T, k)).astype(np.float32)
    got = R.combine(ob, w)
    for t in range(T):
        for c in range(K):
            acc = np.float32(0)
            for j in range(k):
                o = R.bf16_to_f32(ob[t, j, c])
                wk = R.bf16_round(np.float32(w[t, j]))
                acc = np.float32(acc + R.bf16_round(np.float32(o * wk)))
            assert got[t, c] == R.bf16_bits(acc)


def test_sort_routes_invariants():
    rng = np.random.default_rng(3)
    ids = rng.integers(-1, 6, size=(50, 4)).astype(np.int32)
    perm, seg = R.sort_routes(ids, 6)
    flat = ids.reshape(-1)
    assert sorted(perm.tolist()) == sorted(np.nonzero(flat >= 0)[0].tolist())
    for e in range(6):
        part = perm[seg[e]:seg[e + 1]]
        assert np.all(flat[part] == e) and np.all(np.diff(part) > 0)
    assert seg[-1] == (flat >= 0).sum()


def test_route_brute_force():
    rng = np.random.default_rng(4)
    E = 20
    ids = rng.integers(0, E, size=(7, 3)).astype(np.int32)
    log2slot = np.full(E, -1, np.int32)
    log2slot[[2, 5, 11]] = [0, 1, 2]
    log2cpu = np.where(log2slot >= 0, -1, np.arange(E)).astype(np.int32)
    counts = np.zeros(E, np.float32)
    s, c = R.route(ids, log2slot, log2cpu, counts)
    for i in range(7):
        for j in range(3):
            e = ids[i, j]
            assert s[i, j] == (log2slot[e]) and c[i, j] == (-1 if log2slot[e] >= 0 else e)
            assert (s[i, j] >= 0) != (c[i, j] >= 0)
    assert np.array_equal(counts, np.bincount(ids.reshape(-1), minlength=E).astype(np.float32))


def test_ffn_reference_closed_form_and_linearity():
    # one token, one route, N = 1, K = 2: y = w * wd * silu(x.wg) * (x.wu)
    x = R.bf16_bits(np.array([[1.0, -2.0]], np.float32))
    g = np.array([[[0.5, 0.25], [1.0, 1.0]]], np.float32)  # [1, 2N, K]: gate row, up row
    d = np.array([[[2.0], [-1.0]]], np.float32)            # [1, K, N]
    slot = np.array([[0]], np.int32)
    w = np.array([[0.75]], np.float32)
    y = R.ffn_reference(x, slot, w, g, d)
    a = 1.0 * 0.5 - 2.0 * 0.25
    u = 1.0 - 2.0
    h = a / (1 + np.exp(-a)) * u
    assert np.allclose(y, [[0.75 * 2.0 * h, 0.75 * -1.0 * h]], rtol=0, atol=1e-15)
    rng = np.random.default_rng(5)
    xb = R.bf16_bits(rng.standard_normal((6, 8)).astype(np.float32))
    G = rng.standard_normal((3, 4, 8)).astype(np.float32)
    D = rng.standard_normal((3, 8, 2)).astype(np.float32)
    ids = rng.integers(-1, 3, size=(6, 2)).astype(np.int32)
    ww = rng.random((6, 2)).astype(np.float32)
    y1 = R.ffn_reference(xb, ids, ww, G, D)
    y2 = R.ffn_reference(xb, ids, 2 * ww, G, D)
    assert np.allclose(y2, 2 * y1, rtol=1e-12, atol=1e-12)
    # a route's contribution adds: dropping one route changes only its token
    ids2 = ids.copy()
    ids2[0, 0] = -1
    y3 = R.ffn_reference(xb, ids2, ww, G, D)
    assert np.allclose(y3[1:], y1[1:])


def test_silu_and_mul_textbook():
    rng = np.random.default_rng(6)
    hb = R.bf16_bits(rng.standard_normal((4, 16)).astype(np.float32) * 3)
    h = R.bf16_to_f32(hb).astype(np.float64)
    g, u = h[:, :8], h[:, 8:]
    exp = g * (1 / (1 + np.exp(-g))) * u
    got = R.bf16_to_f32(R.silu_and_mul(hb))
    assert np.allclose(got, exp, rtol=2 ** -8, atol=1e-30)


def test_bf16_rounding_ties_to_even():
    x = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8)], np.float32)
    assert np.array_equal(R.bf16_to_f32(R.bf16_bits(x)), np.array([1.0, 1.0 + 2 ** -6, -1.0], np.float32))


@pytest.mark.parametrize("types", [(8, 8, 8), (12, 12, 14), (21, 21, 21)])
def test_cpu_path_agrees_with_ffn_reference(types):
    """The C restatement of the CPU expert path (Q8_K / Q8_0 int8 dots) against the fp64 FFN
    over the exactly dequantised weights: quantising activations costs well under 2e-2."""
    from dataclasses import replace

    import kt_prefill_lend_amd.synth as S
    from oracle import cpu_moe

    if not cpu_moe.LIB_PATH.exists():
        pytest.skip("oracle C library not built")
    base = S.WORKLOADS["q8_0-h2048-n768-e128-k8-hot16"]
    w = replace(base, hidden=512, inter=256, hot=5, experts=12, types=types)
    T = 24
    _, tw, slot, _ = S.routing(w, T)
    xb = S.activations(w, T)
    w13, w2 = S.slot_tensors(w)
    g = R.dequant_rows(w13.reshape(-1, w13.shape[2]), types[0], w.hidden).reshape(w.hot, 2 * w.inter, w.hidden)
    d = R.dequant_rows(w2.reshape(-1, w2.shape[2]), types[2], w.inter).reshape(w.hot, w.hidden, w.inter)
    ref = R.ffn_reference(xb, slot, tw, g, d)
    got = cpu_moe.forward(xb, slot, tw, w13, w2, types[0], types[2], w.inter, threads=2)
    l2, _, cos = R.rel_errors(got, ref)
    assert l2 < 2e-2 and cos > 0.999, (l2, cos)
    # a token with no hot route contributes nothing; the one-thread run is identical
    slot2 = slot.copy()
    slot2[0] = -1
    got2 = cpu_moe.forward(xb, slot2, tw, w13, w2, types[0], types[2], w.inter, threads=1)
    assert np.all(got2[0] == 0)
    assert np.array_equal(got2[1:], got[1:])
