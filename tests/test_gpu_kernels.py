"""GPU parity of the single kernels against the oracle, through the C ABI."""
import numpy as np
import pytest

from conftest import bf16_bits_of, bf16_tensor, to_dev
from helpers import _F16_FIELDS, TYPES, random_blocks
from oracle import gguf_ref as R

pytestmark = pytest.mark.gpu


def _pkg():
    import kt_prefill_lend_amd.kt_gguf_dequant as DQ
    import kt_prefill_lend_amd.kt_gguf_hot as H
    import kt_prefill_lend_amd.kt_gguf_moe_multi as M
    import kt_prefill_lend_amd.kt_hot_cache as C

    return DQ, M, H, C


def zero_scales(blocks: np.ndarray, t: int, rng) -> None:
    """Every third block's fp16 fields become +0 or -0 and (Q6_K) some sub-block scales 0:
    the dequantised zeros must carry the signs of the oracle's plain products."""
    blck, ts = R.BLOCK_INFO[t]
    v = blocks.reshape(blocks.shape[0], -1, ts)
    for off in _F16_FIELDS[t]:
        v[:, ::3, off] = 0
        v[:, ::3, off + 1] = np.where(rng.random(v[:, ::3, off + 1].shape) < 0.5, 0x80, 0).astype(np.uint8)
    if t == R.GGML_Q6_K:
        v[:, 1::3, 192:200] = 0


@pytest.mark.parametrize("t", TYPES)
def test_dequant_bit_exact(dev, t):
    import torch

    DQ, *_ = _pkg()
    rng = np.random.default_rng(100 + t)
    # the stand-alone dequant runs the grouped GEMMs' operand decoder (BPiece<t>): 32-row
    # groups x 256-value columns; the second shape has a partial row group and (Q8_0) a row
    # that ends halfway through a 64-value step
    shapes = [(48, 768 if t == R.GGML_Q8_0 else 512), (33, 288 if t == R.GGML_Q8_0 else 256)]
    for n, (rows, cols) in zip((3, 2), shapes):
        rb = R.row_bytes(cols, t)
        stride = (rows * rb + 64 + 15) // 16 * 16  # padded expert stride
        raw = np.zeros((n, stride), np.uint8)
        for e in range(n):
            blocks = random_blocks(t, rows, cols, rng)
            if rows == 33:
                zero_scales(blocks, t, rng)
            raw[e, :rows * rb] = blocks.reshape(-1)
        out = torch.full((n, rows * cols + 256), -1, dtype=torch.int16, device=dev).view(torch.bfloat16)
        view = out[:, :rows * cols].view(n, rows, cols)
        DQ.dequant_experts(to_dev(raw, dev), stride, t, n, rows, cols, view)
        torch.cuda.synchronize()
        got = bf16_bits_of(out)
        for e in range(n):
            exp = R.dequant_experts(raw[e, :rows * rb], t, 1, rows, cols).reshape(-1)
            assert np.array_equal(got[e, :rows * cols], exp), f"type {t} expert {e} rows {rows} cols {cols}"
            assert np.all(got[e, rows * cols:] == 0xFFFF), "wrote past the expert"


def test_quantize_q8_1_matches_reference_quantizer(dev):
    import torch

    from kt_prefill_lend_amd import _lib

    rng = np.random.default_rng(7)
    T, K = 5, 700
    xb = R.bf16_bits(rng.standard_normal((T, K)).astype(np.float32) * 3)
    xb[1, 64:96] = 0  # an all-zero block
    x = bf16_tensor(xb, dev)
    rb = _lib.lib().ktmi_q8_1_row_bytes(K)
    out = torch.zeros((T, rb), dtype=torch.uint8, device=dev)
    _lib.check(_lib.lib().ktmi_quantize_q8_1(x.data_ptr(), _lib.KTMI_BF16, K, T, out.data_ptr(), 0))
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(T, -1, 36)
    qs, d, s, _ = R.quantize_q8_1(R.bf16_to_f32(xb))
    exp = R.q8_1_pack(qs, d, s).reshape(T, -1, 36)
    assert np.array_equal(got[..., 4:], exp[..., 4:]), "quants"
    assert np.array_equal(got[..., 0:2], exp[..., 0:2]), "d"
    gs = R.f16_bits_to_f32(got[..., 2:4].copy().view(np.uint16)[..., 0])
    assert np.allclose(gs, s, rtol=2e-3, atol=1e-3), "sum"


def _ids_case(rng, tokens, top_k, E):
    ids = np.stack([rng.permutation(E)[:top_k] for _ in range(tokens)]).astype(np.int32)
    ids[rng.random(ids.shape) < 0.25] = -1  # cold routes
    return ids


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("per_route", [False, True])
def test_moe_a8_vec(dev, t, per_route):
    import torch

    _, M, _, _ = _pkg()
    rng = np.random.default_rng(200 + t)
    E, rows, tokens, top_k = 5, 72, 6, 3
    cols = 768 if t == R.GGML_Q8_0 else 512
    W = np.stack([random_blocks(t, rows, cols, rng) for _ in range(E)])
    ids = _ids_case(rng, tokens, top_k, E)
    xb = R.bf16_bits(rng.standard_normal((tokens, cols)).astype(np.float32))
    fn = M.moe_a8_vec_routes if per_route else M.moe_a8_vec_multi
    Y = fn(bf16_tensor(xb, dev), to_dev(W, dev), to_dev(ids.reshape(-1), dev), top_k, t, rows, tokens)
    torch.cuda.synchronize()
    got = Y.float().cpu().numpy()
    ref = R.moe_a8_vec(R.bf16_to_f32(xb), W, ids.reshape(-1), top_k, t, rows, tokens)
    cold = ids.reshape(-1) < 0
    assert np.all(got[cold] == 0)
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 1e-2 * scale + 1e-6, (np.abs(got - ref).max(), scale)
    assert R.rel_errors(got, ref)[0] < 5e-3


def test_moe_a8_vec_pointer_table(dev):
    """W as an int64 table of per-slot addresses gives the slot tensor's sums."""
    import torch

    _, M, _, _ = _pkg()
    t = R.GGML_Q4_K
    rng = np.random.default_rng(5)
    E, rows, cols, tokens, top_k = 4, 32, 512, 2, 2
    W = np.stack([random_blocks(t, rows, cols, rng) for _ in range(E)])
    Wd = to_dev(W, dev)
    # slots at scattered addresses: copies in a bigger buffer, reversed order
    big = torch.zeros((E * 2, rows, W.shape[2]), dtype=torch.uint8, device=dev)
    for s in range(E):
        big[2 * (E - 1 - s)].copy_(Wd[s])
    table = torch.tensor([big[2 * (E - 1 - s)].data_ptr() for s in range(E)], dtype=torch.int64, device=dev)
    ids = to_dev(np.array([0, 3, 2, 0], np.int32), dev)
    x = bf16_tensor(R.bf16_bits(rng.standard_normal((tokens, cols)).astype(np.float32)), dev)
    a = M.moe_a8_vec_multi(x, Wd, ids, top_k, t, rows, tokens)
    b = M.moe_a8_vec_multi(x, table, ids, top_k, t, rows, tokens, table=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_window_equals_per_route(dev):
    """The window build and the per-route build give identical rows (the reference's
    kt-gguf-moe-multi-build.py:28-32 property)."""
    import torch

    _, M, _, _ = _pkg()
    rng = np.random.default_rng(11)
    t, E, rows, cols, tokens, top_k = R.GGML_Q6_K, 3, 64, 512, 9, 2
    W = to_dev(np.stack([random_blocks(t, rows, cols, rng) for _ in range(E)]), dev)
    ids = to_dev(_ids_case(rng, tokens, top_k, E).reshape(-1), dev)
    x = bf16_tensor(R.bf16_bits(rng.standard_normal((tokens, cols)).astype(np.float32)), dev)
    a = M.moe_a8_vec_multi(x, W, ids, top_k, t, rows, tokens)
    b = M.moe_a8_vec_routes(x, W, ids, top_k, t, rows, tokens)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_hot_route(dev):
    import torch

    *_, C = _pkg()
    rng = np.random.default_rng(3)
    E, n = 300, 1000
    ids = rng.integers(0, E, size=(n // 4, 4)).astype(np.int32)
    log2slot = np.full(E, -1, np.int32)
    hot = rng.permutation(E)[:40]
    log2slot[hot] = np.arange(40)
    log2cpu = np.where(log2slot >= 0, -1, np.arange(E)).astype(np.int32)
    counts = np.zeros(E, np.float32)
    counts_d = to_dev(counts, dev)
    s, c = C.route_native(to_dev(ids, dev), to_dev(log2slot, dev), to_dev(log2cpu, dev), counts_d)
    torch.cuda.synchronize()
    es, ec = R.route(ids, log2slot, log2cpu, counts)
    assert np.array_equal(s.cpu().numpy(), es) and np.array_equal(c.cpu().numpy(), ec)
    assert np.array_equal(counts_d.cpu().numpy(), counts)


def test_silu_and_mul(dev):
    import torch

    _, _, H, _ = _pkg()
    rng = np.random.default_rng(4)
    hb = R.bf16_bits(rng.standard_normal((37, 2 * 96)).astype(np.float32) * 4)
    got = bf16_bits_of(H.silu_and_mul(bf16_tensor(hb, dev)))
    torch.cuda.synchronize()
    exp = R.silu_and_mul(hb)
    diff = np.abs(got.astype(np.int32) - exp.astype(np.int32))
    assert diff.max() <= 1  # one bf16 ulp (exp implementation)
    assert (diff == 0).mean() > 0.97


def test_combine_bit_exact(dev):
    import torch

    _, _, H, _ = _pkg()
    rng = np.random.default_rng(6)
    T, k, K = 9, 8, 320
    ob = R.bf16_bits(rng.standard_normal((T, k, K)).astype(np.float32))
    w = rng.random((T, k)).astype(np.float32)
    got = bf16_bits_of(H._combine(bf16_tensor(ob, dev).view(T, k, K), to_dev(w, dev)))
    torch.cuda.synchronize()
    assert np.array_equal(got, R.combine(ob, w))


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("tokens", [2, 4])
def test_dense_a8_vec(dev, t, tokens):
    """dense_a8_vec (hot/kt_gguf_moe_multi.py:98-112): a dense GGUF linear of 520 rows (past
    DENSE_MIN_ROWS, not a multiple of 32) run as a one-expert MoE. Its rows are the MoE GEMV's
    with every token on expert 0, bit for bit, and the oracle's literal vec_dot sums within
    the GEMV tests' bound."""
    import torch

    _, M, _, _ = _pkg()
    rng = np.random.default_rng(300 + 7 * t + tokens)
    rows = 520
    cols = 768 if t == R.GGML_Q8_0 else 512
    Wn = random_blocks(t, rows, cols, rng)
    W = to_dev(Wn, dev)
    xb = R.bf16_bits(rng.standard_normal((tokens, cols)).astype(np.float32))
    x = bf16_tensor(xb, dev)
    assert M.dense_ok(x, W, t)
    y = M.dense_a8_vec(x, W, t)
    zeros = torch.zeros(tokens, dtype=torch.int32, device=dev)
    y_moe = M.moe_a8_vec_multi(x, W.view(1, rows, -1), zeros, 1, t, rows, tokens)
    torch.cuda.synchronize()
    assert y.shape == (tokens, rows) and torch.equal(y, y_moe.view(tokens, rows))
    got = y.float().cpu().numpy()
    ref = R.moe_a8_vec(R.bf16_to_f32(xb), Wn[None], np.zeros(tokens, np.int32), 1, t, rows, tokens)
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 1e-2 * scale + 1e-6, (np.abs(got - ref).max(), scale)
    assert R.rel_errors(got, ref)[0] < 5e-3
