"""Shared input builders for the tests (seeded, small)."""
import numpy as np

from oracle import gguf_ref as R

TYPES = [R.GGML_Q8_0, R.GGML_Q4_K, R.GGML_Q6_K, R.GGML_IQ3_S]
# byte offsets of the fp16 fields inside one block
_F16_FIELDS = {R.GGML_Q8_0: (0,), R.GGML_Q4_K: (0, 2), R.GGML_Q6_K: (208,), R.GGML_IQ3_S: (0,)}


def random_blocks(t: int, rows: int, cols: int, rng: np.random.Generator) -> np.ndarray:
    """uint8 [rows, row_bytes]: uniformly random bytes (every code, sign, grid index and
    scale pattern) with the fp16 scale fields set to finite values of mixed sign."""
    blck, ts = R.BLOCK_INFO[t]
    nb = cols // blck
    b = rng.integers(0, 256, size=(rows, nb, ts), dtype=np.uint8)
    for off in _F16_FIELDS[t]:
        mag = rng.uniform(1e-4, 0.05, size=(rows, nb)).astype(np.float32)
        sign = np.where(rng.random((rows, nb)) < 0.2, -1.0, 1.0).astype(np.float32)
        h = (mag * sign).astype(np.float16).view(np.uint8).reshape(rows, nb, 2)
        b[:, :, off:off + 2] = h
    return b.reshape(rows, nb * ts)


def dequant_w(w13: np.ndarray, w2: np.ndarray, types, hidden: int, inter: int):
    """bf16-rounded fp32 weights of the slot tensors: [S, 2N, K], [S, K, N]."""
    S = w13.shape[0]
    g = R.bf16_round(R.dequant_rows(w13.reshape(S * 2 * inter, -1), types[0], hidden)).reshape(S, 2 * inter, hidden)
    d = R.bf16_round(R.dequant_rows(w2.reshape(S * hidden, -1), types[2], inter)).reshape(S, hidden, inter)
    return g, d


def gemv_layer_oracle(x_bits, topk_w, slot_ids, w13, w2, types, hidden, inter):
    """The decode path's own numerics, step by step in the oracle: q8_1(x) GEMV -> bf16,
    SiLU*mul -> bf16, q8_1(h) GEMV -> bf16, combine."""
    T, k = slot_ids.shape
    ids = slot_ids.reshape(-1)
    x = R.bf16_to_f32(x_bits)
    h13 = R.bf16_bits(R.moe_a8_vec(x, w13, ids, k, types[0], 2 * inter, T).astype(np.float32))
    h = R.silu_and_mul(h13)
    out = R.bf16_bits(R.moe_a8_vec(R.bf16_to_f32(h), w2, ids, 1, types[2], hidden, T * k).astype(np.float32))
    return R.combine(out.reshape(T, k, hidden), topk_w)


def make_expert_gguf(path, layers: int, E: int, N: int, K: int, types, seed: int = 7, metadata: bool = True,
                     world: int = 1):
    """A GGUF file with the routed-expert tensors of `layers` layers: blk.{l}.ffn_{gate,up,
    down}_exps.weight, shapes [E, N*world, K] and [E, K, N*world], random weights ~N(0, 0.02)
    quantised to `types` (gate, up, down). Returns {(layer, proj): uint8 [E, rows, rb]}."""
    from kt_prefill_lend_amd import gguf as G

    rng = np.random.default_rng(seed)
    I = N * world
    raw, tensors = {}, []
    for li in range(layers):
        for proj, t, (rows, cols) in (("gate", types[0], (I, K)), ("up", types[1], (I, K)), ("down", types[2], (K, I))):
            w = (rng.standard_normal((E * rows, cols), dtype=np.float32) * np.float32(0.02))
            q = G.quantize_rows(w, t).reshape(E, rows, -1)
            raw[(li, proj)] = q
            tensors.append((f"blk.{li}.ffn_{proj}_exps.weight", (E, rows, cols), t, q))
    md = {"general.architecture": "toymoe", "general.name": "synthetic experts"}
    if metadata:
        md.update({"toymoe.block_count": layers, "toymoe.expert_count": E, "toymoe.expert_feed_forward_length": I,
                   "toymoe.embedding_length": K})
    G.write_gguf(str(path), md, tensors)
    return raw


def scale_f16_fields(rows: np.ndarray, t: int, factor: float) -> np.ndarray:
    """A copy of GGUF rows uint8 [rows, row_bytes] of type t with every fp16 scale field (d,
    and Q4_K's dmin) multiplied by `factor`, a power of two >= 1: fp16 products by a power of
    two are exact (subnormals included) unless they overflow, which is checked, so each
    dequantised value becomes exactly `factor` times the original."""
    blck, ts = R.BLOCK_INFO[t]
    out = np.ascontiguousarray(rows).copy()
    b = out.reshape(out.shape[0], -1, ts)
    for off in _F16_FIELDS[t]:
        h = np.ascontiguousarray(b[:, :, off:off + 2]).view(np.float16)
        s = (h.astype(np.float32) * np.float32(factor)).astype(np.float16)
        assert np.all(np.isfinite(s)) and np.array_equal(s.astype(np.float32), h.astype(np.float32) * factor)
        b[:, :, off:off + 2] = s.view(np.uint8)
    return out
