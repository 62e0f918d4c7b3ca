"""Writes tests/golden/dequant_golden.npz: seeded GGUF blocks of Q8_0, Q4_K, Q6_K and IQ3_S
with their fp32 dequantised values, decoded here by plain Python loops laid out like
ggml's dequantize_row_* (a second formulation, independent of oracle/gguf_ref.py's index
arithmetic). The reference repository holds no vectors for this path, so these blocks are
pinned by that loop form and by the IQ3_S codebook hash.

    python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
OUT = Path(__file__).resolve().parent / "dequant_golden.npz"


def _grid():
    import re

    txt = (ROOT / "kt-prefill-lend_amd" / "csrc" / "iq3s_grid.inc").read_text()
    body = "\n".join(l for l in txt.splitlines() if not l.lstrip().startswith("//"))
    return [int(v, 16) for v in re.findall(r"0x([0-9a-fA-F]{8})u", body)]


def f16(b, off):
    return float(np.frombuffer(bytes(b[off:off + 2]), dtype=np.float16)[0])


F = np.float32


def deq_q8_0(b):
    d = F(f16(b, 0))
    return [F(d * F(int(np.int8(np.uint8(b[2 + i]))))) for i in range(32)]


def deq_q4_k(b):
    d, dmin = F(f16(b, 0)), F(f16(b, 2))
    s = [int(v) for v in b[4:16]]

    def scale_min(j):
        if j < 4:
            return s[j] & 63, s[j + 4] & 63
        return (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j] >> 6) << 4)

    y = []
    q = 16
    is_ = 0
    for _ in range(0, 256, 64):
        sc, m = scale_min(is_)
        d1, m1 = F(d * F(sc)), F(dmin * F(m))
        sc, m = scale_min(is_ + 1)
        d2, m2 = F(d * F(sc)), F(dmin * F(m))
        y += [F(F(d1 * F(b[q + l] & 0xF)) - m1) for l in range(32)]
        y += [F(F(d2 * F(b[q + l] >> 4)) - m2) for l in range(32)]
        q += 32
        is_ += 2
    return y


def deq_q6_k(b):
    d = F(f16(b, 208))
    y = [F(0)] * 256
    ql, qh, sc = 0, 128, 192
    for n in range(0, 256, 128):
        for l in range(32):
            is_ = l // 16
            q1 = ((b[ql + l] & 0xF) | (((b[qh + l] >> 0) & 3) << 4)) - 32
            q2 = ((b[ql + l + 32] & 0xF) | (((b[qh + l] >> 2) & 3) << 4)) - 32
            q3 = ((b[ql + l] >> 4) | (((b[qh + l] >> 4) & 3) << 4)) - 32
            q4 = ((b[ql + l + 32] >> 4) | (((b[qh + l] >> 6) & 3) << 4)) - 32
            for off, qv, si in ((0, q1, 0), (32, q2, 2), (64, q3, 4), (96, q4, 6)):
                scv = int(np.int8(np.uint8(b[sc + is_ + si])))
                y[n + l + off] = F(F(d * F(scv)) * F(qv))
        ql += 64
        qh += 32
        sc += 8
    return y


def deq_iq3_s(b, grid):
    d = F(f16(b, 0))
    y = []
    qs, qh, signs = 2, 66, 74
    for ib32 in range(0, 8, 2):
        sb = b[106 + ib32 // 2]
        for half, db in ((0, F(d * F(1 + 2 * (sb & 0xF)))), (1, F(d * F(1 + 2 * (sb >> 4))))):
            h = b[qh + half]
            for l in range(4):
                g1 = grid[b[qs + 2 * l] | ((h << (8 - 2 * l)) & 256)]
                g2 = grid[b[qs + 2 * l + 1] | ((h << (7 - 2 * l)) & 256)]
                for j in range(4):
                    v = F(db * F((g1 >> (8 * j)) & 0xFF))
                    y.append(-v if b[signs + l] & (1 << j) else v)
                for j in range(4):
                    v = F(db * F((g2 >> (8 * j)) & 0xFF))
                    y.append(-v if b[signs + l] & (1 << (j + 4)) else v)
            qs += 8
            signs += 4
        qh += 2
    return y


def make(seed=20261201):
    rng = np.random.default_rng(seed)
    grid = _grid()
    out = {}
    spec = {8: (34, (0,), deq_q8_0), 12: (144, (0, 2), deq_q4_k), 14: (210, (208,), deq_q6_k),
            21: (110, (0,), lambda b: deq_iq3_s(b, grid))}
    for t, (ts, f16_offs, fn) in spec.items():
        nb = 12
        raw = rng.integers(0, 256, size=(nb, ts), dtype=np.uint8)
        for i in range(nb):
            for off in f16_offs:
                v = np.float16(rng.uniform(-0.06, 0.06))
                raw[i, off:off + 2] = np.frombuffer(v.tobytes(), np.uint8)
        raw[0, :] = 0  # an all-zero block
        vals = np.array([fn([int(v) for v in raw[i]]) for i in range(nb)], dtype=np.float32)
        out[f"raw_{t}"] = raw
        out[f"val_{t}"] = vals
    np.savez(OUT, **out)
    return OUT


if __name__ == "__main__":
    print(make())
