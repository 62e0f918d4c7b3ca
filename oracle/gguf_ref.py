"""numpy restatement of the reference's hot-expert MoE path. TEST INFRASTRUCTURE ONLY
(only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only
to check results against).

Reference files followed (paths relative to the reference repository; `P:<n>` is line
n of trees/flash-next-gguf/sglang-v0.5.19-flash-next-gguf.patch):

  block layouts ........ hot/kt_gguf_moe_multi/ggml-common.h:55-69 (q8_0, q8_1),
                         :88-94 (q4_K), :105-112 (q6_K), :145-154 (iq3_s)
  block sizes .......... hot/kt_gguf_hot.py:76-91 (BLOCK_INFO, _row_bytes)
  IQ3_S dequant ........ P:11397-11420 (_iq3_s_kernel), grid ggml-common.h:600-665
  q8_1 quantizer ....... hot/kt_gguf_moe_multi/kt_gguf_moe_multi.cu:600-650
  vec_dot sums ......... hot/kt_gguf_moe_multi/vecdotq.cuh:169-183 + 969-983 (Q8_0),
                         :345-376 + 1326-1367 (Q4_K), :481-506 + 1625-1648 (Q6_K),
                         :1875-1899 (IQ3_S)
  window GEMV contract . hot/kt_gguf_moe_multi/kt_gguf_moe_multi.cu:75-217
  SiLU*mul ............. call site hot/kt_gguf_hot.py:260 (sgl_kernel.silu_and_mul)
  combine .............. hot/kt_gguf_hot.py:43-71 (_combine), :300-304 (mul_ + moe_sum)
  route ................ hot/kt_hot_cache.py:62-75, 121-143
  FFN check ............ P:40821-40853 (_reference_check)

How each part is pinned (tests/test_oracle.py, tests/test_host.py):
  * dequant_rows, Q4_K/Q6_K/Q8_0/IQ3_S: (1) the literal restatement of the reference's
    integer vec_dot (`vec_dot_block_literal`, index arithmetic copied in meaning from
    vecdotq.cuh) equals sum(dequant(W) * dequant(q8_1(x))) over random blocks, which
    fails for any wrong nibble, scale, sign or grid index; (2) hand-built known-answer
    blocks, checked against a second, loop-structured decode written in the order of
    ggml's dequantize_row_* (different index formulation); (3) exactness facts: every
    Q8_0/IQ3_S value and every Q4_K product d*sc*q is exact in fp32.
  * IQ3_S grid: sha256 of the table bytes taken from the reference header, strictly
    increasing, every byte odd in 1..15.
  * quantize_q8_1: closed form (amax/127, round-half-away, fp16 d and sum), brute force
    on tiny rows, |x - d*q| <= d/2 bound, zero rows.
  * moe_a8_vec: reduces to per-route vec_dot sums (window == per-route build,
    kt-gguf-moe-multi-build.py:28-32), zero rows for ids < 0, and equals a dense fp64
    x @ W^T on dequantized W and q8_1-dequantized x.
  * combine: brute force per element in fp32 (k order, bf16 roundings of _combine).
  * route / sort_routes: brute force and invariants (every route once, stable order).
  * ffn_reference: closed form on tiny inputs against a per-route fp64 loop, and
    linearity in the route weights.
  * silu_and_mul: parity unpinned against sgl-kernel (not available); checked
    against the textbook x*sigmoid(x) in fp64 to fp32 rounding.
"""
from __future__ import annotations

import hashlib
import re
from pathlib import Path

import numpy as np

GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_Q6_K = 14
GGML_IQ3_S = 21
BLOCK_INFO = {GGML_Q8_0: (32, 34), GGML_Q4_K: (256, 144), GGML_Q6_K: (256, 210), GGML_IQ3_S: (256, 110)}
IQ3S_GRID_SHA256 = "bd1af4945a1717c65610b0284e4628b9a1ba3b306fae3a06f6e5f597356e349f"

_GRID_INC = Path(__file__).resolve().parent.parent / "kt-prefill-lend_amd" / "csrc" / "iq3s_grid.inc"
_grid_cache = None


def iq3s_grid() -> np.ndarray:
    """uint32[512] codebook, parsed from the format-constant data file (checked by hash)."""
    global _grid_cache
    if _grid_cache is None:
        body = "\n".join(l for l in _GRID_INC.read_text().splitlines() if not l.lstrip().startswith("//"))
        vals = [int(v, 16) for v in re.findall(r"0x([0-9a-fA-F]{8})u", body)]
        g = np.array(vals, dtype="<u4")
        if g.size != 512 or hashlib.sha256(g.tobytes()).hexdigest() != IQ3S_GRID_SHA256:
            raise RuntimeError("IQ3_S grid data does not match the ggml table")
        _grid_cache = g
    return _grid_cache


def row_bytes(cols: int, t: int) -> int:
    """hot/kt_gguf_hot.py:88-91."""
    blck, ts = BLOCK_INFO[t]
    assert cols % blck == 0, (cols, t)
    return cols // blck * ts


# ---------------------------------------------------------------- fp conversions

def f16_bits_to_f32(u16) -> np.ndarray:
    return np.asarray(u16, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16_bits(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bit pattern, round to nearest even (NaN kept quiet)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    return np.where(nan, np.uint16(0x7FC0), r).astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x) -> np.ndarray:
    return bf16_to_f32(bf16_bits(x))


# ---------------------------------------------------------------- dequantization
# Output fp32; every op is a single IEEE fp32 op (numpy float32 arithmetic, no FMA).

def _blocks(raw: np.ndarray, t: int, cols: int) -> np.ndarray:
    blck, ts = BLOCK_INFO[t]
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    rows = raw.size // row_bytes(cols, t)
    return raw.reshape(rows, cols // blck, ts)


def _dequant_q8_0(b: np.ndarray) -> np.ndarray:
    """block_q8_0 {half d; int8 qs[32]} (ggml-common.h:55-61): y = d*q."""
    d = f16_bits_to_f32(b[..., 0:2].copy().view(np.uint16)[..., 0])
    q = b[..., 2:34].view(np.int8).astype(np.float32)
    return (d[..., None] * q).astype(np.float32)


def q4_k_scale_min(scales: np.ndarray):
    """6-bit (sc, m) of the 8 sub-blocks from scales[12] (the aux unpack of
    vecdotq.cuh:1342-1351, restated per sub-block)."""
    s = scales.astype(np.int32)
    sc = np.empty(s.shape[:-1] + (8,), np.int32)
    m = np.empty_like(sc)
    for j in range(4):
        sc[..., j] = s[..., j] & 63
        m[..., j] = s[..., j + 4] & 63
    for j in range(4, 8):
        sc[..., j] = (s[..., j + 4] & 15) | ((s[..., j - 4] >> 6) << 4)
        m[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    return sc, m


def _q4_k_fields(b: np.ndarray):
    hd = b[..., 0:4].copy().view(np.uint16)
    d = f16_bits_to_f32(hd[..., 0])
    dmin = f16_bits_to_f32(hd[..., 1])
    sc, m = q4_k_scale_min(b[..., 4:16])
    qs = b[..., 16:144].astype(np.int32)  # [.., 128]
    # element e = 64g + l: l < 32 -> low nibble of qs[32g + l], else high nibble of qs[32g + l - 32]
    q = np.empty(b.shape[:-1] + (256,), np.int32)
    for g in range(4):
        byt = qs[..., 32 * g:32 * g + 32]
        q[..., 64 * g:64 * g + 32] = byt & 15
        q[..., 64 * g + 32:64 * g + 64] = byt >> 4
    return d, dmin, sc, m, q


def _dequant_q4_k(b: np.ndarray) -> np.ndarray:
    """block_q4_K {half2 dm; u8 scales[12]; u8 qs[128]} (ggml-common.h:88-94):
    y = (d*sc_j)*q - (dmin*m_j), j = sub-block of 32."""
    d, dmin, sc, m, q = _q4_k_fields(b)
    j = np.arange(256) // 32
    d1 = (d[..., None] * sc.astype(np.float32)).astype(np.float32)   # exact
    m1 = (dmin[..., None] * m.astype(np.float32)).astype(np.float32)  # exact
    return (d1[..., j] * q.astype(np.float32) - m1[..., j]).astype(np.float32)


def _q6_k_fields(b: np.ndarray):
    ql = b[..., 0:128].astype(np.int32)
    qh = b[..., 128:192].astype(np.int32)
    sc = b[..., 192:208].view(np.int8).astype(np.int32)
    d = f16_bits_to_f32(b[..., 208:210].copy().view(np.uint16)[..., 0])
    e = np.arange(256)
    h, r = e // 128, e % 128
    c, l = r // 32, r % 32
    lo = ql[..., 64 * h + l + 32 * (c & 1)]
    nib = np.where(c < 2, lo & 15, lo >> 4)
    hi = (qh[..., 32 * h + l] >> (2 * c)) & 3
    q = (nib | (hi << 4)) - 32
    s = sc[..., 8 * h + l // 16 + 2 * c]
    return d, s, q


def _dequant_q6_k(b: np.ndarray) -> np.ndarray:
    """block_q6_K {u8 ql[128]; u8 qh[64]; i8 scales[16]; half d} (ggml-common.h:105-112):
    y = (d*sc)*q, q in -32..31."""
    d, s, q = _q6_k_fields(b)
    d1 = (d[..., None] * s.astype(np.float32)).astype(np.float32)
    return (d1 * q.astype(np.float32)).astype(np.float32)


def _iq3_s_fields(b: np.ndarray):
    grid = iq3s_grid().view(np.uint8).reshape(512, 4).astype(np.int32)
    d = f16_bits_to_f32(b[..., 0:2].copy().view(np.uint16)[..., 0])
    qs = b[..., 2:66].astype(np.int32)
    qh = b[..., 66:74].astype(np.int32)
    signs = b[..., 74:106].astype(np.int32)
    scales = b[..., 106:110].astype(np.int32)
    e = np.arange(256)
    ib, l, jj = e // 32, (e % 32) // 8, e % 8
    sub = jj // 4
    idx = qs[..., 8 * ib + 2 * l + sub] | (((qh[..., ib] >> (2 * l + sub)) & 1) << 8)
    g = grid[idx, jj % 4]
    neg = (signs[..., 4 * ib + l] >> jj) & 1
    nib = (scales[..., ib // 2] >> (4 * (ib % 2))) & 15
    return d, nib, g, neg


def _dequant_iq3_s(b: np.ndarray) -> np.ndarray:
    """block_iq3_s {half d; u8 qs[64]; u8 qh[8]; u8 signs[32]; u8 scales[4]}
    (ggml-common.h:145-154), P:11397-11420: db = d*(1+2*nib); y = neg ? -(db*g) : db*g."""
    d, nib, g, neg = _iq3_s_fields(b)
    db = (d[..., None] * (1.0 + 2.0 * nib).astype(np.float32)).astype(np.float32)
    y = (db * g.astype(np.float32)).astype(np.float32)
    return np.where(neg == 1, -y, y).astype(np.float32)


_DEQ = {GGML_Q8_0: _dequant_q8_0, GGML_Q4_K: _dequant_q4_k, GGML_Q6_K: _dequant_q6_k, GGML_IQ3_S: _dequant_iq3_s}


def dequant_rows(raw: np.ndarray, t: int, cols: int) -> np.ndarray:
    """raw uint8 [..., rows, row_bytes(cols, t)] -> fp32 [rows_total, cols]."""
    b = _blocks(raw, t, cols)
    y = _DEQ[t](b)
    return y.reshape(b.shape[0], cols)


def dequant_experts(raw: np.ndarray, t: int, n: int, rows: int, cols: int) -> np.ndarray:
    """P:11471-11498 contract: expert-major raw bytes -> bf16 bits [n, rows, cols]."""
    y = dequant_rows(np.asarray(raw).reshape(n * rows, row_bytes(cols, t)), t, cols)
    return bf16_bits(y).reshape(n, rows, cols)


# ---------------------------------------------------------------- q8_1 activations

def quantize_q8_1(x: np.ndarray):
    """kt_gguf_moe_multi.cu:600-650: per 32 values d = amax/127, q = roundf(x/d)
    (half away from zero), ds = (half(d), half(sum x)); rows zero-padded to a
    multiple of 512. Returns (qs int8 [T, Kp], d fp32 [T, Kp/32] (fp16-rounded),
    s fp32 [T, Kp/32] (fp16-rounded), d_raw fp32 (unrounded, used for q))."""
    x = np.asarray(x, dtype=np.float32)
    T, K = x.shape
    Kp = (K + 511) // 512 * 512
    xp = np.zeros((T, Kp), np.float32)
    xp[:, :K] = x
    blk = xp.reshape(T, Kp // 32, 32)
    amax = np.abs(blk).max(axis=2)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        v = (blk / d[..., None]).astype(np.float32)
    q = np.where(amax[..., None] == 0, 0, np.sign(v) * np.floor(np.abs(v) + np.float32(0.5)))
    qs = q.astype(np.int8).reshape(T, Kp)
    s = blk.sum(axis=2, dtype=np.float32)
    return qs, f16_bits_to_f32(f32_to_f16_bits(d)), f16_bits_to_f32(f32_to_f16_bits(s)), d


def q8_1_pack(qs: np.ndarray, d: np.ndarray, s: np.ndarray) -> np.ndarray:
    """block_q8_1 bytes [T, Kp/32*36] (ds half2 then 32 int8), the reference's scratch layout."""
    T, Kp = qs.shape
    nb = Kp // 32
    out = np.zeros((T, nb, 36), np.uint8)
    out[..., 0:2] = f32_to_f16_bits(d)[..., None].view(np.uint8).reshape(T, nb, 2)
    out[..., 2:4] = f32_to_f16_bits(s)[..., None].view(np.uint8).reshape(T, nb, 2)
    out[..., 4:] = qs.reshape(T, nb, 32).view(np.uint8)
    return out.reshape(T, nb * 36)


# ---------------------------------------------------------------- integer vec_dot

def _i8x4(b4: np.ndarray) -> np.ndarray:
    return b4.view(np.int8).astype(np.int32)


def vec_dot_block_literal(t: int, wb: np.ndarray, q8: np.ndarray) -> float:
    """Sum of the reference's vec_dot_<t>_q8_1 over every iqs a warp visits for one weight
    block, following the index arithmetic of vecdotq.cuh (Q8_0 :969-983, Q4_K :1326-1367,
    Q6_K :1625-1648, IQ3_S :1875-1899) in fp64. wb: the block's bytes; q8: the q8_1 blocks
    it pairs with, uint8 [QK/32, 36]. Slow; for tests on a few blocks."""
    wb = np.asarray(wb, np.uint8)
    ds = q8[:, 0:2].copy().view(np.uint16)[:, 0]
    d8 = f16_bits_to_f32(ds).astype(np.float64)
    qs8 = q8[:, 4:36]
    total = 0.0
    if t == GGML_Q8_0:
        d = float(f16_bits_to_f32(wb[0:2].copy().view(np.uint16)[0]))
        for iqs in range(0, 8, 2):  # QI8_0 = 8, VDR = 2
            sumi = 0
            for i in range(2):
                v = _i8x4(wb[2 + 4 * (iqs + i):2 + 4 * (iqs + i) + 4])
                u = _i8x4(qs8[0, 4 * (iqs + i):4 * (iqs + i) + 4])
                sumi += int((v * u).sum())
            total += d * d8[0] * sumi
    elif t == GGML_Q4_K:
        hd = wb[0:4].copy().view(np.uint16)
        dmx, dmy = float(f16_bits_to_f32(hd[0])), float(f16_bits_to_f32(hd[1]))
        sc16 = wb[4:16].copy().view(np.uint16).astype(np.int32)
        qs = wb[16:144]
        for iqs in range(0, 32, 2):  # QI4_K = 32, VDR = 2
            bq8_offset = 2 * ((iqs // 2) // 4)
            base = 16 * bq8_offset + 4 * ((iqs // 2) % 4)
            v0 = int(qs[base:base + 4].copy().view(np.int32)[0])
            v1 = int(qs[base + 16:base + 20].copy().view(np.int32)[0])
            j = bq8_offset // 2
            if j < 2:
                aux0 = sc16[j] & 0x3F3F
                aux1 = sc16[j + 2] & 0x3F3F
            else:
                aux0 = ((sc16[j + 2] >> 0) & 0x0F0F) | ((sc16[j - 2] & 0xC0C0) >> 2)
                aux1 = ((sc16[j + 2] >> 4) & 0x0F0F) | ((sc16[j] & 0xC0C0) >> 2)
            sc = [aux0 & 0xFF, aux0 >> 8]
            m = [aux1 & 0xFF, aux1 >> 8]
            sumf_d = sumf_m = 0.0
            for i in range(2):  # QR4_K
                blk = bq8_offset + i
                o = 4 * ((iqs // 2) % 4)
                u0 = qs8[blk, o:o + 4].view(np.int8).astype(np.int64)
                u1 = qs8[blk, o + 16:o + 20].view(np.int8).astype(np.int64)
                v0i = np.array([((v0 >> (4 * i)) >> (8 * k)) & 0x0F for k in range(4)], np.int64)
                v1i = np.array([((v1 >> (4 * i)) >> (8 * k)) & 0x0F for k in range(4)], np.int64)
                dot1 = int((v0i * u0).sum() + (v1i * u1).sum())
                dot2 = int(u0.sum() + u1.sum())
                sumf_d += d8[blk] * (dot1 * sc[i])
                sumf_m += d8[blk] * (dot2 * m[i])
            total += dmx * sumf_d - dmy * sumf_m
    elif t == GGML_Q6_K:
        ql, qh = wb[0:128], wb[128:192]
        scales = wb[192:208].view(np.int8).astype(np.int64)
        d = float(f16_bits_to_f32(wb[208:210].copy().view(np.uint16)[0]))
        for iqs in range(32):  # QI6_K = 32, VDR = 1
            bq8_offset = 4 * (iqs // 16) + (iqs % 16) // 8
            scale_offset = 8 * (iqs // 16) + (iqs % 16) // 4
            vh_shift = 2 * ((iqs % 16) // 8)
            vl = ql[4 * iqs:4 * iqs + 4].astype(np.int64)
            hidx = 8 * (iqs // 16) + iqs % 8
            vh = qh[4 * hidx:4 * hidx + 4].astype(np.int64) >> vh_shift
            sumf = 0.0
            for i in range(2):  # QR6_K
                sc = scales[scale_offset + 4 * i]
                vil = (vl >> (4 * i)) & 0x0F
                vih = ((vh >> (4 * i)) & 0x03) << 4
                vi = (vil | vih) - 32
                blk = bq8_offset + 2 * i
                u = qs8[blk, 4 * (iqs % 8):4 * (iqs % 8) + 4].view(np.int8).astype(np.int64)
                sumf += d8[blk] * (int((vi * u).sum()) * sc)
            total += d * sumf
    elif t == GGML_IQ3_S:
        grid = iq3s_grid()
        d = float(f16_bits_to_f32(wb[0:2].copy().view(np.uint16)[0]))
        qs, qh, signs, scl = wb[2:66], wb[66:74].astype(np.int64), wb[74:106].astype(np.int64), wb[106:110]
        for ib32 in range(8):  # QI3_XS = 8, VDR = 1
            q8v = qs8[ib32].view(np.int8).astype(np.int64)
            sumi = 0
            for l in range(4):
                i1 = int(qs[8 * ib32 + 2 * l]) | ((int(qh[ib32]) << (8 - 2 * l)) & 256)
                i2 = int(qs[8 * ib32 + 2 * l + 1]) | ((int(qh[ib32]) << (7 - 2 * l)) & 256)
                g1 = np.array([(int(grid[i1]) >> (8 * k)) & 0xFF for k in range(4)], np.int64)
                g2 = np.array([(int(grid[i2]) >> (8 * k)) & 0xFF for k in range(4)], np.int64)
                sg = int(signs[4 * ib32 + l])
                s0 = np.array([-1 if (sg >> k) & 1 else 1 for k in range(4)], np.int64)
                s1 = np.array([-1 if (sg >> (4 + k)) & 1 else 1 for k in range(4)], np.int64)
                sumi += int((g1 * s0 * q8v[8 * l:8 * l + 4]).sum()) + int((g2 * s1 * q8v[8 * l + 4:8 * l + 8]).sum())
            nib = (int(scl[ib32 // 2]) >> (4 * (ib32 % 2))) & 0xF
            total += d * (1 + 2 * nib) * d8[ib32] * sumi
    else:
        raise ValueError(t)
    return total


def _row_sums_int(t: int, wrows: np.ndarray, cols: int, qs: np.ndarray, d8: np.ndarray) -> np.ndarray:
    """Vectorised per-block value of the reference's vec_dot for every (weight row, token)
    pair: fp64 [rows, T]. wrows uint8 [rows, rb]; qs int8 [T, Kp]; d8 fp32 [T, Kp/32]."""
    b = _blocks(wrows, t, cols)
    R, NB = b.shape[0], b.shape[1]
    T = qs.shape[0]
    x = qs[:, :cols].astype(np.int64).reshape(T, cols // 32, 32)  # q8_1 sub-blocks
    dx = d8[:, :cols // 32].astype(np.float64)
    if t == GGML_Q8_0:
        d = f16_bits_to_f32(b[..., 0:2].copy().view(np.uint16)[..., 0]).astype(np.float64)  # [R, NB]
        q = b[..., 2:34].view(np.int8).astype(np.int64)  # [R, NB, 32]
        isum = np.einsum("rbk,tbk->rtb", q, x)  # [R, T, NB]
        return (d[:, None, :] * dx[None, :, :] * isum).sum(axis=2)
    if t == GGML_Q4_K:
        d, dmin, sc, m, q = _q4_k_fields(b)  # q [R, NB, 256]
        q = q.reshape(R, NB * 8, 32).astype(np.int64)
        isum = np.einsum("rjk,tjk->rtj", q, x)  # [R, T, NB*8]
        xsum = x.sum(axis=2)  # [T, NB*8]
        scj = np.repeat(d.astype(np.float64), 8, axis=1) * sc.reshape(R, -1)  # d * sc_j
        mj = np.repeat(dmin.astype(np.float64), 8, axis=1) * m.reshape(R, -1)
        return (scj[:, None, :] * dx[None] * isum).sum(2) - (mj[:, None, :] * dx[None] * xsum[None]).sum(2)
    if t == GGML_Q6_K:
        d, s, q = _q6_k_fields(b)  # s, q [R, NB, 256]
        q16 = q.reshape(R, NB * 16, 16).astype(np.int64)
        s16 = s.reshape(R, NB * 16, 16)[..., 0].astype(np.float64)
        x16 = x.reshape(T, NB * 16, 16)
        isum = np.einsum("rjk,tjk->rtj", q16, x16)  # [R, T, NB*16]
        dx16 = np.repeat(dx, 2, axis=1)
        return (np.repeat(d.astype(np.float64), 16, axis=1)[:, None, :] * s16[:, None, :] * dx16[None] * isum).sum(2)
    if t == GGML_IQ3_S:
        d, nib, g, neg = _iq3_s_fields(b)
        v = (g * np.where(neg == 1, -1, 1)).reshape(R, NB * 8, 32).astype(np.int64)
        isum = np.einsum("rjk,tjk->rtj", v, x)
        scl = np.repeat(d.astype(np.float64), 8, axis=1) * (1 + 2 * nib.reshape(R, NB * 8, 32)[..., 0])
        return (scl[:, None, :] * dx[None] * isum).sum(2)
    raise ValueError(t)


def moe_a8_vec(X: np.ndarray, W: np.ndarray, ids: np.ndarray, top_k: int, t: int, rows: int, tokens: int) -> np.ndarray:
    """Contract of kt_moe_a8_vec_multi (kt_gguf_moe_multi.cu:653-935, :75-217): X [tokens, cols]
    (fp32 values of the activations), W uint8 [E, rows, rb(cols)], ids int32 [tokens*top_k];
    route p uses token p // top_k and expert ids[p]; ids < 0 give zero rows. Returns the fp64
    value of the reference's fp32 sums, [tokens*top_k, rows] (the kernel stores them in X's
    dtype)."""
    X = np.asarray(X, np.float32)
    cols = X.shape[1]
    qs, d8, _, _ = quantize_q8_1(X)
    ids = np.asarray(ids).reshape(-1)
    Y = np.zeros((tokens * top_k, rows), np.float64)
    for e in sorted(set(int(i) for i in ids if i >= 0)):
        routes = np.nonzero(ids == e)[0]
        toks = routes // top_k
        S = _row_sums_int(t, W[e], cols, qs[toks], d8[toks])  # [rows, n_routes]
        Y[routes] = S.T
    return Y


# ---------------------------------------------------------------- elementwise parts

def silu_and_mul(h_bf16_bits: np.ndarray) -> np.ndarray:
    """[R, 2N] bf16 -> [R, N] bf16 bits: silu(gate) * up in fp32 (gate = first N columns,
    hot/kt_gguf_hot.py:17-21 row order), rounded once. Parity unpinned vs sgl-kernel."""
    h = bf16_to_f32(h_bf16_bits).astype(np.float64)
    N = h.shape[1] // 2
    g, u = h[:, :N], h[:, N:]
    a = (g / (1.0 + np.exp(-g))) * u
    return bf16_bits(a.astype(np.float32))


def combine(out_bf16_bits: np.ndarray, w: np.ndarray) -> np.ndarray:
    """hot/kt_gguf_hot.py:43-71: res[t] = bf16( sum_k fp32( bf16( out[t,k] * bf16(w[t,k]) ) ) ),
    k ascending, fp32 accumulation. out [T, top_k, K] bf16 bits, w [T, top_k] fp32."""
    o = bf16_to_f32(out_bf16_bits)
    wk = bf16_round(np.asarray(w, np.float32))
    T, k, K = o.shape
    acc = np.zeros((T, K), np.float32)
    for j in range(k):
        acc = (acc + bf16_round((o[:, j, :] * wk[:, j:j + 1]).astype(np.float32))).astype(np.float32)
    return bf16_bits(acc)


# ---------------------------------------------------------------- routing

def route(ids: np.ndarray, log2slot: np.ndarray, log2cpu: np.ndarray, counts: np.ndarray):
    """hot/kt_hot_cache.py:62-75, 121-143 for one layer: slot_ids = log2slot[ids],
    cpu_ids = log2cpu[ids], counts[ids] += 1. counts is updated in place."""
    flat = np.asarray(ids).reshape(-1)
    np.add.at(counts, flat, 1.0)
    return log2slot[flat].reshape(np.shape(ids)), log2cpu[flat].reshape(np.shape(ids))


def sort_routes(slot_ids: np.ndarray, n_slots: int):
    """Stable counting sort of routes by slot: perm (route indices, slot-major, ascending
    route index inside a slot, cold routes (-1) dropped) and seg[n_slots+1] offsets."""
    flat = np.asarray(slot_ids).reshape(-1)
    hot = np.nonzero(flat >= 0)[0]
    order = hot[np.argsort(flat[hot], kind="stable")]
    cnt = np.bincount(flat[hot], minlength=n_slots)[:n_slots]
    seg = np.zeros(n_slots + 1, np.int64)
    seg[1:] = np.cumsum(cnt)
    return order.astype(np.int32), seg


# ---------------------------------------------------------------- FFN reference

def ffn_reference(x_bf16_bits: np.ndarray, slot_ids: np.ndarray, w: np.ndarray,
                  w13_deq: np.ndarray, w2_deq: np.ndarray) -> np.ndarray:
    """P:40821-40853 (_reference_check), in fp64: for every slot e, the routes (t, k) with
    slot_ids[t, k] == e: a = silu(x_t Wg^T) * (x_t Wu^T); out_t += (a Wd^T) * w[t, k].
    w13_deq [E, 2N, K] fp32 values (rows [gate; up], hot/kt_gguf_hot.py:17-21),
    w2_deq [E, K, N]. Returns fp64 [T, K]."""
    x = bf16_to_f32(x_bf16_bits).astype(np.float64)
    T, K = x.shape
    N = w13_deq.shape[1] // 2
    ref = np.zeros((T, K), np.float64)
    for e in range(w13_deq.shape[0]):
        rows, cols = np.nonzero(slot_ids == e)
        if rows.size == 0:
            continue
        h = x[rows]
        wg = w13_deq[e, :N].astype(np.float64)
        wu = w13_deq[e, N:].astype(np.float64)
        g = h @ wg.T
        with np.errstate(over="ignore"):  # exp(-g) = inf for g < -709: silu(g) = -0, as it should
            a = g / (1.0 + np.exp(-g)) * (h @ wu.T)
        o = (a @ w2_deq[e].astype(np.float64).T) * np.asarray(w, np.float64)[rows, cols][:, None]
        np.add.at(ref, rows, o)
    return ref


def rel_errors(y: np.ndarray, ref: np.ndarray):
    """(rel L2, rel L1 = mean|err|/mean|ref| (kt-kernel K:4131-4134), cosine)."""
    y = np.asarray(y, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    d = y - ref
    l2 = np.linalg.norm(d) / max(np.linalg.norm(ref), 1e-30)
    l1 = np.abs(d).mean() / max(np.abs(ref).mean(), 1e-30)
    cos = float(y @ ref / max(np.linalg.norm(y) * np.linalg.norm(ref), 1e-30))
    return float(l2), float(l1), cos
