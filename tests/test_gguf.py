"""The GGUF container reader (header, metadata, tensor table, alignment, errors), the
expert reader's TP slicing and bank building, and the hot cache filling its slots from
those banks (all on the CPU)."""
import struct
from types import SimpleNamespace

import numpy as np
import pytest

from helpers import make_expert_gguf
from oracle import gguf_ref as R


def _pkg():
    import kt_prefill_lend_amd.gguf as G
    import kt_prefill_lend_amd.kt_gguf_hot as H

    return G, H


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _hand_built(version=3, magic=0x46554747, align_kv=None, dup_key=False, dup_tensor=False):
    """A GGUF byte string assembled field by field from the format's layout (independent of
    the library's writer): 13 metadata values of every type and two tensors."""
    kv = [
        ("a.u8", 0, struct.pack("<B", 200)), ("a.i8", 1, struct.pack("<b", -5)), ("a.u16", 2, struct.pack("<H", 65000)),
        ("a.i16", 3, struct.pack("<h", -300)), ("a.u32", 4, struct.pack("<I", 4000000000)),
        ("a.i32", 5, struct.pack("<i", -7)), ("a.f32", 6, struct.pack("<f", 0.25)), ("a.bool", 7, struct.pack("<B", 1)),
        ("a.str", 8, _s("héllo")), ("a.arr", 9, struct.pack("<IQ", 8, 2) + _s("x") + _s("yz")),
        ("a.arr32", 9, struct.pack("<IQ", 4, 3) + struct.pack("<3I", 1, 2, 3)),
        ("a.u64", 10, struct.pack("<Q", 2 ** 40 + 1)), ("a.i64", 11, struct.pack("<q", -(2 ** 40))),
        ("a.f64", 12, struct.pack("<d", -1.5)),
    ]
    if align_kv is not None:
        kv.append(("general.alignment",) + align_kv)
    if dup_key:
        kv.append(("a.u8", 0, struct.pack("<B", 1)))
    t0 = np.arange(2 * 34, dtype=np.uint8)        # Q8_0 [1, 2, 32]... 2 rows of 32 values
    t1 = (np.arange(4 * 4, dtype=np.uint8) * 3)  # F32 [4] -> 16 bytes
    names = ["t.q8", "t.q8" if dup_tensor else "t.f32"]
    align = 32 if align_kv is None or align_kv[0] != 4 else struct.unpack("<I", align_kv[1])[0]
    head = struct.pack("<IIQQ", magic, version, 2, len(kv))
    head += b"".join(_s(k) + struct.pack("<I", vt) + v for k, vt, v in kv)
    off1 = (t0.nbytes + align - 1) // align * align
    head += _s(names[0]) + struct.pack("<I", 2) + struct.pack("<2Q", 32, 2) + struct.pack("<IQ", 8, 0)
    head += _s(names[1]) + struct.pack("<I", 1) + struct.pack("<Q", 4) + struct.pack("<IQ", 0, off1)
    data_off = (len(head) + align - 1) // align * align
    body = head + b"\0" * (data_off - len(head)) + t0.tobytes() + b"\0" * (off1 - t0.nbytes) + t1.tobytes()
    return body, data_off, off1, t0, t1


def test_reader_known_answer(tmp_path):
    G, _ = _pkg()
    body, data_off, off1, t0, t1 = _hand_built()
    p = tmp_path / "k.gguf"
    p.write_bytes(body)
    f = G.GGUFFile(str(p))
    m = f.metadata
    assert f.version == 3 and f.alignment == 32 and f.data_offset == data_off
    assert (m["a.u8"], m["a.i8"], m["a.u16"], m["a.i16"], m["a.u32"], m["a.i32"]) == (200, -5, 65000, -300, 4000000000, -7)
    assert m["a.f32"] == 0.25 and m["a.bool"] is True and m["a.str"] == "héllo"
    assert m["a.arr"] == ["x", "yz"] and m["a.arr32"] == [1, 2, 3]
    assert m["a.u64"] == 2 ** 40 + 1 and m["a.i64"] == -(2 ** 40) and m["a.f64"] == -1.5
    assert f.metadata_types["a.arr"] == G.GV_ARRAY and f.metadata_types["a.u64"] == G.GV_UINT64
    q8 = f.tensors["t.q8"]
    assert q8["shape"] == [2, 32] and q8["type"] == 8 and q8["offset"] == data_off and q8["n_bytes"] == 68
    assert f.tensors["t.f32"]["offset"] == data_off + off1 and f.tensors["t.f32"]["n_bytes"] == 16
    assert np.array_equal(f.raw("t.q8"), t0) and np.array_equal(f.raw("t.f32"), t1)
    # a custom alignment moves the data section and the second tensor
    body, data_off, off1, t0, t1 = _hand_built(align_kv=(4, struct.pack("<I", 64)))
    p.write_bytes(body)
    f = G.GGUFFile(str(p))
    assert f.alignment == 64 and f.data_offset % 64 == 0 and f.data_offset == data_off
    assert np.array_equal(f.raw("t.f32"), t1)


@pytest.mark.parametrize("bad,err", [
    (dict(magic=0x46554746), "magic"), (dict(version=1), "version"), (dict(dup_key=True), "duplicate"),
    (dict(dup_tensor=True), "duplicate tensor"), (dict(align_kv=(5, struct.pack("<i", 64))), "uint32"),
    (dict(align_kv=(4, struct.pack("<I", 48))), "power of two"),
])
def test_reader_rejects(tmp_path, bad, err):
    G, _ = _pkg()
    p = tmp_path / "b.gguf"
    p.write_bytes(_hand_built(**bad)[0])
    with pytest.raises((ValueError, KeyError), match=err):
        G.GGUFFile(str(p))


def test_reader_rejects_truncated(tmp_path):
    G, _ = _pkg()
    body = _hand_built()[0]
    p = tmp_path / "t.gguf"
    for cut in (10, 60, len(body) - 8):
        p.write_bytes(body[:cut])
        with pytest.raises(ValueError, match="truncated|past the end"):
            G.GGUFFile(str(p))


def test_writer_round_trip(tmp_path):
    G, _ = _pkg()
    rng = np.random.default_rng(0)
    a = rng.integers(0, 256, 3 * 144, dtype=np.uint8)
    b = rng.integers(0, 256, 210, dtype=np.uint8)
    p = tmp_path / "w.gguf"
    G.write_gguf(str(p), {"k.s": "v", "k.i": 5, "k.big": G.GV(G.GV_UINT64, 7), "k.l": [1.5, 2.5], "k.b": False},
                 [("x", (3, 256), 12, a), ("y", (256,), 14, b)], alignment=128)
    f = G.GGUFFile(str(p))
    assert f.metadata["k.s"] == "v" and f.metadata["k.i"] == 5 and f.metadata["k.big"] == 7
    assert f.metadata_types["k.big"] == G.GV_UINT64 and f.metadata["k.l"] == [1.5, 2.5] and f.metadata["k.b"] is False
    assert f.alignment == 128 and all(t["offset"] % 128 == 0 for t in f.tensors.values())
    assert f.tensors["x"]["shape"] == [3, 256] and np.array_equal(f.raw("x"), a) and np.array_equal(f.raw("y"), b)


@pytest.mark.parametrize("with_keys", [True, False])
def test_expert_reader_slices_and_banks(tmp_path, with_keys):
    """TP slicing (rank r of world 2): gate/up rows [N r, N (r+1)), down the block-aligned
    columns; dequantising the slices gives exactly the matching part of the full tensor."""
    G, H = _pkg()
    E, N, K, world = 5, 256, 512, 2
    types = (R.GGML_Q4_K, R.GGML_Q4_K, R.GGML_Q6_K)
    p = tmp_path / "e.gguf"
    raw = make_expert_gguf(p, 2, E, N, K, types, world=world, metadata=with_keys)
    rd = H.GGUFExperts(str(p))
    assert (rd.E, rd.inter, rd.K, rd.num_layers) == (E, N * world, K, 2)
    assert rd.types(1) == types
    ids = [4, 0, 2]
    for rank in range(world):
        g = rd.slice(1, "gate", N, rank, ids).numpy()
        assert np.array_equal(g, raw[(1, "gate")][ids, N * rank:N * (rank + 1)])
        d = rd.slice(1, "down", N, rank, ids).numpy()
        full = R.dequant_rows(raw[(1, "down")][ids].reshape(len(ids) * K, -1), types[2], N * world)
        part = R.dequant_rows(d.reshape(len(ids) * K, -1), types[2], N)
        assert np.array_equal(part, full[:, N * rank:N * (rank + 1)])
        gate, up, down = rd.banks(1, N, rank, p2l=[3, 1, 4, 0, 2])
        assert gate.shape == (E, N * R.row_bytes(K, types[0])) and down.shape == (E, K * R.row_bytes(N, types[2]))
        assert np.array_equal(up.numpy()[2], raw[(1, "up")][4, N * rank:N * (rank + 1)].reshape(-1))
        assert np.array_equal(down.numpy()[0], rd.slice(1, "down", N, rank, [3]).numpy().reshape(-1))
    assert H._reader(str(p)).E == E  # a GGUF path needs no registration


def test_expert_reader_rejects_unaligned_down(tmp_path):
    _, H = _pkg()
    p = tmp_path / "u.gguf"
    make_expert_gguf(p, 1, 2, 128, 256, (R.GGML_Q8_0, R.GGML_Q8_0, R.GGML_Q4_K), world=2)
    rd = H.GGUFExperts(str(p))
    with pytest.raises(ValueError, match="block-aligned"):
        rd.slice(0, "down", 128, 1, [0])  # Q4_K blocks of 256 values, a 128-column part


def test_hot_cache_fills_from_banks(tmp_path, monkeypatch):
    """Slots seeded from a placement map, filled from the reader's own banks; swaps and
    fill_empty copy the candidate experts' exact bytes; the tables stay consistent."""
    import torch

    import kt_prefill_lend_amd.kt_hot_cache as C

    _, H = _pkg()
    monkeypatch.setattr(C, "OWN_BANKS", "own")
    E, N, K, L, S = 8, 256, 256, 2, 3
    types = (R.GGML_Q8_0, R.GGML_Q8_0, R.GGML_Q6_K)
    p = tmp_path / "h.gguf"
    raw = make_expert_gguf(p, L, E, N, K, types)
    rd = H.GGUFExperts(str(p))
    cache = C.HotCache(L, E, S, "cpu")
    layers = []
    for li in range(L):
        lay = SimpleNamespace(w13_qweight=torch.zeros((S, 2 * N, R.row_bytes(K, types[0])), dtype=torch.uint8),
                              w2_qweight=torch.zeros((S, K, R.row_bytes(N, types[2])), dtype=torch.uint8))
        cache.layers[li] = (SimpleNamespace(reader=rd, N=N, rank=0), lay)
        layers.append(lay)

    def slot_is(li, s, e):
        w13, w2 = layers[li].w13_qweight[s].numpy(), layers[li].w2_qweight[s].numpy()
        return (np.array_equal(w13[:N], raw[(li, "gate")][e]) and np.array_equal(w13[N:], raw[(li, "up")][e])
                and np.array_equal(w2, raw[(li, "down")][e]))

    p2l = [[5, 1, 7, 0, 2, 3, 4, 6], [2, 4, 6, 0, 1, 3, 5, 7]]
    cache.seed(p2l=p2l)
    assert cache.check_tables() == ""
    for li in range(L):
        for s in range(S):
            if p2l[li][s] != s:
                assert slot_is(li, s, p2l[li][s])
    counts = torch.zeros(L, E)
    counts[0, 6] = 50.0  # hot, not resident in layer 0
    counts[0, 1] = 1.0   # the coldest resident of layer 0 (slot 1)
    counts[0, 5], counts[0, 7] = 20.0, 20.0
    plan = cache.plan_swaps(counts)
    assert plan == [(0, 1, 6)]
    for li, s, c in plan:
        cache.assign(li, s, c)
        cache.load_slot(li, s, c)
    cache.push_tables()
    assert cache.check_tables() == "" and slot_is(0, 1, 6)
    assert abs(cache.gpu_share(counts) - (20 + 50 + 20) / 91) < 1e-9
    # an emptied slot is refilled with the hottest non-resident
    cache.assign(1, 2, C.EMPTY)
    counts[1, 7] = 9.0
    assert cache.fill_empty(counts) == 1 and cache.resident[1][2] == 7 and slot_is(1, 2, 7)
    cache.push_tables()
    assert cache.check_tables() == ""
