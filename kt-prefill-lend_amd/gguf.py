"""GGUF expert-block formats: type ids, block geometry, row sizes and host quantisers.

Block geometry follows hot/kt_gguf_hot.py:76-91 (BLOCK_INFO, _row_bytes); the four
types with kernels here are the ones the hot path's configurations use.
"""
from __future__ import annotations

import numpy as np

from . import _lib

GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_Q6_K = 14
GGML_IQ3_S = 21
TYPE_NAMES = {GGML_Q8_0: "Q8_0", GGML_Q4_K: "Q4_K", GGML_Q6_K: "Q6_K", GGML_IQ3_S: "IQ3_S"}
NAME_TYPES = {v: k for k, v in TYPE_NAMES.items()}

# ggml type -> (values per block, bytes per block); the reference's table (kt_gguf_hot.py:76-80)
BLOCK_INFO = {
    8: (32, 34), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
    16: (256, 66), 19: (256, 74), 20: (32, 18), 21: (256, 110), 22: (256, 82), 23: (256, 136),
    18: (256, 98), 42: (64, 18),
}
# types with kernels in libktmi (the rest of BLOCK_INFO are sizes only)
KERNEL_TYPES = frozenset(TYPE_NAMES)


def row_bytes(cols: int, t: int) -> int:
    """Bytes of a row of `cols` values of ggml type t (hot/kt_gguf_hot.py:88-91)."""
    blck, ts = BLOCK_INFO[t]
    assert cols % blck == 0, (cols, t)
    return cols // blck * ts


def quantize_rows(x: np.ndarray, t: int, threads: int = 0) -> np.ndarray:
    """fp32 [rows, cols] -> uint8 [rows, row_bytes(cols, t)] on the host CPU."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    out = np.empty((rows, row_bytes(cols, t)), dtype=np.uint8)
    rc = _lib.lib().ktmi_quantize_rows_host(x.ctypes.data, rows, cols, t, out.ctypes.data, threads)
    _lib.check(rc, "quantize_rows_host")
    return out


# ---------------------------------------------------------------- GGUF container files
#
# The file layout (GGUF v2/v3, little endian):
#   u32 magic "GGUF", u32 version, u64 tensor count, u64 metadata count,
#   metadata: string key, u32 value type, value (strings are u64 length + bytes, arrays
#             u32 element type + u64 count + elements),
#   tensor infos: string name, u32 n_dims, u64 dims[n_dims] (innermost first), u32 ggml
#             type, u64 offset into the data section,
#   padding to general.alignment (32 when absent), then the data section.
# The reader follows the checks of the reference's header parser (K:3712-3810): bad magic,
# unsupported version, duplicate keys or tensors, a non-u32 or non-power-of-two alignment
# are errors.

GGUF_MAGIC = 0x46554747  # b"GGUF"
GGUF_VERSIONS = (2, 3)
GGUF_DEFAULT_ALIGNMENT = 32
(GV_UINT8, GV_INT8, GV_UINT16, GV_INT16, GV_UINT32, GV_INT32, GV_FLOAT32, GV_BOOL, GV_STRING, GV_ARRAY,
 GV_UINT64, GV_INT64, GV_FLOAT64) = range(13)
_GV_SCALAR = {GV_UINT8: "<u1", GV_INT8: "<i1", GV_UINT16: "<u2", GV_INT16: "<i2", GV_UINT32: "<u4",
              GV_INT32: "<i4", GV_FLOAT32: "<f4", GV_BOOL: "<u1", GV_UINT64: "<u8", GV_INT64: "<i8",
              GV_FLOAT64: "<f8"}


class GGUFFile:
    """A GGUF file's metadata and tensor table over a private (copy-on-write) memory map:
    arrays over it are writable views, so torch takes them without a read-only warning, and
    no write through them can reach the file (a written page becomes this process's copy).

    metadata: key -> value (numbers, str, or lists for arrays); metadata_types: key -> value
    type; tensors: name -> {"shape": outermost-first dims, "type": ggml type, "offset":
    absolute byte offset, "n_elements", "n_bytes"}."""

    def __init__(self, path: str):
        import mmap
        import struct

        self.path = path
        with open(path, "rb") as f:
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_COPY)
        mm = self._mm
        size = len(mm)

        def need(off, n):
            if off + n > size:
                raise ValueError(f"{path}: truncated GGUF (needs {off + n} bytes, has {size})")

        def u32(off):
            need(off, 4)
            return struct.unpack_from("<I", mm, off)[0]

        def u64(off):
            need(off, 8)
            return struct.unpack_from("<Q", mm, off)[0]

        def string(off):
            n = u64(off)
            need(off + 8, n)
            return bytes(mm[off + 8:off + 8 + n]).decode("utf-8"), off + 8 + n

        def value(off, vt):
            if vt == GV_STRING:
                return string(off)
            if vt in _GV_SCALAR:
                dt = np.dtype(_GV_SCALAR[vt])
                need(off, dt.itemsize)
                v = np.frombuffer(mm, dtype=dt, count=1, offset=off)[0]
                v = bool(v) if vt == GV_BOOL else v.item()
                return v, off + dt.itemsize
            if vt == GV_ARRAY:
                et, n = u32(off), u64(off + 4)
                off += 12
                if et in _GV_SCALAR and et != GV_BOOL:
                    dt = np.dtype(_GV_SCALAR[et])
                    need(off, n * dt.itemsize)
                    return np.frombuffer(mm, dtype=dt, count=n, offset=off).tolist(), off + n * dt.itemsize
                out = []
                for _ in range(n):
                    v, off = value(off, et)
                    out.append(v)
                return out, off
            raise ValueError(f"{path}: unknown GGUF value type {vt}")

        if u32(0) != GGUF_MAGIC:
            raise ValueError(f"{path}: GGUF magic invalid")
        self.version = u32(4)
        if self.version not in GGUF_VERSIONS:
            raise ValueError(f"{path}: GGUF version {self.version} not supported ({GGUF_VERSIONS})")
        n_tensors, n_kv = u64(8), u64(16)
        off = 24
        self.metadata, self.metadata_types = {}, {}
        for _ in range(n_kv):
            key, off = string(off)
            vt = u32(off)
            off += 4
            if key in self.metadata:
                raise KeyError(f"{path}: duplicate metadata key {key}")
            self.metadata[key], off = value(off, vt)
            self.metadata_types[key] = vt
        infos = []
        for _ in range(n_tensors):
            name, off = string(off)
            nd = u32(off)
            off += 4
            need(off, 8 * nd)
            dims = [int(d) for d in np.frombuffer(mm, dtype="<u8", count=nd, offset=off)]
            off += 8 * nd
            t, toff = u32(off), u64(off + 4)
            off += 12
            infos.append((name, dims, t, toff))
        align = GGUF_DEFAULT_ALIGNMENT
        if "general.alignment" in self.metadata:
            if self.metadata_types["general.alignment"] != GV_UINT32:
                raise ValueError(f"{path}: general.alignment must be a uint32")
            align = int(self.metadata["general.alignment"])
            if align == 0 or align & (align - 1):
                raise ValueError(f"{path}: alignment {align} is not a power of two")
        self.alignment = align
        self.data_offset = (off + align - 1) // align * align
        self.tensors = {}
        for name, dims, t, toff in infos:
            if name in self.tensors:
                raise ValueError(f"{path}: duplicate tensor {name}")
            n = int(np.prod(dims)) if dims else 1
            nbytes = None
            if t in BLOCK_INFO:
                blck, ts = BLOCK_INFO[t]
                if dims[0] % blck:
                    raise ValueError(f"{path}: tensor {name} rows of {dims[0]} values are not whole blocks of {blck}")
                nbytes = n // blck * ts
            elif t in _PLAIN_TYPE_BYTES:
                nbytes = n * _PLAIN_TYPE_BYTES[t]
            start = self.data_offset + int(toff)
            if nbytes is not None and start + nbytes > size:
                raise ValueError(f"{path}: tensor {name} runs past the end of the file")
            self.tensors[name] = {"shape": list(reversed(dims)), "type": int(t), "offset": start,
                                  "n_elements": n, "n_bytes": nbytes}

    def has_tensor(self, name: str) -> bool:
        return name in self.tensors

    def ggml_type(self, name: str) -> int:
        return self.tensors[name]["type"]

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes: a uint8 view over the private file mapping (no copy)."""
        info = self.tensors[name]
        if info["n_bytes"] is None:
            raise ValueError(f"{self.path}: tensor {name} has ggml type {info['type']} of unknown size")
        return np.frombuffer(self._mm, dtype=np.uint8, count=info["n_bytes"], offset=info["offset"])

    def architecture(self) -> str:
        return str(self.metadata.get("general.architecture", ""))

    def model_config(self) -> dict:
        """num_experts, moe_intermediate_size, hidden_size, num_layers: the architecture's
        metadata keys, else the shapes of the routed-expert tensors."""
        arch = self.architecture()

        def key(k):
            return self.metadata.get(f"{arch}.{k}") if arch else None

        layers = 0
        while self.has_tensor(f"blk.{layers}.ffn_gate_exps.weight"):
            layers += 1
        cfg = {"num_experts": key("expert_count"), "moe_intermediate_size": key("expert_feed_forward_length"),
               "hidden_size": key("embedding_length"), "num_layers": key("block_count")}
        g = self.tensors.get("blk.0.ffn_gate_exps.weight")
        if g is not None:  # shape [E, inter, hidden]
            E, inter, hidden = g["shape"]
            cfg["num_experts"] = cfg["num_experts"] or E
            cfg["moe_intermediate_size"] = cfg["moe_intermediate_size"] or inter
            cfg["hidden_size"] = cfg["hidden_size"] or hidden
        cfg["num_layers"] = cfg["num_layers"] or layers
        missing = [k for k, v in cfg.items() if not v]
        if missing:
            raise ValueError(f"{self.path}: no {missing} in the metadata or the expert tensors")
        return {k: int(v) for k, v in cfg.items()}

    def close(self) -> None:
        self._mm.close()


# bytes per element of the plain (unblocked) ggml types
_PLAIN_TYPE_BYTES = {0: 4, 1: 2, 24: 1, 25: 2, 26: 4, 27: 8, 28: 8, 30: 2}


def _gv_encode(v, vt=None) -> bytes:
    import struct

    if vt is None:
        if isinstance(v, bool):
            vt = GV_BOOL
        elif isinstance(v, int):
            vt = GV_UINT32 if 0 <= v < 2 ** 32 else GV_INT64
        elif isinstance(v, float):
            vt = GV_FLOAT32
        elif isinstance(v, str):
            vt = GV_STRING
        elif isinstance(v, (list, tuple)):
            vt = GV_ARRAY
        else:
            raise TypeError(f"no GGUF value type for {type(v)}")
    out = struct.pack("<I", vt)
    return out + _gv_body(v, vt)


def _gv_body(v, vt) -> bytes:
    import struct

    if vt == GV_STRING:
        b = v.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    if vt in _GV_SCALAR:
        return np.array([v], dtype=_GV_SCALAR[vt]).tobytes()
    if vt == GV_ARRAY:
        items = list(v)
        if not items:
            return struct.pack("<IQ", GV_INT32, 0)
        et = _gv_encode(items[0])[:4]
        et = struct.unpack("<I", et)[0]
        return struct.pack("<IQ", et, len(items)) + b"".join(_gv_body(x, et) for x in items)
    raise ValueError(f"unknown GGUF value type {vt}")


class GV:
    """A metadata value with an explicit GGUF value type (GV(GV_UINT64, 7)); plain Python
    values are typed by write_gguf (bool, int -> uint32 or int64, float -> float32, str,
    list -> array of the first element's type)."""

    def __init__(self, vt: int, value):
        self.vt, self.value = vt, value


def write_gguf(path: str, metadata: dict, tensors, alignment: int = GGUF_DEFAULT_ALIGNMENT) -> None:
    """Writes a GGUF v3 file. metadata: key -> value (or GV); tensors: [(name, shape
    outermost first, ggml type, bytes as a uint8 array)], each placed at a multiple of the
    alignment in the data section."""
    import struct

    kv = dict(metadata)
    if alignment != GGUF_DEFAULT_ALIGNMENT:
        kv["general.alignment"] = GV(GV_UINT32, alignment)
    head = [struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(kv))]
    for k, v in kv.items():
        kb = k.encode("utf-8")
        head.append(struct.pack("<Q", len(kb)) + kb)
        head.append(struct.pack("<I", v.vt) + _gv_body(v.value, v.vt) if isinstance(v, GV) else _gv_encode(v))
    offsets, off, blobs = [], 0, []
    for name, shape, t, data in tensors:
        data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
        offsets.append(off)
        blobs.append(data)
        off += (data.nbytes + alignment - 1) // alignment * alignment
    for (name, shape, t, _), toff in zip(tensors, offsets):
        nb = name.encode("utf-8")
        dims = list(reversed([int(d) for d in shape]))
        head.append(struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims)) +
                    struct.pack(f"<{len(dims)}Q", *dims) + struct.pack("<IQ", int(t), toff))
    header = b"".join(head)
    with open(path, "wb") as f:
        f.write(header + b"\0" * ((-len(header)) % alignment))
        for data in blobs:
            f.write(data.tobytes())
            f.write(b"\0" * ((-data.nbytes) % alignment))
