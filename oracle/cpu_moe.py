"""ctypes wrapper of the oracle's C restatement of the CPU expert path (oracle/cpu_moe.c).

TEST INFRASTRUCTURE ONLY: a second oracle for the layer output (tests) and the CPU baseline
that bench.py times beside the GPU. Nothing in the product imports it.

The C code follows kt-kernel's LLAMAFILE MoE forward_many (reference
trees/kt-kernel/kt-kernel-95009ea-flash-next-gguf.patch K:2571-2800): per-token activation
rows quantised once to Q8_K (Q8_0 for Q8_0 weights), int8 block dot products per expert row
block, fp32 SiLU(gate)*up re-quantised for the down projection, fp32 weighted merge.
"""
from __future__ import annotations

import ctypes as C
import os
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libktoracle.so"
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built (make -C oracle)")
        L = C.CDLL(str(LIB_PATH))
        p = C.c_void_p
        L.cpu_moe_forward.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, p, p, p, p, p, C.c_int, C.c_int,
                                      p, C.c_int]
        L.cpu_moe_forward.restype = C.c_int
        L.cpu_moe_max_threads.restype = C.c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(C.c_void_p)


def forward(x_bf16: np.ndarray, slot_ids: np.ndarray, weights: np.ndarray, w13: np.ndarray, w2: np.ndarray,
            type13: int, type2: int, inter: int, threads: int = 0) -> np.ndarray:
    """out fp32 [T, hidden] over the routes with 0 <= slot_ids < n_slots.

    x_bf16 uint16 [T, hidden]; slot_ids int32 [T, k]; weights fp32 [T, k];
    w13 uint8 [S, 2*inter, rb13] rows [gate; up]; w2 uint8 [S, hidden, rb2]."""
    T, K = x_bf16.shape
    top_k = slot_ids.shape[1]
    S = w13.shape[0]
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    s = np.ascontiguousarray(slot_ids, dtype=np.int32)
    wt = np.ascontiguousarray(weights, dtype=np.float32)
    a13 = np.ascontiguousarray(w13)
    a2 = np.ascontiguousarray(w2)
    out = np.zeros((T, K), np.float32)
    rc = lib().cpu_moe_forward(T, K, inter, top_k, S, _ptr(x), _ptr(s), _ptr(wt), _ptr(a13), _ptr(a2), type13, type2,
                               _ptr(out), threads)
    if rc != 0:
        raise RuntimeError("cpu_moe_forward failed")
    return out


def default_threads() -> int:
    """The threads the CPU baseline uses: the CPUs this process may run on (its sched
    affinity, which is the share a job scheduler grants), else every logical CPU."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, n)


def host_info() -> dict:
    """The host the baseline ran on: logical CPUs, the affinity set, and lscpu's model,
    sockets, physical cores and threads per core."""
    import subprocess

    info = {"nproc": os.cpu_count()}
    try:
        info["affinity"] = len(os.sched_getaffinity(0))
    except AttributeError:
        pass
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        kv = {k.strip(): v.strip() for k, _, v in (line.partition(":") for line in out.splitlines()) if _}
        info["model"] = kv.get("Model name")
        sockets = int(kv.get("Socket(s)", "0") or 0)
        per_socket = int(kv.get("Core(s) per socket", "0") or 0)
        info["sockets"] = sockets
        info["physical_cores"] = sockets * per_socket if sockets and per_socket else None
        info["threads_per_core"] = int(kv.get("Thread(s) per core", "0") or 0) or None
    except Exception:  # noqa: BLE001 - lscpu missing: the counts above still stand
        pass
    return info


def _time(fn, min_seconds: float, max_seconds: float):
    fn()  # warm (page faults, the OpenMP pool)
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= min_seconds or el * (reps + 1) / reps > max_seconds:
            return reps, el


def bench(S, w, cpu_tokens: int, T: int, log=print, min_seconds: float = 10.0, max_seconds: float = 30.0,
          distinct: int = 16):
    """The CPU expert path on this host, on the first `cpu_tokens` tokens of the T-token chunk
    of workload `w` (same routing and activations as the GPU run), two legs of at least
    `min_seconds` each:
      * hot routes: the routes of the H hot experts (the GPU's share of the layer, the same
        weights): the rate compared with the GPU (`value`);
      * full layer: every route over all E experts (the CPU's job when no expert is on the
        GPU), E rows of expert weights made from `distinct` quantised experts (each row its
        own memory, so the weights stream from DRAM as E distinct experts would).
    Returns the cpu_baseline record."""
    ids, tw, slot, _ = S.routing(w, T)
    xb = S.activations(w, T)
    n = min(cpu_tokens, T)
    x, sl, wt, lid = xb[:n], slot[:n], tw[:n], ids[:n]
    w13, w2 = S.slot_tensors(w)
    threads = default_threads()
    host = host_info()
    reps, el = _time(lambda: forward(x, sl, wt, w13, w2, w.types[0], w.types[2], w.inter, threads),
                     min_seconds, max_seconds)
    tok_s = n * reps / el
    routes = int((sl >= 0).sum())
    log(f"cpu baseline, hot routes: {n} tokens ({routes} routes) x {reps} in {el:.1f}s on {threads} threads "
        f"-> {tok_s:.1f} tok/s")
    parts = [S.expert_weights(w, e, 0, threads) for e in range(distinct)]
    a13 = np.stack([parts[e % distinct][0] for e in range(w.experts)])
    a2 = np.stack([parts[e % distinct][1] for e in range(w.experts)])
    freps, fel = _time(lambda: forward(x, lid, wt, a13, a2, w.types[0], w.types[2], w.inter, threads),
                       min_seconds, max_seconds)
    ftok_s = n * freps / fel
    log(f"cpu baseline, full layer: {n} tokens ({lid.size} routes over {w.experts} experts) x {freps} in {fel:.1f}s "
        f"-> {ftok_s:.1f} tok/s")
    return {"value": round(tok_s, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"first {n} tokens of the {T}-token chunk, hot routes only ({routes} routes over the "
                      f"{w.hot} hot experts), {reps} repetitions in {el:.1f} s; C restatement of kt-kernel "
                      f"forward_many (Q8_K int8 dots, OpenMP, {threads} threads)",
            "full_layer": {"value": round(ftok_s, 1), "unit": "tokens/s", "routes": int(lid.size),
                           "experts": w.experts, "repetitions": freps, "seconds": round(fel, 1),
                           "weights": f"{distinct} distinct quantised experts over {w.experts} rows"},
            "host": host}
