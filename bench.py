#!/usr/bin/env python3
"""Hot-expert MoE layer benchmark on one MI355X.

Headline: tokens/s of one hot-expert MoE layer at a 16384-token prefill chunk (hidden 2048,
expert intermediate 512, 256 experts, top-8, 40 hot slots, Q4_K gate/up + Q6_K down, Zipf
1.1 routing), inputs resident in HBM. A step is one layer forward (route sort, gate/up
GEMM with SiLU*mul, down GEMM, weighted combine) over the chunk. Prints ONE JSON line.

Besides the headline (`value`, `roofline`, `cpu_baseline`), the line carries the other
legs: `configs` (Q8_0 512 tokens, 2K and 32K chunks, IQ3_S 16K against the MFMA peak),
`decode` (1/4/8/16-token layers against HBM), `stream` (four large layers streamed from
pinned host memory) and `hybrid` (hot routes on the GPU, cold ones on the host cores).

`sustained` repeats the headline measurement after 150 more untimed steps, once the GPU's
clocks have settled under load.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--sustained 100] [--no-cpu]
                    [--no-configs] [--no-decode] [--no-stream] [--no-hybrid]
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
HEADLINE = "q4_k+q6_k-h2048-n512-e256-k8-hot40-prefill"
DECODE = "q4_k-h2048-n512-e256-k8-hot32-decode"
STREAM = "q4_k+q6_k-h7168-n2048-e256-k8-hot24-stream4"
STAGES = ["prep", "gate_up", "mid", "down", "combine"]


def load_pkg():
    name = "kt_prefill_lend_amd"
    if name in sys.modules:
        return sys.modules[name]
    root = ROOT / "kt-prefill-lend_amd"
    spec = importlib.util.spec_from_file_location(name, root / "__init__.py", submodule_search_locations=[str(root)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


class HipEvents:
    """hipEvent_t handles through libamdhip64 (events on the stream the kernels run on)."""

    def __init__(self):
        self.h = C.CDLL("libamdhip64.so")
        self.h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.h.hipEventSynchronize.argtypes = [C.c_void_p]
        self.h.hipEventDestroy.argtypes = [C.c_void_p]

    def create(self, n):
        out = (C.c_void_p * n)()
        for i in range(n):
            e = C.c_void_p()
            assert self.h.hipEventCreate(C.byref(e)) == 0
            out[i] = e
        return out

    def record(self, e, stream):
        assert self.h.hipEventRecord(e, stream) == 0

    def ms(self, a, b):
        f = C.c_float()
        assert self.h.hipEventElapsedTime(C.byref(f), a, b) == 0
        return f.value

    def destroy(self, evs):
        for e in evs:
            self.h.hipEventDestroy(e)


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def time_layer(P, torch, desc_list, x, w, slot, mode, steps, warmup, ev: HipEvents, breakdown_steps=None,
               sample_every=4):
    """Warmup, then `steps` timed layer calls (desc_list rotates weight copies per step) with
    events around the loop and, on every `sample_every`-th call, around its gate/up and down
    GEMMs (4 events, about 1 us of stream time each, so the sampled kernel durations are those
    of the timed steps themselves at a cost of about 1 us per step). Then, enqueued right
    behind them with no host wait in between (the GPU's clocks keep rising over the first ~100
    back-to-back steps, so a pause or a later pass would see a different clock state),
    `breakdown_steps` more calls with an event at every stage boundary, for the per-stage means.
    Returns (ms per step, per-stage mean ms of the breakdown calls, output, mean ms of the
    gate/up and down GEMMs over the sampled timed calls)."""
    H, L = P.kt_gguf_hot, P._lib
    lib = L.lib()
    T, k = slot.shape
    out = torch.empty((T, desc_list[0].hidden), dtype=torch.bfloat16, device=x.device)
    need = max(lib.ktmi_moe_layer_workspace(d, T, k, mode) for d in desc_list)
    ws = torch.empty((need,), dtype=torch.uint8, device=x.device)
    stream = L.stream_ptr(x.device)
    nb = breakdown_steps or steps
    se = ev.create(2)
    stage_ev = ev.create(nb * L.STAGE_EVENTS)
    sampled = []
    if sample_every and steps > 0:  # at least the last step when there are fewer than sample_every
        sampled = [i for i in range(steps) if i % sample_every == sample_every - 1] or [steps - 1]
    kev = ev.create(4 * len(sampled)) if sampled else []  # gate/up start, end, down start, end (boundaries 1-4)
    for i in range(warmup):
        H.moe_layer(desc_list[i % len(desc_list)], x, w, slot, mode, out, ws)
    torch.cuda.synchronize()
    ev.record(se[0], stream)
    n = 0
    for i in range(steps):
        if n < len(sampled) and i == sampled[n]:
            arr = (C.c_void_p * L.STAGE_EVENTS)(None, *kev[4 * n:4 * n + 4], None)
            L.check(lib.ktmi_set_stage_events(arr, L.STAGE_EVENTS))
            H.moe_layer(desc_list[i % len(desc_list)], x, w, slot, mode, out, ws)
            L.check(lib.ktmi_set_stage_events(None, 0))
            n += 1
        else:
            H.moe_layer(desc_list[i % len(desc_list)], x, w, slot, mode, out, ws)
    ev.record(se[1], stream)
    for i in range(nb):
        arr = (C.c_void_p * L.STAGE_EVENTS)(*stage_ev[i * L.STAGE_EVENTS:(i + 1) * L.STAGE_EVENTS])
        L.check(lib.ktmi_set_stage_events(arr, L.STAGE_EVENTS))
        H.moe_layer(desc_list[i % len(desc_list)], x, w, slot, mode, out, ws)
    L.check(lib.ktmi_set_stage_events(None, 0))
    torch.cuda.synchronize()
    total = ev.ms(se[0], se[1])
    ev.destroy(se)
    per = np.zeros((nb, len(STAGES)))
    for i in range(nb):
        b = i * L.STAGE_EVENTS
        for s in range(len(STAGES)):
            per[i, s] = ev.ms(stage_ev[b + s], stage_ev[b + s + 1])
    ev.destroy(stage_ev)
    timed = None
    if sampled:
        timed = {"gate_up": float(np.mean([ev.ms(kev[4 * j], kev[4 * j + 1]) for j in range(len(sampled))])),
                 "down": float(np.mean([ev.ms(kev[4 * j + 2], kev[4 * j + 3]) for j in range(len(sampled))])),
                 "samples": len(sampled)}
        ev.destroy(kev)
    return total / steps, dict(zip(STAGES, per.mean(axis=0).tolist())), out, timed


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=16384)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-stream", action="store_true", help="skip the streamed-layers leg")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other workload shapes (Q8_0 512 tokens, 2K/32K chunks, IQ3_S 16K)")
    ap.add_argument("--no-hybrid", action="store_true", help="skip the GPU + CPU decode leg")
    ap.add_argument("--cpu-tokens", type=int, default=1024, help="tokens of the chunk timed on the CPU")
    ap.add_argument("--sustained", type=int, default=100, metavar="K",
                    help="after the headline, time K more layer steps behind 150 back-to-back untimed ones "
                         "(the GPU's clocks settle under sustained load); 0 skips this leg")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run an fp32 negate of MIB MiB (reads and writes exactly MIB MiB), the known-size "
                         "kernel that scales FETCH_SIZE/WRITE_SIZE counters to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported (there is no multi-GPU "
              f"path: the layer would shard by expert, each GPU holding its own range of hot slots)", file=sys.stderr)
        sys.exit(2)

    import torch

    P = load_pkg()
    import kt_prefill_lend_amd.kt_gguf_hot  # noqa: F401
    import kt_prefill_lend_amd.synth as S

    dev = torch.device("cuda", 0)
    ev = HipEvents()
    if args.copy_probe:
        a = torch.ones(args.copy_probe << 18, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        for _ in range(3):
            torch.neg(a, out=b)
        torch.cuda.synchronize()
        log(f"copy probe: 3 x neg over {args.copy_probe} MiB")
        del a, b
    w = S.WORKLOADS[HEADLINE]
    T = args.tokens
    t0 = time.time()
    ids, tw, slot, hot = S.routing(w, T)
    xb = S.activations(w, T)
    w13, w2 = S.slot_tensors(w)
    log(f"workload {w.name} T={T}: generated in {time.time() - t0:.1f}s, hot routes {(slot >= 0).sum()}")
    x = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
    tw_d = torch.from_numpy(tw).to(dev)
    slot_d = torch.from_numpy(slot).to(dev)
    W13 = torch.from_numpy(w13).to(dev)
    W2 = torch.from_numpy(w2).to(dev)
    H, L = P.kt_gguf_hot, P._lib
    desc = H.layer_desc(W13, W2, w.hidden, w.inter, w.types[0], w.types[2])
    ms, stages, out, timed = time_layer(P, torch, [desc], x, tw_d, slot_d, L.MODE_GROUPED, args.steps, args.warmup, ev)
    r_hot = int((slot >= 0).sum())
    flop_gu = 4.0 * w.hidden * w.inter * r_hot
    flop_dn = 2.0 * w.hidden * w.inter * r_hot
    # the GEMMs' durations in the timed steps themselves (sampled every 4th step)
    kern = {"gate_up": (flop_gu, timed["gate_up"]), "down": (flop_dn, timed["down"])}
    dom = max(kern, key=lambda k: kern[k][1])
    achieved = kern[dom][0] / (kern[dom][1] * 1e-3) / 1e12
    tok_s = T / (ms * 1e-3)
    layer_tflops = (flop_gu + flop_dn) / (ms * 1e-3) / 1e12
    log(f"layer {ms:.3f} ms/step, {tok_s / 1e6:.2f} M tok/s, {layer_tflops:.0f} TFLOP/s "
        f"({100 * layer_tflops / PEAK_BF16_TFLOPS:.1f}% of bf16 peak); GEMMs in the timed steps ms {timed}; "
        f"stages ms (breakdown pass) {stages}")

    def profiled(fname, field):
        # a figure of the dominant kernel from a committed rocprofv3 summary (None if absent)
        f = ROOT / "profiles" / fname
        try:
            rec = json.loads(f.read_text()).get(f"{HEADLINE}:T{T}:{dom}")
            return rec[field] if rec else None
        except Exception:  # noqa: BLE001
            return None

    traffic = profiled("traffic.json", "bytes")  # the median of the profiled runs
    traffic_range = profiled("traffic.json", "bytes_range")
    mfma_busy = profiled("mfma.json", "mfma_busy")
    clock = profiled("mfma.json", "clock_GHz")

    result = {
        "metric": "hot-expert MoE layer tokens/s @16K chunk; % of HBM/MFMA roofline",
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) experts quantised to GGUF, Zipf(1.1) routing)",
        "config": {"workload": w.name, "tokens": T, "hidden": w.hidden, "inter": w.inter, "experts": w.experts,
                   "top_k": w.top_k, "hot_slots": w.hot, "types": "Q4_K gate/up, Q6_K down", "hot_routes": r_hot,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                     "traffic_range": traffic_range,
                     "mfma_busy_counter": mfma_busy, "clock_GHz_counter": clock,
                     "layer_frac": round(layer_tflops / PEAK_BF16_TFLOPS, 4),
                     "kernel_ms_timed": {"gate_up": round(timed["gate_up"], 4), "down": round(timed["down"], 4),
                                         "samples": timed["samples"]},
                     "stage_ms": {k: round(v, 4) for k, v in stages.items()}},
        "cpu_baseline": None,
    }

    if args.sustained:
        # the headline's few warmup steps leave the GPU in its clock ramp (a layer step runs
        # ~0.88 ms from idle and settles near 0.68 ms after ~100 back-to-back steps); this leg
        # reports the settled rate beside it, measured the same way
        sw = 150
        ms2, st2, _, timed2 = time_layer(P, torch, [desc], x, tw_d, slot_d, L.MODE_GROUPED, args.sustained, sw, ev)
        result["sustained"] = {
            "warmup": sw, "steps": args.sustained, "ms_per_step": round(ms2, 4),
            "tokens_per_s": round(T / (ms2 * 1e-3), 1),
            "layer_frac": round((flop_gu + flop_dn) / (ms2 * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "gate_up_frac": round(flop_gu / (timed2["gate_up"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "down_frac": round(flop_dn / (timed2["down"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "kernel_ms_timed": {"gate_up": round(timed2["gate_up"], 4), "down": round(timed2["down"], 4)},
            "stage_ms": {k: round(v, 4) for k, v in st2.items()}}
        log(f"sustained: {result['sustained']}")

    if not args.no_configs:
        result["configs"] = bench_configs(P, torch, S, ev, dev)

    if not args.no_decode:
        result["decode"] = bench_decode(P, torch, S, ev, dev)

    if not args.no_stream:
        result["stream"] = bench_stream(P, torch, S, ev, dev)

    if not args.no_hybrid:
        result["hybrid"] = bench_hybrid(P, torch, S, ev, dev)

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(S, w, args.cpu_tokens, T)

    print(json.dumps(result), flush=True)


def bench_configs(P, torch, S, ev, dev, steps=10, warmup=2, sust_steps=50, sust_warmup=100):
    """The other prefill-sized workloads, one layer each in the mode the library picks: Q8_0
    at 512 tokens, the headline shapes at 2048 and 32768 tokens and IQ3_S at 16384. Reports
    tokens/s and the gate/up and down GEMMs' TFLOP/s against the bf16 MFMA peak (their
    durations sampled in the timed steps). Each leg starts from the clocks the data generation
    left the GPU at; the long chunks (16384 tokens and more) are then timed again behind
    `sust_warmup` back-to-back untimed steps (`sustained`: the clock state of a serving loop)."""
    H, L = P.kt_gguf_hot, P._lib
    lib = L.lib()
    cases = [("q8_0-h2048-n768-e128-k8-hot16", 512), (HEADLINE, 2048), (HEADLINE, 32768),
             ("iq3_s-h2048-n512-e512-k10-hot48", 16384)]
    res = {}
    for name, T in cases:
        w = S.WORKLOADS[name]
        ids, tw, slot, _ = S.routing(w, T)
        x = torch.from_numpy(S.activations(w, T).view(np.int16)).to(dev).view(torch.bfloat16)
        tw_d, slot_d = torch.from_numpy(tw).to(dev), torch.from_numpy(slot).to(dev)
        w13, w2 = S.slot_tensors(w)
        W13, W2 = torch.from_numpy(w13).to(dev), torch.from_numpy(w2).to(dev)
        desc = H.layer_desc(W13, W2, w.hidden, w.inter, w.types[0], w.types[2])
        mode = lib.ktmi_moe_layer_mode(desc, T, w.top_k)
        ms, stages, _, timed = time_layer(P, torch, [desc], x, tw_d, slot_d, mode, steps, warmup, ev)
        if timed:  # the GEMMs' durations in the timed steps
            stages = dict(stages, gate_up=timed["gate_up"], down=timed["down"])
        r_hot = int((slot >= 0).sum())
        f_gu, f_dn = 4.0 * w.hidden * w.inter * r_hot, 2.0 * w.hidden * w.inter * r_hot
        rec = {"tokens": T, "mode": "grouped" if mode == L.MODE_GROUPED else "gemv", "hot_routes": r_hot,
               "ms_per_step": round(ms, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
               "layer_frac_mfma": round((f_gu + f_dn) / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
        for k, f in (("gate_up", f_gu), ("down", f_dn)):
            if stages[k] > 0:
                rec[f"{k}_TFLOPs"] = round(f / (stages[k] * 1e-3) / 1e12, 1)
                rec[f"{k}_frac_mfma"] = round(f / (stages[k] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)
        if T >= 16384 and sust_steps > 0:
            ms2, st2, _, t2 = time_layer(P, torch, [desc], x, tw_d, slot_d, mode, sust_steps, sust_warmup, ev)
            if t2:
                st2 = dict(st2, gate_up=t2["gate_up"], down=t2["down"])
            sus = {"warmup": sust_warmup, "steps": sust_steps, "ms_per_step": round(ms2, 4),
                   "tokens_per_s": round(T / (ms2 * 1e-3), 1),
                   "layer_frac_mfma": round((f_gu + f_dn) / (ms2 * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
            for k, f in (("gate_up", f_gu), ("down", f_dn)):
                if st2[k] > 0:
                    sus[f"{k}_frac_mfma"] = round(f / (st2[k] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)
            rec["sustained"] = sus
        res[f"{name}:T{T}"] = rec
        log(f"config {name} T={T}: {rec}")
        del W13, W2, x
    return res


def bench_decode(P, torch, S, ev, dev, steps=50, warmup=5, rotate_bytes=512e6):
    """Decode-shaped layer (Q4_K, 32 hot slots) at 1/4/8/16 tokens: GB/s against HBM, for the
    decode mode (KTMI_MODE_DECODE, the library's choice from 64 routes) and the GEMV mode (the
    reference kernels' int8 numerics, its choice below 64 routes). Per mode: "hbm", the weights rotating over enough copies that the
    copies' touched bytes exceed `rotate_bytes` (twice the 256 MB Infinity Cache) at every T;
    "warm", one copy; "graph", the same rotated steps captured in one HIP graph and replayed
    (no host issue cost between the layers). GB/s = algorithmic bytes / step time (every launch
    of the step and the gaps between them). "floor": graph-replayed references on the same stream, two
    back-to-back launches of a one-block kernel per step, and a device-to-device copy of the
    step's touched weight bytes from the rotated copies (it reads them and writes as many)."""
    H, L = P.kt_gguf_hot, P._lib
    w = S.WORKLOADS[DECODE]
    w13, w2 = S.slot_tensors(w)
    from kt_prefill_lend_amd.gguf import row_bytes

    exp_bytes = 2 * w.inter * row_bytes(w.hidden, w.types[0]) + w.hidden * row_bytes(w.inter, w.types[2])
    cases = []
    for T in w.tokens:
        ids, tw, slot, _ = S.routing(w, T)
        uniq = len(set(slot[slot >= 0].tolist()))
        cases.append((T, tw, slot, uniq, max(8, int(np.ceil(rotate_bytes / (uniq * exp_bytes))))))
    ncopy = max(c[4] for c in cases)
    W13 = torch.from_numpy(w13).to(dev)
    W2 = torch.from_numpy(w2).to(dev)
    copies = [(W13.clone(), W2.clone()) for _ in range(ncopy)]
    descs = [H.layer_desc(a, b, w.hidden, w.inter, w.types[0], w.types[2]) for a, b in copies]
    log(f"decode: {ncopy} copies of the {w.hot} slots ({ncopy * (w13.nbytes + w2.nbytes) / 1e9:.2f} GB)")
    res = {}
    for T, tw, slot, uniq, nc in cases:
        x = torch.from_numpy(S.activations(w, T).view(np.int16)).to(dev).view(torch.bfloat16)
        tw_d, slot_d = torch.from_numpy(tw).to(dev), torch.from_numpy(slot).to(dev)
        nbytes = uniq * exp_bytes + 2 * T * w.hidden * 2
        out = {}
        for mname, mode in (("decode", L.MODE_DECODE), ("gemv", L.MODE_GEMV)):
            rec = {}
            for name, dl in (("hbm", descs[:nc]), ("warm", descs[:1])):
                ms, stages, _, _ = time_layer(P, torch, dl, x, tw_d, slot_d, mode, steps, warmup, ev, sample_every=0)
                gbs = nbytes / (ms * 1e-3) / 1e9
                rec[name] = {"ms_per_step": round(ms, 4), "GBps": round(gbs, 1),
                             "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                             "stage_ms_with_events": {k: round(v, 4) for k, v in stages.items()}}
            ms = time_layer_graph(P, torch, descs[:nc], x, tw_d, slot_d, mode, steps, ev)
            gbs = nbytes / (ms * 1e-3) / 1e9
            rec["graph"] = {"ms_per_step": round(ms, 4), "GBps": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
            out[mname] = rec
        out["copies"], out["rotated_bytes"] = nc, nc * uniq * exp_bytes
        out["floor"] = decode_floor(P, torch, ev, dev, copies[:nc], slot, uniq, w, steps)
        res[f"T{T}"] = {"hot_routes": int((slot >= 0).sum()), "unique_experts": uniq, "bytes": nbytes, **out}
        log(f"decode T={T}: {res[f'T{T}']}")
    del copies
    return res


def time_layer_graph(P, torch, desc_list, x, w, slot, mode, steps, ev):
    """`steps` layer calls (rotating through desc_list) captured in one HIP graph on a side
    stream; the mean step time of a replay (events around the replay on that stream), after
    two replays to warm up."""
    H, L = P.kt_gguf_hot, P._lib
    lib = L.lib()
    T, k = slot.shape
    out = torch.empty((T, desc_list[0].hidden), dtype=torch.bfloat16, device=x.device)
    ws = torch.empty((max(lib.ktmi_moe_layer_workspace(d, T, k, mode) for d in desc_list),), dtype=torch.uint8,
                     device=x.device)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for d in desc_list[:2]:
            H.moe_layer(d, x, w, slot, mode, out, ws)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(steps):
            H.moe_layer(desc_list[i % len(desc_list)], x, w, slot, mode, out, ws)
    se = ev.create(2)
    with torch.cuda.stream(s):
        g.replay()
        g.replay()
        ev.record(se[0], s.cuda_stream)
        g.replay()
        ev.record(se[1], s.cuda_stream)
    torch.cuda.synchronize()
    ms = ev.ms(se[0], se[1]) / steps
    ev.destroy(se)
    del g
    return ms


def decode_floor(P, torch, ev, dev, copies, slot, uniq, w, steps):
    """Graph-replayed references for a decode step (`steps` of them captured in one HIP graph,
    the mean step of a replay): two back-to-back launches of a one-block kernel (the
    library's remap over 8 ids), and a device-to-device copy of the step's touched weight
    bytes (the unique hot slots' w13 and w2, from the next of the rotated copies each step:
    a read of those bytes from HBM and a write of as many)."""
    L = P._lib
    lib = L.lib()
    ids = torch.zeros(8, dtype=torch.int32, device=dev)
    loc = torch.empty(8, dtype=torch.int32, device=dev)
    hot = sorted(set(slot[slot >= 0].tolist()))
    dst13 = torch.empty((len(hot),) + tuple(copies[0][0].shape[1:]), dtype=torch.uint8, device=dev)
    dst2 = torch.empty((len(hot),) + tuple(copies[0][1].shape[1:]), dtype=torch.uint8, device=dev)
    idx = torch.tensor(hot, dtype=torch.int64, device=dev)
    # the touched slots as contiguous sources in every copy (the copy leg reads exactly them)
    src = [(c13.index_select(0, idx), c2.index_select(0, idx)) for c13, c2 in copies]

    def launches(_i, st):
        for _ in range(2):
            L.check(lib.ktmi_remap_ids(ids.data_ptr(), 8, 0, 4, loc.data_ptr(), st), "remap_ids")

    def copy(i, st):
        a, b = src[i % len(src)]
        dst13.copy_(a, non_blocking=True)
        dst2.copy_(b, non_blocking=True)

    out = {}
    for name, fn in (("two_launches_ms", launches), ("copy_ms", copy)):
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            fn(0, s.cuda_stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                fn(i, s.cuda_stream)
        se = ev.create(2)
        with torch.cuda.stream(s):
            g.replay()
            ev.record(se[0], s.cuda_stream)
            g.replay()
            ev.record(se[1], s.cuda_stream)
        torch.cuda.synchronize()
        out[name] = round(ev.ms(se[0], se[1]) / steps, 4)
        ev.destroy(se)
        del g
    nb = dst13.numel() + dst2.numel()
    out["copy_bytes_read"] = nb
    out["copy_read_GBps"] = round(nb / (out["copy_ms"] * 1e-3) / 1e9, 1)
    del src
    return out


def bench_hybrid(P, torch, S, ev, dev, distinct=16, reps=200, warmup=10, rotate=8):
    """The whole decode layer of the decode workload (256 experts, 32 hot on the GPU, Q4_K)
    at 1 / 4 / 16 tokens: the hot routes on the GPU (GEMV mode), the cold ones on the host
    cores through the library's CPU engine and handoff (submit before the GPU kernels,
    sync_add after). Per step (host clock from the first call to the device synchronisation,
    median over reps): GPU half alone, CPU half alone (engine forward on host arrays) and the
    hybrid layer, the three legs interleaved step by step so that they see the same state
    of the shared host. The calls cycle through `rotate` routings (other seeds), one further
    per call, so the cold experts a call reads were last read `rotate` calls before (their
    union is reported) rather than staying in the host's caches; the CPU engine's rate is
    the bytes of the distinct cold experts a call reads over the CPU-alone time. Experts: `distinct` quantised experts
    copied over the 256 bank rows (every row is its own memory)."""
    H, L = P.kt_gguf_hot, P._lib
    import kt_prefill_lend_amd.kt_cpu_moe as CM
    from kt_prefill_lend_amd.gguf import row_bytes

    w = S.WORKLOADS[DECODE]
    N, K = w.inter, w.hidden
    parts = [S.expert_weights(w, e, 0, 16) for e in range(distinct)]
    gate = torch.from_numpy(np.stack([parts[e % distinct][0][:N].reshape(-1) for e in range(w.experts)])).pin_memory()
    up = torch.from_numpy(np.stack([parts[e % distinct][0][N:].reshape(-1) for e in range(w.experts)])).pin_memory()
    down = torch.from_numpy(np.stack([parts[e % distinct][1].reshape(-1) for e in range(w.experts)])).pin_memory()
    cpu = CM.KTCPUExperts(gate, up, down, K, N, w.types, max_tokens=64, max_top_k=w.top_k)
    w13, w2 = S.slot_tensors(w)
    W13, W2 = torch.from_numpy(w13).to(dev), torch.from_numpy(w2).to(dev)
    desc = H.layer_desc(W13, W2, K, N, w.types[0], w.types[2])
    exp_bytes = 2 * N * row_bytes(K, w.types[0]) + K * row_bytes(N, w.types[2])
    res = {"workload": w.name, "cpu_threads": cpu.threads, "cpu_isa": cpu.isa, "routings": rotate}

    def clock(legs):
        # a step runs every leg once, each ending in a device synchronisation; every call
        # takes the next routing, so whatever a leg reads was last read `rotate` calls
        # before, by any leg; per-leg medians (the shared host's hiccups land in the tail)
        c = 0
        for _ in range(warmup):
            for f in legs:
                f(c)
                c += 1
        torch.cuda.synchronize()
        ts = [[] for _ in legs]
        for _ in range(reps):
            for j, f in enumerate(legs):
                t0 = time.perf_counter()
                f(c)
                torch.cuda.synchronize()
                ts[j].append(time.perf_counter() - t0)
                c += 1
        return [float(np.median(t)) * 1e3 for t in ts]

    for T in (1, 4, 16):
        rs = []
        for r in range(rotate):
            wr = S.small(w, index=w.index + 1000 * r)  # another routing and x per rotation
            ids, tw, slot, _ = S.routing(wr, T)
            cold = np.where(slot < 0, ids, -1).astype(np.int32)
            xb = S.activations(wr, T)
            rs.append(dict(
                x=torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16),
                x_h=torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16),
                tw_d=torch.from_numpy(tw).to(dev), slot_d=torch.from_numpy(slot).to(dev),
                cold_d=torch.from_numpy(cold).to(dev), cold_h=torch.from_numpy(cold), tw_h=torch.from_numpy(tw),
                hot=int((slot >= 0).sum()), n_cold=int((cold >= 0).sum()), cold_set=set(cold[cold >= 0].tolist())))
        out = torch.empty((T, K), dtype=torch.bfloat16, device=dev)
        ws = torch.empty((L.lib().ktmi_moe_layer_workspace(desc, T, w.top_k, L.MODE_GEMV),), dtype=torch.uint8, device=dev)

        def gpu_half(i):
            d = rs[i % rotate]
            H.moe_layer(desc, d["x"], d["tw_d"], d["slot_d"], L.MODE_GEMV, out, ws)

        def cpu_half(i):
            d = rs[i % rotate]
            cpu.forward(d["x_h"], d["cold_h"], d["tw_h"])

        def hybrid(i):
            d = rs[i % rotate]
            cpu.submit(d["x"], d["cold_d"], d["tw_d"])
            H.moe_layer(desc, d["x"], d["tw_d"], d["slot_d"], L.MODE_GEMV, out, ws)
            cpu.sync_add(out)

        gpu_ms, cpu_ms, hy_ms = clock([gpu_half, cpu_half, hybrid])
        n_cold = float(np.mean([len(d["cold_set"]) for d in rs]))
        union = set().union(*[d["cold_set"] for d in rs])
        r = {"hot_routes": float(np.mean([d["hot"] for d in rs])), "cold_routes": float(np.mean([d["n_cold"] for d in rs])),
             "cold_experts": n_cold, "cold_experts_union": len(union),
             "cold_union_MB": round(len(union) * exp_bytes / 1e6, 1),
             "gpu_ms": round(gpu_ms, 4), "cpu_ms": round(cpu_ms, 4), "hybrid_ms": round(hy_ms, 4),
             "handoff_ms": round(hy_ms - cpu_ms, 4),
             "cpu_GBps": round(n_cold * exp_bytes / (cpu_ms * 1e-3) / 1e9, 1),
             "overlap": round((gpu_ms + cpu_ms - hy_ms) / max(min(gpu_ms, cpu_ms), 1e-9), 3)}
        res[f"T{T}"] = r
        log(f"hybrid T={T}: {r}")
    cpu.close()
    return res


def bench_stream(P, torch, S, ev, dev, distinct=4, reps=3):
    """Large-expert layers streamed from pinned host memory (hidden 7168, intermediate 2048,
    24 hot Q4_K/Q6_K experts per layer, 6144-token chunk, 4 layers): each layer's experts
    are one group; layer l+1's copy overlaps layer l's grouped layer. Weights: 24 distinct
    experts, made from `distinct` quantised ones (quantising 24 at this size takes minutes)
    by rotating their rows, a different rotation per slot, so that no two slots hold the
    same matrices. Reports the H2D copy time per layer, the compute time per layer on resident
    weights, the pipelined time of the 4 layers, and the overlap efficiency
    (serial - pipelined) / (serial - ideal), ideal = max(copies, computes) + min(copy, compute)."""
    import kt_prefill_lend_amd.kt_stream_prefill as SP

    H, L = P.kt_gguf_hot, P._lib
    w = S.WORKLOADS[STREAM]
    T = w.tokens[0]
    nl = w.layers
    t0 = time.time()
    parts = [S.expert_weights(w, e, 0, 16) for e in range(distinct)]
    # slot e: base e % distinct with its gate/up and down rows rotated by 97 (e // distinct)
    w13 = np.stack([np.roll(parts[e % distinct][0], 97 * (e // distinct), axis=0) for e in range(w.hot)])
    w2 = np.stack([np.roll(parts[e % distinct][1], 97 * (e // distinct), axis=0) for e in range(w.hot)])
    assert len({w13[e, :8].tobytes() for e in range(w.hot)}) == w.hot  # 24 distinct experts
    banks = [SP.Bank.from_slot_rows(torch.from_numpy(w13), torch.from_numpy(w2), w.inter, w.types) for _ in range(nl)]
    ids, tw, slot, _ = S.routing(w, T)
    x = torch.from_numpy(S.activations(w, T).view(np.int16)).to(dev).view(torch.bfloat16)
    tw_d, slot_d = torch.from_numpy(tw).to(dev), torch.from_numpy(slot).to(dev)
    log(f"stream: {nl} layers x {w.hot} experts, {banks[0].gate.nbytes * 2 + banks[0].down.nbytes:,} B per layer pinned,"
        f" prepared in {time.time() - t0:.1f}s")
    st = SP.KTStreamPrefillGGUF.standalone(w.inter, w.hidden, w.top_k, w.types, group_size=w.hot, device=dev,
                                           layers=range(nl))
    for i, b in enumerate(banks):
        st.set_bank(i, b)
    stream = L.stream_ptr(dev)
    # copies alone: events on the copy stream around reps * nl stagings
    st.sync_copies()
    torch.cuda.synchronize()
    cs = st.copy_stream()
    ce = ev.create(2)
    ev.record(ce[0], cs)
    for r in range(reps):
        for i in range(nl):
            st._stage((r * nl + i) % 2, i, 0, w.hot)
    ev.record(ce[1], cs)
    st.sync_copies()
    copy_ms = ev.ms(ce[0], ce[1]) / (reps * nl)
    ev.destroy(ce)
    layer_bytes = banks[0].gate.nbytes * 2 + banks[0].down.nbytes
    # compute alone, on resident weights
    W13, W2 = torch.from_numpy(w13).to(dev), torch.from_numpy(w2).to(dev)
    desc = H.layer_desc(W13, W2, w.hidden, w.inter, w.types[0], w.types[2])
    ms_c, _, _, _ = time_layer(P, torch, [desc], x, tw_d, slot_d, L.MODE_GROUPED, reps * nl, 2, ev, breakdown_steps=1,
                               sample_every=0)
    del W13, W2
    # the pipeline: nl layers, one group each
    items = [(i, x, tw_d, slot_d) for i in range(nl)]
    st.run_layers(items)  # warm
    torch.cuda.synchronize()
    # each pass timed from a drained device, so its first layer's copy overlaps nothing
    # (back-to-back passes would hide it behind the previous pass's last layer)
    se = ev.create(2)
    total = 0.0
    for _ in range(reps):
        ev.record(se[0], stream)
        st.run_layers(items)
        ev.record(se[1], stream)
        torch.cuda.synchronize()
        total += ev.ms(se[0], se[1]) / reps
    ev.destroy(se)
    st.close()
    serial = nl * (copy_ms + ms_c)
    ideal = max(nl * copy_ms, nl * ms_c) + min(copy_ms, ms_c)
    eff = (serial - total) / (serial - ideal) if serial > ideal else 1.0
    r_hot = int((slot >= 0).sum())
    res = {"workload": w.name, "tokens": T, "layers": nl, "hot_routes": r_hot, "layer_bytes": layer_bytes,
           "copy_ms_per_layer": round(copy_ms, 3), "h2d_GBps": round(layer_bytes / (copy_ms * 1e-3) / 1e9, 1),
           "compute_ms_per_layer": round(ms_c, 3),
           "compute_TFLOPs": round(6.0 * w.hidden * w.inter * r_hot / (ms_c * 1e-3) / 1e12, 1),
           "pipelined_ms": round(total, 3), "serial_ms": round(serial, 3), "ideal_ms": round(ideal, 3),
           "overlap_efficiency": round(eff, 3)}
    log(f"stream: {res}")
    return res


def cpu_baseline(S, w, cpu_tokens, T):
    """The CPU expert path (a C restatement of kt-kernel's forward_many) on the same
    workload's first `cpu_tokens` tokens, hot routes only, on this host's cores."""
    try:
        sys.path.insert(0, str(ROOT))
        from oracle import cpu_moe
    except Exception as e:  # noqa: BLE001
        log(f"cpu baseline unavailable: {e}")
        return None
    return cpu_moe.bench(S, w, cpu_tokens, T, log)


if __name__ == "__main__":
    main()
