"""Counted `s_waitcnt vmcnt(n)` waits checked against the gfx950 assembly the compiler emits.

A counted wait lets the n youngest vector-memory instructions stay in flight; it is correct
only if at least n such instructions were issued after the load it waits for. The kernels
derive n from per-format load counts (BPiece<t>::NLOAD, Unit::NLD); these tests compile the
sources for gfx950 and count the instructions actually emitted.

* decode_gate_up: the x pieces are waited for with n <= the weight loads issued after them.
* grouped_gemm (every type, gate/up and down, both route-tile heights; the 256-route kernels
  also hold the 128-route body, which they run for a slot's short last tile, and every
  K loop of a kernel is checked): at the end of K step k the activation tile of step k+1,
  whose direct buffer->LDS loads were issued during step k-2, must have landed, so the
  step-end wait's n must not exceed the vector-memory instructions issued after that
  tile's last direct load (cyclically over the 4 steps of the unrolled super-block loop,
  and in issue order over the prologue, the first super-block, which is peeled off the
  loop and whose first step also issues tiles 1 to 3, and the loop's first iteration);
  and no vmcnt(0) may drain the prefetch inside the K loop. The last super-block is peeled
  off after the loop: its first step is an ordinary one, the three after it issue no direct
  loads (their tiles would be past the tile's K), and the waits of its first three steps are
  checked the same way, after the loop's last iteration and after the peeled first
  super-block (a two-column tile runs no loop iteration).
"""
import os
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "kt-prefill-lend_amd" / "csrc"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

pytestmark = pytest.mark.skipif(not shutil.which(HIPCC) and not Path(HIPCC).exists(), reason="hipcc not available")

VMEM = re.compile(r"^\s*(global_load|buffer_load)")
DMA = re.compile(r"^\s*buffer_load\w*\s.*\blds\b")


def _asm(src: str, tmp_path) -> list:
    out = tmp_path / (Path(src).stem + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", str(CSRC / src), f"-I{CSRC}", "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=900)
    return out.read_text().split("\n")


def _vmcnt(line: str) -> int:
    return int(re.search(r"vmcnt\((\d+)\)", line).group(1))


def test_decode_gate_up_counted_wait_covers_the_weight_loads(tmp_path):
    lines = _asm("decode_layer.hip", tmp_path)
    starts = [i for i, l in enumerate(lines) if re.match(r"^_ZN4ktmi12_GLOBAL__N_114decode_gate_up\w*:", l)]
    assert len(starts) >= 16
    for st in starts:
        end = next(i for i in range(st + 1, len(lines)) if "s_endpgm" in lines[i])
        marks = [i for i in range(st, end) if "sched_barrier mask(0x00000000)" in lines[i]]
        assert len(marks) >= 2, lines[st]
        a, b = marks[0], marks[1]  # the weight loads sit between the first two
        loads = sum(1 for i in range(a, b) if VMEM.match(lines[i]))
        wait = next(lines[i] for i in range(b, end) if "s_waitcnt" in lines[i])
        n = _vmcnt(wait)
        assert 0 < n <= loads, (lines[st].split(":")[0], n, loads)


def _k_loops(lines, st, end):
    """The K loops of a kernel: per loop body holding MFMAs, the innermost loop (the
    super-block loop), in code order."""
    labels = {}
    for i in range(st, end):
        m = re.match(r"^(\.LBB\w+):", lines[i])
        if m:
            labels[m.group(1)] = i
    loops = []
    for i in range(st, end):
        m = re.search(r"s_cbranch_\w+\s+(\.LBB\w+)", lines[i])
        if m and m.group(1) in labels and labels[m.group(1)] < i and any("v_mfma" in lines[j] for j in range(labels[m.group(1)], i)):
            loops.append((labels[m.group(1)], i))
    # drop loops that contain another one
    return sorted(ab for ab in loops if not any(o != ab and ab[0] <= o[0] and o[1] <= ab[1] for o in loops))


def test_grouped_gemm_counted_waits_cover_the_activation_tiles(tmp_path):
    lines = _asm("moe_gemm.hip", tmp_path)
    starts = [i for i, l in enumerate(lines) if re.match(r"^_ZN4ktmi12_GLOBAL__N_112grouped_gemm\w*:", l)]
    assert len(starts) == 16  # 4 types x (gate/up, down) x (256-, 128-route tiles)
    for st in starts:
        name = lines[st].split(":")[0]
        end = next(i for i in range(st + 1, len(lines)) if lines[i].startswith(".Lfunc_end"))
        loops = _k_loops(lines, st, end)
        fj8 = re.search(r"grouped_gemmILi\d+ELb\dELi8E", name) is not None
        assert len(loops) == (2 if fj8 else 1), (name, "K loops", loops)
        for a, b in loops:
            _check_k_loop(lines, name, a, b)
            _check_last_super_block(lines, name, a, b)


def _check_k_loop(lines, name, a, b):
    body = lines[a:b]
    assert not [l for l in body if re.search(r"s_waitcnt.*vmcnt\(0\)", l)], (name, "vmcnt(0) in the K loop")
    bars = [j for j, l in enumerate(body) if l.strip() == "s_barrier"]
    assert len(bars) == 4, (name, "4 K steps per super-block", len(bars))
    steps, prev = [], bars[-1] - len(body)
    for s in range(4):  # step s: the instructions after the previous step's barrier up to its own
        steps.append([j % len(body) for j in range(prev + 1, bars[s])])
        prev = bars[s]
    waits = []
    for s in range(4):
        w = next(body[j] for j in reversed(steps[s]) if "s_waitcnt" in body[j] and "vmcnt" in body[j])
        waits.append(_vmcnt(w))
        k2 = steps[(s - 2) % 4]
        dmas = [p for p, j in enumerate(k2) if DMA.match(body[j])]
        assert dmas, (name, "no direct loads in step", (s - 2) % 4)
        after = sum(1 for j in k2[dmas[-1] + 1:] if VMEM.match(body[j]))
        after += sum(1 for j in steps[(s - 1) % 4] if VMEM.match(body[j]))
        after += sum(1 for j in steps[s] if VMEM.match(body[j]))
        assert 0 < waits[s] <= after, (name, "step", s, waits[s], after)
    # before the loop: the prologue (tile 0's AJ direct loads, then its wait and a barrier)
    # and the first super-block's 4 steps, peeled off the loop (their first MFMAs start the
    # accumulators at 0; step 0 also issues tiles 1, 2 and 3): the 5 barriers right before
    # the loop
    aj = sum(1 for l in body if DMA.match(l)) // 4
    pb = [j for j in range(a) if lines[j].strip() == "s_barrier"][-5:]
    assert len(pb) == 5 and aj > 0, (name, "the prologue's barrier + 4 peeled steps")
    bar0 = pb[0]
    dmas = [j for j in range(bar0) if DMA.match(lines[j])][-aj:]
    assert len(dmas) == aj, (name, "tile 0 in the prologue")
    # the prologue's tail from tile 0's first direct load, the 4 peeled steps, then the
    # loop's first iteration: direct loads in tile order, aj per tile
    pro = lines[dmas[0]:bar0]
    seq = [pro] + [lines[pb[s] + 1:pb[s + 1]] for s in range(4)] + [[body[j] for j in steps[s]] for s in range(4)]
    flat = [(q, l) for q, part in enumerate(seq) for l in part]
    dma_at = [i for i, (_, l) in enumerate(flat) if DMA.match(l)]
    assert len(dma_at) >= 9 * aj, (name, "tiles 0..8 issued by the first 8 steps", len(dma_at))
    # seq part q >= 1 is step q - 1; its closing wait needs tile q (tile 0 for the prologue)
    for q in range(len(seq)):
        w_at = max(i for i, (qq, l) in enumerate(flat) if qq == q and "s_waitcnt" in l and "vmcnt" in l)
        last = dma_at[(q + 1) * aj - 1]
        assert last < w_at, (name, "tile", q, "issued after the wait for it")
        after = sum(1 for i in range(last + 1, w_at) if VMEM.match(flat[i][1]))
        assert 0 < _vmcnt(flat[w_at][1]) <= after, (name, "wait of part", q, _vmcnt(flat[w_at][1]), after)


def _steps_of_loop(lines, a, b):
    body = lines[a:b]
    bars = [j for j, l in enumerate(body) if l.strip() == "s_barrier"]
    steps, prev = [], bars[-1] - len(body)
    for s in range(4):
        steps.append([body[j % len(body)] for j in range(prev + 1, bars[s])])
        prev = bars[s]
    return steps


def _check_last_super_block(lines, name, a, b):
    """The peeled last super-block after the K loop (see the module docstring): its steps'
    closing waits, with the loop's last iteration or the peeled first super-block before it."""
    tb = [j for j in range(b + 1, len(lines)) if lines[j].strip() == "s_barrier"][:3]
    assert len(tb) == 3, (name, "3 barriers after the loop")
    tail = [lines[b + 1:tb[0]], lines[tb[0] + 1:tb[1]], lines[tb[1] + 1:tb[2]]]
    aj = sum(1 for l in lines[a:b] if DMA.match(l)) // 4
    assert [sum(1 for l in st if DMA.match(l)) for st in tail] == [aj, 0, 0], (name, "direct loads of the last steps")
    assert all(any("v_mfma" in l for l in st) for st in tail), (name, "MFMAs in the last steps")
    pb = [j for j in range(a) if lines[j].strip() == "s_barrier"][-5:]
    first = [lines[pb[s] + 1:pb[s + 1]] for s in range(4)]
    for pred in (_steps_of_loop(lines, a, b), first):
        seq = pred + tail
        for s in range(3):  # tail step s (sequence index 4 + s) needs the tile issued at index 2 + s
            flat = [l for part in seq[2 + s:4 + s] for l in part] + seq[4 + s]
            src = seq[2 + s]
            dmas = [i for i, l in enumerate(src) if DMA.match(l)]
            assert dmas, (name, "tail step", s, "no tile issued two steps before")
            w_at = max(i for i, l in enumerate(flat) if "s_waitcnt" in l and "vmcnt" in l)
            after = sum(1 for i in range(dmas[-1] + 1, w_at) if VMEM.match(flat[i]))
            assert 0 < _vmcnt(flat[w_at]) <= after, (name, "tail step", s, _vmcnt(flat[w_at]), after)
