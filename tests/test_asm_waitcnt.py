"""The decode gate/up kernel waits for its x pieces with a counted `s_waitcnt vmcnt(n)`: n must
not exceed the number of weight-load instructions the compiler emitted after the x loads
(Unit::NLD per unit), or the wait would let x be read before it lands. This compiles
decode_layer.hip for gfx950 and checks every instantiation's count in the assembly."""
import os
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "kt-prefill-lend_amd" / "csrc"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not shutil.which(HIPCC) and not Path(HIPCC).exists(), reason="hipcc not available")
def test_decode_gate_up_counted_wait_covers_the_weight_loads(tmp_path):
    out = tmp_path / "decode_layer.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", str(CSRC / "decode_layer.hip"), f"-I{CSRC}", "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    lines = out.read_text().split("\n")
    starts = [i for i, l in enumerate(lines) if re.match(r"^_ZN4ktmi12_GLOBAL__N_114decode_gate_up\w*:", l)]
    assert len(starts) >= 16
    for st in starts:
        end = next(i for i in range(st + 1, len(lines)) if "s_endpgm" in lines[i])
        marks = [i for i in range(st, end) if "sched_barrier mask(0x00000000)" in lines[i]]
        assert len(marks) >= 2, lines[st]
        a, b = marks[0], marks[1]  # the weight loads sit between the first two
        loads = sum(1 for i in range(a, b) if re.search(r"\b(global_load|buffer_load)", lines[i]))
        wait = next(lines[i] for i in range(b, end) if "s_waitcnt" in lines[i])
        n = int(re.search(r"vmcnt\((\d+)\)", wait).group(1))
        assert 0 < n <= loads, (lines[st].split(":")[0], n, loads)
