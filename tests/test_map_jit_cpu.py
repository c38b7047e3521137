"""The source ts_hip_map compiles at run time for an elementwise program
(ts_hip_map_jit_source), checked on the CPU: it compiles for gfx950 with the
flags the library passes to hipRTC, and the code has no packed fp32
instructions, no scratch and no indexed register moves (every register of the
program is a plain register)."""
from __future__ import annotations

import ctypes
import pathlib
import re
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
HIPCC = "/opt/rocm/bin/hipcc"
# the options ts_hip_map.hip hands to hipRTC (hipRTC includes the HIP runtime
# header by itself)
RTC_OPTIONS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
               "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-include", "hip/hip_runtime.h"]


def _c2_program(F):
    """The config-2 step as the host library builds it: a, b, c and the seed
    constant in, the forward recomputed, ga, gb, gc stored and y summed."""
    p = F.MapProgram()
    p.n_inputs = 4
    for k in range(3):
        p.inputs[k] = 256 * (k + 1)
    p.const_inputs = p.scalar_inputs = 1 << 3
    p.const_values[3] = 1.0
    C = F.MAP_CODES
    ops = [("add", 0, 1, 4), ("mul", 4, 2, 5), ("div", 0, 2, 6), ("sub", 5, 6, 5), ("relu", 5, 5, 6),
           ("relu_bwd", 6, 3, 3), ("neg", 3, 3, 7), ("div", 7, 2, 8), ("mul", 3, 2, 9), ("add", 8, 9, 8),
           ("mul", 7, 0, 0), ("mul", 2, 2, 7), ("div", 0, 7, 0), ("neg", 0, 0, 0), ("mul", 3, 4, 4),
           ("add", 0, 4, 0)]
    p.n_ops = len(ops)
    for k, (code, a, b, d) in enumerate(ops):
        p.ops[k] = F.MapOp(C[code], a, b, 1 if code == "div" else 0, 0.0, d)
    p.n_outputs = 3
    for o, r in enumerate((8, 9, 0)):
        p.outputs[o] = 4096 + 256 * o
        p.output_regs[o] = r
    p.reduce_reg = 6
    return p


@pytest.mark.skipif(shutil.which(HIPCC) is None, reason="hipcc is not installed")
def test_compiled_source_builds_without_packed_fp32(tmp_path):
    from train_station_amd import _ffi as F
    hip = F.hip
    p = _c2_program(F)
    n = hip.ts_hip_map_jit_source(ctypes.byref(p), 1, None, 0)
    assert n > 1
    buf = ctypes.create_string_buffer(n)
    assert hip.ts_hip_map_jit_source(ctypes.byref(p), 1, buf, n) == n
    src = tmp_path / "compiled.hip"
    src.write_text(buf.value.decode())
    out = tmp_path / "compiled.s"
    cmd = [HIPCC, *RTC_OPTIONS, "-I", str(ROOT / "include"), "-I", str(ROOT / "train-station_amd" / "csrc"),
           "-S", "--cuda-device-only", "-Werror=array-bounds", "-o", str(out), str(src)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    asm = out.read_text()
    assert not re.search(r"v_pk_(add|mul|fma)_f32", asm)
    assert "gpr_idx" not in asm and "v_movrel" not in asm
    assert re.search(r"\.private_segment_fixed_size:\s+0\b", asm)
    # a malformed program (an op reads a register nothing wrote) has no source
    p.ops[0] = F.MapOp(F.MAP_CODES["add"], 12, 1, 0, 0.0, 4)
    assert hip.ts_hip_map_jit_source(ctypes.byref(p), 1, None, 0) == 0
