# SPDX-License-Identifier: BSD-3-Clause
"""Checks on the gfx950 assembly of the kernels' hand-written asm, on the CPU.

The split-K partial stores are issued from inline asm (splitk_store4 in
xtc_amd/csrc/splitk.hpp).  The compiler does not insert the wait states an
MFMA result needs before a memory instruction reads it when the reader is
inline asm, so the asm brings its own.  Here a kernel that stores an MFMA
result straight away is compiled for gfx950 and the wait states between the
MFMA and the store are counted (s_nop N counts N + 1, any other instruction
one): at least 19, the requirement of a 16-pass XDL op.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "xtc_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

PROBE = r"""
#include "splitk.hpp"
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
__global__ void store_after_mfma16(const float* a, const float* b, float* p) {
  f32x4 acc = {0, 0, 0, 0};
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[threadIdx.x], b[threadIdx.x], acc, 0, 0, 0);
  xtc_hip::splitk_store4(p + 4 * threadIdx.x, acc);
}
__global__ void store_after_mfma32(const float* a, const float* b, float* p) {
  f32x16 acc = {};
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[threadIdx.x], b[threadIdx.x], acc, 0, 0, 0);
  f32x4 v = {acc[0], acc[1], acc[2], acc[3]};
  xtc_hip::splitk_store4(p + 4 * threadIdx.x, v);
}
"""


def _wait_states_before(lines: list[str], idx: int) -> int:
    """Wait states between the last v_mfma before lines[idx] and lines[idx]."""
    total = 0
    for line in reversed(lines[:idx]):
        op = line.split()[0]
        if op.startswith("v_mfma"):
            return total
        m = re.match(r"s_nop\s+(\d+)", line)
        total += int(m.group(1)) + 1 if m else 1
    return total


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
def test_splitk_asm_store_waits_for_the_mfma(tmp_path):
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    out = tmp_path / "probe.s"
    subprocess.run(
        [HIPCC, "--offload-arch=gfx950", "-O3", "-S", "--cuda-device-only", f"-I{CSRC}", str(src), "-o", str(out),
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"],
        check=True, capture_output=True,
    )
    lines = [ln.strip() for ln in out.read_text().splitlines()]
    lines = [ln for ln in lines if ln and not ln.startswith((";", ".", "//")) and not ln.endswith(":")]
    stores = [i for i, ln in enumerate(lines) if ln.startswith("global_store_dwordx4") and "sc1" in ln]
    assert len(stores) == 2
    for i in stores:
        assert _wait_states_before(lines, i) >= 19, lines[max(0, i - 6) : i + 1]
