"""Compile-time invariants of the layer kernel that its speed depends on (CPU: hipcc only).

moe_layer_kernel's item functions are separate calls: one more live register
in any of them pushes callee-saved registers to scratch (saved at entry,
restored at exit, measurably slower) or drops the kernel below two waves per
SIMD (half the persistent grid).  The compiler's resource remarks for the
library's own flags must show no scratch and two waves per SIMD.
"""
import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "home-seek_amd"))


def _resources(src_name: str, tmp_path) -> dict:
    """{kernel or function name: (scratch bytes per lane, waves per SIMD)} from hipcc's resource remarks."""
    import _build
    src = ROOT / "home-seek_amd" / "csrc" / src_name
    cmd = [_build.HIPCC, *_build.HIP_FLAGS, "--offload-device-only", "-Rpass-analysis=kernel-resource-usage", "-c",
           str(src), "-o", str(tmp_path / (src.stem + ".o"))]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-2000:]
    blocks = re.split(r"remark: [^\n]*Function Name: ", res.stderr)[1:]
    found = {}
    for b in blocks:
        name = b.split()[0]
        scratch = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", b)
        occ = re.search(r"Occupancy \[waves/SIMD\]: (\d+)", b)
        found[name] = (int(scratch.group(1)) if scratch else None, int(occ.group(1)) if occ else None)
    return found


@pytest.mark.skipif(shutil.which("/opt/rocm/bin/hipcc") is None, reason="hipcc not present")
def test_layer_kernel_no_scratch_two_waves_per_simd(tmp_path):
    found = _resources("hsmoe_moe_layer.hip", tmp_path)
    layer = [n for n in found if "moe_layer_kernel" in n]
    assert layer, f"no resource remark for moe_layer_kernel in {list(found)}"
    scratch, occ = found[layer[0]]
    assert scratch == 0, f"moe_layer_kernel uses {scratch} bytes of scratch per lane"
    assert occ is not None and occ >= 2, f"moe_layer_kernel occupancy {occ} waves/SIMD"


@pytest.mark.skipif(shutil.which("/opt/rocm/bin/hipcc") is None, reason="hipcc not present")
def test_prefill_kernels_no_scratch(tmp_path):
    """Every instantiation of the prefill gate/up and down kernels (FP4 at 4
    waves per SIMD for gate/up, FP8 and bf16 for the shared expert) keeps its
    registers: a spill would slow prefill with no test noticing."""
    found = _resources("hsmoe_moe_prefill.hip", tmp_path)
    kern = {n: v for n, v in found.items() if "prefill_gate_up_kernel" in n or "prefill_down_kernel" in n}
    assert any("prefill_gate_up_kernel" in n for n in kern) and any("prefill_down_kernel" in n for n in kern), list(found)
    bad = {n: v for n, v in kern.items() if v[0] != 0}
    assert not bad, f"prefill kernels with scratch: {bad}"
