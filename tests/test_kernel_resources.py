"""Register and scratch budget of the fused kernels (compiled here, no GPU).

The row-pipeline kernels keep every live value in registers: a value the
register allocator puts in scratch memory is reloaded with a wait for every
load the wave has in flight, which stalls the producers' and decoders' row
pipelines.  Their workgroups of 16 waves (four per SIMD) leave each wave 128
of the SIMD's 512 VGPRs, those of 12 waves (egress kind family 2) 168.  This
compiles the device code of the two fused sources with the library's flags
and checks, for every kernel, what the compiler's metadata reports: no
scratch (private segment 0, no VGPR spills) and a VGPR count that fits the
kernel's waves.
"""
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "vlx-tee_amd"))
import build as B  # noqa: E402  (vlx-tee_amd/build.py: the library's compiler flags)

HIPCC = shutil.which("hipcc") or ("/opt/rocm/bin/hipcc" if Path("/opt/rocm/bin/hipcc").exists() else None)
pytestmark = pytest.mark.skipif(HIPCC is None, reason="hipcc not available")

# kernel name fragment -> VGPRs a wave may use (512 per SIMD lane / waves per SIMD)
BUDGET = {
    "egress_fused_kernelILi0ELi0E": 128, "egress_fused_kernelILi1ELi0E": 128,
    "egress_fused_kernelILi0ELi1E": 128, "egress_fused_kernelILi1ELi1E": 128,
    "egress_fused_kernelILi0ELi2E": 168, "egress_fused_kernelILi1ELi2E": 168,
    "ingress_fused_kernelILi0ELi0E": 128, "ingress_fused_kernelILi1ELi0E": 128,
    "ingress_fused_kernelILi0ELi1E": 128, "ingress_fused_kernelILi1ELi1E": 128,
    "egress_small_kernel": 512, "ingress_small_kernel": 512,
}


def _kernels(asm: str) -> dict:
    """Per kernel: the metadata fields of its entry in .amdgpu_metadata."""
    meta = asm[asm.index(".amdgpu_metadata"):]
    out = {}
    for block in re.split(r"\n  - ", meta):
        m = re.search(r"\.name:\s+(\S+)", block)
        if not m:
            continue
        fields = dict(re.findall(r"\.(private_segment_fixed_size|vgpr_count|vgpr_spill_count|agpr_count):\s+(\d+)",
                                 block))
        out[m.group(1)] = {k: int(v) for k, v in fields.items()}
    return out


@pytest.fixture(scope="module")
def metadata(tmp_path_factory):
    d = tmp_path_factory.mktemp("asm")

    def compile_one(name):
        out = d / (name + ".s")
        cmd = [HIPCC, *B.HIPCC_FLAGS, "--cuda-device-only", "-S", "-I", str(ROOT / "include"),
               str(ROOT / "vlx-tee_amd" / "csrc" / (name + ".hip")), "-o", str(out)]
        subprocess.run(cmd, check=True, capture_output=True)
        return _kernels(out.read_text())

    with ThreadPoolExecutor(2) as pool:
        parts = list(pool.map(compile_one, ["ztcp_egress", "ztcp_ingress"]))
    return {k: v for p in parts for k, v in p.items()}


def test_every_budgeted_kernel_is_present(metadata):
    for frag in BUDGET:
        assert any(frag in name for name in metadata), frag


@pytest.mark.parametrize("frag", sorted(BUDGET))
def test_no_scratch_and_registers_fit(metadata, frag):
    hits = {n: m for n, m in metadata.items() if frag in n}
    assert hits, frag
    for name, m in hits.items():
        assert m["private_segment_fixed_size"] == 0, (name, m)
        assert m["vgpr_spill_count"] == 0, (name, m)
        assert m["vgpr_count"] + m.get("agpr_count", 0) <= BUDGET[frag], (name, m)
