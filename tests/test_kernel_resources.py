"""CPU: resource use of the built device code (no GPU needed).

Reads the code-object metadata of every kernel in ``libdflash_hip.so`` (the gfx950 code
objects of its offload bundles) and checks that no kernel keeps per-lane scratch beyond the
few register spills the prefill tile kernels are known to have.  A device function that the
compiler stops inlining while it takes the kernel's parameter block by reference makes the
whole block live in scratch (hundreds of bytes per lane, written by every lane at every
launch): that slowed the verify kernels by over 20 us per launch when it happened, with no
other symptom.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "qwen3.5-35b-dflash_amd" / "libdflash_hip.so"
LLVM = Path("/opt/rocm/llvm/bin")
TOOLS = [LLVM / t for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf")]
# the prefill tile kernels run at 256 VGPRs with a few spilled registers
SPILL_ALLOWANCE = {"w4_tile_kernel": 128}
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _kernels(tmp_path):
    fatbin = tmp_path / "fatbin.bin"
    subprocess.run([str(TOOLS[0]), f"--dump-section=.hip_fatbin={fatbin}", str(LIB), str(tmp_path / "host.so")],
                   check=True, capture_output=True)
    data = fatbin.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    kernels = {}
    for i, s in enumerate(starts):
        bundle, obj = tmp_path / f"b{i}.bin", tmp_path / f"co{i}.elf"
        bundle.write_bytes(data[s:starts[i + 1] if i + 1 < len(starts) else len(data)])
        subprocess.run([str(TOOLS[1]), "--unbundle", "--type=o", f"--input={bundle}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={obj}"], check=True,
                       capture_output=True)
        notes = subprocess.run([str(TOOLS[2]), "--notes", str(obj)], check=True, capture_output=True,
                               text=True).stdout
        for block in notes.split(".agpr_count:")[1:]:
            name = re.search(r"\.name:\s+(\S+)", block).group(1)
            kernels[name] = {
                "scratch": int(re.search(r"\.private_segment_fixed_size:\s+(\d+)", block).group(1)),
                "dynamic_stack": re.search(r"\.uses_dynamic_stack:\s+(\S+)", block).group(1) == "true",
            }
    return kernels


@pytest.mark.skipif(not LIB.exists() or not all(t.exists() for t in TOOLS),
                    reason="needs the built library and the ROCm LLVM tools")
def test_no_kernel_keeps_its_parameters_in_scratch(tmp_path):
    kernels = _kernels(tmp_path)
    assert len(kernels) >= 60, sorted(kernels)
    assert any("w4_verify_kernel" in n for n in kernels) and any("w4_tile_kernel" in n for n in kernels)
    bad = []
    for name, r in kernels.items():
        allowance = next((v for k, v in SPILL_ALLOWANCE.items() if k in name), 0)
        if r["scratch"] > allowance or r["dynamic_stack"]:
            bad.append((name, r))
    assert not bad, bad
