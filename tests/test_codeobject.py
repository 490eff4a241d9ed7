"""CPU test of the built gfx950 code objects: every kernel in the libraries
runs without a private (scratch) segment and spills no registers.  The code
object is taken out of the library's .hip_fatbin section with the ROCm LLVM
tools and its AMDGPU metadata notes are read back."""

import os
import re
import subprocess
import tempfile

import pytest

from harp_amd import _lib

LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def kernel_notes(lib_path):
    """AMDGPU metadata of every kernel in the library.  The linked
    .hip_fatbin section holds one offload bundle per translation unit, one
    after the other: each is unbundled and read."""
    notes = ""
    with tempfile.TemporaryDirectory() as d:
        fb = os.path.join(d, "fatbin")
        subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fb}", str(lib_path), os.devnull],
                       check=True, capture_output=True)
        data = open(fb, "rb").read()
        starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
        for i, st in enumerate(starts):
            part, co = os.path.join(d, f"b{i}"), os.path.join(d, f"co{i}.o")
            with open(part, "wb") as f:
                f.write(data[st:starts[i + 1] if i + 1 < len(starts) else len(data)])
            subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={part}",
                            f"--targets={TARGET}", f"--output={co}"], check=True, capture_output=True)
            notes += subprocess.run([f"{LLVM}/llvm-readelf", "--notes", co], check=True, capture_output=True,
                                    text=True).stdout
    kernels = {}
    cur = None
    for line in notes.splitlines():
        m = re.match(r"\s*-?\s*\.(\w+):\s+(\S+)", line)
        if not m:
            continue
        key, val = m.groups()
        if key == "agpr_count" and line.strip().startswith("-"):
            cur = {}
        if cur is None:
            continue
        cur[key] = val
        if key == "name":
            kernels[val] = cur
    return kernels


@pytest.mark.skipif(not os.path.exists(f"{LLVM}/clang-offload-bundler"), reason="ROCm LLVM tools not installed")
@pytest.mark.parametrize("lib", [_lib.ABI_LIB, _lib.KERNELS / "libharp_bench_probe.so"],
                         ids=["libharp_ra", "libharp_bench_probe"])
def test_no_scratch_and_no_spills(lib):
    if not lib.exists():
        pytest.skip(f"{lib} not built")
    ks = kernel_notes(lib)
    assert ks, "no kernels found in the code object"
    hot = [n for n in ks if re.search(r"(fwd|dq|dkdv)_kernel", n)]
    if lib == _lib.ABI_LIB:
        assert len(hot) == 15, hot  # 5 head-dim variants x 3 kernels
        # every translation unit's kernels are read: the hand-scheduled
        # head-dim-128 kernels and the fused projection too
        for name in ("fwd_asm_kernel", "dq_asm_kernel", "dkdv_asm_kernel", "proj_kernel"):
            assert any(name in n for n in ks), name
    for name, k in ks.items():
        assert int(k["private_segment_fixed_size"]) == 0, (name, k)
        assert int(k["vgpr_spill_count"]) == 0 and int(k["sgpr_spill_count"]) == 0, (name, k)
