"""Build the gfx950 libraries in-tree (no JIT cache, no setuptools).

Outputs (all under ``kernels/`` at the repository root, next to each other
so the operator libraries find the C-ABI library through ``$ORIGIN``):

* ``libharp_ra.so``              HIP kernels + the C ABIs of include/harp_ring_attn.h
                                 and include/harp_qk_norm_rope.h
                                 (hipcc, --offload-arch=gfx950).
* ``libring_attention_ops.so``   the PyTorch operator library (namespace
                                 ``ring_attention_ops``), the drop-in for the
                                 reference's kernels/libring_attention_ops.so
                                 (gemm/ring_attention/Makefile:9-12, 36-37).
* ``libharp_async_op.so``        the PyTorch operator library for the QK RMSNorm
                                 and RoPE operators (namespace ``async_op``,
                                 async_rt/csrc/async_op_api.cc:54-57), on the GPU.

Run ``python -m harp_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "harp_amd" / "csrc"
INCLUDE = ROOT / "include"
OUT = ROOT / "kernels"
ABI_LIB = OUT / "libharp_ra.so"
OPS_LIB = OUT / "libring_attention_ops.so"
ASYNC_OPS_LIB = OUT / "libharp_async_op.so"

HIP_SOURCES = ["ra_kernels.hip", "fwd_asm.hip", "dq_asm.hip", "dkdv_asm.hip", "ra_abi.hip", "qk_kernels.hip", "qk_abi.hip", "proj_kernels.hip"]
HIP_HEADERS = ["ra_common.h", "ra_kernels.h", "qk_kernels.h", "proj_kernels.h", "fwd_asm.inc", "fwd_asm_gen.py",
               "dq_asm.inc", "dq_asm_gen.py", "dkdv_asm.inc",
               "dkdv_asm_gen.py", "asm_sched.py"]
OPS_SOURCE = "torch_ring_attention_ops.cpp"
ASYNC_OPS_SOURCE = "torch_async_op.cpp"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
OFFLOAD_ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    f"--offload-arch={OFFLOAD_ARCH}",
    # packed-fp32 VALU ops are kept out of every gfx950 code object
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    # machine scheduler aiming at instruction-level parallelism within the
    # regions the kernels' scheduling fences leave it: 0.4% faster step than
    # the default strategy at the headline shape, same register use
    "-mllvm",
    "-amdgpu-sched-strategy=max-ilp",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in res.stdout.splitlines() if "packed-fp32-ops" not in ln and ln.strip()
    )
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out:
        print(out)


def generate_asm(verbose: bool = False) -> None:
    """csrc/fwd_asm.inc, dq_asm.inc and dkdv_asm.inc: the hand-scheduled
    forward, dQ and dK/dV loops, from their generators."""
    for gen in ("fwd_asm_gen.py", "dq_asm_gen.py", "dkdv_asm_gen.py"):
        _run([sys.executable, str(CSRC / gen)], verbose)


def build_abi(verbose: bool = False) -> Path:
    generate_asm(verbose)
    OUT.mkdir(parents=True, exist_ok=True)
    tmp = ABI_LIB.with_suffix(".so.tmp")
    cmd = [str(ROCM / "bin" / "hipcc"), *HIPCC_FLAGS, f"-I{INCLUDE}"]
    cmd += [str(CSRC / s) for s in HIP_SOURCES]
    cmd += ["-o", str(tmp)]
    _run(cmd, verbose)
    os.replace(tmp, ABI_LIB)
    return ABI_LIB


def build_ops(verbose: bool = False, source: str = OPS_SOURCE, lib: Path = OPS_LIB,
              ext_name: str = "ring_attention_ops") -> Path:
    import torch.utils.cpp_extension as ce

    OUT.mkdir(parents=True, exist_ok=True)
    torch_lib = Path(ce.library_paths()[0])
    incs = ce.include_paths()
    tmp = lib.with_suffix(".so.tmp")
    abi = int(__import__("torch")._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        "g++",
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        f"-DTORCH_EXTENSION_NAME={ext_name}",
        *[f"-I{p}" for p in incs],
        f"-I{ROCM / 'include'}",
        f"-I{INCLUDE}",
        str(CSRC / source),
        f"-L{OUT}",
        "-lharp_ra",
        f"-L{torch_lib}",
        "-lc10",
        "-lc10_hip",
        "-ltorch_cpu",
        "-ltorch",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{torch_lib}",
        "-o",
        str(tmp),
    ]
    _run(cmd, verbose)
    os.replace(tmp, lib)
    return lib


def build_async_ops(verbose: bool = False) -> Path:
    """kernels/libharp_async_op.so: the async_op operators (QK RMSNorm, RoPE)."""
    return build_ops(verbose, ASYNC_OPS_SOURCE, ASYNC_OPS_LIB, "harp_async_op")


def build(verbose: bool = False) -> None:
    """Compile every library unconditionally (the build check)."""
    build_abi(verbose)
    build_ops(verbose)
    build_async_ops(verbose)


def sources_newer_than_libs() -> bool:
    """True when a source file is newer than a built library (or one is missing)."""
    libs = [ABI_LIB, OPS_LIB, ASYNC_OPS_LIB]
    if not all(p.exists() for p in libs):
        return True
    newest_lib = min(p.stat().st_mtime for p in libs)
    srcs = [CSRC / s for s in HIP_SOURCES + HIP_HEADERS + [OPS_SOURCE, ASYNC_OPS_SOURCE]]
    srcs += [INCLUDE / "harp_ring_attn.h", INCLUDE / "harp_qk_norm_rope.h"]
    return any(s.stat().st_mtime > newest_lib for s in srcs)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(f"built {ABI_LIB} and {OPS_LIB}")
