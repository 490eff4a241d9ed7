"""The Linear-layer GEMMs around the ring-attention block, on the GPU.

HARP runs its Linear layers (q/k/v/out projections, the FFN, adaLN) through
its own SME GEMM library, ``xhblas_gemm`` (gemm/bgemm/bgemm.cpp:419-424,
header gemm/bgemm/bgemm.h:20-26), tuned for a fixed table of shapes
(gemm/README.md:12-70).  :func:`xhblas_gemm` keeps that entry point's
arguments and status codes for device tensors:

* ``C[M, N] = alpha * op(A)[M, K] @ op(B)[K, N]``, row-major only
  (``order`` 101); ``op(X)`` is ``X`` for ``trans`` 111 (``A`` stored
  ``[M, K]``, ``lda == K``) and ``X^T`` for 112 (``A`` stored ``[K, M]``,
  ``lda == M``); likewise ``B`` (``ldb`` = its row length), ``ldc == N``
  (bgemm.cpp:316-356).
* bf16 inputs and output, fp32 accumulation.  The reference truncates the
  fp32 result to bf16 (bgemm.cpp:127-146); the library GEMMs round to
  nearest, at most one bf16 unit apart (not reproduced on purpose, as the
  ring-attention kernels do not reproduce the reference's truncations).
* ``beta`` must be 0 (status -8, bgemm.cpp:348-350); ``K == 0`` or
  ``alpha == 0`` zero ``C``; ``M == 0`` or ``N == 0`` do nothing.
* ``sign == 1`` with ``ba``: ``ba[N]`` is a bias added before ``alpha``
  (the accumulator starts at ``ba``, bgemm_demo1/bgemm.cpp:364-380);
  ``sign == 2`` with ``ba``: after the product, ``ba[j] = sum_i A[i*M + j]``
  over the ``K`` rows of a transposed ``A`` (the bias gradient of a Linear
  backward, bgemm.cpp:405-416).
* Any shape is accepted: the reference returns -6 for shapes outside its
  table (bgemm.cpp:342-345); the GPU GEMMs need no per-shape kernels.

The product runs on the ROCm BLAS libraries through torch (hipBLASLt, or
rocBLAS where it measured faster for that shape: :data:`BACKEND_BY_SHAPE`,
filled from ``python -m harp_amd.gemm --bench`` on the MI355X).  Nothing
here falls back to the CPU: CPU tensors raise.
"""

from __future__ import annotations

import argparse
import json
from typing import Dict, Optional, Tuple

import torch

ROW_MAJOR, COL_MAJOR = 101, 102
NO_TRANS, TRANS, CONJ_TRANS = 111, 112, 113

# gemm/README.md:12-70, (M, N, K, transA, transB) with T = TRANS, N = NO_TRANS
_T, _N = TRANS, NO_TRANS
REFERENCE_SHAPES = {
    "demo1": [
        (10240, 3840, 768, _T, _N), (3840, 2560, 1024, _T, _N), (3840, 768, 1024, _T, _N),
        (3072, 64, 3840, _N, _T), (3840, 64, 1024, _T, _N), (10240, 3840, 256, _T, _N),
        (3840, 3840, 768, _T, _N), (3840, 3840, 256, _T, _N), (768, 3840, 10240, _N, _T),
        (768, 3840, 10240, _N, _N), (768, 10240, 3840, _N, _T), (3840, 10240, 768, _T, _N),
        (768, 10240, 3840, _N, _N), (1024, 3840, 2560, _N, _T), (256, 3840, 10240, _N, _T),
        (256, 10240, 3840, _N, _T), (768, 3840, 3840, _N, _T), (256, 3840, 10240, _N, _N),
        (768, 3840, 3840, _N, _N), (1024, 3840, 768, _N, _T), (3840, 10240, 256, _T, _N),
        (256, 10240, 3840, _N, _N), (1024, 3840, 64, _N, _T), (256, 3840, 3840, _N, _T),
        (256, 3840, 3840, _N, _N), (64, 3840, 3072, _T, _N), (3072, 3840, 64, _N, _N),
    ],
    "demo2": [(1024, 2560, 3840, _N, _N), (1024, 64, 3840, _N, _N), (1024, 768, 3840, _N, _N)],
    "outer": [(15360, 256, 1, _T, _N), (3840, 256, 1, _T, _N), (1024, 256, 1, _T, _N), (256, 1024, 1, _T, _N)],
    "vector": [
        (1, 256, 15360, _N, _N), (1, 15360, 256, _N, _T), (1, 256, 1024, _N, _T), (1, 1024, 256, _N, _T),
        (1, 256, 1024, _N, _N), (1, 3840, 256, _N, _T), (1, 256, 3840, _N, _N), (1, 1024, 256, _N, _N),
    ],
}

# The reference's published times for the demo1 / demo2 shapes on its SME
# host, seconds per call (gemm/README.md:74-110), for side-by-side reporting.
REFERENCE_SECONDS = {
    (10240, 3840, 768, _T, _N): 0.004775, (3840, 2560, 1024, _T, _N): 0.001910, (3840, 768, 1024, _T, _N): 0.000778,
    (3072, 64, 3840, _N, _T): 0.000535, (3840, 64, 1024, _T, _N): 0.000151, (10240, 3840, 256, _T, _N): 0.002255,
    (3840, 3840, 768, _T, _N): 0.002148, (3840, 3840, 256, _T, _N): 0.001001, (768, 3840, 10240, _N, _T): 0.005477,
    (768, 3840, 10240, _N, _N): 0.005559, (768, 10240, 3840, _N, _T): 0.005007, (3840, 10240, 768, _T, _N): 0.004977,
    (768, 10240, 3840, _N, _N): 0.005037, (1024, 3840, 2560, _N, _T): 0.002409, (256, 3840, 10240, _N, _T): 0.002391,
    (256, 10240, 3840, _N, _T): 0.002275, (768, 3840, 3840, _N, _T): 0.002127, (256, 3840, 10240, _N, _N): 0.002442,
    (768, 3840, 3840, _N, _N): 0.002248, (1024, 3840, 768, _N, _T): 0.000736, (3840, 10240, 256, _T, _N): 0.001657,
    (256, 10240, 3840, _N, _N): 0.002253, (1024, 3840, 64, _N, _T): 0.000155, (256, 3840, 3840, _N, _T): 0.001101,
    (256, 3840, 3840, _N, _N): 0.001079, (64, 3840, 3072, _T, _N): 0.000402, (3072, 3840, 64, _N, _N): 0.000445,
    (1024, 2560, 3840, _N, _N): 0.002372, (1024, 64, 3840, _N, _N): 0.001929, (1024, 768, 3840, _N, _N): 0.001094,
}

# Shapes (M, N, K, transA, transB) measured more than 3% faster on rocBLAS
# than on hipBLASLt on the MI355X (python -m harp_amd.gemm --bench, graph-timed
# device milliseconds: 0.0863 vs 0.0916, 0.0874 vs 0.0906, 0.0795 vs 0.0834);
# every other shape uses hipBLASLt (the two are within 3% there).
BACKEND_BY_SHAPE: Dict[Tuple[int, int, int, int, int], str] = {
    (10240, 3840, 768, _T, _N): "rocblas",
    (768, 3840, 10240, _N, _N): "rocblas",
    (3840, 10240, 768, _T, _N): "rocblas",
}

_BACKENDS = {"hipblaslt": "cublaslt", "rocblas": "cublas"}  # torch's names for the ROCm libraries


def _normalize(t: int) -> int:
    return TRANS if t == CONJ_TRANS else t  # real data: conjugate transpose = transpose


def _op(x: torch.Tensor, trans: int, rows: int, cols: int) -> torch.Tensor:
    """op(X) as a [rows, cols] view of the dense row-major storage."""
    if trans == NO_TRANS:
        return x.reshape(-1)[: rows * cols].view(rows, cols)
    return x.reshape(-1)[: rows * cols].view(cols, rows).t()


class _Backend:
    """Select the BLAS library for the GEMMs issued inside the block."""

    def __init__(self, name: Optional[str]):
        self.name = name

    def __enter__(self):
        if self.name is None:
            return self
        self.prev = torch.backends.cuda.preferred_blas_library()
        torch.backends.cuda.preferred_blas_library(_BACKENDS[self.name])
        return self

    def __exit__(self, *exc):
        if self.name is not None:
            torch.backends.cuda.preferred_blas_library(self.prev)


def xhblas_gemm(order: int, trans_a: int, trans_b: int, M: int, N: int, K: int, alpha: float,
                A: torch.Tensor, lda: int, B: torch.Tensor, ldb: int, beta: float, C: torch.Tensor, ldc: int,
                ba: Optional[torch.Tensor] = None, sign: int = 0, backend: Optional[str] = None) -> int:
    """C = alpha * op(A) @ op(B) on device bf16 tensors; returns the reference's
    status (0 ok, -1 order, -2 / -3 transpose, -4 negative size, -5 leading
    dimension, -8 beta != 0).  ``backend`` forces "hipblaslt" or "rocblas"."""
    trans_a, trans_b = _normalize(trans_a), _normalize(trans_b)
    if order != ROW_MAJOR:
        return -1
    if trans_a not in (NO_TRANS, TRANS):
        return -2
    if trans_b not in (NO_TRANS, TRANS):
        return -3
    if M < 0 or N < 0 or K < 0:
        return -4
    # the reference's order (bgemm.cpp:324-349): leading dimensions before
    # beta; it returns -6 for a shape outside its table, where every shape
    # runs here
    a_cols = K if trans_a == NO_TRANS else M
    b_cols = N if trans_b == NO_TRANS else K
    if lda != a_cols or ldb != b_cols or ldc != N:
        return -5
    if beta != 0.0:
        return -8
    if M == 0 or N == 0:
        return 0
    for name, t in (("A", A), ("B", B), ("C", C)):
        if not t.is_cuda:
            raise RuntimeError(f"xhblas_gemm: {name} must be on a HIP device (there is no CPU path)")
        if t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise RuntimeError(f"xhblas_gemm: {name} must be a contiguous bfloat16 tensor")
    if A.numel() < M * K or B.numel() < K * N or C.numel() < M * N:
        raise RuntimeError("xhblas_gemm: a buffer is smaller than its matrix")
    c = C.reshape(-1)[: M * N].view(M, N)
    if K == 0 or alpha == 0.0:
        c.zero_()
        return 0
    a = _op(A, trans_a, M, K)
    b = _op(B, trans_b, K, N)
    key = (M, N, K, trans_a, trans_b)
    with _Backend(backend if backend is not None else BACKEND_BY_SHAPE.get(key, "hipblaslt")):
        if sign == 1 and ba is not None:
            # accumulator starts at the bias: alpha * (op(A) op(B) + ba)
            torch.addmm(ba.reshape(-1)[:N].view(1, N).expand(M, N), a, b, beta=alpha, alpha=alpha, out=c)
        else:
            torch.mm(a, b, out=c)
            if alpha != 1.0:
                c.mul_(alpha)
    if sign == 2 and ba is not None:
        # bias gradient: column sums of the transposed A's K rows
        ba.reshape(-1)[:M].copy_(A.reshape(-1)[: K * M].view(K, M).float().sum(0))
    return 0


def _bench_shape(shape, backend: str, iters: int = 20) -> float:
    """Device milliseconds per call: ``iters`` calls captured into one HIP
    graph and replayed, so host-side dispatch does not bound small shapes.
    (Timing only: the replays' outputs are not used.)"""
    M, N, K, ta, tb = shape
    g = torch.Generator(device="cuda").manual_seed(3407)
    A = torch.randn(M * K, device="cuda", generator=g).to(torch.bfloat16)
    B = torch.randn(K * N, device="cuda", generator=g).to(torch.bfloat16)
    C = torch.empty(M * N, device="cuda", dtype=torch.bfloat16)
    lda = K if ta == NO_TRANS else M
    ldb = N if tb == NO_TRANS else K

    def call():
        assert xhblas_gemm(ROW_MAJOR, ta, tb, M, N, K, 1.0, A, lda, B, ldb, 0.0, C, N, backend=backend) == 0

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            call()
    graph.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    best = float("inf")
    for _ in range(3):
        ev[0].record()
        graph.replay()
        ev[1].record()
        torch.cuda.synchronize()
        best = min(best, ev[0].elapsed_time(ev[1]) / iters)
    return best


def bench_table(iters: int = 20) -> list:
    """Per reference shape: ms and TFLOP/s on hipBLASLt and on rocBLAS, the
    faster one, and the reference's SME time where it publishes one."""
    rows = []
    peak = 2516.6
    for group, shapes in REFERENCE_SHAPES.items():
        for shape in shapes:
            M, N, K, ta, tb = shape
            flop = 2.0 * M * N * K
            res = {}
            for be in ("hipblaslt", "rocblas"):
                ms = _bench_shape(shape, be, iters)
                res[be] = ms
            best = min(res, key=res.get)
            ref_s = REFERENCE_SECONDS.get(shape)
            rows.append({
                "group": group, "M": M, "N": N, "K": K,
                "transA": "T" if ta == TRANS else "N", "transB": "T" if tb == TRANS else "N",
                "hipblaslt_ms": round(res["hipblaslt"], 4), "rocblas_ms": round(res["rocblas"], 4),
                "best": best, "best_tflops": round(flop / (res[best] * 1e-3) / 1e12, 1),
                "frac_bf16_peak": round(flop / (res[best] * 1e-3) / 1e12 / peak, 4),
                "reference_sme_ms": None if ref_s is None else round(ref_s * 1e3, 3),
            })
            print(json.dumps(rows[-1]), flush=True)
    return rows


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description="GEMM table at the reference's Linear shapes (gemm/README.md)")
    ap.add_argument("--bench", action="store_true")
    ap.add_argument("--iters", type=int, default=20)
    args = ap.parse_args()
    if args.bench:
        bench_table(args.iters)
