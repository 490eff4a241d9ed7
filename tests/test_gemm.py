"""xhblas_gemm (harp_amd.gemm), the GPU counterpart of the reference's Linear
GEMM entry point (gemm/bgemm/bgemm.cpp:316-424): status codes on the host
(CPU tests), and on the GPU every shape of the reference's table
(gemm/README.md:12-70) against an fp32 product of the same bf16 inputs, plus
the bias (sign 1) and bias-gradient (sign 2) options."""

import pytest
import torch

from harp_amd import gemm as G

R, NT, T = G.ROW_MAJOR, G.NO_TRANS, G.TRANS
DUMMY = torch.zeros(1, dtype=torch.bfloat16)  # never touched: validation returns first


@pytest.mark.parametrize(
    "args,code",
    [
        (dict(order=G.COL_MAJOR), -1),
        (dict(trans_a=7), -2),
        (dict(trans_b=7), -3),
        (dict(M=-1), -4),
        (dict(M=0), 0),  # nothing to do
        (dict(N=0, ldb=0, ldc=0), 0),
        (dict(beta=1.0), -8),
        (dict(lda=65), -5),
        (dict(ldb=17), -5),
        (dict(ldc=31), -5),
        # bgemm.cpp:324-349 checks the leading dimensions before beta and
        # before anything is done, degenerate sizes included
        (dict(M=0, lda=65), -5),
        (dict(N=0, ldc=31), -5),
        (dict(lda=65, beta=1.0), -5),
        (dict(M=0, beta=1.0), -8),
    ],
)
def test_status_codes_match_the_reference(args, code):
    a = dict(order=R, trans_a=NT, trans_b=NT, M=8, N=32, K=64, alpha=1.0, A=DUMMY, lda=64, B=DUMMY, ldb=32,
             beta=0.0, C=DUMMY, ldc=32)
    a.update(args)
    assert G.xhblas_gemm(**a) == code


def test_cpu_tensors_raise():
    A = torch.zeros(8 * 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        G.xhblas_gemm(R, NT, NT, 8, 32, 64, 1.0, A, 64, A, 32, 0.0, A, 32)


def test_reference_table_is_complete():
    # gemm/README.md:12-70: 27 + 3 + 4 + 8 shapes; every timed shape has a table entry
    assert [len(v) for v in G.REFERENCE_SHAPES.values()] == [27, 3, 4, 8]
    listed = {s for v in G.REFERENCE_SHAPES.values() for s in v}
    assert set(G.REFERENCE_SECONDS) <= listed and len(G.REFERENCE_SECONDS) == 30


def _inputs(M, N, K, ta, tb, seed):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(M * K, generator=g).to(torch.bfloat16)
    B = torch.randn(K * N, generator=g).to(torch.bfloat16)
    a = A.view(M, K) if ta == NT else A.view(K, M).t()
    b = B.view(K, N) if tb == NT else B.view(N, K).t()
    return A, B, a.double(), b.double()


ALL_SHAPES = [s for v in G.REFERENCE_SHAPES.values() for s in v]


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ALL_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}x{s[2]}{'TN'[s[3] == NT]}{'TN'[s[4] == NT]}")
def test_reference_shapes_match_fp64(shape):
    """A reference shape on hipBLASLt, on rocBLAS and on the per-shape choice,
    each within bf16 rounding of the fp64 product of the same bf16 inputs
    (computed on the GPU in fp64)."""
    M, N, K, ta, tb = shape
    A, B, _, _ = _inputs(M, N, K, ta, tb, seed=M + N + K)
    Ad, Bd = A.cuda(), B.cuda()
    a = (Ad.view(M, K) if ta == NT else Ad.view(K, M).t()).double()
    b = (Bd.view(K, N) if tb == NT else Bd.view(N, K).t()).double()
    ref = 0.5 * (a @ b)
    # elementwise bound: two bf16 units of |ref| plus an fp32-accumulation term
    tol = 2 * 2.0 ** -8 * ref.abs() + 0.5e-5 * (a.abs() @ b.abs())
    lda = K if ta == NT else M
    ldb = N if tb == NT else K
    for backend in ("hipblaslt", "rocblas", None):
        C = torch.full((M * N,), float("nan"), dtype=torch.bfloat16, device="cuda")
        assert G.xhblas_gemm(R, ta, tb, M, N, K, 0.5, Ad, lda, Bd, ldb, 0.0, C, N, backend=backend) == 0
        got = C.double().view(M, N)
        rel = ((got - ref).norm() / ref.norm()).item()
        # one bf16 rounding of the result: relative RMS error about 2^-9 / sqrt(3)
        assert rel <= 4e-3, (shape, backend, rel)
        assert bool(((got - ref).abs() <= tol).all()), (shape, backend)


@pytest.mark.gpu
def test_bias_and_bias_gradient():
    M, N, K = 768, 3840, 256
    A, B, a, b = _inputs(M, N, K, T, NT, seed=99)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    C = torch.empty(M * N, dtype=torch.bfloat16, device="cuda")
    # sign 1: the accumulator starts at the bias, alpha scales both
    assert G.xhblas_gemm(R, T, NT, M, N, K, 2.0, A.cuda(), M, B.cuda(), N, 0.0, C, N, ba=bias.cuda(), sign=1) == 0
    ref = 2.0 * (a @ b + bias.double()[None, :])
    got = C.cpu().double().view(M, N)
    assert ((got - ref).norm() / ref.norm()).item() <= 4e-3
    # sign 2: ba[j] = sum over the K rows of the transposed A, column j
    ba = torch.full((M,), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert G.xhblas_gemm(R, T, NT, M, N, K, 1.0, A.cuda(), M, B.cuda(), N, 0.0, C, N, ba=ba, sign=2) == 0
    want = A.view(K, M).double().sum(0)
    assert torch.allclose(ba.cpu().double(), want, rtol=2.0 ** -7, atol=1e-2)


@pytest.mark.gpu
def test_zero_k_and_zero_alpha_clear_c():
    C = torch.ones(64 * 32, dtype=torch.bfloat16, device="cuda")
    A = torch.ones(64 * 8, dtype=torch.bfloat16, device="cuda")
    assert G.xhblas_gemm(R, NT, NT, 64, 32, 8, 0.0, A, 8, A, 32, 0.0, C, 32) == 0
    assert (C == 0).all()
