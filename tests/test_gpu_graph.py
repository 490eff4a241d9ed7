"""HIP-graph capture of the block's operators: ring-attention forward, delta
and backward (torch.ops.ring_attention_ops), the fused QK RMSNorm + RoPE
forward and backward (torch.ops.async_op) and the fused q/k/v projection
kernel (harp_amd.qkv) are recorded once into a
torch.cuda.CUDAGraph on static tensors and replayed on new inputs.  No
operator allocates device memory outside torch's allocator or clears memory
with hipMemsetAsync, so each replay must equal the eager result on the same
inputs bit for bit.  Between replays the test runs its own eager work and
synchronizes, and it checks every replay."""

import math

import pytest
import torch

import harp_amd
from harp_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _inputs(seed, B=1, H=2, T=256, D=64, N=2):
    g = torch.Generator().manual_seed(seed)

    def tok(t):  # token-major storage seen as [B, H, T, D]
        return (torch.randn((B, t, H, D), generator=g)).to(torch.bfloat16).to(DEV).transpose(1, 2)

    return tok(T), tok(N * T), tok(N * T), tok(T)


def _ring_step(q, k, v, do, N, out, m, l, dq, dk, dv):
    """Forward, delta and backward through the operators, into given tensors."""
    ops = torch.ops.ring_attention_ops
    scale = 1.0 / math.sqrt(q.size(-1))
    m.fill_(float("-inf"))
    ops.ring_attention_forward(q, k, v, out, m, l, N, scale)
    D = ops.ring_attention_delta(do, out)
    ops.ring_attention_backward(q, dq, k, dk, v, dv, do, m, l, D, N, scale)


@pytest.mark.parametrize("D", [64, 128])  # compiled kernels; the hand-scheduled D = 128 loops
def test_ring_attention_graph_replays_equal_eager(D):
    harp_amd.load_ops()
    _lib.timing_enable(False)  # no per-launch timing events inside the capture
    N = 2
    q, k, v, do = _inputs(0, D=D)
    out = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    B, H, T, _ = q.shape
    m = torch.empty((B, H, T, 1), dtype=torch.bfloat16, device=DEV)
    l = torch.empty((B, H, T, 1), dtype=torch.float32, device=DEV)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    outs = (out, m, l, dq, dk, dv)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside capture, as torch requires
        _ring_step(q, k, v, do, N, *outs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _ring_step(q, k, v, do, N, *outs)

    for seed in (1, 2, 3):
        nq, nk, nv, ndo = _inputs(seed, D=D)
        for dst, src in ((q, nq), (k, nk), (v, nv), (do, ndo)):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]
        # eager on the same inputs, into fresh tensors
        ref = [torch.empty_like(t) for t in outs]
        _ring_step(nq, nk, nv, ndo, N, *ref)
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "m", "l", "dq", "dk", "dv"), got, ref):
            assert torch.equal(a, b), (seed, name)


def test_qk_norm_rope_graph_replays_equal_eager():
    harp_amd.load_async_ops()
    ops = torch.ops.async_op
    B, H, S, D = 1, 4, 128, 128
    g = torch.Generator().manual_seed(5)

    def tok():
        return torch.randn((B, S, H, D), generator=g).to(torch.bfloat16).to(DEV).transpose(1, 2)

    x, dy = tok(), tok()
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(DEV)
    ang = torch.arange(S, dtype=torch.float64)[:, None] * (10000.0 ** (-2.0 * torch.arange(D // 2) / D))[None, :]
    f = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).to(DEV)
    y, dx = torch.empty_like(x), torch.empty_like(x)
    rms = torch.empty(B * H * S, dtype=torch.float32, device=DEV)
    gw = torch.empty(D, dtype=torch.bfloat16, device=DEV)

    def step(x_, dy_, y_, rms_, dx_, gw_):
        ops.qk_norm_rope_forward(x_, w, f, y_, rms_, 1e-6)
        ops.qk_norm_rope_backward(x_, dy_, w, rms_, f, dx_, gw_)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(x, dy, y, rms, dx, gw)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(x, dy, y, rms, dx, gw)

    for _ in range(3):
        nx, ndy = tok(), tok()
        x.copy_(nx)
        dy.copy_(ndy)
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (y, rms, dx, gw)]
        ref = [torch.empty_like(t) for t in (y, rms, dx, gw)]
        step(nx, ndy, *ref)
        torch.cuda.synchronize()
        for name, a, b in zip(("y", "rms", "dx", "grad_weight"), got, ref):
            assert torch.equal(a, b), name


def test_fused_producer_graph_replays_equal_eager():
    """The fused q/k/v projection kernel (harp_amd.qkv.qkv_project, with the
    pre-norm products and rms kept) at a shape whose half-empty last round
    goes to the tail launch: two launches in the graph."""
    from harp_amd import qkv

    B, S, dim, H = 1, 90 * 256, 128, 2
    g = torch.Generator().manual_seed(11)
    x = torch.randn((B, S, dim), generator=g).to(torch.bfloat16).to(DEV)
    ws = [(torch.randn((H * 128, dim), generator=g) / dim ** 0.5).to(torch.bfloat16).to(DEV) for _ in range(3)]
    w = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(DEV)
    ang = torch.arange(S, dtype=torch.float64)[:, None] * (10000.0 ** (-2.0 * torch.arange(64) / 128))[None, :]
    f = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).to(DEV)
    norms = [(w, 1e-6), (w, 1e-6), (None, 0.0)]

    def step(x_):
        outs, lins, rmss = qkv.qkv_project(x_, ws, norms, f, keep_for_backward=True)
        return list(outs) + [lins[0], lins[1], rmss[0], rmss[1]]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step(x)

    for _ in range(3):
        nx = torch.randn((B, S, dim), generator=g).to(torch.bfloat16).to(DEV)
        x.copy_(nx)
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in static]
        ref = step(nx)
        torch.cuda.synchronize()
        for name, a, b in zip(("q", "k", "v", "q_lin", "k_lin", "rms_q", "rms_k"), got, ref):
            assert torch.equal(a, b), name
