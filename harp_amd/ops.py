"""Python call pattern of the ring-attention block on the HIP path.

* :class:`RingAttention` mirrors ``CPURingAttention``
  (src/models/z_image/module/attn.py:15-49): same arguments, same caller-
  allocated ``out`` (fp32, q's token-major strides), bf16 ``m_i`` and fp32
  ``l_i``, same saved tensors, same ``D = rowsum(dO * O)`` preprocess (here one
  kernel, ``ring_attention_delta``), same op calls by name through
  ``torch.ops.ring_attention_ops``.
* :func:`abi_forward` / :func:`abi_backward` / :func:`abi_delta` call
  libharp_ra.so's C ABI directly (ctypes), with per-chunk pointers, so the KV
  chunks of the ring need not be contiguous.

Single-GPU ring semantics: ``k``/``v`` carry all ``sp_size`` chunks of the
ring concatenated along dim 2 (``k.size(2) / sp_size`` rows each, passed to
the operators as ``kv_chunk_len``); chunk ``c`` is visited at step
``(c - ring_rank) % sp_size`` (ring_attn.cpp:2497).
"""

from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib


def _ops():
    _lib.load_ops()
    return torch.ops.ring_attention_ops


class RingAttention(torch.autograd.Function):
    """Autograd Function with the reference's call pattern (attn.py:15-49)."""

    @staticmethod
    def forward(ctx, local_q, local_k, local_v, sp_size, ring_rank=0, kv_lens=None):
        ctx.sp_size = sp_size
        ctx.ring_rank = ring_rank
        ctx.kv_lens = kv_lens
        if local_k.size(2) % sp_size:
            raise ValueError(f"k/v hold all sp_size={sp_size} chunks along dim 2: k.size(2)={local_k.size(2)} "
                             "is not a multiple of sp_size")
        ctx.chunk_len = local_k.size(2) // sp_size
        scale = 1.0 / math.sqrt(local_q.size(-1))  # attn.py:20
        ctx.scale = scale
        mm_type = local_q.dtype
        B, H, T, _ = local_q.shape
        # attn.py:24-27 allocates out with zeros_like (token-major strides); every
        # element is written by the kernel, so empty_like keeps the layout without a fill
        out = torch.empty_like(local_q, dtype=torch.float32)
        m_i = torch.full((B, H, T, 1), float("-inf"), device=local_q.device, dtype=torch.bfloat16)
        l_i = torch.empty((B, H, T, 1), device=local_q.device, dtype=torch.float32)
        _ops().ring_attention_forward(local_q, local_k, local_v, out, m_i, l_i, sp_size, scale, ring_rank, kv_lens,
                                      ctx.chunk_len)
        ctx.save_for_backward(local_q, local_k, local_v, out, m_i, l_i)
        return out.to(mm_type)

    @staticmethod
    def backward(ctx, grad_out):
        local_q, local_k, local_v, out, m_i, l_i = ctx.saved_tensors
        grad_out = _kernel_view(grad_out.to(torch.bfloat16))
        D = _ops().ring_attention_delta(grad_out, out)  # attn.py:41
        grad_q = torch.empty_like(local_q, dtype=torch.bfloat16)
        grad_k = torch.empty_like(local_k, dtype=torch.bfloat16)
        grad_v = torch.empty_like(local_v, dtype=torch.bfloat16)
        _ops().ring_attention_backward(
            local_q, grad_q, local_k, grad_k, local_v, grad_v, grad_out, m_i, l_i, D,
            ctx.sp_size, ctx.scale, ctx.ring_rank, ctx.kv_lens, ctx.chunk_len,
        )
        return grad_q, grad_k, grad_v, None, None, None


def _kernel_view(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` if the kernels can read it in place (unit D stride, other
    strides multiples of 8 elements, 16-byte aligned), else a contiguous copy."""
    ok = (
        t.stride(3) == 1
        and all(s % 8 == 0 and s >= 0 for s in t.stride()[:3])
        and t.data_ptr() % 16 == 0
    )
    return t if ok else t.contiguous()


def ring_attention(q, k, v, sp_size: int, ring_rank: int = 0, kv_lens: Optional[Sequence[int]] = None):
    """Functional form: softmax(QK^T/sqrt(D)) V over all ring chunks, with autograd."""
    return RingAttention.apply(q, k, v, sp_size, ring_rank, None if kv_lens is None else list(kv_lens))


# ---------------------------------------------------------------------------
# Direct C-ABI calls (ctypes), used by tests and the benchmark
# ---------------------------------------------------------------------------

def _strides(t: torch.Tensor):
    return _lib.i64_array(t.stride())


def _stream_ptr(stream: Optional[torch.cuda.Stream]) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _lens_arg(kv_lens):
    return None if kv_lens is None else _lib.i32_array(kv_lens)


_SIZE_MAX = 2**64 - 1


def forward_workspace_bytes(B, H, T, D, sp_size, chunk_len, kv_lens=None) -> int:
    """Device scratch bytes the forward needs on the current device (raises
    on invalid sizes)."""
    n = int(_lib.load_abi().harp_ra_forward_workspace_bytes(B, H, T, D, sp_size, chunk_len, _lens_arg(kv_lens)))
    if n == _SIZE_MAX:
        raise ValueError(_lib.last_error())
    return n


def backward_workspace_bytes(B, H, T, D, sp_size, chunk_len, kv_lens=None) -> int:
    """Device scratch bytes the backward needs on the current device (raises
    on invalid sizes)."""
    n = int(_lib.load_abi().harp_ra_backward_workspace_bytes(B, H, T, D, sp_size, chunk_len, _lens_arg(kv_lens)))
    if n == _SIZE_MAX:
        raise ValueError(_lib.last_error())
    return n


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _ws_ptr(ws: torch.Tensor):
    return ws.data_ptr() if ws.numel() else None


def abi_forward(
    q: torch.Tensor,
    k_chunks: Sequence[torch.Tensor],
    v_chunks: Sequence[torch.Tensor],
    out: torch.Tensor,
    m_i: torch.Tensor,
    l_i: torch.Tensor,
    scale: float,
    ring_rank: int = 0,
    kv_lens: Optional[Sequence[int]] = None,
    workspace: Optional[torch.Tensor] = None,
    stream: Optional[torch.cuda.Stream] = None,
) -> None:
    lib = _lib.load_abi()
    B, H, T, D = q.shape
    n = len(k_chunks)
    chunk_len = k_chunks[0].shape[2]
    if workspace is None:
        workspace = _workspace(forward_workspace_bytes(B, H, T, D, n, chunk_len, kv_lens), q.device)
    m_code = _lib.HARP_RA_BF16 if m_i.dtype == torch.bfloat16 else _lib.HARP_RA_F32
    rc = lib.harp_ra_forward(
        q.data_ptr(), _strides(q),
        _lib.ptr_array([c.data_ptr() for c in k_chunks]), _lib.ptr_array([c.data_ptr() for c in v_chunks]),
        _strides(k_chunks[0]), chunk_len, _lens_arg(kv_lens),
        out.data_ptr(), _strides(out), m_i.data_ptr(), m_code, l_i.data_ptr(),
        B, H, T, D, n, ring_rank, float(scale),
        _ws_ptr(workspace), workspace.numel(), _stream_ptr(stream),
    )
    _lib.check(rc, "harp_ra_forward")


def abi_delta(grad_out: torch.Tensor, out: torch.Tensor, delta: torch.Tensor, stream=None) -> None:
    lib = _lib.load_abi()
    B, H, T, D = out.shape
    rc = lib.harp_ra_delta(grad_out.data_ptr(), _strides(grad_out), out.data_ptr(), _strides(out),
                           delta.data_ptr(), B, H, T, D, _stream_ptr(stream))
    _lib.check(rc, "harp_ra_delta")


def abi_backward(
    q: torch.Tensor,
    dq: torch.Tensor,
    k_chunks: Sequence[torch.Tensor],
    v_chunks: Sequence[torch.Tensor],
    dk_chunks: Sequence[torch.Tensor],
    dv_chunks: Sequence[torch.Tensor],
    grad_out: torch.Tensor,
    m_i: torch.Tensor,
    l_i: torch.Tensor,
    delta: torch.Tensor,
    scale: float,
    ring_rank: int = 0,
    kv_lens: Optional[Sequence[int]] = None,
    workspace: Optional[torch.Tensor] = None,
    stream: Optional[torch.cuda.Stream] = None,
) -> None:
    lib = _lib.load_abi()
    B, H, T, D = q.shape
    n = len(k_chunks)
    chunk_len = k_chunks[0].shape[2]
    if workspace is None:
        workspace = _workspace(backward_workspace_bytes(B, H, T, D, n, chunk_len, kv_lens), q.device)

    def code(t):
        return _lib.HARP_RA_BF16 if t.dtype == torch.bfloat16 else _lib.HARP_RA_F32

    rc = lib.harp_ra_backward(
        q.data_ptr(), _strides(q), dq.data_ptr(), _strides(dq), code(dq),
        _lib.ptr_array([c.data_ptr() for c in k_chunks]), _lib.ptr_array([c.data_ptr() for c in v_chunks]),
        _strides(k_chunks[0]),
        _lib.ptr_array([c.data_ptr() for c in dk_chunks]), _lib.ptr_array([c.data_ptr() for c in dv_chunks]),
        _strides(dk_chunks[0]), code(dk_chunks[0]),
        chunk_len, _lens_arg(kv_lens),
        grad_out.data_ptr(), _strides(grad_out),
        m_i.data_ptr(), code(m_i), l_i.data_ptr(), delta.data_ptr(),
        B, H, T, D, n, ring_rank, float(scale),
        _ws_ptr(workspace), workspace.numel(), _stream_ptr(stream),
    )
    _lib.check(rc, "harp_ra_backward")


def concat_chunks(chunks: Sequence[torch.Tensor]) -> torch.Tensor:
    """Concatenate [B,H,Tc,D] chunks along T into one token-major [B,H,N*Tc,D] view
    (physical [B, N*Tc, H, D]), the k/v layout the torch operators take."""
    B, H, Tc, D = chunks[0].shape
    phys = torch.empty((B, len(chunks) * Tc, H, D), dtype=chunks[0].dtype, device=chunks[0].device)
    view = phys.transpose(1, 2)
    for i, c in enumerate(chunks):
        view[:, :, i * Tc:(i + 1) * Tc].copy_(c)
    return view
