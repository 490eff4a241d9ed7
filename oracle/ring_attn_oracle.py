"""CPU oracle for HARP's ring-attention block (forward + backward).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or, for the baseline, as the timed CPU restatement).  The product path
(``harp_amd``) never imports it and has no CPU fallback.

What it restates
----------------
The reference kernel is ``gemm/ring_attention/ring_attn.cpp`` (ARMv9 SME, not
buildable on x86: it needs ``arm_sme.h``, KBLAS and MPI).  Its arithmetic is:

* forward, ``ring_attention_forward`` (ring_attn.cpp:2412-2575): for every head
  and ring step ``s`` with chunk ``c = (s + rank) % sp_size`` (:2497):
  ``S = scale * Q K_c^T`` (:2513-2516); step 0 sets ``m = rowmax(S)``,
  ``l = sum exp(S - m)`` and ``O = P V_c`` (:2517-2537); later steps take
  ``m' = max(rowmax S, m)``, ``corr = exp(m - m')``, ``l = sum exp(S - m') + l*corr``,
  ``O = O*corr + P V_c`` (:2538-2567); finally ``O /= l`` (:2569-2573).
* backward, ``ring_attention_backward`` (ring_attn.cpp:2577-2829), KV-stationary:
  for the chunk a rank owns, per query chunk, ``S = scale Q K^T`` (:2767-2772),
  ``dP = dO V^T`` (:2773-2778), ``P = exp(S - m)/l`` and
  ``dS = P (dP - D) scale`` (``sve_exp_li``, :1199-1338, called at :2780-2788),
  ``dQpart = dS K`` (:2794-2799), ``dK += dS^T Q`` and ``dV += P^T dO``
  (:2800-2814); ``dQ = sum over owners of dQpart`` (:2817-2828).
* ``D = rowsum(dO * O)`` is computed by the Python caller
  (src/models/z_image/module/attn.py:41) and passed to the backward op.

The oracle evaluates this math in the requested dtype (float64 by default) on
the same bf16 inputs the GPU sees.  It deliberately does NOT reproduce the
reference's rounding shortcuts (bf16-truncated S/dP, FEXPA exp, bf16 m_i,
bf16 dK/dV accumulation, bf16 softmax scale): the parity contract is fp32-or-
better math on bf16 inputs.  ``reference_rounding=True`` on
:func:`ring_forward` restates the two cheapest of those shortcuts (bf16 S by
truncation, bf16 m) for diagnostics only; it is never the pass/fail oracle.

Single-GPU emulation of one rank's share: ``q`` is the local query chunk
(T rows), ``k_chunks``/``v_chunks`` are the N = sp_size KV chunks of the ring.
The forward is Q-stationary over the chunks in ring order starting at
``ring_rank``; the backward returns dQ for the local rows and Q_local's
contribution to dK/dV of every chunk (the KV-stationary sum of the reference
restricted to one query chunk).

Key padding: ``kv_valid_lens[c]`` keys of chunk ``c`` are valid; the rest are
masked (their P is exactly 0).  This is the boolean key-padding-mask semantics
of ``F.scaled_dot_product_attention`` used by the reference model's
non-ring attention (src/models/z_image/standalone_transformer.py:259-269).

How each function is pinned (tests/test_oracle.py):
* ring_forward: vs torch.nn.functional.scaled_dot_product_attention (fp64) on
  the concatenated, masked KV; vs brute-force fp64 loops on tiny shapes;
  invariance under chunk order / ring_rank; LSE associativity.
* ring_backward: vs fp64 autograd through SDPA; vs central finite differences
  on tiny fp64 inputs; D identity rowsum(dO*O) == rowsum(P*dP).
* delta: vs an explicit einsum and the rowsum(P*dP) identity.
"""

from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import torch

LOG2E = 1.4426950408889634

__all__ = [
    "ring_forward",
    "ring_backward",
    "delta",
    "lse_from_ml",
    "make_inputs",
    "cpu_baseline_fwd_bwd",
]


def _chunk_order(n: int, ring_rank: int) -> List[int]:
    # ring_attn.cpp:2497 (forward) and :2724 (backward): step s visits (s + rank) % n
    return [(s + ring_rank) % n for s in range(n)]


def _valid(kv_valid_lens: Optional[Sequence[int]], chunks: Sequence[torch.Tensor]) -> List[int]:
    if kv_valid_lens is None:
        return [c.shape[2] for c in chunks]
    lens = [int(x) for x in kv_valid_lens]
    assert len(lens) == len(chunks)
    for n, c in zip(lens, chunks):
        assert 0 <= n <= c.shape[2]
    return lens


def ring_forward(
    q: torch.Tensor,
    k_chunks: Sequence[torch.Tensor],
    v_chunks: Sequence[torch.Tensor],
    scale: float,
    ring_rank: int = 0,
    kv_valid_lens: Optional[Sequence[int]] = None,
    dtype: torch.dtype = torch.float64,
    reference_rounding: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Online-softmax ring forward (ring_attn.cpp:2488-2574).

    q: [B,H,T,D]; k_chunks/v_chunks: N tensors [B,H,Tc,D].  Returns
    (O [B,H,T,D], m [B,H,T,1], l [B,H,T,1]) in ``dtype`` with
    ``m + log(l) = LSE`` (natural log) and O already divided by l.
    """
    n = len(k_chunks)
    lens = _valid(kv_valid_lens, k_chunks)
    qf = q.to(dtype)
    B, H, T, D = q.shape
    m = torch.full((B, H, T, 1), -math.inf, dtype=dtype)
    l = torch.zeros((B, H, T, 1), dtype=dtype)
    o = torch.zeros((B, H, T, D), dtype=dtype)
    for step, c in enumerate(_chunk_order(n, ring_rank)):
        kc = k_chunks[c][:, :, : lens[c]].to(dtype)
        vc = v_chunks[c][:, :, : lens[c]].to(dtype)
        if kc.shape[2] == 0:
            continue
        s = scale * torch.matmul(qf, kc.transpose(-1, -2))  # :2513-2516
        if reference_rounding:
            # Q1: bf16 output of the SME GEMM by truncation (ring_attn.cpp:203-237)
            s = _bf16_trunc(s.float()).to(dtype)
        rowmax = s.amax(dim=-1, keepdim=True)  # quick_max :1031-1081
        if reference_rounding:
            rowmax = rowmax.to(torch.bfloat16).to(dtype)  # Q5: m kept in bf16 (:2521)
        m_new = torch.maximum(m, rowmax)  # :2540-2543
        m_sub = torch.where(torch.isinf(m_new), torch.zeros_like(m_new), m_new)
        corr = torch.exp(m - m_sub)  # :2544
        p = torch.exp(s - m_sub)  # sve_exp :1083-1177
        l = l * corr + p.sum(dim=-1, keepdim=True)  # :2545-2547
        o = o * corr + torch.matmul(p, vc)  # sve_out :1179-1197, sbgemm :2563-2566
        m = m_new
    o = o / l  # :2569-2573
    return o, m, l


def lse_from_ml(m: torch.Tensor, l: torch.Tensor) -> torch.Tensor:
    """LSE = m + log(l): the statistic the backward recomputes P from
    (P = exp(S - m) / l in sve_exp_li, ring_attn.cpp:1199-1338)."""
    return m.to(torch.float64) + torch.log(l.to(torch.float64))


def delta(grad_out: torch.Tensor, out: torch.Tensor, dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """D = rowsum(dO * O) over the head dim, as attn.py:41 computes it."""
    return torch.sum(grad_out.to(dtype) * out.to(dtype), dim=-1, keepdim=True)


def ring_backward(
    q: torch.Tensor,
    k_chunks: Sequence[torch.Tensor],
    v_chunks: Sequence[torch.Tensor],
    grad_out: torch.Tensor,
    m: torch.Tensor,
    l: torch.Tensor,
    D: torch.Tensor,
    scale: float,
    ring_rank: int = 0,
    kv_valid_lens: Optional[Sequence[int]] = None,
    dtype: torch.dtype = torch.float64,
) -> Tuple[torch.Tensor, List[torch.Tensor], List[torch.Tensor]]:
    """KV-stationary ring backward restricted to one query chunk.

    Follows ring_attn.cpp:2723-2828: for every KV chunk c (the chunk a rank
    owns), with the local query chunk on the query side:
      S = scale Q K_c^T; dP = dO V_c^T; P = exp(S - m)/l;
      dS = P (dP - D) scale; dQ += dS K_c; dK_c = dS^T Q; dV_c = P^T dO.
    Returns (dQ [B,H,T,D], [dK_c], [dV_c]) in ``dtype``; pad keys
    (beyond kv_valid_lens) get zero gradient.
    """
    n = len(k_chunks)
    lens = _valid(kv_valid_lens, k_chunks)
    qf = q.to(dtype)
    dof = grad_out.to(dtype)
    mf = m.to(dtype)
    lf = l.to(dtype)
    Df = D.to(dtype)
    dq = torch.zeros(qf.shape, dtype=dtype)
    dks: List[torch.Tensor] = [torch.zeros(kc.shape, dtype=dtype) for kc in k_chunks]
    dvs: List[torch.Tensor] = [torch.zeros(vc.shape, dtype=dtype) for vc in v_chunks]
    for c in _chunk_order(n, ring_rank):
        nv = lens[c]
        if nv == 0:
            continue
        kc = k_chunks[c][:, :, :nv].to(dtype)
        vc = v_chunks[c][:, :, :nv].to(dtype)
        s = scale * torch.matmul(qf, kc.transpose(-1, -2))  # :2767-2772
        dp = torch.matmul(dof, vc.transpose(-1, -2))  # :2773-2778
        p = torch.exp(s - mf) / lf  # sve_exp_li: exp(S - m) / l
        ds = p * (dp - Df) * scale  # sve_exp_li: P (dP - D) scale
        dq += torch.matmul(ds, kc)  # :2794-2799 then owner sum :2819-2827
        dks[c][:, :, :nv] = torch.matmul(ds.transpose(-1, -2), qf)  # :2801-2806
        dvs[c][:, :, :nv] = torch.matmul(p.transpose(-1, -2), dof)  # :2809-2814
    return dq, dks, dvs


def _bf16_trunc(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> bf16 by truncation of the low 16 bits (the SME kernel's
    ``uzp2`` of the high halves, ring_attn.cpp:203-237)."""
    bits = x.contiguous().view(torch.int32) & ~0xFFFF
    return bits.view(torch.float32)


def make_inputs(
    B: int,
    H: int,
    T: int,
    D: int,
    n_chunks: int,
    seed: int = 3407,
    value_scale: float = 1.0,
    chunk_len: Optional[int] = None,
) -> Tuple[torch.Tensor, List[torch.Tensor], List[torch.Tensor], torch.Tensor]:
    """Seeded synthetic inputs in the benchmark's draw order.

    fp32 randn from ``torch.Generator().manual_seed(seed)`` (times
    ``value_scale``) cast to bf16, drawn in the order Q_local, K chunks
    0..N-1, V chunks 0..N-1, dO_local.  Each tensor is physically token-major
    ``[B, T, H, D]`` and returned as the ``[B, H, T, D]`` view, the layout of
    the reference's q/k/v (torch_ring_attention_ops.cpp:40-67).
    """
    tc = T if chunk_len is None else chunk_len
    g = torch.Generator().manual_seed(seed)

    def draw(rows: int) -> torch.Tensor:
        x = torch.randn((B, rows, H, D), generator=g, dtype=torch.float32)
        if value_scale != 1.0:
            x = x * value_scale
        return x.to(torch.bfloat16).transpose(1, 2)

    q = draw(T)
    ks = [draw(tc) for _ in range(n_chunks)]
    vs = [draw(tc) for _ in range(n_chunks)]
    do = draw(T)
    return q, ks, vs, do


def cpu_baseline_fwd_bwd(
    q: torch.Tensor,
    k_chunks: Sequence[torch.Tensor],
    v_chunks: Sequence[torch.Tensor],
    grad_out: torch.Tensor,
    scale: float,
) -> None:
    """The reference's algorithm as PyTorch CPU ops, for the timed CPU baseline.

    Mirrors ring_attn.cpp with its mixed precision: per ring step a bf16
    matmul for S (:2513-2516), fp32 online softmax with running max / sum
    merge (:2517-2567), bf16 P into ``O += P V`` in fp32 (:2534-2566), O /= l;
    then the KV-stationary backward (:2723-2828) with bf16 GEMM operands and
    fp32 accumulation; D = rowsum(dO * O) as attn.py:41.
    """
    n = len(k_chunks)
    B, H, T, D = q.shape
    m = torch.full((B, H, T, 1), -math.inf)
    l = torch.zeros((B, H, T, 1))
    o = torch.zeros((B, H, T, D))
    for c in range(n):
        s = torch.matmul(q, k_chunks[c].transpose(-1, -2)).float() * scale
        m_new = torch.maximum(m, s.amax(dim=-1, keepdim=True))
        corr = torch.exp(m - m_new)
        p = torch.exp(s - m_new)
        l = l * corr + p.sum(dim=-1, keepdim=True)
        o = o * corr + torch.matmul(p.to(torch.bfloat16), v_chunks[c]).float()
        m = m_new
    o = o / l
    dmat = torch.sum(grad_out.float() * o, dim=-1, keepdim=True)
    lse = m + torch.log(l)
    dq = torch.zeros((B, H, T, D))
    for c in range(n):
        s = torch.matmul(q, k_chunks[c].transpose(-1, -2)).float() * scale
        dp = torch.matmul(grad_out, v_chunks[c].transpose(-1, -2)).float()
        p = torch.exp(s - lse)
        ds = (p * (dp - dmat) * scale).to(torch.bfloat16)
        pb = p.to(torch.bfloat16)
        dq += torch.matmul(ds, k_chunks[c]).float()
        torch.matmul(ds.transpose(-1, -2), q)  # dK_c
        torch.matmul(pb.transpose(-1, -2), grad_out)  # dV_c
