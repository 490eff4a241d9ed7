"""Shared helpers for parity tests: seeded inputs, the relative-error metric
and the tolerances of the parity contract."""

from __future__ import annotations

import torch

# Parity bars (bf16 inputs, fp32-or-better reference): O and LSE within 2e-2,
# dQ / dK / dV within 3e-2, in relative Frobenius norm.
TOL_O = 2e-2
TOL_LSE = 2e-2
TOL_GRAD = 3e-2


def rel_fro(x: torch.Tensor, ref: torch.Tensor) -> float:
    x = x.double().cpu()
    ref = ref.double().cpu()
    den = torch.linalg.vector_norm(ref).item()
    num = torch.linalg.vector_norm(x - ref).item()
    return num / den if den > 0 else num


def rel_max(x: torch.Tensor, ref: torch.Tensor) -> float:
    x = x.double().cpu()
    ref = ref.double().cpu()
    den = ref.abs().max().item()
    return (x - ref).abs().max().item() / den if den > 0 else (x - ref).abs().max().item()


def token_major(B: int, T: int, H: int, D: int, device, dtype=torch.bfloat16) -> torch.Tensor:
    """Empty [B,H,T,D] view over token-major [B,T,H,D] storage."""
    return torch.empty((B, T, H, D), device=device, dtype=dtype).transpose(1, 2)
