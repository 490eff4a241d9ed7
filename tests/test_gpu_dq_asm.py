"""GPU parity of the head-dim-128 dQ kernel (dq_asm.hip, the hand-scheduled
loop) on the paths its loop takes rarely: every exit point of the loop
unrolled over eight LDS block buffers, partial last blocks of a chunk (pad
keys whose zero K rows must contribute nothing), queries past T in the last
query block, chunks shorter than a block or empty, fp32 and bf16 dQ outputs,
and KV splits (partial dQ buffers summed on the host side of the split).
Bars as the other parity tests: dQ, dK, dV <= 3e-2 relative Frobenius error
against the fp64 oracle (oracle/ring_attn_oracle.py, ring_attn.cpp:2577-2829).
"""

import math

import pytest
import torch

from oracle import ring_attn_oracle as orc
from tests.gpu_harness import run_hip
from tests.parity import TOL_GRAD, rel_fro
from tests.test_gpu_parity import _check_all, _oracle_full

pytestmark = pytest.mark.gpu

D = 128


def _grad_check(res, ref):
    for name in ("dq", "dk", "dv"):
        err = rel_fro(res[name], ref[name])
        print(f"  {name}: rel {err:.2e}", flush=True)
        assert err <= TOL_GRAD, (name, err)


@pytest.mark.parametrize("nb", list(range(1, 10)))
@pytest.mark.parametrize("ragged", [False, True])
def test_every_loop_exit(nb, ragged):
    """One chunk of nb 32-key blocks (the last one partial when ragged): the
    loop leaves from slot (nb - 1) % 8; 70 queries leave most of the block's
    256 query rows past T."""
    n_keys = 32 * nb - (5 if ragged else 0)
    print(f"[dq exit nb={nb} keys={n_keys}]", flush=True)
    q, ks, vs, do = orc.make_inputs(1, 2, 70, D, 1, seed=200 + nb, chunk_len=n_keys)
    scale = 1.0 / math.sqrt(D)
    res = run_hip(q, ks, vs, do, scale)
    ref = _oracle_full(q, ks, vs, do, scale)
    _grad_check(res, ref)


@pytest.mark.parametrize("grad_dtype", [torch.bfloat16, torch.float32])
def test_tiny_and_empty_chunks(grad_dtype):
    """Chunks of 1, 0, 33, 0, 64 and 95 valid keys (chunk length 96) at two
    ring ranks: the copy cursor crosses chunks inside one slot and skips
    empty ones; every chunk but one ends in a partial block."""
    lens = [1, 0, 33, 0, 64, 95]
    for rank in (0, 3):
        print(f"[dq tiny chunks rank {rank} {grad_dtype}]", flush=True)
        q, ks, vs, do = orc.make_inputs(2, 3, 300, D, len(lens), seed=60 + rank, chunk_len=96)
        scale = 1.0 / math.sqrt(D)
        res = run_hip(q, ks, vs, do, scale, ring_rank=rank, kv_lens=lens, grad_dtype=grad_dtype)
        ref = _oracle_full(q, ks, vs, do, scale, rank=rank, lens=lens)
        _check_all(res, ref)


def test_kv_split_small_grid():
    """One 256-query block per head and eight chunks: the host splits the
    ring over grid dimension y; each split writes its own dQ partial."""
    q, ks, vs, do = orc.make_inputs(1, 1, 256, D, 8, seed=91, chunk_len=160)
    lens = [160, 131, 160, 7, 160, 160, 96, 160]
    scale = 1.0 / math.sqrt(D)
    res = run_hip(q, ks, vs, do, scale, ring_rank=5, kv_lens=lens)
    ref = _oracle_full(q, ks, vs, do, scale, rank=5, lens=lens)
    _check_all(res, ref)


def test_large_scores():
    """Scores of a few hundred (scale 1 instead of 1/sqrt(D)): P is exp2 of
    a large negative number for most keys and exactly 1 at the row maximum;
    the clamp must not alter valid probabilities."""
    g = torch.Generator().manual_seed(5)
    B, H, T, tc = 1, 2, 100, 150
    q = (2.0 * torch.randn((B, H, T, D), generator=g)).to(torch.bfloat16)
    ks = [(2.0 * torch.randn((B, H, tc, D), generator=g)).to(torch.bfloat16) for _ in range(2)]
    vs = [torch.randn((B, H, tc, D), generator=g).to(torch.bfloat16) for _ in range(2)]
    do = torch.randn((B, H, T, D), generator=g).to(torch.bfloat16)
    res = run_hip(q, ks, vs, do, 1.0)
    ref = _oracle_full(q, ks, vs, do, 1.0)
    _grad_check(res, ref)
