"""GPU parity of the head-dim-128 forward (fwd_asm.hip, the hand-scheduled
loop) on the paths its loop takes rarely: every exit point of the loop
unrolled over eight LDS block buffers, partial last blocks of a chunk (the
masked slot twins), chunks shorter than a block or empty (the cursor moving
through several chunks in one step), the lazy rescale after the first block
(row maxima that grow along the keys), and KV splits.  Bars as the other
parity tests: O and LSE <= 2e-2 relative Frobenius error against the fp64
oracle (oracle/ring_attn_oracle.py, ring_attn.cpp:2412-2575)."""

import math

import pytest
import torch

from oracle import ring_attn_oracle as orc
from tests.gpu_harness import run_hip
from tests.parity import TOL_LSE, TOL_O, rel_fro
from tests.test_gpu_parity import _check_all, _oracle_full

pytestmark = pytest.mark.gpu

D = 128


def _fwd_check(res, ref):
    for name, tol in (("o", TOL_O), ("lse", TOL_LSE)):
        err = rel_fro(res[name], ref[name])
        print(f"  {name}: rel {err:.2e}", flush=True)
        assert err <= tol, (name, err)


@pytest.mark.parametrize("nb", list(range(1, 10)))
@pytest.mark.parametrize("ragged", [False, True])
def test_every_loop_exit(nb, ragged):
    """One chunk of nb 32-key blocks (the last one partial when ragged): the
    loop leaves from slot (nb - 1) % 8."""
    n_keys = 32 * nb - (5 if ragged else 0)
    print(f"[exit nb={nb} keys={n_keys}]", flush=True)
    q, ks, vs, do = orc.make_inputs(1, 2, 70, D, 1, seed=100 + nb, chunk_len=n_keys)
    scale = 1.0 / math.sqrt(D)
    res = run_hip(q, ks, vs, do, scale, backward=False)
    ref = _oracle_full(q, ks, vs, do, scale)
    _fwd_check(res, ref)


def test_tiny_and_empty_chunks_every_rank():
    """Chunks of 1, 0, 33, 0, 64 and 95 valid keys (chunk length 96): the copy
    cursor crosses chunks inside one slot, skips empty ones, and most chunks
    end in a partial block."""
    lens = [1, 0, 33, 0, 64, 95]
    for rank in range(len(lens)):
        print(f"[tiny chunks rank {rank}]", flush=True)
        q, ks, vs, do = orc.make_inputs(2, 3, 300, D, len(lens), seed=40 + rank, chunk_len=96)
        scale = 1.0 / math.sqrt(D)
        res = run_hip(q, ks, vs, do, scale, ring_rank=rank, kv_lens=lens, via="abi" if rank % 2 else "ops")
        ref = _oracle_full(q, ks, vs, do, scale, rank=rank, lens=lens)
        _check_all(res, ref)


def test_rescale_as_the_maximum_grows():
    """Scores that rise along the keys by more than the 2^8 lazy-rescale
    threshold, block after block and chunk after chunk: O and l are rescaled
    many times after the first block."""
    g = torch.Generator().manual_seed(7)
    B, H, T, N, tc = 1, 2, 130, 4, 200
    u = torch.randn((1, H, 1, D), generator=g)
    u = u / u.norm(dim=-1, keepdim=True)
    q = (6.0 * u + 0.3 * torch.randn((B, H, T, D), generator=g)).to(torch.bfloat16)
    ks, vs = [], []
    for c in range(N):
        ramp = torch.linspace(0.0, 1.0, tc).view(1, 1, tc, 1)
        # scores (q . k x scale) rise by about 8 per chunk, 11.5 in log2
        # units: over the ring the row maximum passes the threshold 4-5 times
        k = (8.0 * (c + ramp)) * u * math.sqrt(D) / 6.0 + 0.3 * torch.randn((B, H, tc, D), generator=g)
        ks.append(k.to(torch.bfloat16))
        vs.append(torch.randn((B, H, tc, D), generator=g).to(torch.bfloat16))
    do = torch.randn((B, H, T, D), generator=g).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    ref = _oracle_full(q, ks, vs, do, scale)
    res = run_hip(q, ks, vs, do, scale, backward=False)
    _fwd_check(res, ref)


def test_kv_split_small_grid():
    """One 256-query block per head and eight chunks: the host splits the
    ring over several launches' worth of blocks (grid dimension y), each
    split runs its own ring steps and the partials are merged."""
    q, ks, vs, do = orc.make_inputs(1, 1, 256, D, 8, seed=77, chunk_len=160)
    lens = [160, 131, 160, 7, 160, 160, 96, 160]
    scale = 1.0 / math.sqrt(D)
    res = run_hip(q, ks, vs, do, scale, ring_rank=3, kv_lens=lens)
    ref = _oracle_full(q, ks, vs, do, scale, rank=3, lens=lens)
    _check_all(res, ref)
