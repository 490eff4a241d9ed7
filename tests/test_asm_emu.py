"""CPU check of the generated dK/dV loop (dkdv_asm_gen.py) through the
instruction-level model in tests/asm_emu.py: one 256-key block, every query
block count up to two trips around the five LDS buffers, a ragged last query
block, pad keys, and a block past the valid keys.  dK, dV against fp64
(ring_attn.cpp:2577-2829 for one chunk); pad keys must come out 0."""

import numpy as np
import pytest

from tests import asm_emu as emu


def _case(T, len_valid, seed):
    rng = np.random.default_rng(seed)
    L = 256
    scale = 1 / np.sqrt(128)
    q = emu.f2bf(rng.standard_normal((T, 128)).astype(np.float32))
    k = emu.f2bf(rng.standard_normal((L, 128)).astype(np.float32))
    v = emu.f2bf(rng.standard_normal((L, 128)).astype(np.float32))
    do = emu.f2bf(rng.standard_normal((T, 128)).astype(np.float32))
    dkr, dvr, lse, dl = emu.reference(q, k, v, do, scale, len_valid)
    dk, dv, _ = emu.run_block(q, k, v, do, (-lse / scale).astype(np.float32), (-dl).astype(np.float32), scale,
                              len_valid)
    return dk, dv, dkr, dvr


@pytest.mark.parametrize("T", [32, 96, 160, 330])
def test_loop_matches_fp64(T):
    dk, dv, dkr, dvr = _case(T, 256, seed=T)
    for name, a, b in (("dk", dk, dkr), ("dv", dv, dvr)):
        err = np.linalg.norm(a - b) / np.linalg.norm(b)
        assert err < 1e-2, (name, err)


def test_pad_keys_zero():
    """200 valid keys: keys 200-255 are pads and must be written as 0."""
    dk, dv, dkr, dvr = _case(64, 200, seed=3)
    assert not dk[200:].any() and not dv[200:].any()
    for a, b in ((dk[:200], dkr), (dv[:200], dvr)):
        assert np.linalg.norm(a - b) / np.linalg.norm(b) < 1e-2


def test_planted_layout_error_is_caught():
    """The model is sensitive to the generator's layout: swapping the two
    key groups' K operands in the set-up must fail the comparison."""
    rng = np.random.default_rng(9)
    T, L = 32, 256
    scale = 1 / np.sqrt(128)
    q = emu.f2bf(rng.standard_normal((T, 128)).astype(np.float32))
    k = emu.f2bf(rng.standard_normal((L, 128)).astype(np.float32))
    v = emu.f2bf(rng.standard_normal((L, 128)).astype(np.float32))
    do = emu.f2bf(rng.standard_normal((T, 128)).astype(np.float32))
    dkr, dvr, lse, dl = emu.reference(q, k, v, do, scale, L)
    k_bad = k.copy()
    k_bad[0:32], k_bad[32:64] = k[32:64].copy(), k[0:32].copy()  # wave 0's key groups swapped in K only
    dk, dv, _ = emu.run_block(q, k_bad, v, do, (-lse / scale).astype(np.float32), (-dl).astype(np.float32), scale, L)
    assert np.linalg.norm(dv - dvr) / np.linalg.norm(dvr) > 0.1
