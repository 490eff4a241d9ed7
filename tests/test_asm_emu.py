"""CPU check of the generated hand-scheduled loops through the
instruction-level model in tests/asm_emu.py, against fp64
(ring_attn.cpp:2412-2575 forward, :2577-2829 backward):
  dK/dV (dkdv_asm_gen.py): one 256-key block, query block counts that leave
    the loop from each of its five slots and over two trips around the LDS
    buffers, a ragged last query block, pad keys;
  dQ and forward (dq_asm_gen.py, fwd_asm_gen.py): every loop exit with and
    without a partial last block, the copy cursor through tiny and empty
    chunks in ring order, the forward's lazy rescale;
and planted mistakes (a layout swap, a dropped cursor advance, a rescale
that does not compute the flagged block again) shown to fail."""

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


@pytest.mark.parametrize("T", [32, 64, 96, 128, 160, 330])  # leaves from every slot (nb - 1) % 5
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


# ---- dQ and forward loops ---------------------------------------------------

def _qkv(T, lens, rows, seed, ramp=0.0):
    rng = np.random.default_rng(seed)
    bf = lambda *sh: emu.f2bf(rng.standard_normal(sh).astype(np.float32))
    q, do = bf(T, 128), bf(T, 128)
    ks, vs = [], []
    for c in range(len(lens)):
        k = rng.standard_normal((rows, 128)).astype(np.float32)
        if ramp:  # scores that rise along the keys (the forward's lazy rescale)
            u = emu.bf2f(q[0].astype(np.uint32)).astype(np.float32)
            k += np.outer(ramp * (c + np.linspace(0, 1, rows)), u / np.linalg.norm(u) ** 2 * np.sqrt(128))
        ks.append(emu.f2bf(k))
        vs.append(bf(rows, 128))
    return q, do, ks, vs


def _dq_ref(q, do, ks, vs, lens, scale):
    O, lse, m, P, K, V = emu.attention_reference(q, ks, vs, lens, scale)
    dO = emu.bf2f(do.astype(np.uint32)).astype(np.float64)
    D = (dO * O).sum(1)
    dq = (P * (dO @ V.T - D[:, None])) @ K * scale
    return dq, lse, D


def _rel(a, b):
    return np.linalg.norm(a - b) / np.linalg.norm(b)


@pytest.mark.parametrize("nb", list(range(1, 10)))
@pytest.mark.parametrize("ragged", [False, True])
def test_dq_and_fwd_every_loop_exit(nb, ragged):
    """One chunk of nb 32-key blocks: both loops leave from slot (nb - 1) % 8;
    70 queries leave most of the block's 256 rows past T."""
    n = 32 * nb - (5 if ragged else 0)
    q, do, ks, vs = _qkv(70, [n], n, seed=nb)
    scale = 1 / np.sqrt(128)
    dqr, lse, D = _dq_ref(q, do, ks, vs, [n], scale)
    dq = emu.run_dq_block(q, do, ks, vs, [n], [0], (-lse / scale).astype(np.float32), (-D).astype(np.float32),
                          scale)
    assert _rel(dq, dqr) < 1e-2
    O, lse_r, m_r, *_ = emu.attention_reference(q, ks, vs, [n], scale)
    Of, mf, lf = emu.run_fwd_block(q, ks, vs, [n], [0], scale)
    assert _rel(Of, O) < 1e-2
    assert np.abs(mf + np.log(lf) - lse_r).max() < 1e-4
    # m is the exps' reference point: at most 8 log2 units below the row max
    assert (mf <= m_r + 1e-4).all() and (mf >= m_r - 8 * np.log(2.0) - 1e-4).all()


@pytest.mark.parametrize("rank", [0, 2, 4])
def test_cursor_through_tiny_and_empty_chunks(rank):
    """Chunks of 33, 0, 96, 1 and 64 keys (96 rows each) in ring order from
    `rank`: the copy cursor crosses chunks inside a slot and skips empty ones."""
    lens = [33, 0, 96, 1, 64]
    order = [(s + rank) % len(lens) for s in range(len(lens))]
    q, do, ks, vs = _qkv(70, lens, 96, seed=10 + rank)
    scale = 1 / np.sqrt(128)
    dqr, lse, D = _dq_ref(q, do, ks, vs, lens, scale)
    dq = emu.run_dq_block(q, do, ks, vs, lens, order, (-lse / scale).astype(np.float32), (-D).astype(np.float32),
                          scale)
    assert _rel(dq, dqr) < 1e-2
    O, lse_r, m_r, *_ = emu.attention_reference(q, ks, vs, lens, scale)
    Of, mf, lf = emu.run_fwd_block(q, ks, vs, lens, order, scale)
    assert _rel(Of, O) < 1e-2
    assert np.abs(mf + np.log(lf) - lse_r).max() < 1e-4


def test_fwd_rescale_as_the_maximum_grows():
    """Scores rising by more than the 2^8 lazy-rescale threshold chunk after
    chunk: the out-of-line rescale runs several times."""
    lens = [96, 96, 96, 96]
    q, do, ks, vs = _qkv(40, lens, 96, seed=3, ramp=12.0)
    scale = 1 / np.sqrt(128)
    O, lse_r, m_r, *_ = emu.attention_reference(q, ks, vs, lens, scale)
    Of, mf, lf = emu.run_fwd_block(q, ks, vs, lens, [0, 1, 2, 3], scale)
    assert emu.LAST_COUNTS.get("v_accvgpr_read_b32", 0) > 0  # the rescale of O ran
    assert _rel(Of, O) < 1e-2
    assert np.abs(mf + np.log(lf) - lse_r).max() < 1e-4


def test_planted_cursor_error_is_caught():
    """Dropping the cursor's row advance from one slot's copy code (every
    later block re-read at the same rows) must fail the dQ comparison."""
    lens = [200]
    q, do, ks, vs = _qkv(40, lens, 200, seed=7)
    scale = 1 / np.sqrt(128)
    dqr, lse, D = _dq_ref(q, do, ks, vs, lens, scale)
    lines = emu.GQ.build()
    k = next(i for i, ln in enumerate(lines) if ln.startswith("s_add_u32 s72, s72, %[blkb]"))
    bad = lines[:k] + lines[k + 2:]  # the K row pointer's add and add-with-carry
    dq = emu.run_dq_block(q, do, ks, vs, lens, [0], (-lse / scale).astype(np.float32), (-D).astype(np.float32),
                          scale, lines=bad)
    assert _rel(dq, dqr) > 0.05


@pytest.mark.filterwarnings("ignore:invalid value encountered in matmul")  # the stale inf P
def test_planted_missing_recompute_in_the_rescale_is_caught():
    """The forward's rescale must compute the flagged block's P again against
    the new reference point (the first block's exps overflow against the
    starting -FLT_MAX): dropping the packs of that recompute must fail."""
    lens = [96, 96]
    q, do, ks, vs = _qkv(40, lens, 96, seed=4)
    scale = 1 / np.sqrt(128)
    O, lse_r, m_r, *_ = emu.attention_reference(q, ks, vs, lens, scale)
    lines = emu.GF.build()
    bad, in_resc = [], False
    for ln in lines:
        if ln.startswith(".Lfa_rescale"):
            in_resc = True
        elif ln.startswith("s_mov_b64 s[64:65], 0"):
            in_resc = False
        if in_resc and ln.startswith("v_cvt_pk_bf16_f32"):
            continue
        bad.append(ln)
    assert len(bad) < len(lines)
    Of, mf, lf = emu.run_fwd_block(q, ks, vs, lens, [0, 1], scale, lines=bad)
    err = _rel(Of, O)
    assert not np.isfinite(err) or err > 0.05
