"""CPU bounds check of the epilogue of the head-dim-128 Q-stationary kernels
(fwd_asm.hip writes O, dq_asm.hip writes dQ): the address functions the
kernels call (harp_amd/csrc/q_epilogue.h), compiled for the host by
tests/q_epilogue_bounds.cpp and walked over every lane of every block of a
grid, with each LDS and global address checked against its allocation.

Geometries: BASELINE config 5's ragged T (token-major and head-major
outputs), the KV-split partial buffers at HARP's own T = 256 / H = 30, tiny
and ragged T, and a bf16 dQ view at a +1 element offset with padded rows
(refused by the C ABI: its stores would not be 8-byte aligned)."""

import os
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "q_epilogue_bounds.cpp")
D = 128
# fwd_asm.hip / dq_asm.hip: max(the loop's 2 x 64 KiB block buffers, the
# staging rows: 4 waves x 64 rows x 132 floats)
LDS_BYTES = max(2 * 65536, 4 * 64 * 132 * 4)


@pytest.fixture(scope="module")
def walker():
    d = tempfile.mkdtemp(prefix="q_epi_")
    exe = os.path.join(d, "walk")
    subprocess.run(["g++", "-O2", "-std=c++17", SRC, "-o", exe], check=True, capture_output=True)
    return exe


def walk(exe, B, H, T, n_split, eb, offset, sb, sh, st, split, alloc, lds=LDS_BYTES):
    out = subprocess.run([exe] + [str(x) for x in (B, H, T, n_split, eb, lds, offset, sb, sh, st, split, alloc)],
                         check=True, capture_output=True, text=True).stdout
    return {k: int(v) for k, v in (t.split("=") for t in out.split())}


def _clean(r):
    for k in ("lds_oob", "stage_twice", "stage_missing", "read_twice", "read_unwritten", "global_oob",
              "global_twice", "global_missing"):
        assert r[k] == 0, (k, r)


@pytest.mark.parametrize("layout", ["token_major", "head_major"])
def test_config5_rows(walker, layout):
    B, H, T = 1, 24, 4429
    sb = T * H * D
    sh, st = (D, H * D) if layout == "token_major" else (T * D, D)
    r = walk(walker, B, H, T, 1, 4, 0, sb, sh, st, 0, B * sb)
    _clean(r)
    assert r["stores"] == B * H * T * 32  # every row by 32 lanes of four elements
    assert r["misaligned"] == 0


def test_split_partials_at_harp_shape(walker):
    """The fp32 [n][B, H, T, D] partials of an eight-way KV split."""
    B, H, T, n = 1, 30, 256, 8
    per = B * H * T * D
    r = walk(walker, B, H, T, n, 4, 0, H * T * D, T * D, D, per, n * per)
    _clean(r)
    assert r["stores"] == n * B * H * T * 32


@pytest.mark.parametrize("T", [1, 65, 255, 257, 700])
def test_ragged_t(walker, T):
    B, H = 2, 3
    r = walk(walker, B, H, T, 1, 4, 0, H * T * D, T * D, D, 0, B * H * T * D)
    _clean(r)


def test_unaligned_bf16_view(walker):
    """bf16 dQ at a +1 element offset with row stride H (D + 1): in bounds,
    but the stores are not 8-byte aligned, which is why the C ABI refuses
    such bf16 dQ views at head dim 128."""
    B, H, T = 1, 2, 100
    row = H * (D + 1)
    r = walk(walker, B, H, T, 1, 2, 1, T * row, D + 1, row, 0, B * T * row + 1)
    _clean(r)
    assert r["misaligned"] > 0


def test_planted_errors_are_caught(walker):
    """A row stride one element short (rows overlap), an allocation one row
    short and an LDS allocation one 16-byte write short of the last staged
    element (the last row's 4-float pad is never touched) must each show up."""
    B, H, T = 1, 2, 300
    row = H * D
    assert walk(walker, B, H, T, 1, 4, 0, T * row, D, row - 1, 0, B * T * row)["global_twice"] > 0
    assert walk(walker, B, H, T, 1, 4, 0, T * row, D, row, 0, B * T * row - row)["global_oob"] > 0
    assert walk(walker, B, H, T, 1, 4, 0, T * row, D, row, 0, B * T * row, lds=4 * 64 * 132 * 4 - 32)["lds_oob"] > 0
