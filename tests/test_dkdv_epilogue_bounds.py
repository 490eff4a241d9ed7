"""CPU bounds check of the head-dim-128 dK/dV kernel's bf16 epilogue: the
address functions the kernel calls (harp_amd/csrc/dkdv_epilogue.h), compiled
for the host by tests/dkdv_epilogue_bounds.cpp and walked over every lane of
every block of a grid, with each LDS and global address checked against its
allocation.

Geometries: the one in which a withdrawn variant of this epilogue (fp32
outputs also staged, per-row element-store fallbacks) faulted the GPU --
B1 H2, chunks of 300 rows with 300 / 250 valid keys, dK / dV views at a +1
element offset with row stride H (D + 1) -- and the views the C ABI accepts
at head dim 128 (token-major, padded rows, BASELINE config 5's chunks)."""

import os
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "dkdv_epilogue_bounds.cpp")
D = 128
# dkdv_asm.hip: five 16 KiB query buffers, the 256-row padded V tile (272-byte
# rows) and four waves' statistics areas (5 x 512 bytes)
LDS_BYTES = 5 * 16384 + 256 * 272 + 4 * 5 * 512


@pytest.fixture(scope="module")
def walker():
    d = tempfile.mkdtemp(prefix="dkdv_epi_")
    exe = os.path.join(d, "walk")
    subprocess.run(["g++", "-O2", "-std=c++17", SRC, "-o", exe], check=True, capture_output=True)
    return exe


def walk(exe, B, H, rows, lens, offset, sb, sh, st, alloc):
    out = subprocess.run([exe, str(B), str(H), str(rows), str(LDS_BYTES), str(offset), str(sb), str(sh), str(st),
                          str(alloc)] + [str(x) for x in lens], check=True, capture_output=True, text=True).stdout
    return {k: int(v) for k, v in (t.split("=") for t in out.split())}


def _clean(r):
    for k in ("lds_oob", "stage_twice", "stage_missing", "read_twice", "read_unwritten", "global_oob",
              "global_twice", "global_missing"):
        assert r[k] == 0, (k, r)


def test_faulting_geometry_stays_in_bounds(walker):
    """The geometry of the withdrawn variant's fault: every address the
    shipped arithmetic forms is inside its allocation; the stores are not
    8-byte aligned (why the C ABI now refuses such views at head dim 128)."""
    B, H, rows = 1, 2, 300
    row = H * (D + 1)
    r = walk(walker, B, H, rows, [300, 250], 1, rows * row, D + 1, row, B * rows * row)
    _clean(r)
    # two chunks x H x 300 rows, each row stored by 32 lanes of 4 elements
    assert r["stores"] == 2 * B * H * rows * 32
    assert r["misaligned"] > 0


@pytest.mark.parametrize("pad", [0, 4])
def test_token_major_and_padded_rows(walker, pad):
    B, H, rows = 2, 3, 520
    row = H * (D + pad)
    r = walk(walker, B, H, rows, [1, 0, 257, 511], 0, rows * row, D + pad, row, B * rows * row)
    _clean(r)
    assert r["misaligned"] == 0


def test_config5_chunks(walker):
    B, H, rows = 1, 24, 4480
    r = walk(walker, B, H, rows, [4429] * 4, 0, rows * H * D, D, H * D, B * rows * H * D)
    _clean(r)
    assert r["misaligned"] == 0


def test_planted_stride_error_is_caught(walker):
    """A row stride one element short of the view's (rows overlap) and an
    allocation one row short must both show up."""
    B, H, rows = 1, 2, 300
    row = H * D
    r = walk(walker, B, H, rows, [300], 0, rows * row, D, row - 1, B * rows * row)
    assert r["global_twice"] > 0
    r = walk(walker, B, H, rows, [300], 0, rows * row, D, row, B * rows * row - row)
    assert r["global_oob"] > 0
