"""CPU bounds check of the output epilogues of the compiled kernels (head
dims other than 128: fwd_kernel writes O, dq_kernel dQ, dkdv_kernel dK and
dV): the address functions the kernels call (harp_amd/csrc/cq_epilogue.h),
compiled for the host by tests/cq_epilogue_bounds.cpp and walked over every
lane of every block, with each LDS and global address checked against its
allocation.

Geometries: BASELINE configs 2 (D = 64, KV-split partials) and 3 (D = 72
padded to 96), ragged T and chunk lengths, fp32 and bf16 outputs, and bf16
views at a +1 element offset with odd row strides (the element-by-element
store path the kernels take for views that are not 8-byte aligned)."""

import os
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "cq_epilogue_bounds.cpp")
# ra_kernels.hip: fwd_kernel / dq_kernel stage waves 0-3 in the K tiles and
# 4-7 in the V tiles (each 2 buffers x 2 sub-tiles x 64 x 128 bf16);
# dkdv_kernel in the Q / dO buffers (2 x 2 x 64 x 128 bf16) and the V tiles
# (4 x 64 rows of DP + 8 bf16)
QKV_TILES = 2 * 2 * 64 * 128 * 2


def v_tiles(dp):
    return 4 * 64 * (dp + 8) * 2  # at DP 80 (the 16-wide tail) the V tile is PadTile<80>


@pytest.fixture(scope="module")
def walker():
    d = tempfile.mkdtemp(prefix="cq_epi_")
    exe = os.path.join(d, "walk")
    subprocess.run(["g++", "-O2", "-std=c++17", SRC, "-o", exe], check=True, capture_output=True)
    return exe


def walk(exe, kind, DP, D, B, H, rows, n_split, eb, wide, halves, offset, sb, sh, st, split, alloc, chunks=()):
    args = [kind, DP, D, B, H, rows, n_split, eb, int(wide), halves[0], halves[1], offset, sb, sh, st, split, alloc]
    out = subprocess.run([exe] + [str(x) for x in args] + [str(c) for c in chunks], check=True, capture_output=True,
                         text=True).stdout
    return {k: int(v) for k, v in (t.split("=") for t in out.split())}


def _clean(r):
    for k in ("lds_oob", "stage_pad", "stage_twice", "stage_missing", "read_twice", "read_unwritten", "read_missing",
              "global_oob", "global_twice", "global_missing"):
        assert r[k] == 0, (k, r)


Q_HALVES = (QKV_TILES, QKV_TILES)


@pytest.mark.parametrize("DP,D,B,H,T,n_split", [
    (64, 64, 1, 16, 2048, 2),   # config 2: the forward's and dQ's fp32 split partials
    (80, 72, 2, 16, 4096, 1),   # config 3: the 16-wide d tail
    (80, 80, 1, 3, 77, 3),
    (96, 96, 1, 3, 77, 3),
    (32, 24, 2, 2, 300, 1),
])
def test_q_fp32_head_major_and_splits(walker, DP, D, B, H, T, n_split):
    per = B * H * T * D
    r = walk(walker, "q", DP, D, B, H, T, n_split, 4, True, Q_HALVES, 0, H * T * D, T * D, D, per, n_split * per)
    _clean(r)
    assert r["stores"] == n_split * B * H * T * D // 4


@pytest.mark.parametrize("eb", [4, 2])
def test_q_token_major_config3(walker, eb):
    """dQ (bf16 and fp32) of config 3 in the operators' token-major
    layout, 16-wide d tail: 8-byte aligned 4-element stores."""
    B, H, T, D = 2, 16, 4096, 72
    r = walk(walker, "q", 80, D, B, H, T, 1, eb, True, Q_HALVES, 0, T * H * D, D, H * D, 0, B * T * H * D)
    _clean(r)
    assert r["misaligned"] == 0


def test_q_unaligned_bf16_view_takes_the_element_path(walker):
    B, H, T, D = 1, 3, 100, 64
    row = H * (D + 1)
    r = walk(walker, "q", 64, D, B, H, T, 1, 2, True, Q_HALVES, 1, T * row, D + 1, row, 0, B * T * row + 1)
    assert r["misaligned"] > 0  # why the kernel does not take the 4-element path here
    r = walk(walker, "q", 64, D, B, H, T, 1, 2, False, Q_HALVES, 1, T * row, D + 1, row, 0, B * T * row + 1)
    _clean(r)
    assert r["stores"] == B * H * T * D


@pytest.mark.parametrize("DP,D,B,H,chunks", [
    (64, 64, 1, 16, [2048] * 4),        # config 2
    (80, 72, 2, 16, [4096, 4096]),      # config 3 (two of its eight chunks): the 16-wide d tail
    (80, 80, 1, 2, [300, 97, 1, 256]),  # ragged chunk lengths
    (96, 88, 1, 2, [300, 97, 1, 256]),
    (32, 32, 2, 3, [520]),
])
@pytest.mark.parametrize("eb", [2, 4])
def test_k_token_major(walker, DP, D, B, H, chunks, eb):
    rows = max(chunks)
    r = walk(walker, "k", DP, D, B, H, rows, 1, eb, True, (QKV_TILES, v_tiles(DP)), 0, rows * H * D, D, H * D, 0,
             B * rows * H * D, chunks)
    _clean(r)
    assert r["misaligned"] == 0
    assert r["stores"] == sum(B * H * c * D // 4 for c in chunks)


def test_k_unaligned_bf16_views_take_the_element_path(walker):
    """dK / dV at a +1 element offset with row stride H (D + 1), as the GPU
    test of unaligned views at head dim 64 passes them."""
    B, H, D, rows = 1, 2, 64, 300
    row = H * (D + 1)
    halves = (QKV_TILES, v_tiles(64))
    r = walk(walker, "k", 64, D, B, H, rows, 1, 2, False, halves, 1, rows * row, D + 1, row, 0, B * rows * row + 1,
             [300, 250])
    _clean(r)
    assert r["stores"] == B * H * (300 + 250) * D


def test_planted_errors_are_caught(walker):
    """A V-tile array one staging row short, a row stride one element short
    (rows overlap) and an allocation one row short must each show up."""
    B, H, D, rows = 1, 2, 64, 256
    row = H * D
    args = dict(DP=64, D=D, B=B, H=H, rows=rows, n_split=1, eb=2, wide=True, offset=0, sb=rows * row, sh=D,
                split=0, chunks=[rows])
    good = (QKV_TILES, v_tiles(64))
    assert walk(walker, "k", halves=(good[0], good[1] - 4 * 72), st=row, alloc=B * rows * row, **args)["lds_oob"] > 0
    assert walk(walker, "k", halves=good, st=row - 1, alloc=B * rows * row, **args)["global_twice"] > 0
    assert walk(walker, "k", halves=good, st=row, alloc=B * rows * row - row, **args)["global_oob"] > 0
