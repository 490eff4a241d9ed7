// Address arithmetic of the output epilogues of the compiled kernels
// (ra_kernels.hip: fwd_kernel, dq_kernel, dkdv_kernel; head dims other than
// 128), as host-and-device functions: the kernels compute every staging,
// read-back and output address through them, and the host bounds check
// (tests/cq_epilogue_bounds.cpp) compiles the same functions and walks every
// lane of every block.
//
// A block is 8 waves of 32 rows (queries in fwd / dQ, keys in dK / dV).  Its
// outputs are staged through LDS after the loop: waves 0-3 in one of the
// kernel's LDS arrays, waves 4-7 in another (half(wave)), each wave in 32
// rows of kSR floats.  Every row is then read back 16 bytes per lane, lanes
// covering consecutive 4-element chunks of consecutive rows, and stored as
// contiguous pieces of the output row instead of one element per lane and
// instruction.  DP = 32 * (d blocks), or 32 n + 16 with a 16-wide last
// block, is the padded head dim, D <= DP the real one (a multiple of 8, so a
// 4-element chunk is all in or all out).
#pragma once

#include <stdint.h>

#include "acc_layout.h"

namespace harp_ra {
namespace cq_epi {

constexpr int kWaves = 8;
constexpr int kRows = 32;  // rows per wave

// Which of the two staging arrays a wave uses, and its first float there.
HARP_HD int half(int wave) { return wave >> 2; }

template <int DP, int SR>
struct Rows {
  static constexpr int kSR = SR;                       // floats per staging row
  static constexpr int kChunks = DP / 4;               // 16-byte chunks per row
  static constexpr int kIters = kRows * kChunks / 64;  // read-back iterations per lane
  static constexpr int kHalfBytes = 4 * kRows * kSR * 4;  // four waves' staging
  static_assert(DP % 16 == 0 && (kRows * kChunks) % 64 == 0, "whole read-back iterations");
  HARP_HD static int stage_base(int wave) { return (wave & 3) * kRows * kSR; }
  // read-back iteration it of lane `lane`: row and chunk within the wave's rows
  HARP_HD static int read_row(int it, int lane) { return (it * 64 + lane) / kChunks; }
  HARP_HD static int read_chunk(int it, int lane) { return (it * 64 + lane) % kChunks; }
  HARP_HD static int stage_read(int it, int lane) { return read_row(it, lane) * kSR + 4 * read_chunk(it, lane); }
  // element-by-element read-back (bf16 views that are not 8-byte aligned):
  // iteration it (0 .. DP/2 - 1) of lane `lane` reads one float
  static constexpr int kElemIters = kRows * DP / 64;
  HARP_HD static int elem_row(int it, int lane) { return (it * 64 + lane) / DP; }
  HARP_HD static int elem_col(int it, int lane) { return (it * 64 + lane) % DP; }
  HARP_HD static int stage_elem(int it, int lane) { return elem_row(it, lane) * kSR + elem_col(it, lane); }
};

// fwd / dQ: the accumulator holds the transpose (lane = query, register r of d
// block db = element 32 db + c_row(r, lane / 32)); registers 4 i .. 4 i + 3
// are four consecutive elements, staged by one 16-byte write.  Rows DP + 4
// floats apart: the 16 rows of a write phase start on distinct banks.
template <int DP>
struct QRows : Rows<DP, DP + 4> {
  HARP_HD static int stage_write(int db, int i, int lane) {
    return (lane & 31) * (DP + 4) + db * 32 + c_row(4 * i, lane >> 5);
  }
  // a 16-wide last d block (DP = 32 n + 16), 16 x 16 accumulator layout:
  // the four registers of lane `lane` in tile u are query row 16 u + lane %
  // 16, elements DP - 16 + 4 (lane / 16) .. + 3, staged by one 16-byte write
  HARP_HD static int stage_write_tail(int u, int lane) {
    return (16 * u + (lane & 15)) * (DP + 4) + DP - 16 + 4 * (lane >> 4);
  }
};

// dK / dV: lane = d column 32 db + lane % 32, register r = key row
// c_row(r, lane / 32); staged one float per lane and register.  Rows DP + 8
// floats apart: rows 4 apart (the two lane halves of one write) fall 32 banks
// apart.
template <int DP>
struct KRows : Rows<DP, DP + 8> {
  HARP_HD static int stage_write(int db, int r, int lane) {
    return c_row(r, lane >> 5) * (DP + 8) + db * 32 + (lane & 31);
  }
  // a 16-wide last d block (DP = 32 n + 16), 16 x 16 accumulator layout:
  // register i of lane `lane` in tile t is key row 16 t + 4 (lane / 16) + i,
  // column DP - 16 + lane % 16
  HARP_HD static int stage_write_tail(int t, int i, int lane) {
    return (16 * t + 4 * (lane >> 4) + i) * (DP + 8) + DP - 16 + (lane & 15);
  }
};

}  // namespace cq_epi
}  // namespace harp_ra
