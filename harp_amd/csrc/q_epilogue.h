// Address arithmetic of the epilogue shared by the head-dim-128
// Q-stationary kernels (fwd_asm.hip: O; dq_asm.hip: dQ), as host-and-device
// functions: the kernels compute every staging, read-back and output address
// through them, and the host bounds check (tests/q_epilogue_bounds.cpp)
// compiles the same functions and walks every lane of every block.
//
// A wave ends its loop with the 128 x 64 fp32 transpose of its rows' output
// in AGPRs: lane l holds query row 32 qg + l % 32 and, in accumulator
// register r of d block db, element d = 32 db + c_row(r, l / 32).  Registers
// r = 4 i .. 4 i + 3 are four consecutive elements, so each lane stages them
// with one 16-byte LDS write into its query's staging row; every row is then
// read back by 32 lanes, 16 bytes each, and stored as one contiguous row.
#pragma once

#include <stdint.h>

#include "acc_layout.h"

namespace harp_ra {
namespace q_epi {

constexpr int kWaves = 4;
constexpr int kRowsPerWave = 64;
constexpr int kStageRow = 132;  // floats per staging row (128 + 4: the 16 rows of a write phase hit distinct banks)
constexpr int kStageBytes = kWaves * kRowsPerWave * kStageRow * 4;

// First float of wave w's 64-row staging area.
HARP_HD int stage_base(int wave) { return wave * kRowsPerWave * kStageRow; }

// Float index, within the wave's staging area, of the first of the four
// consecutive elements that lane `lane` stages for query group qg, d block
// db and register quad i (registers 4 i .. 4 i + 3).
HARP_HD int stage_write(int qg, int db, int i, int lane) {
  return (qg * 32 + (lane & 31)) * kStageRow + db * 32 + c_row(4 * i, lane >> 5);
}

// Read-back: iteration it (0..31) of lane `lane` reads four consecutive
// floats of staging row 2 it + lane / 32, starting at d = 4 (lane % 32).
HARP_HD int stage_read(int it, int lane) { return (it * 2 + (lane >> 5)) * kStageRow + (lane & 31) * 4; }

// Query row (0 .. T-1 when in range) that read-back iteration `it` stores.
HARP_HD int out_query(int qtile0, int wave, int it, int lane) {
  return qtile0 + wave * kRowsPerWave + it * 2 + (lane >> 5);
}

// Element offset, from the output's base pointer, of the first of the four
// elements (d = 4 (lane % 32) .. + 3) that the lane stores for query row qi,
// with `bh_base` = b * stride_b + h * stride_h (+ the split's offset).
HARP_HD int64_t out_elem(int64_t bh_base, int qi, int64_t stride_t, int lane) {
  return bh_base + (int64_t)qi * stride_t + (lane & 31) * 4;
}

}  // namespace q_epi
}  // namespace harp_ra
