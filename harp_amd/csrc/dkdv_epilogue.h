// Address arithmetic of the head-dim-128 dK/dV kernel's epilogue
// (dkdv_asm.hip), as host-and-device functions: the kernel computes every
// staging, read-back and output address through them, and the host bounds
// check (tests/dkdv_epilogue_bounds.cpp) compiles the same functions and
// walks every lane of every block over a geometry.
#pragma once

#include <stdint.h>

#include "acc_layout.h"

namespace harp_ra {
namespace dkdv_epi {

constexpr int kWaves = 4;
constexpr int kKeysPerWave = 64;
constexpr int kStageRow = 136;  // floats per staging row (128 + 8: rows 4 apart fall 32 banks apart)

// First float of wave w's 64-row staging area.
HARP_HD int stage_base(int wave) { return wave * kKeysPerWave * kStageRow; }

// Float index, within the wave's staging area, that lane `lane` writes for
// accumulator register r of key group kg (32 keys) and 32-wide d block db.
HARP_HD int stage_write(int kg, int db, int r, int lane) {
  return (kg * 32 + c_row(r, lane >> 5)) * kStageRow + db * 32 + (lane & 31);
}

// Read-back: iteration it (0..31) of lane `lane` reads four consecutive
// floats of staging row it * 2 + lane / 32, starting at d = 4 (lane % 32).
HARP_HD int stage_read(int it, int lane) { return (it * 2 + (lane >> 5)) * kStageRow + (lane & 31) * 4; }

// Key row within the chunk that read-back iteration `it` of the lane stores.
HARP_HD int out_row(int kblk0, int wave, int it, int lane) {
  return kblk0 + wave * kKeysPerWave + it * 2 + (lane >> 5);
}

// Element offset, from the chunk's base pointer, of the first of the four
// outputs (d = 4 (lane % 32) .. + 3) that the lane stores for key row kk of
// (b, h) with element offset `bh_base` = b * stride_b + h * stride_h.
HARP_HD int64_t out_elem(int64_t bh_base, int kk, int64_t stride_t, int lane) {
  return bh_base + (int64_t)kk * stride_t + (lane & 31) * 4;
}

}  // namespace dkdv_epi
}  // namespace harp_ra
