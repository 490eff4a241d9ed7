// Host walk of the head-dim-128 dK/dV kernel's bf16 epilogue addresses
// (dkdv_asm.hip), compiled from the same functions the kernel calls
// (harp_amd/csrc/dkdv_epilogue.h).  Test infrastructure: run by
// tests/test_dkdv_epilogue_bounds.py with g++.
//
// For every block of the grid (key tile, head, batch), every wave and lane,
// it checks:
//   * every staging write and read-back address lies inside the kernel's LDS
//     allocation, each wave's 64 x 128 staging tile is written exactly once
//     and read back exactly once;
//   * every global store (four bf16 outputs) lies inside the caller's
//     allocation for the dK / dV chunk, no output element is written twice
//     over the grid, and every element of rows < chunk rows, d < 128 is
//     written (pad keys as zero by the kernel);
// and counts the stores whose address is not 8-byte aligned (the wide store
// needs it; the C ABI refuses such views at head dim 128).
//
// usage: dkdv_epilogue_bounds B H chunk_rows lds_bytes view_offset
//        stride_b stride_h stride_t alloc_elems len0 [len1 ...]
// (element units of bf16; the view's base is the allocation + view_offset)
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../harp_amd/csrc/dkdv_epilogue.h"

using namespace harp_ra;

int main(int argc, char** argv) {
  if (argc < 11) {
    std::fprintf(stderr, "usage: %s B H chunk_rows lds_bytes offset sb sh st alloc len0 [len1 ...]\n", argv[0]);
    return 2;
  }
  const int B = std::atoi(argv[1]), H = std::atoi(argv[2]), rows = std::atoi(argv[3]);
  const long long lds_bytes = std::atoll(argv[4]), off = std::atoll(argv[5]);
  const long long sb = std::atoll(argv[6]), sh = std::atoll(argv[7]), st = std::atoll(argv[8]);
  const long long alloc = std::atoll(argv[9]);
  std::vector<int> lens;
  for (int i = 10; i < argc; ++i) lens.push_back(std::atoi(argv[i]));
  const int n = (int)lens.size();
  const int block_keys = dkdv_epi::kWaves * dkdv_epi::kKeysPerWave;
  const int tiles_per_chunk = (rows + block_keys - 1) / block_keys;

  long long lds_oob = 0, stage_twice = 0, stage_missing = 0, read_twice = 0, read_unwritten = 0;
  long long global_oob = 0, global_twice = 0, global_missing = 0, misaligned = 0, stores = 0;
  for (int c = 0; c < n; ++c) {
    std::vector<unsigned char> hit((size_t)alloc, 0);
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h)
        for (int t = 0; t < tiles_per_chunk; ++t) {
          const int kblk0 = t * block_keys;
          const long long base = (long long)b * sb + (long long)h * sh;
          for (int wave = 0; wave < dkdv_epi::kWaves; ++wave) {
            // staging: the wave's 64 rows x 128 floats, written then read back
            std::vector<int> wr(dkdv_epi::kKeysPerWave * dkdv_epi::kStageRow, 0), rd(wr.size(), 0);
            for (int lane = 0; lane < 64; ++lane)
              for (int kg = 0; kg < 2; ++kg)
                for (int db = 0; db < 4; ++db)
                  for (int r = 0; r < 16; ++r) {
                    const int i = dkdv_epi::stage_write(kg, db, r, lane);
                    const long long a = 4LL * (dkdv_epi::stage_base(wave) + i);
                    if (i < 0 || a < 0 || a + 4 > lds_bytes || i >= (int)wr.size()) {
                      ++lds_oob;
                      continue;
                    }
                    ++wr[i];
                  }
            for (int lane = 0; lane < 64; ++lane)
              for (int it = 0; it < dkdv_epi::kKeysPerWave / 2; ++it) {
                const int i = dkdv_epi::stage_read(it, lane);
                const long long a = 4LL * (dkdv_epi::stage_base(wave) + i);
                if (i < 0 || a < 0 || a + 16 > lds_bytes || i + 4 > (int)rd.size()) {
                  ++lds_oob;
                  continue;
                }
                for (int e = 0; e < 4; ++e) {
                  ++rd[i + e];
                  if (!wr[i + e]) ++read_unwritten;
                }
                // the global store of this read-back row
                const int kk = dkdv_epi::out_row(kblk0, wave, it, lane);
                if (kk >= rows) continue;
                const long long el = off + dkdv_epi::out_elem(base, kk, st, lane);
                ++stores;
                if ((el * 2) % 8) ++misaligned;
                if (el < 0 || el + 4 > alloc) {
                  ++global_oob;
                  continue;
                }
                for (int e = 0; e < 4; ++e)
                  if (hit[(size_t)(el + e)]++) ++global_twice;
              }
            for (int row = 0; row < dkdv_epi::kKeysPerWave; ++row)
              for (int col = 0; col < 128; ++col) {
                const int i = row * dkdv_epi::kStageRow + col;
                if (wr[i] != 1) ++(wr[i] ? stage_twice : stage_missing);
                if (rd[i] > 1) ++read_twice;
              }
          }
        }
    // every element of every (b, h) row below the chunk's row count
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h)
        for (int kk = 0; kk < rows; ++kk)
          for (int d = 0; d < 128; ++d) {
            const long long el = off + (long long)b * sb + (long long)h * sh + (long long)kk * st + d;
            if (el < 0 || el >= alloc || !hit[(size_t)el]) ++global_missing;
          }
  }
  std::printf(
      "lds_oob=%lld stage_twice=%lld stage_missing=%lld read_twice=%lld read_unwritten=%lld global_oob=%lld "
      "global_twice=%lld global_missing=%lld misaligned=%lld stores=%lld\n",
      lds_oob, stage_twice, stage_missing, read_twice, read_unwritten, global_oob, global_twice, global_missing,
      misaligned, stores);
  return 0;
}
