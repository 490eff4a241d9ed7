// Host walk of the epilogue addresses of the head-dim-128 Q-stationary
// kernels (fwd_asm.hip: O; dq_asm.hip: dQ), compiled from the same functions
// the kernels call (harp_amd/csrc/q_epilogue.h).  Test infrastructure: run by
// tests/test_q_epilogue_bounds.py with g++.
//
// For every block of the grid (query tile, head, batch, KV split), every
// wave and lane, it checks:
//   * every staging write (16 bytes) and read-back (16 bytes) lies inside the
//     kernel's LDS allocation; each wave's 64 x 128 staging tile is written
//     exactly once and read back exactly once, and nothing is read back
//     before it is written;
//   * every global store (four elements) lies inside the caller's
//     allocation, no output element is written twice over the grid, and
//     every element of rows < T, d < 128 of every split is written;
// and counts the stores whose address is not 8-byte aligned (the wide bf16
// store needs it; the kernel then stores element by element).
//
// usage: q_epilogue_bounds B H T n_split elem_bytes lds_bytes view_offset
//        stride_b stride_h stride_t split_stride alloc_elems
// (element units; the view's base is the allocation + view_offset)
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../harp_amd/csrc/q_epilogue.h"

using namespace harp_ra;

int main(int argc, char** argv) {
  if (argc != 13) {
    std::fprintf(stderr, "usage: %s B H T n_split elem_bytes lds_bytes offset sb sh st split alloc\n", argv[0]);
    return 2;
  }
  const int B = std::atoi(argv[1]), H = std::atoi(argv[2]), T = std::atoi(argv[3]), n_split = std::atoi(argv[4]);
  const int eb = std::atoi(argv[5]);
  const long long lds_bytes = std::atoll(argv[6]), off = std::atoll(argv[7]);
  const long long sb = std::atoll(argv[8]), sh = std::atoll(argv[9]), st = std::atoll(argv[10]);
  const long long split = std::atoll(argv[11]), alloc = std::atoll(argv[12]);
  const int block_rows = q_epi::kWaves * q_epi::kRowsPerWave;
  const int tiles = (T + block_rows - 1) / block_rows;

  long long lds_oob = 0, stage_twice = 0, stage_missing = 0, read_twice = 0, read_unwritten = 0;
  long long global_oob = 0, global_twice = 0, global_missing = 0, misaligned = 0, stores = 0;
  std::vector<unsigned char> hit((size_t)alloc, 0);
  for (int s = 0; s < n_split; ++s)
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h)
        for (int qt = 0; qt < tiles; ++qt) {
          const long long base = (long long)s * split + (long long)b * sb + (long long)h * sh;
          for (int wave = 0; wave < q_epi::kWaves; ++wave) {
            std::vector<int> wr(q_epi::kRowsPerWave * q_epi::kStageRow, 0), rd(wr.size(), 0);
            for (int lane = 0; lane < 64; ++lane)
              for (int qg = 0; qg < 2; ++qg)
                for (int db = 0; db < 4; ++db)
                  for (int i = 0; i < 4; ++i) {
                    const int x = q_epi::stage_write(qg, db, i, lane);
                    const long long a = 4LL * (q_epi::stage_base(wave) + x);
                    if (x < 0 || a < 0 || a % 16 || a + 16 > lds_bytes || x + 4 > (int)wr.size()) {
                      ++lds_oob;
                      continue;
                    }
                    for (int e = 0; e < 4; ++e) ++wr[x + e];
                  }
            for (int lane = 0; lane < 64; ++lane)
              for (int it = 0; it < q_epi::kRowsPerWave / 2; ++it) {
                const int x = q_epi::stage_read(it, lane);
                const long long a = 4LL * (q_epi::stage_base(wave) + x);
                if (x < 0 || a < 0 || a % 16 || a + 16 > lds_bytes || x + 4 > (int)rd.size()) {
                  ++lds_oob;
                  continue;
                }
                for (int e = 0; e < 4; ++e) {
                  ++rd[x + e];
                  if (!wr[x + e]) ++read_unwritten;
                }
                const int qi = q_epi::out_query(qt * block_rows, wave, it, lane);
                if (qi >= T) continue;
                const long long el = off + q_epi::out_elem(base, qi, st, lane);
                ++stores;
                if ((el * eb) % 8) ++misaligned;
                if (el < 0 || el + 4 > alloc) {
                  ++global_oob;
                  continue;
                }
                for (int e = 0; e < 4; ++e)
                  if (hit[(size_t)(el + e)]++) ++global_twice;
              }
            for (int row = 0; row < q_epi::kRowsPerWave; ++row)
              for (int col = 0; col < 128; ++col) {
                const int x = row * q_epi::kStageRow + col;
                if (wr[x] != 1) ++(wr[x] ? stage_twice : stage_missing);
                if (rd[x] > 1) ++read_twice;
              }
          }
        }
  for (int s = 0; s < n_split; ++s)
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h)
        for (int t = 0; t < T; ++t)
          for (int d = 0; d < 128; ++d) {
            const long long el = off + (long long)s * split + (long long)b * sb + (long long)h * sh + (long long)t * st + d;
            if (el < 0 || el >= alloc || !hit[(size_t)el]) ++global_missing;
          }
  std::printf(
      "lds_oob=%lld stage_twice=%lld stage_missing=%lld read_twice=%lld read_unwritten=%lld global_oob=%lld "
      "global_twice=%lld global_missing=%lld misaligned=%lld stores=%lld\n",
      lds_oob, stage_twice, stage_missing, read_twice, read_unwritten, global_oob, global_twice, global_missing,
      misaligned, stores);
  return 0;
}
