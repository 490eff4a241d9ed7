// Host walk of the output-epilogue addresses of the compiled kernels
// (ra_kernels.hip: fwd_kernel and dq_kernel "q", dkdv_kernel "k"), compiled
// from the same functions the kernels call (harp_amd/csrc/cq_epilogue.h).
// Test infrastructure: run by tests/test_cq_epilogue_bounds.py with g++.
//
// For every block of the grid, every wave and lane, it checks:
//   * every staging write and read-back lies inside the LDS array of the
//     wave's half (its byte size given), each wave's 32 x DP staging tile is
//     written exactly once and read back exactly once (the 16-byte read-back,
//     or the one-element read-back of the narrow store path), and nothing is
//     read before it is written;
//   * every global store lies inside the caller's allocation, no output
//     element is written twice over the grid, and every element of every
//     output row (d < D) is written;
// and counts the 4-element stores whose address is not 8-byte aligned.  DP 80
// is the layout at head dims 72 / 80: two 32-wide d blocks and a 16-wide last
// one staged from the 16 x 16 accumulator layout.
//
// usage: cq_epilogue_bounds kind DP D B H rows n_split elem_bytes wide
//        half0_bytes half1_bytes view_offset stride_b stride_h stride_t
//        split_stride alloc_elems [chunk rows...]
// kind q: rows = T, n_split KV splits, split_stride elements between them.
// kind k: rows = chunk rows; the trailing list gives each chunk's rows (one
// allocation per chunk, each checked alone); n_split and split_stride unused.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../harp_amd/csrc/cq_epilogue.h"

using namespace harp_ra;

struct Counts {
  long long lds_oob = 0, stage_pad = 0, stage_twice = 0, stage_missing = 0, read_twice = 0, read_unwritten = 0,
            read_missing = 0;
  long long global_oob = 0, global_twice = 0, global_missing = 0, misaligned = 0, stores = 0;
};

template <class E, int DP, bool Q>
void walk_block(Counts& n, int wave_rows0, int valid_rows, int D, int eb, bool wide, const long long half_bytes[2],
                long long base, long long st, long long alloc, std::vector<unsigned char>& hit) {
  constexpr int DBLK = DP / 32;  // 32-wide d blocks; DP % 32 == 16: a 16-wide last one (dK / dV)
  for (int wave = 0; wave < cq_epi::kWaves; ++wave) {
    const long long lim = half_bytes[cq_epi::half(wave)];
    std::vector<int> wr(cq_epi::kRows * E::kSR, 0), rd(wr.size(), 0);
    auto in_lds = [&](int x, int len) {
      const long long a = 4LL * (E::stage_base(wave) + (long long)x);
      return x >= 0 && a >= 0 && a + 4LL * len <= lim && x + len <= (int)wr.size();
    };
    for (int lane = 0; lane < 64; ++lane)
      for (int db = 0; db < DBLK; ++db)
        for (int k = 0; k < (Q ? 4 : 16); ++k) {
          const int x = E::stage_write(db, k, lane), len = Q ? 4 : 1;
          if (!in_lds(x, len) || (Q && x % 4)) {
            ++n.lds_oob;
            continue;
          }
          for (int e = 0; e < len; ++e) ++wr[x + e];
        }
    if constexpr (DP % 32 == 16) {  // the 16-wide last d block, 16 x 16 accumulator layout
      for (int lane = 0; lane < 64; ++lane)
        for (int t = 0; t < 2; ++t)
          for (int i = 0; i < (Q ? 1 : 4); ++i) {
            int x, len;
            if constexpr (Q) {
              x = E::stage_write_tail(t, lane), len = 4;
            } else {
              x = E::stage_write_tail(t, i, lane), len = 1;
            }
            if (!in_lds(x, len) || (Q && x % 4)) {
              ++n.lds_oob;
              continue;
            }
            for (int e = 0; e < len; ++e) ++wr[x + e];
          }
    }
    const int first_row = wave_rows0 + wave * cq_epi::kRows;
    auto store = [&](int row, int col, int len) {
      const int rr = first_row + row;
      if (rr >= valid_rows || col >= D) return;
      const long long el = base + (long long)rr * st + col;
      ++n.stores;
      if (len == 4 && (el * eb) % 8) ++n.misaligned;
      if (el < 0 || el + len > alloc) {
        ++n.global_oob;
        return;
      }
      for (int e = 0; e < len; ++e)
        if (hit[(size_t)(el + e)]++) ++n.global_twice;
    };
    for (int lane = 0; lane < 64; ++lane) {
      if (wide) {
        for (int it = 0; it < E::kIters; ++it) {
          const int x = E::stage_read(it, lane);
          if (!in_lds(x, 4) || x % 4) {
            ++n.lds_oob;
            continue;
          }
          for (int e = 0; e < 4; ++e) {
            ++rd[x + e];
            if (!wr[x + e]) ++n.read_unwritten;
          }
          store(E::read_row(it, lane), 4 * E::read_chunk(it, lane), 4);
        }
      } else {
        for (int it = 0; it < E::kElemIters; ++it) {
          const int x = E::stage_elem(it, lane);
          if (!in_lds(x, 1)) {
            ++n.lds_oob;
            continue;
          }
          ++rd[x];
          if (!wr[x]) ++n.read_unwritten;
          store(E::elem_row(it, lane), E::elem_col(it, lane), 1);
        }
      }
    }
    for (int row = 0; row < cq_epi::kRows; ++row)
      for (int col = 0; col < E::kSR; ++col) {
        const int x = row * E::kSR + col;
        if (col >= DP) {  // the row's padding: never written or read
          if (wr[x] || rd[x]) ++n.stage_pad;
          continue;
        }
        if (wr[x] != 1) ++(wr[x] ? n.stage_twice : n.stage_missing);
        if (rd[x] != 1) ++(rd[x] ? n.read_twice : n.read_missing);
      }
  }
}

template <int DP>
int run(char kind, int D, int B, int H, int rows, int n_split, int eb, bool wide, const long long half_bytes[2],
        long long off, long long sb, long long sh, long long st, long long split, long long alloc,
        const std::vector<int>& chunk_rows, Counts& n) {
  const int block_rows = cq_epi::kWaves * cq_epi::kRows;
  if (kind == 'q') {
    std::vector<unsigned char> hit((size_t)alloc, 0);
    const int tiles = (rows + block_rows - 1) / block_rows;
    for (int s = 0; s < n_split; ++s)
      for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
          for (int qt = 0; qt < tiles; ++qt)
            walk_block<cq_epi::QRows<DP>, DP, true>(n, qt * block_rows, rows, D, eb, wide, half_bytes,
                                                     off + s * split + b * sb + h * sh, st, alloc, hit);
    for (int s = 0; s < n_split; ++s)
      for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
          for (int t = 0; t < rows; ++t)
            for (int d = 0; d < D; ++d) {
              const long long el = off + s * split + b * sb + h * sh + t * st + d;
              if (el < 0 || el >= alloc || !hit[(size_t)el]) ++n.global_missing;
            }
  } else {
    for (int cr : chunk_rows) {
      std::vector<unsigned char> hit((size_t)alloc, 0);
      const int tiles = (cr + block_rows - 1) / block_rows;
      for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
          for (int kt = 0; kt < tiles; ++kt)
            walk_block<cq_epi::KRows<DP>, DP, false>(n, kt * block_rows, cr, D, eb, wide, half_bytes,
                                                      off + b * sb + h * sh, st, alloc, hit);
      for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
          for (int t = 0; t < cr; ++t)
            for (int d = 0; d < D; ++d) {
              const long long el = off + b * sb + h * sh + t * st + d;
              if (el < 0 || el >= alloc || !hit[(size_t)el]) ++n.global_missing;
            }
    }
  }
  return 0;
}

int main(int argc, char** argv) {
  if (argc < 18) {
    std::fprintf(stderr, "usage: %s kind DP D B H rows n_split eb wide half0 half1 off sb sh st split alloc [rows...]\n",
                 argv[0]);
    return 2;
  }
  const char kind = argv[1][0];
  const int DP = std::atoi(argv[2]), D = std::atoi(argv[3]), B = std::atoi(argv[4]), H = std::atoi(argv[5]);
  const int rows = std::atoi(argv[6]), n_split = std::atoi(argv[7]), eb = std::atoi(argv[8]);
  const bool wide = std::atoi(argv[9]) != 0;
  const long long half_bytes[2] = {std::atoll(argv[10]), std::atoll(argv[11])};
  const long long off = std::atoll(argv[12]), sb = std::atoll(argv[13]), sh = std::atoll(argv[14]);
  const long long st = std::atoll(argv[15]), split = std::atoll(argv[16]), alloc = std::atoll(argv[17]);
  std::vector<int> chunk_rows;
  for (int i = 18; i < argc; ++i) chunk_rows.push_back(std::atoi(argv[i]));
  Counts n;
  switch (DP) {
    case 32: run<32>(kind, D, B, H, rows, n_split, eb, wide, half_bytes, off, sb, sh, st, split, alloc, chunk_rows, n); break;
    case 64: run<64>(kind, D, B, H, rows, n_split, eb, wide, half_bytes, off, sb, sh, st, split, alloc, chunk_rows, n); break;
    case 96: run<96>(kind, D, B, H, rows, n_split, eb, wide, half_bytes, off, sb, sh, st, split, alloc, chunk_rows, n); break;
    case 80:  // the 16-wide d tail (head dims 72 / 80)
      run<80>(kind, D, B, H, rows, n_split, eb, wide, half_bytes, off, sb, sh, st, split, alloc, chunk_rows, n); break;
    default: std::fprintf(stderr, "DP must be 32, 64, 80 or 96\n"); return 2;
  }
  std::printf(
      "lds_oob=%lld stage_pad=%lld stage_twice=%lld stage_missing=%lld read_twice=%lld read_unwritten=%lld "
      "read_missing=%lld global_oob=%lld global_twice=%lld global_missing=%lld misaligned=%lld stores=%lld\n",
      n.lds_oob, n.stage_pad, n.stage_twice, n.stage_missing, n.read_twice, n.read_unwritten, n.read_missing,
      n.global_oob, n.global_twice, n.global_missing, n.misaligned, n.stores);
  return 0;
}
