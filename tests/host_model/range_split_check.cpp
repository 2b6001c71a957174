// Host-side model of the persistent decode kernel's work split, compiled
// with g++ (and AddressSanitizer / UndefinedBehaviorSanitizer) by
// tests/test_host_model.py.  It includes the header the kernels use
// (lite-vllm_amd/csrc/lv_split.h) and checks, against brute force:
//   * the ranges [start(b), start(b+1)) partition [0, total) for every grid
//     size, and owner(p) is the range holding p, for every p;
//   * the piece bookkeeping of the decode kernel and its reduce kernel
//     agree: every row's pieces are written once each, into slots
//     (piece_slot: pieces 0 / 1 row-indexed, later ones in their
//     workgroup's slot) that no other row uses, the header word
//     (row_header) carries the row's piece count and prefix splits, and the
//     reduce kernel reads exactly the written slots (from the header alone
//     for up to two pieces, from the offsets beyond), for random ragged rows
//     with and without walked blocks;
//   * every slot index stays inside the workspace the host sizes for it
//     (2 slots per row + 1 per workgroup).
// Exit status 0 = all checks passed; a message and status 1 otherwise.
#include <cstdio>
#include <cstdlib>
#include <map>
#include <random>
#include <set>
#include <vector>

#include "lv_split.h"

static int g_fail = 0;
#define CHECK(c, ...)                                               \
  do {                                                              \
    if (!(c)) {                                                     \
      if (g_fail < 20) {                                            \
        std::fprintf(stderr, "FAIL %s:%d ", __FILE__, __LINE__);    \
        std::fprintf(stderr, __VA_ARGS__);                          \
        std::fprintf(stderr, "\n");                                 \
      }                                                             \
      ++g_fail;                                                     \
    }                                                               \
  } while (0)

static void check_split(int total, int grid) {
  const lv::RangeSplit r = lv::make_range_split(total, grid);
  CHECK(r.start(0) == 0, "start(0) total=%d grid=%d", total, grid);
  CHECK(r.start(grid) == total, "start(grid)=%d total=%d grid=%d", r.start(grid), total, grid);
  for (int b = 0; b < grid; ++b) CHECK(r.start(b) <= r.start(b + 1), "non-monotone at b=%d", b);
  int b = 0;
  for (int p = 0; p < total; ++p) {
    while (r.start(b + 1) <= p) ++b;
    CHECK(r.owner(p) == b && b < grid, "owner(%d)=%d want %d (total %d grid %d)", p, r.owner(p),
          b, total, grid);
  }
}

// Decode kernel / reduce kernel piece bookkeeping for one batch.
static void check_pieces(const std::vector<int>& walked, int grid, std::mt19937& rng) {
  const int n = (int)walked.size();
  std::vector<int> off(n + 1, 0);
  for (int i = 0; i < n; ++i) off[i + 1] = off[i] + walked[i];
  const int total = off[n];
  const lv::RangeSplit r = lv::make_range_split(total, grid);
  const int num_slots = 2 * n + grid;
  std::map<int, int> slot_owner;                 // slot -> row
  std::map<int, std::set<int>> pieces;           // row -> its slots
  std::vector<int> whole_by(n, -1);
  for (int g = 0; g < grid; ++g) {
    const int r0 = r.start(g), r1 = r.start(g + 1);
    if (r0 >= r1) continue;
    for (int sq = 0; sq < n; ++sq) {
      const int a = off[sq], b = off[sq + 1];
      if (a == b || b <= r0 || a >= r1) continue;   // no blocks in this range
      if (a >= r0 && b <= r1) {
        CHECK(whole_by[sq] < 0, "row %d whole in two ranges", sq);
        whole_by[sq] = g;
        continue;
      }
      const int rank = r.piece_rank(a, g);
      const int exact = g - r.owner(a);
      CHECK(rank == (exact < 2 ? exact : 2), "row %d piece %d: rank %d", sq, exact, rank);
      const int slot = lv::piece_slot(sq, rank, g, n);
      CHECK(slot >= 0 && slot < num_slots, "slot %d outside the workspace (%d)", slot, num_slots);
      CHECK(!slot_owner.count(slot), "slot %d written by rows %d and %d", slot, slot_owner[slot],
            sq);
      slot_owner[slot] = sq;
      pieces[sq].insert(slot);
    }
  }
  for (int sq = 0; sq < n; ++sq) {
    const int a = off[sq], b = off[sq + 1];
    const int nsplit = (int)(rng() % 17);
    const int h = lv::row_header(a, b, r, nsplit);
    CHECK(lv::header_splits(h) == nsplit, "row %d: header splits", sq);
    const int np = lv::header_pieces(h);
    if (a == b) {
      CHECK(np == 0 && !pieces.count(sq) && whole_by[sq] < 0, "empty row %d", sq);
      continue;
    }
    if (np == 1) {
      CHECK(whole_by[sq] == r.owner(a) && !pieces.count(sq), "row %d: header says whole", sq);
      continue;
    }
    CHECK(np == 2 || np == 3, "row %d: header pieces %d", sq, np);
    std::set<int> read;
    if (np == 2) {
      read = {2 * sq, 2 * sq + 1};               // the reduce kernel's fast path
      CHECK(r.owner(b - 1) - r.owner(a) == 1, "row %d: two pieces", sq);
    } else {
      const int g0 = r.owner(a), cnt = r.owner(b - 1) - g0 + 1;
      CHECK(cnt >= 3, "row %d: header 3, %d pieces", sq, cnt);
      for (int i = 0; i < cnt; ++i) read.insert(lv::piece_slot(sq, i < 2 ? i : 2, g0 + i, n));
    }
    CHECK(read == pieces[sq], "row %d: reduce reads %zu slots, kernel wrote %zu", sq,
          read.size(), pieces[sq].size());
    for (int k : read)
      CHECK(slot_owner.count(k) && slot_owner[k] == sq, "row %d reads a slot of another row", sq);
  }
}

int main() {
  const int grids[] = {1, 2, 3, 7, 8, 64, 255, 256, 257, 1024};
  for (int grid : grids)
    for (int total : {0, 1, 2, 5, 63, 64, 255, 256, 257, 1000, 4099, 37000})
      check_split(total, grid);
  std::mt19937 rng(12345);
  for (int trial = 0; trial < 600; ++trial) {
    const int n = 1 + (int)(rng() % 300);
    std::vector<int> walked(n);
    const int maxb = 1 + (int)(rng() % 200);
    for (int& w : walked) w = (rng() % 7 == 0) ? 0 : (int)(rng() % maxb);
    check_pieces(walked, grids[rng() % 10], rng);
  }
  if (g_fail) {
    std::fprintf(stderr, "%d checks failed\n", g_fail);
    return 1;
  }
  std::printf("range split and piece bookkeeping: all checks passed\n");
  return 0;
}
