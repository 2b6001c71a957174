// Split of the persistent decode kernel's flattened block list over its
// grid, shared by the decode kernel and its reduce kernel (plain C++ as
// well, so a CPU test can compile it with g++).
#pragma once

#ifndef __HIPCC__
#ifndef __host__
#define __host__
#endif
#ifndef __device__
#define __device__
#endif
#include <algorithm>
using std::min;
#endif

namespace lv {

// Equal contiguous ranges: workgroup b walks flattened blocks
// [start(b), start(b + 1)), start(b) = min(total, b * per),
// per = ceil(total / grid).  The entry point keeps num_decodes * max_blocks
// (>= total) below 2^31 - 2^16, so 32-bit arithmetic suffices (the reduce
// kernel divides by per; a 64-bit division is a long instruction sequence).
struct RangeSplit {
  int per, total;
  __host__ __device__ int start(int b) const {
    return (int)min((long long)total, (long long)b * per);
  }
  // The workgroup whose range holds flattened position p (0 <= p < total).
  __host__ __device__ int owner(int p) const { return p / per; }
  // min(2, w - owner(p)) for the first block p of a row that workgroup w
  // walks part of (w's range is not empty, p < start(w + 1)); no division.
  __host__ __device__ int piece_rank(int p, int w) const {
    const int r0 = w * per;
    return p >= r0 ? 0 : (p >= r0 - per ? 1 : 2);
  }
};

__host__ __device__ inline RangeSplit make_range_split(int total, int grid) {
  RangeSplit r;
  r.total = total;
  r.per = total > 0 ? (total + grid - 1) / grid : 1;
  return r;
}

// Pieces of a row that spans several ranges.  The row's piece i is walked by
// workgroup owner(first block) + i.  Pieces 0 and 1 (every such row has both)
// go to row-indexed slots 2 * row and 2 * row + 1, so the reduce kernel finds
// them without knowing the split; piece i >= 2 goes to slot 2 * num_rows + w
// of its workgroup w (a workgroup walks at most one piece with i >= 1: the
// first of its range).  rank = piece_rank(...).
__host__ __device__ inline int piece_slot(int row, int rank, int w, int num_rows) {
  return rank < 2 ? 2 * row + rank : 2 * num_rows + w;
}

// Per-row word the decode kernel writes for the reduce kernel, for a row
// whose walked blocks are [a, b): bits 0-7 hold the number of pieces capped
// at 3 (0: no walked blocks, 1: one piece, finished by the decode kernel,
// 2: pieces 0 and 1, 3: three or more), bits 8-15 the number of its
// shared-prefix splits.
__host__ __device__ inline int row_header(int a, int b, const RangeSplit& r, int nsplit) {
  const int np = a == b ? 0 : min(r.owner(b - 1) - r.owner(a) + 1, 3);
  return np | (nsplit << 8);
}
__host__ __device__ inline int header_pieces(int h) { return h & 0xff; }
__host__ __device__ inline int header_splits(int h) { return (h >> 8) & 0xff; }

}  // namespace lv
