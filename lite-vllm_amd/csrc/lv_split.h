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
};

__host__ __device__ inline RangeSplit make_range_split(int total, int grid) {
  RangeSplit r;
  r.total = total;
  r.per = total > 0 ? (total + grid - 1) / grid : 1;
  return r;
}

}  // namespace lv
