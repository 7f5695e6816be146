// Float64 sums and prefix sums in NumPy's exact operation order.
//
// The reference normalises and validates probability vectors with
// `values.sum(dtype=np.float64)` and `np.cumsum` (src/deepseekrpc/sampling.py
// :109-139).  Reproducing their rounding bit for bit needs their order:
//
//  * np.add.reduce over a contiguous float64 vector walks it in buffers of
//    8,192 elements (the iterator's default buffer size) and adds the buffers'
//    results in order.  Each buffer is summed pairwise: a range of more than
//    128 elements splits at n/2 rounded down to a multiple of 8 and its halves
//    are added; a range of 8..128 elements keeps 8 running sums over strided
//    elements, combined as ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then adds the
//    n mod 8 leftovers in order; a range under 8 adds its elements to 0.0 in
//    order.  (NumPy's pairwise summation, numpy/_core/src/umath/loops_utils.h;
//    checked bit for bit against NumPy 2.2 on random vectors of 1 to 129,280
//    elements by the tests.)
//  * np.cumsum is a sequential running sum.
//
// One workgroup handles a vector of at most 16 buffers: wave w owns buffer w.
// Its lane 0 lists the buffer's leaves (ranges of at most 128 elements, each
// at least 64 long when the buffer is), the lanes sum the leaves, and lane 0
// adds them back up along the same tree.  Not on the sampling hot path.
#pragma once

#include "dsr_common.h"

namespace dsr {

constexpr int kNpBuffer = 8192;   // NumPy's default iterator buffer, in elements
constexpr int kNpLeaf = 128;      // pairwise-summation block
constexpr int kNpMaxLeaves = 128; // leaves of one buffer: each leaf holds >= 64 elements
constexpr int64_t kNpMaxLength = (int64_t)kWaves * kNpBuffer;

struct NpSumShared {
  int32_t leaf_lo[kWaves][kNpMaxLeaves];
  int32_t leaf_len[kWaves][kNpMaxLeaves];
  double leaf_sum[kWaves][kNpMaxLeaves];
  double buffer_sum[kWaves];
  int leaves[kWaves];
};

// Leaves of the pairwise tree over [lo, lo + n), left to right.
template <int D>
__device__ __noinline__ void np_list_leaves(int lo, int n, int32_t* out_lo, int32_t* out_len, int& count) {
  if (n <= kNpLeaf) {
    out_lo[count] = lo;
    out_len[count] = n;
    ++count;
    return;
  }
  int h = n / 2;
  h -= h % 8;
  np_list_leaves<D - 1>(lo, h, out_lo, out_len, count);
  np_list_leaves<D - 1>(lo + h, n - h, out_lo, out_len, count);
}
template <>
__device__ __noinline__ void np_list_leaves<0>(int lo, int n, int32_t* out_lo, int32_t* out_len, int& count) {
  out_lo[count] = lo;
  out_len[count] = n;
  ++count;
}

// The tree's sum from its leaf sums, consumed left to right.
template <int D>
__device__ __noinline__ double np_tree_sum(int n, const double* leaf, int& next) {
  if (n <= kNpLeaf) return leaf[next++];
  int h = n / 2;
  h -= h % 8;
  const double a = np_tree_sum<D - 1>(h, leaf, next);
  const double b = np_tree_sum<D - 1>(n - h, leaf, next);
  return a + b;
}
template <>
__device__ __noinline__ double np_tree_sum<0>(int, const double* leaf, int& next) {
  return leaf[next++];
}

// A buffer of 8,192 splits at most 6 times before its ranges fit a leaf.
constexpr int kNpDepth = 8;

// One leaf: 8 strided running sums (n >= 8) or a plain running sum (n < 8).
template <class Load>
__device__ double np_leaf_sum(Load load, int64_t base, int n) {
  if (n < 8) {
    double r = 0.0;
    for (int i = 0; i < n; ++i) r += load(base + i);
    return r;
  }
  double r0 = load(base + 0), r1 = load(base + 1), r2 = load(base + 2), r3 = load(base + 3);
  double r4 = load(base + 4), r5 = load(base + 5), r6 = load(base + 6), r7 = load(base + 7);
  int i = 8;
  for (; i < n - (n % 8); i += 8) {
    r0 += load(base + i + 0);
    r1 += load(base + i + 1);
    r2 += load(base + i + 2);
    r3 += load(base + i + 3);
    r4 += load(base + i + 4);
    r5 += load(base + i + 5);
    r6 += load(base + i + 6);
    r7 += load(base + i + 7);
  }
  double res = ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7));
  for (; i < n; ++i) res += load(base + i);
  return res;
}

// np.add.reduce of load(0 .. n-1), n <= kNpMaxLength, for the whole
// workgroup (every thread must call it; every thread gets the result).
template <class Load>
__device__ double np_sum(Load load, int64_t n, NpSumShared& sh) {
  const int w = wave_id(), lane = lane_id();
  const int64_t lo = (int64_t)w * kNpBuffer;
  const int len = lo < n ? (int)((n - lo) < kNpBuffer ? (n - lo) : kNpBuffer) : 0;
  if (len > 0 && lane == 0) {
    int count = 0;
    np_list_leaves<kNpDepth>(0, len, sh.leaf_lo[w], sh.leaf_len[w], count);
    sh.leaves[w] = count;
  }
  __syncthreads();
  if (len > 0) {
    for (int j = lane; j < sh.leaves[w]; j += 64)
      sh.leaf_sum[w][j] = np_leaf_sum(load, lo + sh.leaf_lo[w][j], sh.leaf_len[w][j]);
  }
  __syncthreads();
  if (len > 0 && lane == 0) {
    int next = 0;
    sh.buffer_sum[w] = np_tree_sum<kNpDepth>(len, sh.leaf_sum[w], next);
  }
  __syncthreads();
  double total = 0.0;
  const int buffers = (int)((n + kNpBuffer - 1) / kNpBuffer);
  for (int b = 0; b < buffers; ++b) total = b == 0 ? sh.buffer_sum[0] : total + sh.buffer_sum[b];
  __syncthreads();
  return total;
}

}  // namespace dsr
