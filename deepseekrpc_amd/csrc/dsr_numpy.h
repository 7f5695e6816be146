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
// A full buffer's tree is balanced (64 leaves of 128), so its wave sums it
// with no list: 8 lanes per leaf keep the leaf's 8 strided running sums, and
// xor butterflies over 1, 2, 4 lanes combine them in NumPy's order, then
// over 8, 16, 32 lanes give the sums of 1,024 elements, which the tree's top
// three levels add.  (Floating-point addition is commutative, so a lane
// pair's two sums agree bit for bit.)  A shorter last buffer's wave lists
// its tree level by level (a scan per level, no recursion), sums each leaf
// the same way (8 lanes, leftovers after the butterfly) and adds the tree
// back up level by level.
#pragma once

#include "dsr_wave.h"

namespace dsr {

constexpr int kNpBuffer = 8192;   // NumPy's default iterator buffer, in elements
constexpr int kNpLeaf = 128;      // pairwise-summation block
constexpr int kNpMaxLeaves = 128; // leaves of a buffer shorter than 8,192: each holds >= 64 elements
constexpr int kNpLevels = 8;      // a short buffer's tree: the root, then at most 7 levels of splits
constexpr int64_t kNpMaxLength = (int64_t)kWaves * kNpBuffer;

struct NpSumShared {
  int32_t node_lo[kNpLevels][kNpMaxLeaves];   // a short buffer's tree, level by level, in order
  int32_t node_len[kNpLevels][kNpMaxLeaves];
  int32_t node_pos[kNpLevels][kNpMaxLeaves];  // where a node's range sits in the next level
  int32_t nodes[kNpLevels];
  double val[kNpLevels][kNpMaxLeaves];        // node sums, from the leaves up
  double buffer_sum[kWaves];
};

// np.add.reduce of load(0 .. n-1), n <= kNpMaxLength, for the whole
// workgroup (every thread must call it; every thread gets the result).
// load(i) is called exactly once per element, and visit(i, x) then sees it,
// in some thread; within a thread the visits come in increasing i.  Inlined,
// so that what the callbacks capture stays in registers.
template <class Load, class Visit>
__device__ __forceinline__ double np_sum(Load load, int64_t n, NpSumShared& sh, Visit visit) {
  const int w = wave_id(), lane = lane_id();
  const int g = lane >> 3, k = lane & 7;  // leaf within a group of 8, running sum within the leaf
  const int64_t lo = (int64_t)w * kNpBuffer;
  const int len = lo < n ? (int)((n - lo) < kNpBuffer ? (n - lo) : kNpBuffer) : 0;  // uniform per wave
  const bool listed = len >= 8 && len < kNpBuffer;  // at most one wave: the last buffer
  // A short buffer's tree, breadth first: level l + 1 holds level l's ranges
  // in order, each one longer than a leaf replaced by its two halves (the
  // split rounded down to a multiple of 8), so the last level lists the
  // leaves.  The loop runs a fixed number of levels: once every range is a
  // leaf a level copies the one above it.
  if (listed && lane == 0) {
    sh.nodes[0] = 1;
    sh.node_lo[0][0] = 0;
    sh.node_len[0][0] = len;
  }
  __syncthreads();
  for (int l = 0; l + 1 < kNpLevels; ++l) {  // every thread takes part in the barriers
    if (listed) {
      const int cnt = sh.nodes[l];
      const int i0 = lane, i1 = lane + 64;
      const int m0 = i0 < cnt ? sh.node_len[l][i0] : 0, m1 = i1 < cnt ? sh.node_len[l][i1] : 0;
      const uint32_t c0 = i0 < cnt ? (m0 > kNpLeaf ? 2u : 1u) : 0u;
      const uint32_t c1 = i1 < cnt ? (m1 > kNpLeaf ? 2u : 1u) : 0u;
      const uint32_t s0 = wave_scan_dpp(c0), s1 = wave_scan_dpp(c1);
      const uint32_t t0 = lane_value(s0, 63), t1 = lane_value(s1, 63);
      auto emit = [&](int i, int m, uint32_t c, uint32_t e) {
        if (c == 0 || e + c > (uint32_t)kNpMaxLeaves) return;  // the bound never binds: leaves hold >= 64
        const int a = sh.node_lo[l][i];
        sh.node_pos[l][i] = (int)e;
        if (c == 2) {
          int h = m / 2;
          h -= h % 8;
          sh.node_lo[l + 1][e] = a;
          sh.node_len[l + 1][e] = h;
          sh.node_lo[l + 1][e + 1] = a + h;
          sh.node_len[l + 1][e + 1] = m - h;
        } else {
          sh.node_lo[l + 1][e] = a;
          sh.node_len[l + 1][e] = m;
        }
      };
      emit(i0, m0, c0, s0 - c0);
      emit(i1, m1, c1, t0 + s1 - c1);
      if (lane == 0) sh.nodes[l + 1] = (int)(t0 + t1 < (uint32_t)kNpMaxLeaves ? t0 + t1 : kNpMaxLeaves);
    }
    __syncthreads();
  }
  if (len == kNpBuffer) {
    // A full buffer's tree is balanced: 64 leaves of 128.  The sum of leaves
    // 8q .. 8q + 7 (elements 1,024 q .. 1,024 q + 1,023):
    auto group = [&](int q) -> double {
      const int64_t base = lo + 128 * (8 * q + g) + k;  // leaf 8q + g, running sum k
      double v[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) v[t] = load(base + 8 * t);
      double r = v[0];
      visit(base, v[0]);
#pragma unroll
      for (int t = 1; t < 16; ++t) {
        r += v[t];
        visit(base + 8 * t, v[t]);
      }
#pragma unroll
      for (int m = 1; m < 64; m <<= 1) r += __shfl_xor(r, m);
      return r;
    };
    const double s0 = group(0), s1 = group(1), s2 = group(2), s3 = group(3);
    const double s4 = group(4), s5 = group(5), s6 = group(6), s7 = group(7);
    if (lane == 0) sh.buffer_sum[w] = ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7));
  } else if (listed) {
    constexpr int L = kNpLevels - 1;
    const int leaves = sh.nodes[L];
    for (int q0 = 0; q0 < leaves; q0 += 8) {  // uniform over the wave
      const int j = q0 + g;
      const bool has = j < leaves;
      const int llo = has ? sh.node_lo[L][j] : 0, llen = has ? sh.node_len[L][j] : 0;
      const int nb = llen >> 3;  // full 8-element rows of the leaf (every leaf here holds >= 8)
      const int64_t base = lo + llo + k;
      double v[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) v[t] = t < nb ? load(base + 8 * t) : 0.0;
      double r = v[0];
      if (nb > 0) visit(base, v[0]);
#pragma unroll
      for (int t = 1; t < 16; ++t) {
        if (t < nb) {
          r += v[t];
          visit(base + 8 * t, v[t]);
        }
      }
      r += __shfl_xor(r, 1);
      r += __shfl_xor(r, 2);
      r += __shfl_xor(r, 4);
      if (has && k == 0) {
        for (int i = 8 * nb; i < llen; ++i) {  // the leftovers, in order
          const double x = load(lo + llo + i);
          r += x;
          visit(lo + llo + i, x);
        }
        sh.val[L][j] = r;
      }
    }
  } else if (len > 0 && lane == 0) {  // fewer than 8 elements: a running sum from 0.0
    double r = 0.0;
    for (int i = 0; i < len; ++i) {
      const double x = load(lo + i);
      r += x;
      visit(lo + i, x);
    }
    sh.buffer_sum[w] = r;
  }
  __syncthreads();
  // The short buffer's tree from the leaves up: a split range is its left
  // half's sum plus its right half's.
  for (int l = kNpLevels - 2; l >= 0; --l) {
    if (listed) {
      const int cnt = sh.nodes[l];
      for (int i = lane; i < cnt; i += 64) {
        const int p = sh.node_pos[l][i];
        const double a = sh.val[l + 1][p];
        sh.val[l][i] = sh.node_len[l][i] > kNpLeaf ? a + sh.val[l + 1][p + 1] : a;
      }
    }
    __syncthreads();
  }
  if (listed && lane == 0) sh.buffer_sum[w] = sh.val[0][0];
  __syncthreads();
  double total = 0.0;
  const int buffers = (int)((n + kNpBuffer - 1) / kNpBuffer);
  for (int b = 0; b < buffers; ++b) total = b == 0 ? sh.buffer_sum[0] : total + sh.buffer_sum[b];
  __syncthreads();
  return total;
}

template <class Load>
__device__ __forceinline__ double np_sum(Load load, int64_t n, NpSumShared& sh) {
  return np_sum(load, n, sh, [](int64_t, double) {});
}

// One buffer, load(lo .. lo + len - 1) with 0 < len <= 8,192, summed in
// NumPy's order by a workgroup of kNpBufWaves waves, so that the buffers of
// a vector go to separate workgroups (their results are then added in
// order: sum = b0, then sum + b1, ...).  Wave v of a full buffer takes
// leaves 8v .. 8v + 7 (elements 1,024 v .. 1,024 v + 1,023) as np_sum's
// wave takes them and the tree's top three levels add the eight results; a
// shorter buffer's tree is listed by wave 0 and its leaves shared out eight
// per wave.  Every thread of the workgroup calls it and gets the result;
// visit(i, x) sees every element once, within a thread in increasing i.
constexpr int kNpBufWaves = 8;
constexpr int kNpBufThreads = 64 * kNpBufWaves;

struct NpBufShared {
  int32_t node_lo[kNpLevels][kNpMaxLeaves];
  int32_t node_len[kNpLevels][kNpMaxLeaves];
  int32_t node_pos[kNpLevels][kNpMaxLeaves];
  int32_t nodes[kNpLevels];
  double val[kNpLevels][kNpMaxLeaves];
  double gsum[kNpBufWaves];
  double result;
};

template <class Load, class Visit>
__device__ __forceinline__ double np_buffer_sum(Load load, int64_t lo, int len, NpBufShared& sh, Visit visit) {
  const int w = wave_id(), lane = lane_id();
  const int g = lane >> 3, k = lane & 7;
  if (len == kNpBuffer) {
    const int64_t base = lo + 128 * (8 * w + g) + k;  // leaf 8w + g, running sum k
    double v[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) v[t] = load(base + 8 * t);
    double r = v[0];
    visit(base, v[0]);
#pragma unroll
    for (int t = 1; t < 16; ++t) {
      r += v[t];
      visit(base + 8 * t, v[t]);
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) r += __shfl_xor(r, m);
    if (lane == 0) sh.gsum[w] = r;
    __syncthreads();
    const double* q = sh.gsum;
    const double total = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
    __syncthreads();  // the shared arrays may be used again on return
    return total;
  }
  if (len < 8) {  // a running sum from 0.0
    if (threadIdx.x == 0) {
      double r = 0.0;
      for (int i = 0; i < len; ++i) {
        const double x = load(lo + i);
        r += x;
        visit(lo + i, x);
      }
      sh.result = r;
    }
    __syncthreads();
    const double total = sh.result;
    __syncthreads();
    return total;
  }
  // The tree, breadth first, by wave 0 (np_sum's listing); every thread
  // takes part in the barriers.
  if (w == 0 && lane == 0) {
    sh.nodes[0] = 1;
    sh.node_lo[0][0] = 0;
    sh.node_len[0][0] = len;
  }
  __syncthreads();
  for (int l = 0; l + 1 < kNpLevels; ++l) {
    if (w == 0) {
      const int cnt = sh.nodes[l];
      const int i0 = lane, i1 = lane + 64;
      const int m0 = i0 < cnt ? sh.node_len[l][i0] : 0, m1 = i1 < cnt ? sh.node_len[l][i1] : 0;
      const uint32_t c0 = i0 < cnt ? (m0 > kNpLeaf ? 2u : 1u) : 0u;
      const uint32_t c1 = i1 < cnt ? (m1 > kNpLeaf ? 2u : 1u) : 0u;
      const uint32_t s0 = wave_scan_dpp(c0), s1 = wave_scan_dpp(c1);
      const uint32_t t0 = lane_value(s0, 63), t1 = lane_value(s1, 63);
      auto emit = [&](int i, int m, uint32_t c, uint32_t e) {
        if (c == 0 || e + c > (uint32_t)kNpMaxLeaves) return;  // the bound never binds: leaves hold >= 64
        const int a = sh.node_lo[l][i];
        sh.node_pos[l][i] = (int)e;
        if (c == 2) {
          int h = m / 2;
          h -= h % 8;
          sh.node_lo[l + 1][e] = a;
          sh.node_len[l + 1][e] = h;
          sh.node_lo[l + 1][e + 1] = a + h;
          sh.node_len[l + 1][e + 1] = m - h;
        } else {
          sh.node_lo[l + 1][e] = a;
          sh.node_len[l + 1][e] = m;
        }
      };
      emit(i0, m0, c0, s0 - c0);
      emit(i1, m1, c1, t0 + s1 - c1);
      if (lane == 0) sh.nodes[l + 1] = (int)(t0 + t1 < (uint32_t)kNpMaxLeaves ? t0 + t1 : kNpMaxLeaves);
    }
    __syncthreads();
  }
  constexpr int L = kNpLevels - 1;
  const int leaves = sh.nodes[L];
  for (int q0 = 8 * w; q0 < leaves; q0 += 8 * kNpBufWaves) {  // uniform over the wave
    const int j = q0 + g;
    const bool has = j < leaves;
    const int llo = has ? sh.node_lo[L][j] : 0, llen = has ? sh.node_len[L][j] : 0;
    const int nb = llen >> 3;  // full 8-element rows of the leaf (every leaf here holds >= 8)
    const int64_t base = lo + llo + k;
    double v[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) v[t] = t < nb ? load(base + 8 * t) : 0.0;
    double r = v[0];
    if (nb > 0) visit(base, v[0]);
#pragma unroll
    for (int t = 1; t < 16; ++t) {
      if (t < nb) {
        r += v[t];
        visit(base + 8 * t, v[t]);
      }
    }
    r += __shfl_xor(r, 1);
    r += __shfl_xor(r, 2);
    r += __shfl_xor(r, 4);
    if (has && k == 0) {
      for (int i = 8 * nb; i < llen; ++i) {  // the leftovers, in order
        const double x = load(lo + llo + i);
        r += x;
        visit(lo + llo + i, x);
      }
      sh.val[L][j] = r;
    }
  }
  __syncthreads();
  for (int l = kNpLevels - 2; l >= 0; --l) {  // from the leaves up
    if (w == 0) {
      const int cnt = sh.nodes[l];
      for (int i = lane; i < cnt; i += 64) {
        const int p = sh.node_pos[l][i];
        const double a = sh.val[l + 1][p];
        sh.val[l][i] = sh.node_len[l][i] > kNpLeaf ? a + sh.val[l + 1][p + 1] : a;
      }
    }
    __syncthreads();
  }
  const double total = sh.val[0][0];
  __syncthreads();
  return total;
}

}  // namespace dsr
