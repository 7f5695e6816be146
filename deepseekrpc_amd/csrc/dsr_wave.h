// Low-latency wave64 and workgroup primitives for gfx950 built on DPP.
//
// Wave reductions use quad_perm / row_half_mirror / row_mirror DPP moves
// inside each 16-lane row and v_readlane across the four rows; wave scans use
// row_shr and row_bcast:15 / row_bcast:31.  These are VALU modifiers, far
// cheaper than LDS-routed shuffles.  All functions must be called by every
// lane of the wave (full EXEC).  Association orders are fixed, so floating-
// point results are reproducible.
//
// BlockSync gives workgroup reductions and scans that cost one barrier each:
// partial results go to one of two alternating slot arrays, so a slot is
// never rewritten while another wave may still read it.
#pragma once

#include "dsr_common.h"

namespace dsr {

// Workgroup barrier that orders LDS only: outstanding global loads keep
// streaming into registers across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF, bool BOUND_CTRL = true>
__device__ __forceinline__ uint32_t dpp32(uint32_t old, uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)x, CTRL, ROW_MASK, BANK_MASK, BOUND_CTRL);
}

template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF, bool BOUND_CTRL = true>
__device__ __forceinline__ uint64_t dpp64(uint64_t old, uint64_t x) {
  const uint32_t lo = dpp32<CTRL, ROW_MASK, BANK_MASK, BOUND_CTRL>((uint32_t)old, (uint32_t)x);
  const uint32_t hi = dpp32<CTRL, ROW_MASK, BANK_MASK, BOUND_CTRL>((uint32_t)(old >> 32), (uint32_t)(x >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// Bit-level carriers so one template serves u32, i64, u64 and f64.
template <class T> struct Bits;
template <> struct Bits<uint32_t> {
  static __device__ __forceinline__ uint32_t to(uint32_t x) { return x; }
  static __device__ __forceinline__ uint32_t from(uint32_t x) { return x; }
  template <int C, int RM = 0xF, int BM = 0xF, bool BC = true>
  static __device__ __forceinline__ uint32_t dpp(uint32_t o, uint32_t x) { return dpp32<C, RM, BM, BC>(o, x); }
  static __device__ __forceinline__ uint32_t readlane(uint32_t x, int l) {
    return (uint32_t)__builtin_amdgcn_readlane((int)x, l);
  }
};
template <> struct Bits<long long> {
  static __device__ __forceinline__ uint64_t to(long long x) { return (uint64_t)x; }
  static __device__ __forceinline__ long long from(uint64_t x) { return (long long)x; }
  template <int C, int RM = 0xF, int BM = 0xF, bool BC = true>
  static __device__ __forceinline__ uint64_t dpp(uint64_t o, uint64_t x) { return dpp64<C, RM, BM, BC>(o, x); }
  static __device__ __forceinline__ uint64_t readlane(uint64_t x, int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), l);
    return ((uint64_t)hi << 32) | lo;
  }
};
template <> struct Bits<double> {
  static __device__ __forceinline__ uint64_t to(double x) { return (uint64_t)__double_as_longlong(x); }
  static __device__ __forceinline__ double from(uint64_t x) { return __longlong_as_double((long long)x); }
  template <int C, int RM = 0xF, int BM = 0xF, bool BC = true>
  static __device__ __forceinline__ uint64_t dpp(uint64_t o, uint64_t x) { return dpp64<C, RM, BM, BC>(o, x); }
  static __device__ __forceinline__ uint64_t readlane(uint64_t x, int l) { return Bits<long long>::readlane(x, l); }
};
template <> struct Bits<unsigned long long> {
  static __device__ __forceinline__ uint64_t to(unsigned long long x) { return (uint64_t)x; }
  static __device__ __forceinline__ unsigned long long from(uint64_t x) { return (unsigned long long)x; }
  template <int C, int RM = 0xF, int BM = 0xF, bool BC = true>
  static __device__ __forceinline__ uint64_t dpp(uint64_t o, uint64_t x) { return dpp64<C, RM, BM, BC>(o, x); }
  static __device__ __forceinline__ uint64_t readlane(uint64_t x, int l) { return Bits<long long>::readlane(x, l); }
};

template <class T, int C>
__device__ __forceinline__ T dpp_move(T x) {
  return Bits<T>::from(Bits<T>::template dpp<C>(0, Bits<T>::to(x)));
}

// Reduction inside each 16-lane row; every lane of the row ends with its row's result.
template <class T, class Op>
__device__ __forceinline__ T row_reduce(T x, Op op) {
  x = op(x, dpp_move<T, 0xB1>(x));   // quad_perm [1,0,3,2]
  x = op(x, dpp_move<T, 0x4E>(x));   // quad_perm [2,3,0,1]
  x = op(x, dpp_move<T, 0x141>(x));  // row_half_mirror
  x = op(x, dpp_move<T, 0x140>(x));  // row_mirror
  return x;
}

template <class T>
__device__ __forceinline__ T lane_value(T x, int l) {
  return Bits<T>::from(Bits<T>::readlane(Bits<T>::to(x), l));
}

// Whole-wave reduction; the (uniform) result is returned to every lane.
template <class T, class Op>
__device__ __forceinline__ T wave_reduce_dpp(T x, Op op) {
  x = row_reduce(x, op);
  return op(op(lane_value(x, 0), lane_value(x, 16)), op(lane_value(x, 32), lane_value(x, 48)));
}

// Inclusive prefix over the 64 lanes in lane order.
template <class T>
__device__ __forceinline__ T wave_scan_dpp(T v) {
  using B = Bits<T>;
  v = v + B::from(B::template dpp<0x111>(0, B::to(v)));        // row_shr:1
  v = v + B::from(B::template dpp<0x112>(0, B::to(v)));        // row_shr:2
  v = v + B::from(B::template dpp<0x114>(0, B::to(v)));        // row_shr:4
  v = v + B::from(B::template dpp<0x118>(0, B::to(v)));        // row_shr:8
  v = v + B::from(B::template dpp<0x142, 0xA>(0, B::to(v)));   // row_bcast:15 into rows 1, 3
  v = v + B::from(B::template dpp<0x143, 0xC>(0, B::to(v)));   // row_bcast:31 into rows 2, 3
  return v;
}

// Running maximum over the 64 lanes in lane order.
__device__ __forceinline__ double wave_maxscan_dpp(double v) {
  using B = Bits<double>;
  const double lo = -(double)INFINITY;
  const uint64_t lob = B::to(lo);
  v = fmax(v, B::from(B::template dpp<0x111, 0xF, 0xF, false>(lob, B::to(v))));
  v = fmax(v, B::from(B::template dpp<0x112, 0xF, 0xF, false>(lob, B::to(v))));
  v = fmax(v, B::from(B::template dpp<0x114, 0xF, 0xF, false>(lob, B::to(v))));
  v = fmax(v, B::from(B::template dpp<0x118, 0xF, 0xF, false>(lob, B::to(v))));
  v = fmax(v, B::from(B::template dpp<0x142, 0xA, 0xF, false>(lob, B::to(v))));
  v = fmax(v, B::from(B::template dpp<0x143, 0xC, 0xF, false>(lob, B::to(v))));
  return v;
}

// Inclusive prefix inside each 16-lane row only.
template <class T>
__device__ __forceinline__ T row_scan_dpp(T v) {
  using B = Bits<T>;
  v = v + B::from(B::template dpp<0x111>(0, B::to(v)));
  v = v + B::from(B::template dpp<0x112>(0, B::to(v)));
  v = v + B::from(B::template dpp<0x114>(0, B::to(v)));
  v = v + B::from(B::template dpp<0x118>(0, B::to(v)));
  return v;
}

struct SyncSlots {
  double f[2][kWaves];
  long long i[2][kWaves];
  uint32_t u[2][kWaves];
};

// Workgroup reductions / scans with one barrier each.  Every thread of the
// workgroup must make the same sequence of calls.  Each call takes the slot
// set of the next parity, so a wave that runs ahead into the next call never
// overwrites slots that a slower wave is still reading.
class BlockSync {
 public:
  __device__ explicit BlockSync(SyncSlots& s) : s_(s), ph_(0) {}

  template <class T, class Op>
  __device__ T reduce(T x, T identity, Op op) {
    T* slot = slots<T>(next());
    x = wave_reduce_dpp(x, op);
    if (lane_id() == 0) slot[wave_id()] = x;
    lds_barrier();
    T y = lane_id() < kWaves ? slot[lane_id()] : identity;
    y = row_reduce(y, op);
    return lane_value(y, 0);
  }

  __device__ double sum(double x) { return reduce(x, 0.0, OpSum()); }
  __device__ long long sum(long long x) { return reduce(x, 0ll, OpSum()); }
  __device__ long long max(long long x) { return reduce(x, LLONG_MIN, OpMax()); }
  __device__ long long min(long long x) { return reduce(x, LLONG_MAX, OpMin()); }
  __device__ uint32_t max(uint32_t x) { return reduce(x, 0u, OpMax()); }
  __device__ uint32_t min(uint32_t x) { return reduce(x, 0xFFFFFFFFu, OpMin()); }
  __device__ uint32_t sum(uint32_t x) { return reduce(x, 0u, OpSum()); }

  // The sum of a 64-bit integer and the maximum of a double behind one barrier.
  __device__ void sum_max(long long& s, double& m) {
    const int p = next();
    long long* si = s_.i[p];
    double* sf = s_.f[p];
    const long long ws = wave_reduce_dpp(s, OpSum());
    const double wm = wave_reduce_dpp(m, OpMax());
    if (lane_id() == 0) {
      si[wave_id()] = ws;
      sf[wave_id()] = wm;
    }
    lds_barrier();
    const long long a = lane_id() < kWaves ? si[lane_id()] : 0ll;
    const double b = lane_id() < kWaves ? sf[lane_id()] : -(double)INFINITY;
    s = lane_value(row_reduce(a, OpSum()), 0);
    m = lane_value(row_reduce(b, OpMax()), 0);
  }

  // Exclusive prefix over threads in thread order, and the workgroup total.
  template <class T>
  __device__ T scan(T x, T& total) {
    T* slot = slots<T>(next());
    const T incl = wave_scan_dpp(x);
    if (lane_id() == 63) slot[wave_id()] = incl;
    lds_barrier();
    T y = lane_id() < kWaves ? slot[lane_id()] : (T)0;
    const T wincl = row_scan_dpp(y);
    total = lane_value(wincl, kWaves - 1);
    const T base = lane_value(wincl - y, wave_id());
    return (base + incl) - x;
  }

  // Exclusive prefix of x in thread order (with its total) and the sum of y,
  // behind one barrier.
  __device__ uint32_t scan_sum(uint32_t x, double y, uint32_t& xtotal, double& ysum) {
    const int p = next();
    uint32_t* su = s_.u[p];
    double* sf = s_.f[p];
    const uint32_t incl = wave_scan_dpp(x);
    const double ws = wave_reduce_dpp(y, OpSum());
    if (lane_id() == 63) su[wave_id()] = incl;
    if (lane_id() == 0) sf[wave_id()] = ws;
    lds_barrier();
    const uint32_t u = lane_id() < kWaves ? su[lane_id()] : 0u;
    const uint32_t wincl = row_scan_dpp(u);
    xtotal = lane_value(wincl, kWaves - 1);
    const uint32_t base = lane_value(wincl - u, wave_id());
    double f = lane_id() < kWaves ? sf[lane_id()] : 0.0;
    f = row_reduce(f, OpSum());
    ysum = lane_value(f, 0);
    return base + incl - x;
  }

  // Exclusive prefixes (thread order) of a 64-bit and a 32-bit integer, with
  // their totals, behind one barrier.  Integer sums are exact, so the
  // intervals [ex, ex + x) tile [0, total) exactly.
  __device__ long long scan2(long long a, uint32_t b, long long& atotal, uint32_t& bex, uint32_t& btotal) {
    const int p = next();
    long long* si = s_.i[p];
    uint32_t* su = s_.u[p];
    const long long ai = wave_scan_dpp(a);
    const uint32_t bi = wave_scan_dpp(b);
    if (lane_id() == 63) {
      si[wave_id()] = ai;
      su[wave_id()] = bi;
    }
    lds_barrier();
    const long long ya = lane_id() < kWaves ? si[lane_id()] : 0ll;
    const uint32_t yb = lane_id() < kWaves ? su[lane_id()] : 0u;
    const long long wa = row_scan_dpp(ya);
    const uint32_t wb = row_scan_dpp(yb);
    atotal = lane_value(wa, kWaves - 1);
    btotal = lane_value(wb, kWaves - 1);
    bex = lane_value(wb - yb, wave_id()) + bi - b;
    return lane_value(wa - ya, wave_id()) + ai - a;
  }

  // scan2 with an unsigned 64-bit first operand (sums up to 2^64 - 1).
  __device__ unsigned long long scan2u(unsigned long long a, uint32_t b, unsigned long long& atotal, uint32_t& bex,
                                       uint32_t& btotal) {
    const int p = next();
    long long* si = s_.i[p];
    uint32_t* su = s_.u[p];
    const unsigned long long ai = wave_scan_dpp(a);
    const uint32_t bi = wave_scan_dpp(b);
    if (lane_id() == 63) {
      si[wave_id()] = (long long)ai;
      su[wave_id()] = bi;
    }
    lds_barrier();
    const unsigned long long ya = lane_id() < kWaves ? (unsigned long long)si[lane_id()] : 0ull;
    const uint32_t yb = lane_id() < kWaves ? su[lane_id()] : 0u;
    const unsigned long long wa = row_scan_dpp(ya);
    const uint32_t wb = row_scan_dpp(yb);
    atotal = lane_value(wa, kWaves - 1);
    btotal = lane_value(wb, kWaves - 1);
    bex = lane_value(wb - yb, wave_id()) + bi - b;
    return lane_value(wa - ya, wave_id()) + ai - a;
  }

  // Index-order CDF of non-negative x behind one barrier.  Returns this
  // thread's inclusive value; `ex` is exactly the previous thread's inclusive
  // value (0 for thread 0), so the intervals [ex, inc) tile [0, total)
  // without gaps or overlaps.  inc never decreases in thread order (a running
  // maximum removes the ulp-level dips of the tree-shaped scan) and threads
  // with x == 0 get empty intervals.  Wave bases are summed sequentially, in
  // the same order in every lane.  Also returns the workgroup sum of `tally`.
  __device__ double cdf_scan(double x, double& ex, double& total, uint32_t tally, uint32_t& tally_sum) {
    const int p = next();
    double* sf = s_.f[p];
    uint32_t* su = s_.u[p];
    double incl = wave_scan_dpp(x);
    incl = x > 0.0 ? incl : -(double)INFINITY;
    incl = fmax(wave_maxscan_dpp(incl), 0.0);
    const uint32_t tw = wave_reduce_dpp(tally, OpSum());
    if (lane_id() == 63) sf[wave_id()] = incl;
    if (lane_id() == 0) su[wave_id()] = tw;
    lds_barrier();
    double base = 0.0, mine = 0.0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      if (w == wave_id()) mine = base;
      base = base + sf[w];
    }
    total = base;
    uint32_t u = lane_id() < kWaves ? su[lane_id()] : 0u;
    u = row_reduce(u, OpSum());
    tally_sum = lane_value(u, 0);
    double prev = __shfl_up(incl, 1);
    ex = lane_id() == 0 ? mine : mine + prev;
    return mine + incl;
  }

 private:
  __device__ int next() { ph_ ^= 1; return ph_; }
  template <class T> __device__ T* slots(int p);
  SyncSlots& s_;
  int ph_;
};

template <> __device__ __forceinline__ double* BlockSync::slots<double>(int p) { return s_.f[p]; }
template <> __device__ __forceinline__ long long* BlockSync::slots<long long>(int p) { return s_.i[p]; }
template <> __device__ __forceinline__ uint32_t* BlockSync::slots<uint32_t>(int p) { return s_.u[p]; }

// Position of this lane among the set lanes of a ballot.
__device__ __forceinline__ uint32_t lanes_below(unsigned long long b) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
}

// ---------------------------------------------------------------------------
// Workgroup reductions and scans over BlockScratch slots.  Each call is
// bracketed by full barriers (__syncthreads, which also orders global
// memory): the workspace passes that call them re-read rows other threads
// wrote.  The wave parts run on DPP.

template <class T>
__device__ __forceinline__ T wave_sum(T x) { return wave_reduce_dpp(x, OpSum()); }

template <class T, class Op>
__device__ __forceinline__ T block_reduce(T x, T* slot, T identity, Op op) {
  x = wave_reduce_dpp(x, op);
  if (lane_id() == 0) slot[wave_id()] = x;
  __syncthreads();
  T y = lane_id() < kWaves ? slot[lane_id()] : identity;
  y = row_reduce(y, op);
  const T r = lane_value(y, 0);
  __syncthreads();
  return r;
}

__device__ __forceinline__ double block_sum(double x, BlockScratch& s) {
  return block_reduce(x, s.f64, 0.0, OpSum());
}

__device__ __forceinline__ double block_max(double x, BlockScratch& s) {
  return block_reduce(x, s.f64, -(double)INFINITY, OpMax());
}

__device__ __forceinline__ long long block_sum_i64(long long x, BlockScratch& s) {
  return block_reduce(x, s.i64, 0ll, OpSum());
}

__device__ __forceinline__ long long block_min_i64(long long x, BlockScratch& s) {
  return block_reduce(x, s.i64, LLONG_MAX, OpMin());
}

__device__ __forceinline__ long long block_max_i64(long long x, BlockScratch& s) {
  return block_reduce(x, s.i64, LLONG_MIN, OpMax());
}

__device__ __forceinline__ int block_or(int x, BlockScratch& s) {
  return block_max_i64(x ? 1 : 0, s) != 0;
}

// Exclusive prefix over threads in thread order (fixed association order);
// `total` gets the workgroup total.
template <class T>
__device__ __forceinline__ T block_exclusive_scan(T x, T* slot, T& total) {
  const T v = wave_scan_dpp(x);
  if (lane_id() == 63) slot[wave_id()] = v;
  __syncthreads();
  const T y = lane_id() < kWaves ? slot[lane_id()] : (T)0;
  const T wincl = row_scan_dpp(y);
  total = lane_value(wincl, kWaves - 1);
  const T base = lane_value(wincl - y, wave_id());
  __syncthreads();
  return (base + v) - x;
}

__device__ __forceinline__ long long block_exclusive_scan_i64(long long x, BlockScratch& s, long long& total) {
  return block_exclusive_scan(x, s.i64, total);
}

__device__ __forceinline__ double block_exclusive_scan_f64(double x, BlockScratch& s, double& total) {
  return block_exclusive_scan(x, s.f64, total);
}

}  // namespace dsr
