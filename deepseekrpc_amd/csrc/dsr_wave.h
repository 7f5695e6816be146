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

// Bit-level carriers so one template serves u32, i64 and f64.
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
// workgroup must make the same sequence of calls.
class BlockSync {
 public:
  __device__ explicit BlockSync(SyncSlots& s) : s_(s), ph_(0) {}

  template <class T, class Op>
  __device__ T reduce(T x, T identity, Op op) {
    T* slot = slots<T>();
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

  // Exclusive prefix over threads in thread order, and the workgroup total.
  template <class T>
  __device__ T scan(T x, T& total) {
    T* slot = slots<T>();
    const T incl = wave_scan_dpp(x);
    if (lane_id() == 63) slot[wave_id()] = incl;
    lds_barrier();
    T y = lane_id() < kWaves ? slot[lane_id()] : (T)0;
    const T wincl = row_scan_dpp(y);
    total = lane_value(wincl, kWaves - 1);
    const T base = lane_value(wincl - y, wave_id());
    return (base + incl) - x;
  }

  // Plain barrier that also advances the slot parity.
  __device__ void barrier() { lds_barrier(); }

 private:
  template <class T> __device__ T* slots();
  SyncSlots& s_;
  int ph_;
};

template <> __device__ __forceinline__ double* BlockSync::slots<double>() { ph_ ^= 1; return s_.f[ph_]; }
template <> __device__ __forceinline__ long long* BlockSync::slots<long long>() { ph_ ^= 1; return s_.i[ph_]; }
template <> __device__ __forceinline__ uint32_t* BlockSync::slots<uint32_t>() { ph_ ^= 1; return s_.u[ph_]; }

// k-th largest (1-based, k <= 64) of one 16-bit value per lane, by a bitwise
// search over ballots; the result is uniform across the wave.
__device__ __forceinline__ uint32_t wave_kth_largest_u16(uint32_t v, uint32_t k) {
  uint32_t prefix = 0;
#pragma unroll
  for (int b = 15; b >= 0; --b) {
    const uint32_t cand = prefix | (1u << b);
    const uint32_t n = (uint32_t)__popcll(__ballot(v >= cand));
    if (n >= k) prefix = cand;
  }
  return prefix;
}

// Adds `amount` to hist[bin] for every active lane, one LDS atomic per
// distinct bin in the wave (lanes sharing a bin are combined first).
__device__ __forceinline__ void hist_add_u32(uint32_t* hist, uint32_t bin, bool active) {
  unsigned long long todo = __ballot(active);
  while (todo) {
    const int leader = __ffsll((long long)todo) - 1;
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)bin, leader);
    const unsigned long long same = __ballot(active && bin == b);
    if (lane_id() == leader) atomicAdd(&hist[b], (uint32_t)__popcll(same));
    todo &= ~same;
  }
}

__device__ __forceinline__ void hist_add_u64(unsigned long long* hist, uint32_t bin, bool active,
                                             unsigned long long amount) {
  unsigned long long todo = __ballot(active);
  while (todo) {
    const int leader = __ffsll((long long)todo) - 1;
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)bin, leader);
    const bool mine = active && bin == b;
    const unsigned long long same = __ballot(mine);
    const long long part = wave_reduce_dpp((long long)(mine ? amount : 0ull), OpSum());
    if (lane_id() == leader) atomicAdd(&hist[b], (unsigned long long)part);
    todo &= ~same;
  }
}

}  // namespace dsr
