// Device-side building blocks shared by the sampling kernels (gfx950, wave64).
//
// Every block-wide reduction here runs in a fixed order (xor butterflies
// inside a wave, then the per-wave partials summed in wave order), so a
// floating-point result is bit-reproducible from run to run.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dsr_sampling.h"

namespace dsr {

constexpr int kThreads = 1024;            // one workgroup per row
constexpr int kWaves = kThreads / 64;     // 16 wave64s

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// Scratch shared by the block primitives.  Every primitive writes its slot,
// barriers, reads, and barriers again, so calls can follow each other freely.
struct BlockScratch {
  double f64[kWaves];
  unsigned long long u64[kWaves];
  long long i64[kWaves];
  double bcast_f[4];
  long long bcast_i[4];
};

template <class T>
__device__ __forceinline__ T wave_sum(T x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

template <class T>
__device__ __forceinline__ T wave_max(T x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    T y = __shfl_xor(x, o);
    x = y > x ? y : x;
  }
  return x;
}

template <class T>
__device__ __forceinline__ T wave_min(T x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    T y = __shfl_xor(x, o);
    x = y < x ? y : x;
  }
  return x;
}

__device__ __forceinline__ double block_sum(double x, BlockScratch& s) {
  x = wave_sum(x);
  if (lane_id() == 0) s.f64[wave_id()] = x;
  __syncthreads();
  double r = 0.0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) r += s.f64[w];
  __syncthreads();
  return r;
}

__device__ __forceinline__ double block_max(double x, BlockScratch& s) {
  x = wave_max(x);
  if (lane_id() == 0) s.f64[wave_id()] = x;
  __syncthreads();
  double r = s.f64[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = s.f64[w] > r ? s.f64[w] : r;
  __syncthreads();
  return r;
}

__device__ __forceinline__ long long block_sum_i64(long long x, BlockScratch& s) {
  x = wave_sum(x);
  if (lane_id() == 0) s.i64[wave_id()] = x;
  __syncthreads();
  long long r = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) r += s.i64[w];
  __syncthreads();
  return r;
}

__device__ __forceinline__ long long block_min_i64(long long x, BlockScratch& s) {
  x = wave_min(x);
  if (lane_id() == 0) s.i64[wave_id()] = x;
  __syncthreads();
  long long r = s.i64[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = s.i64[w] < r ? s.i64[w] : r;
  __syncthreads();
  return r;
}

__device__ __forceinline__ long long block_max_i64(long long x, BlockScratch& s) {
  x = wave_max(x);
  if (lane_id() == 0) s.i64[wave_id()] = x;
  __syncthreads();
  long long r = s.i64[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = s.i64[w] > r ? s.i64[w] : r;
  __syncthreads();
  return r;
}

__device__ __forceinline__ int block_or(int x, BlockScratch& s) {
  return block_max_i64(x ? 1 : 0, s) != 0;
}

// Exclusive prefix sum over threads in thread order; `total` gets the sum.
__device__ __forceinline__ long long block_exclusive_scan_i64(long long x, BlockScratch& s, long long& total) {
  long long v = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    long long y = __shfl_up(v, o);
    if (lane_id() >= o) v += y;
  }
  if (lane_id() == 63) s.i64[wave_id()] = v;
  __syncthreads();
  long long base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    long long t = s.i64[w];
    base += w < wave_id() ? t : 0;
    tot += t;
  }
  __syncthreads();
  total = tot;
  return base + v - x;
}

// Exclusive prefix sum of doubles in thread order (fixed association order).
__device__ __forceinline__ double block_exclusive_scan_f64(double x, BlockScratch& s, double& total) {
  double v = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    double y = __shfl_up(v, o);
    if (lane_id() >= o) v += y;
  }
  if (lane_id() == 63) s.f64[wave_id()] = v;
  __syncthreads();
  double base = 0.0, tot = 0.0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    double t = s.f64[w];
    if (w < wave_id()) base += t;
    tot += t;
  }
  __syncthreads();
  total = tot;
  // v is the inclusive prefix inside the wave; drop this thread's own term.
  double incl = base + v;
  return incl - x;
}

// Order-preserving 64-bit key of a double: larger value -> larger key,
// -0.0 and +0.0 share one key (NumPy sorts them as equal).
__device__ __forceinline__ uint64_t order_key(double x) {
  uint64_t b = (x == 0.0) ? 0ull : (uint64_t)__double_as_longlong(x);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

__device__ __forceinline__ double key_value(uint64_t k) {
  uint64_t b = (k >> 63) ? (k & 0x7FFFFFFFFFFFFFFFull) : ~k;
  return __longlong_as_double((long long)b);
}

__device__ __forceinline__ double load_logit(const void* base, int dtype, int64_t off) {
  if (dtype == DSR_BF16) {
    uint32_t b = ((const uint16_t*)base)[off];
    return (double)__uint_as_float(b << 16);
  }
  if (dtype == DSR_F32) return (double)((const float*)base)[off];
  return ((const double*)base)[off];
}

__device__ __forceinline__ bool policy_ok(const dsr_policy_t& p) {
  // Bounds of SamplingPolicy.__post_init__ (sampling.py:38-43); NaN fails every test.
  return p.temperature >= 0.0 && p.temperature <= 100.0 && p.top_p >= 0.0 && p.top_p <= 1.0 &&
         p.min_p >= 0.0 && p.min_p <= 1.0 && p.repetition_penalty >= 0.01 && p.repetition_penalty <= 100.0 &&
         p.presence_penalty >= -2.0 && p.presence_penalty <= 2.0 && p.frequency_penalty >= -2.0 &&
         p.frequency_penalty <= 2.0 && p.top_k >= 0 && p.top_k <= DSR_MAX_VOCAB && p.reserved == 0;
}

}  // namespace dsr
