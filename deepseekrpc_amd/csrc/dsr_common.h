// Device-side building blocks shared by the sampling kernels (gfx950, wave64).
//
// Every block-wide reduction here runs in a fixed order (xor butterflies
// inside a wave, then the 16 per-wave partials combined by a butterfly over
// lanes 0..15), so a floating-point result is bit-reproducible from run to
// run.  The cross-wave step reads one partial per lane, which keeps register
// pressure low in kernels that hold a whole row in VGPRs.
#pragma once

#include <hip/hip_runtime.h>
#include <limits.h>
#include <math.h>
#include <stdint.h>

#include "dsr_sampling.h"

namespace dsr {

constexpr int kThreads = 1024;            // one workgroup per row
constexpr int kWaves = kThreads / 64;     // 16 wave64s

// Doubles per workspace row: the vocabulary rounded up to 32 tokens.
__host__ __device__ inline int64_t ws_stride(int64_t V) { return (V + 31) & ~(int64_t)31; }

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// Scratch shared by the block primitives.  Every primitive writes its slot,
// barriers, reads, and barriers again, so calls can follow each other freely.
struct BlockScratch {
  double f64[kWaves];
  long long i64[kWaves];
  double bcast_f[4];
  long long bcast_i[4];
};

struct OpSum {
  template <class T> __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct OpMax {
  template <class T> __device__ __forceinline__ T operator()(T a, T b) const { return b > a ? b : a; }
};
struct OpMin {
  template <class T> __device__ __forceinline__ T operator()(T a, T b) const { return b < a ? b : a; }
};
struct OpOr {
  template <class T> __device__ __forceinline__ T operator()(T a, T b) const { return a | b; }
};

// Order-preserving 64-bit key of a double: larger value -> larger key,
// -0.0 and +0.0 share one key (NumPy sorts them as equal).
__device__ __forceinline__ uint64_t order_key(double x) {
  uint64_t b = (x == 0.0) ? 0ull : (uint64_t)__double_as_longlong(x);
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

__device__ __forceinline__ double load_logit(const void* base, int dtype, int64_t off) {
  if (dtype == DSR_BF16) {
    uint32_t b = ((const uint16_t*)base)[off];
    return (double)__uint_as_float(b << 16);
  }
  if (dtype == DSR_F32) return (double)((const float*)base)[off];
  return ((const double*)base)[off];
}

// 2^(j/64), j = 0..63, correctly rounded (computed in 50-digit decimal arithmetic).
__device__ const double kExp2Frac[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0};

// exp(z) for float64 z <= 0 by Tang's table-driven method (P. T. P. Tang,
// "Table-driven implementation of the exponential function in IEEE
// floating-point arithmetic", ACM TOMS 15(2), 1989): z = (64m + j) ln2/64 + r
// with |r| <= ln2/128 (Cody-Waite reduction, ln2/64 split so that k * hi is
// exact), exp(z) = 2^m * 2^(j/64) * p(r), p the degree-5 Taylor polynomial of
// exp (truncation below 2^-54 relative).  `tab` holds 2^(j/64), j = 0..63
// (exp_table_init copies kExp2Frac).  Relative error a few ulps; z = -inf gives 0.  Used where
// a decision is certified with a tolerance far above that, never where the
// reference's own float64 exp must be mirrored.
__device__ __forceinline__ void exp_table_init(double* tab) {
  for (int j = threadIdx.x; j < 64; j += blockDim.x) tab[j] = kExp2Frac[j];
}

__device__ __forceinline__ double exp_nonpos(double z, const double* tab) {
  const double kInvL = 92.33248261689366;        // 64 / ln 2
  const double kLhi = 0x1.62e42ff000000p-7;      // ln 2 / 64, leading 29 bits
  const double kLlo = -0x1.718432a1b0e26p-41;    // ln 2 / 64 - kLhi
  z = fmax(z, -746.0);                           // below -745.14 the result underflows to 0
  const double kd = rint(z * kInvL);
  const int k = (int)kd;
  double r = fma(-kd, kLhi, z);
  r = fma(-kd, kLlo, r);
  double p = fma(1.0 / 120.0, r, 1.0 / 24.0);
  p = fma(p, r, 1.0 / 6.0);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  return ldexp(tab[k & 63] * p, k >> 6);
}

// One Generator.random() of NumPy's PCG64 bit generator (O'Neill's PCG
// family: a 128-bit linear congruential state with the XSL-RR output, as
// numpy/random/src/pcg64 implements it): s <- s * M + inc (mod 2^128),
// x = hi(s) ^ lo(s), out = rotr64(x, hi(s) >> 58), u = (out >> 11) * 2^-53.
// st holds s and inc as little-endian 128-bit integers (lo, hi, inc lo,
// inc hi); next receives the advanced state in the same layout.
__device__ __forceinline__ double pcg64_random(const uint64_t* st, uint64_t next[4]) {
  const unsigned __int128 M = ((unsigned __int128)0x2360ED051FC65DA4ull << 64) | 0x4385DF649FCCF645ull;
  const unsigned __int128 inc = ((unsigned __int128)st[3] << 64) | st[2];
  unsigned __int128 s = ((unsigned __int128)st[1] << 64) | st[0];
  s = s * M + inc;
  const uint64_t hi = (uint64_t)(s >> 64), lo = (uint64_t)s;
  const uint32_t rot = (uint32_t)(hi >> 58);
  const uint64_t x = hi ^ lo;
  const uint64_t out = (x >> rot) | (x << ((64u - rot) & 63u));
  next[0] = lo;
  next[1] = hi;
  next[2] = st[2];
  next[3] = st[3];
  return (double)(out >> 11) * 0x1.0p-53;
}

// The first n draws of a PCG64 state, in order (n <= 8); the state itself is
// left as it is.
__device__ __forceinline__ void pcg64_draws(const uint64_t* st, int n, double* u) {
  uint64_t cur[4] = {st[0], st[1], st[2], st[3]}, next[4];
  for (int i = 0; i < n && i < 8; ++i) {
    u[i] = pcg64_random(cur, next);
    cur[0] = next[0];
    cur[1] = next[1];
  }
}

// Advances a PCG64 state in place by n draws (one thread).
__device__ __forceinline__ void pcg64_advance(uint64_t* st, int n) {
  uint64_t cur[4] = {st[0], st[1], st[2], st[3]}, next[4];
  for (int i = 0; i < n; ++i) {
    pcg64_random(cur, next);
    cur[0] = next[0];
    cur[1] = next[1];
  }
  if (n > 0) {
    st[0] = cur[0];
    st[1] = cur[1];
  }
}

// A row's draw source: its PCG64 state (rng_state) in the kernels
// instantiated with RNG = true (launched when the caller gives states), else
// its pre-drawn uniform.
template <bool RNG>
__device__ __forceinline__ bool has_draws(const dsr_sample_args_t& a) { return RNG || a.uniforms; }

__device__ __forceinline__ void store_rng(const dsr_sample_args_t& a, int64_t row, const uint64_t next[4]) {
  uint64_t* o = a.rng_state + 4 * row;
  o[0] = next[0];
  o[1] = next[1];
}

__device__ __forceinline__ bool policy_ok(const dsr_policy_t& p) {
  // Bounds of SamplingPolicy.__post_init__ (sampling.py:38-43); NaN fails every test.
  return p.temperature >= 0.0 && p.temperature <= 100.0 && p.top_p >= 0.0 && p.top_p <= 1.0 &&
         p.min_p >= 0.0 && p.min_p <= 1.0 && p.repetition_penalty >= 0.01 && p.repetition_penalty <= 100.0 &&
         p.presence_penalty >= -2.0 && p.presence_penalty <= 2.0 && p.frequency_penalty >= -2.0 &&
         p.frequency_penalty <= 2.0 && p.top_k >= 0 && p.top_k <= DSR_MAX_VOCAB && p.reserved == 0;
}

}  // namespace dsr
