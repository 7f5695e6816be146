// Kernels and C ABI of the token-sampling hot path (gfx950).
//
//   dsr_sample_rows    -> SamplingPolicy.probabilities + categorical
//                         (sampling.py:48-128), one workgroup per row; fp32 /
//                         f64 top-k rows are first cut into slices, one
//                         workgroup each (dsr_split.h).
//   dsr_verify_drafts  -> SamplingWork.verify -> verify_drafts
//                         (terminal_sampling.py:170-183, sampling.py:247-294):
//                         one workgroup per conditional distribution, then
//                         one per request for the sequential accept chain.
//   dsr_prob_*         -> categorical / correction_distribution / the accept
//                         test on float64 probability vectors.
//   dsr_vocab_head     -> the terminal stage's vocabulary projection and its
//                         finiteness check (stage_graph.py:356-362), with the
//                         verifier's per-row statistics in the epilogue
//                         (dsr_head.h); dsr_verify_drafts_head reads them.
#include <hip/hip_runtime.h>
#include <limits.h>
#include <mutex>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "dsr_f32.h"
#include "dsr_fast.h"
#include "dsr_topk.h"
#include "dsr_full.h"
#include "dsr_general.h"
#include "dsr_head.h"
#include "dsr_history.h"
#include "dsr_numpy.h"
#include "dsr_split.h"
#include "dsr_verify.h"

namespace dsr {

static_assert(DSR_MAX_VOCAB <= kNpMaxLength, "NumPy-order sums cover at most 16 buffers");

// ---------------------------------------------------------------------------
// dsr_sample_rows: general path.

// W[0, n) holds the final probabilities; position j is token map(j).
template <bool RNG, class Map = IdentityMap>
__device__ __forceinline__ void finish_row(const dsr_sample_args_t& a, int64_t row, const double* W, int64_t n, int st,
                                           const DistOut& d, unsigned flags, GenShared& sh, Map map = Map()) {
  int64_t token = -1;
  int consumed = 0;
  if (st == DSR_OK && has_draws<RNG>(a)) {
    if (d.npos == 1) {
      token = d.first;  // sampling.py:120-122: no uniform is drawn
    } else {
      uint64_t next[4];
      const double u = RNG ? pcg64_random(a.rng_state + 4 * row, next) : a.uniforms[row];
      if (!(u >= 0.0 && u < 1.0)) {
        st = DSR_E_UNIFORM;
      } else {
        token = cdf_search(W, n, u, d.npos, sh, flags);
        if (token >= 0) token = map(token);
        consumed = 1;
      }
      if (RNG) {
        __syncthreads();  // every thread has read the state
        if (threadIdx.x == 0) store_rng(a, row, next);
      }
    }
  }
  if (threadIdx.x == 0) {
    a.out_token[row] = st == DSR_OK ? (int32_t)token : -1;
    a.out_consumed[row] = (uint8_t)(st == DSR_OK ? consumed : 0);
    a.out_status[row] = st;
    if (a.out_flags) a.out_flags[row] = (uint8_t)flags;
  }
}

__device__ __forceinline__ RowSpec sample_row_spec(const dsr_sample_args_t& a, int64_t row, double* W) {
  RowSpec r;
  r.V = a.vocab;
  r.dtype = a.dtype;
  const size_t esz = a.dtype == DSR_BF16 ? 2 : (a.dtype == DSR_F32 ? 4 : 8);
  r.logits = (const char*)a.logits + (size_t)row * (size_t)a.ld * esz;
  r.pol = a.policy[row];
  r.pen_n = 0;
  r.pen_ids = r.pen_count = r.pen_gen = nullptr;
  if (a.pen_off) {
    int64_t o = a.pen_off[row];
    r.pen_n = a.pen_off[row + 1] - o;
    r.pen_ids = a.pen_ids + o;
    r.pen_count = a.pen_count + o;
    r.pen_gen = a.pen_gen + o;
  }
  r.prefix = nullptr;
  r.prefix_n = 0;
  r.bias_n = 0;
  r.bias_ids = nullptr;
  r.bias_val = nullptr;
  if (a.bias_off) {
    int64_t o = a.bias_off[row];
    r.bias_n = a.bias_off[row + 1] - o;
    r.bias_ids = a.bias_ids + o;
    r.bias_val = a.bias_val + o;
  }
  r.allow = a.allow_bits ? a.allow_bits + row * a.allow_ld : nullptr;
  r.W = W;
  r.kept_bits = a.out_kept_bits ? a.out_kept_bits + row * a.kept_ld : nullptr;
  r.kept_words = (a.vocab + 31) >> 5;
  r.probs_f32 = a.out_probs_f32 ? a.out_probs_f32 + row * a.probs_ld : nullptr;
  r.probs_f64 = a.out_probs_f64 ? a.out_probs_f64 + row * a.probs_ld : nullptr;
  return r;
}

template <bool RNG>
__global__ __launch_bounds__(kThreads) void k_sample_general(dsr_sample_args_t a) {
  __shared__ GenShared sh;
  const int64_t row = blockIdx.x;
  double* W = (double*)a.workspace + row * ws_stride(a.vocab);
  RowSpec r = sample_row_spec(a, row, W);
  unsigned flags = DSR_FLAG_GENERAL;
  DistOut d;
  int st = general_distribution(r, sh, flags, d);
  finish_row<RNG>(a, row, W, a.vocab, st, d, flags, sh);
}

// Split-row path, stage two: one workgroup per row finishes from the slices'
// candidates, or redoes the row on the general path in the same workgroup.
template <bool RNG>
__global__ __launch_bounds__(kThreads) void k_split_finish(dsr_sample_args_t a, int smax) {
  __shared__ GenShared sh;
  __shared__ double cz[kSplitCap];   // the candidates' values, then (v - max) / T
  __shared__ double kz[kSplitMaxK];  // the kept tokens' values, then probabilities, in index order
  __shared__ int32_t kid[kSplitMaxK];
  const int64_t row = blockIdx.x;
  double* W = (double*)a.workspace + row * ws_stride(a.vocab);
  RowSpec r = sample_row_spec(a, row, W);
  unsigned flags = DSR_FLAG_GENERAL;
  SplitGeom g;
  const bool split = split_geom(r.pol, a.vocab, smax, row_plain(a, row), g);
  if (split && g.nof) {
    int why = 0;
    if (split_no_filter<RNG>(a, row, r, g, sh, why)) return;
    __syncthreads();
    flags |= (unsigned)why << 4;
  } else if (split) {
    unsigned sflags = DSR_FLAG_SPLIT;
    DistOut d;
    int64_t n = 0;
    int why = 0;
    const int st = split_distribution(r, g, sh, cz, kz, kid, sflags, d, n, why);
    if (st >= 0) {
      finish_row<RNG>(a, row, kz, n, st, d, sflags, sh, [](int64_t j) { return (int64_t)kid[j]; });
      return;
    }
    __syncthreads();  // every thread is done with the candidate list
    flags |= (unsigned)why << 4;
  }
  DistOut d;
  int st = general_distribution(r, sh, flags, d);
  finish_row<RNG>(a, row, W, a.vocab, st, d, flags, sh);
}

// One-workgroup FP32 top-k path; rows it does not take are redone by the
// general path inside the same workgroup.
template <bool RNG>
__global__ __launch_bounds__(kThreads) void k_sample_f32(dsr_sample_args_t a, const dsr_head_part_t* parts) {
  __shared__ F32Shared sh;
  const int64_t row = blockIdx.x;
  double* W = (double*)a.workspace + row * ws_stride(a.vocab);
  RowSpec r = sample_row_spec(a, row, W);
  unsigned flags = DSR_FLAG_F32_TOPK;
  DistOut d;
  int64_t n = 0;
  int why = 0;
  int st = kHeadFull;
  if (parts) {
    st = f32_distribution_head(a, row, parts, r, sh, flags, d, n, why);
    if (st == kHeadFull) __syncthreads();  // the records' pass is done with LDS
  }
  if (st == kHeadFull) st = f32_distribution(a, row, r, sh, flags, d, n, why);
  if (st == kDecided) return;  // a short list's wave wrote the outputs
  if (st >= 0) {
    const int32_t* kid = sh.t.kid;
    finish_row<RNG>(a, row, sh.t.kz, n, st, d, flags, sh.gen, [kid](int64_t j) { return (int64_t)kid[j]; });
    return;
  }
  __syncthreads();  // every thread is done with the list
  flags = DSR_FLAG_GENERAL | ((unsigned)why << 4);
  DistOut dg;
  const int sg = general_distribution(r, sh.gen, flags, dg);
  finish_row<RNG>(a, row, W, a.vocab, sg, dg, flags, sh.gen);
}

// Zeroes [0, V) of each probability row of a dsr_sample_rows call ahead of
// k_sample_f32, which writes only the kept tokens' entries: the rows are
// spread over the whole chip (a row of 129,280 float64 probabilities is a
// megabyte, about 40 us for the one workgroup that samples it).
constexpr int kZeroChunk = 4096;
constexpr int kZeroThreads = 256;

__global__ __launch_bounds__(kZeroThreads) void k_zero_probs(float* f32, double* f64, int64_t ld, int64_t V,
                                                             int chunks) {
  const int64_t r = blockIdx.x / chunks;
  const int64_t lo = (int64_t)(blockIdx.x % chunks) * kZeroChunk;
  const int64_t hi = lo + kZeroChunk < V ? lo + kZeroChunk : V;
  for (int64_t i = lo + threadIdx.x; i < hi; i += kZeroThreads) {
    if (f32) f32[r * ld + i] = 0.0f;
    if (f64) f64[r * ld + i] = 0.0;
  }
}

// Fast path for bf16 rows; rows it does not take are redone by the general
// path inside the same workgroup.
template <bool RNG>
__global__ __launch_bounds__(kThreads) void k_sample_bf16_fast(dsr_sample_args_t a) {
  __shared__ TopkShared sh;
  const int64_t row = blockIdx.x;
  const int why = topk_sample_row<RNG>(a, row, sh);
  // A whole row under kModeDeferWhole is the next launch's (k_sample_bf16_full).
  if (why == 0 || (why == kHandTopK && (a.hints & kModeDeferWhole))) return;
  __syncthreads();
  GenShared& gs = *reinterpret_cast<GenShared*>(&sh);
  double* W = (double*)a.workspace + row * ws_stride(a.vocab);
  RowSpec r = sample_row_spec(a, row, W);
  unsigned flags = DSR_FLAG_GENERAL | ((unsigned)why << 4);
  DistOut d;
  int st = general_distribution(r, gs, flags, d);
  finish_row<RNG>(a, row, W, a.vocab, st, d, flags, gs);
}

// Full-vocabulary path for bf16 rows that carry a token history (no bias);
// rows it does not take are redone by the general path in the same workgroup.
struct FullKernelShared {
  union {
    FullShared f;
    GenShared g;
  };
};

template <bool RNG>
__global__ __launch_bounds__(kThreads) void k_sample_bf16_full(dsr_sample_args_t a) {
  __shared__ FullKernelShared sh;
  const int64_t row = blockIdx.x;
  // After the top-k register kernel: only the rows it left (uniform; read
  // before the row's loads are issued, so other rows cost no HBM traffic).
  if ((a.hints & kModeOnlyWhole) && !whole_row(a.policy[row].temperature, a.policy[row].top_k, a.vocab)) return;
  const int why = full_sample_row<RNG>(a, row, sh.f);
  if (why == 0) return;
  __syncthreads();
  double* W = (double*)a.workspace + row * ws_stride(a.vocab);
  RowSpec r = sample_row_spec(a, row, W);
  unsigned flags = DSR_FLAG_GENERAL | ((unsigned)why << 4);
  DistOut d;
  int st = general_distribution(r, sh.g, flags, d);
  finish_row<RNG>(a, row, W, a.vocab, st, d, flags, sh.g);
}

// ---------------------------------------------------------------------------
// Probability-vector kernels (single workgroup).

__device__ __forceinline__ void prob_stats_row(const double* p, int64_t n, double* out_sum, int32_t* out,
                                               GenShared& sh, NpSumShared& np) {
  int bad = 0;
  long long npos = 0, first = LLONG_MAX;
  RowMax mx;  // every thread visits its elements in increasing index order
  // The sum the reference tests against 1 +- 1e-10 (sampling.py:111-113), in
  // NumPy's order, with the other statistics taken from the same loads.
  const double s = np_sum([&](int64_t i) { return p[i]; }, n, np, [&](int64_t i, double x) {
    if (!isfinite(x) || x < 0.0) bad = 1;
    if (x > 0.0) {
      ++npos;
      if (i < first) first = i;
    }
    mx.add(i, x);
  });
  bad = block_or(bad, sh.b);
  npos = block_sum_i64(npos, sh.b);
  first = block_min_i64(first, sh.b);
  const double M = block_max(mx.m, sh.b);
  const long long am = block_min_i64(mx.m == M ? mx.first : LLONG_MAX, sh.b);
  if (threadIdx.x == 0) {
    out_sum[0] = s;
    out[0] = bad ? 0 : 1;
    out[1] = (int32_t)npos;
    out[2] = first == LLONG_MAX ? -1 : (int32_t)first;
    out[3] = am == LLONG_MAX ? -1 : (int32_t)am;
  }
}

__global__ __launch_bounds__(kThreads) void k_prob_stats(const double* p, int64_t n, double* out_sum,
                                                         int32_t* out) {
  __shared__ GenShared sh;
  __shared__ NpSumShared np;
  prob_stats_row(p, n, out_sum, out, sh, np);
}

// Up to DSR_STATS_MAX_ROWS vectors at once, one workgroup each: row r's
// statistics go to out[3 r] (the sum) and out[3 r + 1 .. 3 r + 2] (the four
// int32 results).
struct StatsRows {
  const double* p[DSR_STATS_MAX_ROWS];
};

__global__ __launch_bounds__(kThreads) void k_prob_stats_rows(StatsRows r, int64_t n, double* out) {
  __shared__ GenShared sh;
  __shared__ NpSumShared np;
  const int row = blockIdx.x;
  prob_stats_row(r.p[row], n, out + 3 * row, (int32_t*)(out + 3 * row + 1), sh, np);
}

// First i with c_i / c_last > u for the sequential running sum c of the
// vector p(0 .. n-1) (np.cumsum, then searchsorted "right";
// sampling.py:126-128), by one lane.
template <class F>
__device__ int64_t sequential_cdf_search(F p, int64_t n, double u) {
  double last = 0.0;
  for (int64_t i = 0; i < n; ++i) last += p(i);
  double c = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    c += p(i);
    if (c / last > u) return i;
  }
  return n - 1;  // not reached: c_last / c_last = 1 > u
}

// categorical (sampling.py:118-128) over one float64 vector p(0 .. n-1), one
// workgroup.  Wave w owns elements [8192 w, 8192 (w + 1)) as 16 chunks of
// 512.  One coalesced pass gives every chunk's sum (8 strided loads per lane,
// then a wave sum) and the positive count; the crossing of u * total is then
// found by wave, by chunk, and inside the chunk by its wave's running scan.
// These sums take another order than np.cumsum: where u sits within that
// rounding band of a cell edge (or no crossing shows), the sequential sum
// decides.  Every thread gets the token and the flags.
constexpr int kCatChunk = 512;
constexpr int kCatChunks = 16;
static_assert((int64_t)kWaves * kCatChunks * kCatChunk >= DSR_MAX_VOCAB, "one workgroup covers the vocabulary");

struct CatShared {
  double csum[kWaves][kCatChunks];
  double wsum[kWaves];
  long long wpos[kWaves];
  long long found[2];
};

template <class F>
__device__ void prob_categorical_row(F p, int64_t n, double u, CatShared& cs, int64_t& token, unsigned& flags) {
  const int w = wave_id(), lane = lane_id();
  const int64_t lo = (int64_t)w * kCatChunks * kCatChunk;
  long long np = 0;
  double wtot = 0.0;
#pragma unroll 1
  for (int c = 0; c < kCatChunks; c += 2) {  // two chunks' loads in flight at a time
    double x[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int64_t i = lo + (int64_t)c * kCatChunk + 64 * q + lane;
      x[q] = i < n ? p(i) : 0.0;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      double part = 0.0;
#pragma unroll
      for (int q = 8 * h; q < 8 * h + 8; ++q) {
        part += x[q];
        np += x[q] > 0.0 ? 1 : 0;
      }
      const double s = wave_reduce_dpp(part, OpSum());  // the same value in every lane
      if (lane == 0) cs.csum[w][c + h] = s;
      wtot += s;
    }
  }
  const long long wnp = wave_reduce_dpp(np, OpSum());
  if (lane == 0) {
    cs.wsum[w] = wtot;
    cs.wpos[w] = wnp;
  }
  if (threadIdx.x == 0) cs.found[1] = 1;
  __syncthreads();
  double total = 0.0;
  long long npos = 0;
  for (int v = 0; v < kWaves; ++v) {
    total += cs.wsum[v];
    npos += cs.wpos[v];
  }
  const double thr = u * total;
  int ow = -1;  // the last wave with mass whose running sum before it is at most thr
  double obase = 0.0, base = 0.0;
  for (int v = 0; v < kWaves; ++v) {
    if (cs.wsum[v] > 0.0 && base <= thr) {
      ow = v;
      obase = base;
    }
    base += cs.wsum[v];
  }
  if (w == ow) {  // uniform over the wave
    int oc = -1;  // the same over its chunks
    double ocb = 0.0, cb = obase;
    for (int c = 0; c < kCatChunks; ++c) {
      const double s = cs.csum[w][c];
      if (s > 0.0 && cb <= thr) {
        oc = c;
        ocb = cb;
      }
      cb += s;
    }
    int64_t tok = -1;
    int margin = 1;
    if (oc >= 0) {
      const int64_t clo = lo + (int64_t)oc * kCatChunk, chi = clo + kCatChunk < n ? clo + kCatChunk : n;
      const double tol = ((double)npos + 16.0) * 0x1p-51 * total;
      wave_slice_cdf(p, clo, chi, ocb, thr, tol, tok, margin);
    }
    if (lane == 0) {
      cs.found[0] = tok;
      cs.found[1] = margin;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0 && cs.found[1]) cs.found[0] = sequential_cdf_search(p, n, u);
  __syncthreads();
  token = cs.found[0];
  flags = cs.found[1] ? DSR_FLAG_MARGIN : 0u;
}

__global__ __launch_bounds__(kThreads) void k_prob_categorical(const double* p, int64_t n, double u, int32_t* out) {
  __shared__ CatShared cs;
  int64_t tok;
  unsigned flags;
  prob_categorical_row([&](int64_t i) { return p[i]; }, n, u, cs, tok, flags);
  if (threadIdx.x == 0) {
    out[0] = (int32_t)tok;
    out[1] = (int32_t)flags;
  }
}

__global__ __launch_bounds__(kThreads) void k_prob_correction(const double* p, const double* q, int64_t n,
                                                              double* out, int32_t* st) {
  __shared__ NpSumShared np;
  // residual.sum() in NumPy's order as the residual is formed and stored,
  // then residual / total (sampling.py:134-139).
  const double total = np_sum([&](int64_t i) { return fmax(p[i] - q[i], 0.0); }, n, np,
                              [&](int64_t i, double x) { out[i] = x; });
  const bool ok = total > 0.0 && isfinite(total);
  if (ok) row_pass<double>(n, [&](int64_t i) { return out[i]; }, [&](int64_t i, double x) { out[i] = x / total; });
  if (threadIdx.x == 0) st[0] = ok ? DSR_OK : DSR_E_CORRECTION;
}

__global__ void k_prob_accept(const double* p, const double* q, int32_t x, double u, int32_t* out) {
  if (threadIdx.x == 0) {
    const double qx = q[x];
    out[0] = qx > 0.0 ? 1 : 0;
    double ratio = p[x] / qx;
    ratio = ratio < 1.0 ? ratio : 1.0;
    out[1] = (qx > 0.0 && u < ratio) ? 1 : 0;
  }
}

// ---------------------------------------------------------------------------
// dsr_rows_finite: np.isfinite(row).all() of FP32 rows (the terminal window
// check, terminal_sampling.py:25).  A row is spread over workgroups of 4,096
// values (one CU pulls a 517 KB row at about 28 GB/s: 18.5 us for one
// workgroup per row), and a thread that finds a value whose exponent field
// is all ones stores 0 to the row's flag, which the caller set to 1: no
// reduction and no second launch.  16-byte loads when the row starts on a
// 16-byte boundary.
constexpr int kFiniteChunk = 4096;
constexpr int kFiniteThreads = 256;

__device__ __forceinline__ uint32_t nonfinite_bits(uint32_t u) { return (u & 0x7F800000u) == 0x7F800000u; }

__global__ __launch_bounds__(kFiniteThreads) void k_rows_finite(const float* x, int64_t n, int64_t ld, int chunks,
                                                                int32_t* out) {
  const int64_t r = blockIdx.x / chunks;
  const int64_t lo = (int64_t)(blockIdx.x % chunks) * kFiniteChunk;
  const int64_t hi = lo + kFiniteChunk < n ? lo + kFiniteChunk : n;
  const float* row = x + r * ld;
  uint32_t bad = 0;
  if (((uintptr_t)row & 15u) == 0) {
    const uint4* v = (const uint4*)(row + lo);
    const int64_t nv = (hi - lo) / 4;
    uint4 q[kFiniteChunk / 4 / kFiniteThreads];
#pragma unroll
    for (int u = 0; u < kFiniteChunk / 4 / kFiniteThreads; ++u) {
      const int64_t i = threadIdx.x + (int64_t)u * kFiniteThreads;
      q[u] = i < nv ? v[i] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kFiniteChunk / 4 / kFiniteThreads; ++u)
      bad |= nonfinite_bits(q[u].x) | nonfinite_bits(q[u].y) | nonfinite_bits(q[u].z) | nonfinite_bits(q[u].w);
    for (int64_t i = lo + 4 * nv + threadIdx.x; i < hi; i += kFiniteThreads) bad |= nonfinite_bits(__float_as_uint(row[i]));
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += kFiniteThreads) bad |= nonfinite_bits(__float_as_uint(row[i]));
  }
  if (bad) out[r] = 0;
}

// ---------------------------------------------------------------------------
// dsr_verify_probs: verify_drafts (sampling.py:247-294) on float64 rows the
// caller has built, in four launches:
//  1. k_vprobs_stats, one workgroup per 8,192-element buffer of every row:
//     the buffer's NumPy-ordered sum, whether every entry is finite and
//     >= 0, its positive count, first positive index, maximum and first
//     index of the maximum;
//  2. k_vprobs_chain, one wave per request: each row's statistics (buffer
//     sums added in order, as np.add.reduce adds them), the checks in the
//     reference's order and the accept chain; greedy requests end here;
//  3. k_vprobs_draw, one workgroup per buffer of a pending replacement or
//     bonus draw: the NumPy-ordered buffer sum of max(p - q, 0) (or of p),
//     its support and the sums of its 512-element chunks;
//  4. k_vprobs_finish, one wave per request: the correction total, the
//     single-support case, the target draw and the CDF search over
//     max(p - q, 0) / total formed on the fly.
// The correction vector's own _distribution check is not repeated: its
// entries r_i / total are each within half an ulp of exact and sum to 1
// within 2^-47, far inside 1e-10, and r_i / total > 0 exactly when r_i > 0
// (total <= 1 + 1e-10 cannot round a positive quotient to zero).

constexpr int kVpBuffers = 16;  // 8,192-element buffers per row
static_assert((int64_t)kVpBuffers * kNpBuffer >= DSR_MAX_VOCAB, "the buffers cover a row");
constexpr int kVpChunks = kNpBuffer / kCatChunk;  // 512-element CDF chunks per buffer
static_assert(kVpChunks == 2 * kNpBufWaves, "two chunks per wave of a draw workgroup");

struct VpStat {  // one buffer of one row
  double sum, max;
  int32_t ok, npos, first, amax;
};
struct VpDraw {  // one buffer of a pending draw
  double sum;
  int32_t npos, first;
  double csum[kVpChunks];
};

struct VpLayout {
  VpStat* stat;   // [rows, 2K+1, kVpBuffers]
  Decision* dec;  // [rows]
  VpDraw* draw;   // [rows, kVpBuffers]
};

__host__ __device__ inline size_t vprobs_ws_bytes(int64_t rows, int32_t K) {
  return (size_t)rows * ((size_t)(2 * K + 1) * kVpBuffers * sizeof(VpStat) + kDecisionBytes +
                         kVpBuffers * sizeof(VpDraw));
}

__host__ __device__ inline VpLayout vprobs_layout(void* ws, int64_t rows, int32_t K) {
  VpLayout L;
  char* p = (char*)ws;
  L.stat = (VpStat*)p;
  p += (size_t)rows * (2 * K + 1) * kVpBuffers * sizeof(VpStat);
  L.dec = (Decision*)p;
  p += (size_t)rows * kDecisionBytes;
  L.draw = (VpDraw*)p;
  return L;
}

// Row `slot` of request `row`: targets 0..K, drafts K+1..2K.
__device__ __forceinline__ const double* probs_row(const dsr_verify_probs_args_t& a, int64_t row, int slot) {
  return slot <= a.K ? a.target[row * (a.K + 1) + slot] : a.draft[row * a.K + (slot - a.K - 1)];
}

// A reduction over the kNpBufWaves waves of a workgroup; every call needs its
// own slot array.
template <class T, class Op>
__device__ __forceinline__ T buf_reduce(T x, T* slot, T id, Op op) {
  x = wave_reduce_dpp(x, op);
  if (lane_id() == 0) slot[wave_id()] = x;
  __syncthreads();
  T y = id;
#pragma unroll
  for (int w = 0; w < kNpBufWaves; ++w) y = op(y, slot[w]);
  return y;
}

// Step 1.  A target row whose builder failed is not read (its records stay
// unread too); a NULL row reads as an invalid distribution.
__global__ __launch_bounds__(kNpBufThreads) void k_vprobs_stats(dsr_verify_probs_args_t a, VpLayout L) {
  __shared__ NpBufShared nb;
  __shared__ double rmax[kNpBufWaves];
  __shared__ long long rbad[kNpBufWaves], rnpos[kNpBufWaves], rfirst[kNpBufWaves], ramax[kNpBufWaves];
  const int slots = 2 * a.K + 1;
  const uint32_t item = blockIdx.x;
  const int b = (int)(item % kVpBuffers);
  const uint32_t rs = item / kVpBuffers;
  const int64_t row = rs / slots;
  const int slot = (int)(rs % slots);
  const int64_t lo = (int64_t)b * kNpBuffer;
  if (lo >= a.vocab) return;
  if (slot <= a.K && a.target_status && a.target_status[row * (a.K + 1) + slot] != DSR_OK) return;
  VpStat* out = L.stat + item;
  const double* p = probs_row(a, row, slot);
  if (!p) {
    if (threadIdx.x == 0) out->ok = 0;
    return;
  }
  // 32-bit: hipcc (ROCm 7.2) built the 64-bit form of this minimum as an
  // s_cselect on a stale SCC, giving 8,192 for the short last buffer.
  const int len = min((int)(a.vocab - lo), kNpBuffer);
  long long bad = 0, npos = 0, first = LLONG_MAX, am = LLONG_MAX;
  double m = -INFINITY;
  const double sum = np_buffer_sum([&](int64_t i) { return p[i]; }, lo, len, nb, [&](int64_t i, double x) {
    if (!(isfinite(x) && x >= 0.0)) bad = 1;
    if (x > 0.0) {
      ++npos;
      if (i < first) first = i;
    }
    if (x > m) {
      m = x;
      am = i;
    }
  });
  bad = buf_reduce(bad, rbad, 0ll, OpMax());
  npos = buf_reduce(npos, rnpos, 0ll, OpSum());
  first = buf_reduce(first, rfirst, LLONG_MAX, OpMin());
  const double M = buf_reduce(m, rmax, -(double)INFINITY, OpMax());
  am = buf_reduce(m == M ? am : LLONG_MAX, ramax, LLONG_MAX, OpMin());
  if (threadIdx.x == 0) {
    out->sum = sum;
    out->max = M;
    out->ok = bad ? 0 : 1;
    out->npos = (int32_t)npos;
    out->first = first == LLONG_MAX ? -1 : (int32_t)first;
    out->amax = am == LLONG_MAX ? -1 : (int32_t)am;
  }
}

// Step 2.  Lane b holds buffer b of the row being combined.
__global__ __launch_bounds__(64) void k_vprobs_chain(dsr_verify_probs_args_t a, VpLayout L) {
  constexpr int kSlots = 2 * DSR_MAX_DRAFTS + 1;
  __shared__ Decision d;
  __shared__ double gua[DSR_MAX_DRAFTS];
  __shared__ int32_t sst[kSlots], samax[kSlots];
  __shared__ VpStat stats[kSlots * kVpBuffers];
  __shared__ double pv[2 * DSR_MAX_DRAFTS];  // target j, then draft j, at draft j's token
  __shared__ int32_t tst[DSR_MAX_DRAFTS + 1];  // the target rows' build statuses
  // The request, staged: draft ids, pre-drawn accept uniforms, the output
  // limit and greedy flag, the EOS range and its first kEosStage ids, and the
  // accept domain's PCG64 state (the one thread that runs the chain then
  // reads no global memory on its way).
  constexpr int kEosStage = 64;
  __shared__ int32_t sids[DSR_MAX_DRAFTS], seos[kEosStage], smeta[2];
  __shared__ double sua[DSR_MAX_DRAFTS];
  __shared__ int64_t seoff[2];
  __shared__ uint64_t srng[4];
  const int64_t row = blockIdx.x;
  const int K = a.K, slots = 2 * K + 1, l = lane_id();
  const int nbuf = (int)((a.vocab + kNpBuffer - 1) / kNpBuffer);
  if (l <= K) tst[l] = a.target_status ? a.target_status[row * (K + 1) + l] : (int32_t)DSR_OK;
  if (l < K) {
    sids[l] = a.draft_ids[row * K + l];
    if (a.u_accept) sua[l] = a.u_accept[row * K + l];
  }
  if (l == 32) smeta[0] = a.output_limit[row];
  if (l == 33) smeta[1] = a.greedy ? (int32_t)a.greedy[row] : 0;
  if (l >= 34 && l < 36) seoff[l - 34] = a.eos_off ? a.eos_off[row + (l - 34)] : 0;
  if (l >= 40 && l < 44 && a.rng_accept) srng[l - 40] = a.rng_accept[4 * row + (l - 40)];
  __syncthreads();
  auto status_in = [&](int slot) { return slot <= K ? tst[slot] : (int32_t)DSR_OK; };
  const int64_t e0 = seoff[0], n_eos = seoff[1] - seoff[0];
  if (l < n_eos && l < kEosStage) seos[l] = a.eos_ids[e0 + l];
  // Every load the chain needs, issued at once: the buffers' statistics of
  // each row, and the two probabilities of each draft's token (a row that
  // failed to build, or a token outside the vocabulary, is not read).
  for (int i = l; i < slots * kVpBuffers; i += 64) {
    const int slot = i / kVpBuffers, b = i % kVpBuffers;
    if (b < nbuf && status_in(slot) == DSR_OK) stats[i] = L.stat[(row * slots + slot) * kVpBuffers + b];
  }
  if (l < 2 * K) {
    const int j = l < K ? l : l - K;
    const int slot = l < K ? j : K + 1 + j;
    const int32_t x = sids[j];
    const double* p = status_in(slot) == DSR_OK ? probs_row(a, row, slot) : nullptr;
    pv[l] = p && x >= 0 && x < a.vocab ? p[x] : 0.0;
  }
  __syncthreads();
  // Lane s settles row s from its buffers' statistics, all rows at once.
  if (l < slots) {
    int st = status_in(l);
    int32_t amax = -1;
    if (st == DSR_OK) {
      double total = 0.0, M = -INFINITY;  // np.add.reduce adds the buffers' sums in order
      bool ok = true;
      long long am = LLONG_MAX;
      for (int b = 0; b < nbuf; ++b) {
        const VpStat x = stats[l * kVpBuffers + b];
        total = b == 0 ? x.sum : total + x.sum;
        ok = ok && x.ok;
        if (x.max > M) {
          M = x.max;
          am = x.amax;
        } else if (x.max == M && (long long)x.amax < am) {
          am = x.amax;
        }
      }
      amax = am == LLONG_MAX ? -1 : (int32_t)am;
      // _distribution (sampling.py:109-115): finite, >= 0, sum within 1e-10 of 1.
      st = ok && fabs(total - 1.0) <= 1e-10 ? DSR_OK : DSR_E_DISTRIBUTION;
    }
    sst[l] = st;
    samax[l] = amax;
  }
  __syncthreads();
  if (l != 0) return;
  auto status_of = [&](int slot) { return (int)sst[slot]; };
  const bool greedy = smeta[1] != 0;
  Request rq;  // request_of's fields, from the staged copies
  rq.ids = sids;
  rq.ua = sua;
  rq.eos = n_eos <= kEosStage ? seos : a.eos_ids + e0;
  rq.n_eos = (int)n_eos;
  rq.limit = smeta[0];
  if (a.rng_accept) {  // the accept domain's next K draws, consumed in order
    pcg64_draws(srng, K, gua);
    rq.ua = gua;
  }
  verify_precheck(a, rq, status_of, d);
  if (d.status == DSR_OK)
    verify_chain(
        a, rq, greedy, 0.0, status_of, [&](int slot, int j) { return slot <= K ? pv[j] : pv[K + j]; },
        [&](int j) { return (int64_t)samax[j]; }, [](int) {}, d);
  if (d.status == DSR_OK && d.next != 0 && greedy) {  // the target's argmax (sampling.py:286,290)
    verify_append(a, rq, d, samax[d.draw_j], 0);
    d.next = 0;
  }
  L.dec[row] = d;
  if (d.status != DSR_OK || d.next == 0) write_decision(a, row, d);
}

// Step 3.  Wave w also sums chunks 2w and 2w + 1 of the buffer (any order:
// the search in step 4 allows for it).
__global__ __launch_bounds__(kNpBufThreads) void k_vprobs_draw(dsr_verify_probs_args_t a, VpLayout L) {
  __shared__ NpBufShared nb;
  __shared__ long long rnpos[kNpBufWaves], rfirst[kNpBufWaves];
  const int64_t row = blockIdx.x / kVpBuffers;
  const int b = (int)(blockIdx.x % kVpBuffers);
  const Decision* dp = L.dec + row;
  if (dp->status != DSR_OK || dp->next == 0) return;
  const int64_t lo = (int64_t)b * kNpBuffer;
  if (lo >= a.vocab) return;
  // 32-bit: hipcc (ROCm 7.2) built the 64-bit form of this minimum as an
  // s_cselect on a stale SCC, giving 8,192 for the short last buffer.
  const int len = min((int)(a.vocab - lo), kNpBuffer);
  const int j = dp->draw_j;
  const double* P = probs_row(a, row, j);
  const double* Q = dp->next == 1 ? probs_row(a, row, a.K + 1 + j) : nullptr;
  auto r = [&](int64_t i) { return Q ? fmax(P[i] - Q[i], 0.0) : P[i]; };
  long long npos = 0, first = LLONG_MAX;
  const double sum = np_buffer_sum(r, lo, len, nb, [&](int64_t i, double x) {
    if (x > 0.0) {
      ++npos;
      if (i < first) first = i;
    }
  });
  npos = buf_reduce(npos, rnpos, 0ll, OpSum());
  first = buf_reduce(first, rfirst, LLONG_MAX, OpMin());
  VpDraw* out = L.draw + blockIdx.x;
  const int w = wave_id(), l = lane_id();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = 2 * w + h;
    const int64_t clo = lo + (int64_t)c * kCatChunk;
    double part = 0.0;
#pragma unroll
    for (int t = 0; t < kCatChunk / 64; ++t) {
      const int64_t i = clo + 64 * t + l;
      part += i < lo + len ? r(i) : 0.0;
    }
    part = wave_reduce_dpp(part, OpSum());
    if (l == 0) out->csum[c] = part;
  }
  if (threadIdx.x == 0) {
    out->sum = sum;
    out->npos = (int32_t)npos;
    out->first = first == LLONG_MAX ? -1 : (int32_t)first;
  }
}

// Step 4.  Lane l holds chunks 4l .. 4l + 3 of the row (chunk c covers
// elements 512 c .. 512 c + 511), scaled by 1 / total for a correction; the
// chunk holding the crossing of u times their sum is walked with the exact
// entries max(p - q, 0) / total, and a decision within the rounding band of
// a cell edge is settled by the sequential cumulative sum (np.cumsum).
__global__ __launch_bounds__(64) void k_vprobs_finish(dsr_verify_probs_args_t a, VpLayout L) {
  const int64_t row = blockIdx.x;
  Decision d = L.dec[row];
  if (d.status != DSR_OK || d.next == 0) return;
  const int K = a.K, l = lane_id(), j = d.draw_j;
  const int nbuf = (int)((a.vocab + kNpBuffer - 1) / kNpBuffer);
  const VpDraw* parts = L.draw + row * kVpBuffers;
  const bool resid = d.next == 1;
  const double* P = probs_row(a, row, j);
  const double* Q = resid ? probs_row(a, row, K + 1 + j) : nullptr;
  double bs = 0.0;
  long long np_ = 0, f = LLONG_MAX;
  if (l < nbuf) {
    bs = parts[l].sum;
    np_ = parts[l].npos;
    f = parts[l].npos > 0 ? (long long)parts[l].first : LLONG_MAX;
  }
  double total = lane_value(bs, 0);  // np.add.reduce's order over the buffers
  for (int b = 1; b < nbuf; ++b) total += lane_value(bs, b);
  const long long npos = wave_reduce_dpp(np_, OpSum());
  const long long first = wave_reduce_dpp(f, OpMin());
  int64_t rep = -1;
  int used = 0, status = DSR_OK, margin = 0;
  if (resid && !(total > 0.0 && isfinite(total))) {
    status = DSR_E_CORRECTION;  // correction_distribution (sampling.py:137-138)
  } else if (npos == 1) {
    rep = first;  // a single positive entry: no uniform is drawn (sampling.py:120-122)
  } else {
    double u = 0.0;
    if (a.rng_target) pcg64_draws(a.rng_target + 4 * row, 1, &u);
    else u = a.u_target[row];
    if (!(u >= 0.0 && u < 1.0)) {
      status = DSR_E_UNIFORM;
    } else {
      used = 1;
      const double scale = resid ? total : 1.0;
      auto q = [&](int64_t i) { return resid ? fmax(P[i] - Q[i], 0.0) / scale : P[i]; };
      double cs[4], lane_sum = 0.0;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int c = 4 * l + t, b = c / kVpChunks;
        cs[t] = b < nbuf ? parts[b].csum[c % kVpChunks] / scale : 0.0;
        lane_sum += cs[t];
      }
      const double incl = wave_scan_dpp(lane_sum);
      const double tq = lane_value(incl, 63);
      const double thr = u * tq;
      // The last chunk with mass starting at or below thr.
      double st = incl - lane_sum, cbase = 0.0;
      int cand = -1;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (cs[t] > 0.0 && st <= thr) {
          cand = 4 * l + t;
          cbase = st;
        }
        st += cs[t];
      }
      const unsigned long long cb = __ballot(cand >= 0);
      if (cb) {
        const int owner = 63 - __clzll((long long)cb);
        const int c = __shfl(cand, owner);
        const double base = __shfl(cbase, owner);
        const int64_t clo = (int64_t)c * kCatChunk;
        const int64_t chi = clo + kCatChunk < a.vocab ? clo + kCatChunk : a.vocab;
        const double tol = ((double)npos + 16.0) * 0x1p-51 * tq;
        wave_slice_cdf(q, clo, chi, base, thr, tol, rep, margin);
      } else {
        margin = 1;
      }
      if (margin && l == 0) rep = sequential_cdf_search(q, a.vocab, u);
      rep = (int64_t)__shfl((long long)rep, 0);
    }
  }
  if (l == 0) {
    if (margin) d.flags |= DSR_FLAG_MARGIN;
    Request rq = request_of(a, row);
    if (status != DSR_OK) d.status = status;
    else verify_append(a, rq, d, rep, used);
    write_decision(a, row, d);
  }
}

}  // namespace dsr

// ---------------------------------------------------------------------------
// C ABI.

using namespace dsr;

static int32_t launched() { return hipGetLastError() == hipSuccess ? 0 : DSR_ERR_LAUNCH; }

extern "C" {

int32_t dsr_abi_version(void) { return DSR_ABI_VERSION; }

const char* dsr_status_message(int32_t code) {
  switch (code) {
    case DSR_OK: return "ok";
    case DSR_E_LOGITS: return "sampling needs one bounded finite-or-masked floating logit vector";
    case DSR_E_MASKED: return "sampling controls masked every vocabulary token";
    case DSR_E_NO_MASS: return "sampling controls produced no positive probability";
    case DSR_E_UNIFORM: return "sampling uniform must lie in [0,1)";
    case DSR_E_COUNTS: return "sampling frequency counts do not match the vocabulary";
    case DSR_E_BIAS: return "invalid logit bias mapping";
    case DSR_E_PROPOSAL_ZERO: return "a proposed token has zero probability under its claimed conditional proposal";
    case DSR_E_CORRECTION: return "a rejected proposal has no positive correction distribution";
    case DSR_E_TOKEN: return "verification token must be an integer in the vocabulary";
    case DSR_E_DISTRIBUTION: return "verifier requires a normalized complete FP64 probability vector";
    case DSR_E_POLICY: return "invalid sampling policy";
    case DSR_E_GENERATED: return "generated token counts must be a subset of complete sampling history";
    case DSR_E_HISTORY: return "history needs bounded exact integer token IDs";
    case DSR_E_APPEND: return "a history append holds at most 16384 tokens per row";
    case DSR_E_HINT: return "request contradicts the call's DSR_HINT_VERIFY_FAST promise";
    default: return "unknown sampling status";
  }
}

size_t dsr_sample_workspace_bytes(int64_t rows, int64_t vocab) {
  if (rows < 0 || vocab < 1) return 0;
  return (size_t)rows * (size_t)ws_stride(vocab) * sizeof(double);
}

size_t dsr_verify_workspace_bytes(int64_t rows, int32_t K, int64_t vocab) {
  if (rows < 0 || vocab < 1 || K < 0) return 0;
  return verify_ws_bytes(rows, K, vocab);
}

// The DSR_HINT_* bits a caller may set; any other bit is rejected, so the
// field can take new meanings later without an ABI change.
static constexpr uint32_t kHintBits = DSR_HINT_WHOLE_SOME | DSR_HINT_WHOLE_ALL | DSR_HINT_VERIFY_FAST | DSR_HINT_TOPK_ALL;

static bool dtype_ok(int32_t d) { return d == DSR_BF16 || d == DSR_F32 || d == DSR_F64; }

static int32_t sample_rows(const dsr_sample_args_t* args, const dsr_head_part_t* parts, void* stream);

int32_t dsr_sample_rows(const dsr_sample_args_t* args, void* stream) { return sample_rows(args, nullptr, stream); }

int32_t dsr_sample_rows_head(const dsr_sample_args_t* args, const dsr_head_part_t* parts, void* stream) {
  return sample_rows(args, parts, stream);
}

static int32_t sample_rows(const dsr_sample_args_t* args, const dsr_head_part_t* parts, void* stream) {
  if (!args) return DSR_ERR_ARG;
  const dsr_sample_args_t& a = *args;
  const int64_t words = (a.vocab + 31) / 32;
  if (!a.logits || !a.policy || !a.out_token || !a.out_consumed || !a.out_status || !dtype_ok(a.dtype) ||
      a.rows < 0 || a.rows > INT_MAX || a.vocab < 1 || a.vocab > DSR_MAX_VOCAB || a.ld < a.vocab ||
      (a.hints & ~kHintBits))
    return DSR_ERR_ARG;
  if (a.pen_off && (!a.pen_ids || !a.pen_count || !a.pen_gen)) return DSR_ERR_ARG;
  if (a.bias_off && (!a.bias_ids || !a.bias_val)) return DSR_ERR_ARG;
  if (a.allow_bits && a.allow_ld < words) return DSR_ERR_ARG;
  if ((a.out_probs_f32 || a.out_probs_f64) && a.probs_ld < a.vocab) return DSR_ERR_ARG;
  if (a.out_kept_bits && a.kept_ld < words) return DSR_ERR_ARG;
  if (!a.workspace || a.workspace_bytes < dsr_sample_workspace_bytes(a.rows, a.vocab) ||
      ((uintptr_t)a.workspace & 7u))
    return DSR_ERR_WORKSPACE;
  if (a.rows == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)a.rows);
  auto launch_fast = [&](uint32_t mode) {
    dsr_sample_args_t k = a;
    k.hints = mode;
    if (k.rng_state) hipLaunchKernelGGL(k_sample_bf16_fast<true>, grid, dim3(kThreads), 0, s, k);
    else hipLaunchKernelGGL(k_sample_bf16_fast<false>, grid, dim3(kThreads), 0, s, k);
  };
  auto launch_full = [&](uint32_t mode) {
    dsr_sample_args_t k = a;
    k.hints = mode;
    if (k.rng_state) hipLaunchKernelGGL(k_sample_bf16_full<true>, grid, dim3(kThreads), 0, s, k);
    else hipLaunchKernelGGL(k_sample_bf16_full<false>, grid, dim3(kThreads), 0, s, k);
  };
  if (fast_path_eligible(a)) {
    // A bf16 batch with no history or bias: whole rows (no top-k register
    // cut) go to the full-vocabulary kernel when the caller says it has some.
    if (a.hints & DSR_HINT_WHOLE_ALL) {
      launch_full(0u);
    } else if (a.hints & DSR_HINT_WHOLE_SOME) {
      launch_fast(kModeDeferWhole);
      launch_full(kModeOnlyWhole);
    } else {
      launch_fast(0u);
    }
  } else if (full_path_eligible(a)) {
    launch_full(0u);
  } else if (f32_path_eligible(a)) {
    if (a.out_probs_f32 || a.out_probs_f64) {
      const int64_t chunks = (a.vocab + kZeroChunk - 1) / kZeroChunk;
      hipLaunchKernelGGL(k_zero_probs, dim3((unsigned)(a.rows * chunks)), dim3(kZeroThreads), 0, s, a.out_probs_f32,
                         a.out_probs_f64, a.probs_ld, a.vocab, (int)chunks);
    }
    const dsr_head_part_t* hp = parts && f32_head_eligible(a) ? parts : nullptr;
    if (a.rng_state) hipLaunchKernelGGL(k_sample_f32<true>, dim3((unsigned)a.rows), dim3(kThreads), 0, s, a, hp);
    else hipLaunchKernelGGL(k_sample_f32<false>, dim3((unsigned)a.rows), dim3(kThreads), 0, s, a, hp);
  } else if (split_path_eligible(a)) {
    const int smax = split_max_slices(a.rows);
    hipLaunchKernelGGL(k_split_select, dim3((unsigned)(a.rows * smax)), dim3(kThreads), 0, s, a, smax);
    if (a.rng_state) hipLaunchKernelGGL(k_split_finish<true>, dim3((unsigned)a.rows), dim3(kThreads), 0, s, a, smax);
    else hipLaunchKernelGGL(k_split_finish<false>, dim3((unsigned)a.rows), dim3(kThreads), 0, s, a, smax);
  } else {
    if (a.rng_state) hipLaunchKernelGGL(k_sample_general<true>, dim3((unsigned)a.rows), dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL(k_sample_general<false>, dim3((unsigned)a.rows), dim3(kThreads), 0, s, a);
  }
  return launched();
}

// ---------------------------------------------------------------------------
// Allocation-free variant of dsr_sample_rows.  Its workspace is a file-scope
// device array, one copy per device, held until the process ends.  Host code
// never passes the array's name to a kernel (on the host that name is only a
// stand-in): each device's address is looked up once, with that device
// current, and kept.

static __device__ __align__(256) unsigned char scratch[DSR_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex scratch_lock;
void* scratch_address[kMaxScratchDevices];  // per device; null until looked up
}  // namespace

// The scratch array of the current device; 0 or DSR_ERR_LAUNCH.
static int32_t current_scratch(void** out) {
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxScratchDevices) return DSR_ERR_LAUNCH;
  std::lock_guard<std::mutex> hold(scratch_lock);
  if (!scratch_address[device]) {
    void* address = nullptr;
    if (hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)) != hipSuccess || !address) return DSR_ERR_LAUNCH;
    scratch_address[device] = address;
  }
  *out = scratch_address[device];
  return 0;
}

int32_t dsr_sample_rows_noalloc(const dsr_sample_args_t* args, void* stream) {
  if (!args) return DSR_ERR_ARG;
  if (args->workspace || args->workspace_bytes) return DSR_ERR_ARG;  // the device array is the workspace
  if (args->rows < 0 || args->vocab < 1) return DSR_ERR_ARG;
  if (dsr_sample_workspace_bytes(args->rows, args->vocab) > (size_t)DSR_NOALLOC_SCRATCH_BYTES)
    return DSR_ERR_WORKSPACE;
  void* ws = nullptr;
  const int32_t rc = current_scratch(&ws);
  if (rc) return rc;
  dsr_sample_args_t a = *args;
  a.workspace = ws;
  a.workspace_bytes = DSR_NOALLOC_SCRATCH_BYTES;
  return dsr_sample_rows(&a, stream);
}

}  // extern "C"

// dsr_verify_drafts and dsr_verify_drafts_head: with head records (tp) the
// fast path's statistics come from k_head_shares instead of k_verify_stats.
static int32_t verify_launch(const dsr_verify_args_t& a, const dsr_head_part_t* tp, const dsr_head_part_t* dp,
                             void* stream) {
  if (!a.target || (a.K > 0 && (!a.draft || !a.draft_ids || (!a.u_accept && !a.rng_accept))) || !a.policy ||
      (!a.u_target && !a.rng_target) ||
      !a.output_limit || !a.out_accepted || !a.out_ids || !a.out_count || !a.out_pending || !a.out_stop ||
      !a.out_used_accept || !a.out_used_target || !a.out_status || !dtype_ok(a.dtype) || a.K < 0 ||
      a.K > DSR_MAX_DRAFTS || a.rows < 0 || a.vocab < 1 || a.vocab > DSR_MAX_VOCAB || a.ld < a.vocab ||
      a.reserved != 0 || (a.hints & ~kHintBits))
    return DSR_ERR_ARG;
  if (a.pen_off && (!a.pen_ids || !a.pen_count || !a.pen_gen)) return DSR_ERR_ARG;
  if (a.bias_off && (!a.bias_ids || !a.bias_val)) return DSR_ERR_ARG;
  if (a.eos_off && !a.eos_ids) return DSR_ERR_ARG;
  if (a.allow_bits && a.allow_ld < (a.vocab + 31) / 32) return DSR_ERR_ARG;
  const int64_t slots = 2 * (int64_t)a.K + 1;
  if ((int64_t)a.rows * slots * kVerifySplit > INT_MAX || (int64_t)a.rows * kDrawSplit > INT_MAX) return DSR_ERR_ARG;
  if (!a.workspace || a.workspace_bytes < dsr_verify_workspace_bytes(a.rows, a.K, a.vocab) ||
      ((uintptr_t)a.workspace & 7u))
    return DSR_ERR_WORKSPACE;
  if (a.rows == 0) return 0;
  VerifyLayout L = verify_layout(a.workspace, a.rows, a.K, a.vocab);
  L.fast_inputs = !a.pen_off && !a.bias_off && !a.allow_bits;
  hipStream_t s = (hipStream_t)stream;
  // A call whose requests all take the fast path needs no general-path
  // distributions; a request breaking that promise gets DSR_E_HINT.
  L.dists_built = !(L.fast_inputs && (a.hints & DSR_HINT_VERIFY_FAST));
  if (L.dists_built) {
    hipLaunchKernelGGL(k_verify_dists, dim3((unsigned)(a.rows * slots)), dim3(kThreads), 0, s, a, L);
    if (hipGetLastError() != hipSuccess) return DSR_ERR_LAUNCH;
  }
  // 16-byte loads when every row starts on a 16-byte boundary.
  const size_t elt = a.dtype == DSR_BF16 ? 2 : (a.dtype == DSR_F32 ? 4 : 8);
  const bool vec = ((uintptr_t)a.target & 15u) == 0 && (a.K == 0 || ((uintptr_t)a.draft & 15u) == 0) &&
                   ((size_t)a.ld * elt) % 16 == 0;
  if (L.fast_inputs && tp) {
    hipLaunchKernelGGL(k_head_shares, dim3((unsigned)(a.rows * slots)), dim3(64), 0, s, a, L, tp, dp);
    if (hipGetLastError() != hipSuccess) return DSR_ERR_LAUNCH;
  } else if (L.fast_inputs) {
    const dim3 grid((unsigned)(a.rows * slots * kVerifySplit));
    if (a.dtype == DSR_BF16) {
      if (vec) hipLaunchKernelGGL((k_verify_stats<DSR_BF16, true>), grid, dim3(kStatThreads), 0, s, a, L);
      else hipLaunchKernelGGL((k_verify_stats<DSR_BF16, false>), grid, dim3(kStatThreads), 0, s, a, L);
    } else if (a.dtype == DSR_F32) {
      if (vec) hipLaunchKernelGGL((k_verify_stats<DSR_F32, true>), grid, dim3(kStatThreads), 0, s, a, L);
      else hipLaunchKernelGGL((k_verify_stats<DSR_F32, false>), grid, dim3(kStatThreads), 0, s, a, L);
    } else {
      if (vec) hipLaunchKernelGGL((k_verify_stats<DSR_F64, true>), grid, dim3(kStatThreads), 0, s, a, L);
      else hipLaunchKernelGGL((k_verify_stats<DSR_F64, false>), grid, dim3(kStatThreads), 0, s, a, L);
    }
    if (hipGetLastError() != hipSuccess) return DSR_ERR_LAUNCH;
  }
  hipLaunchKernelGGL(k_verify_chain, dim3((unsigned)a.rows), dim3(kThreads), 0, s, a, L);
  if (L.fast_inputs) {
    if (hipGetLastError() != hipSuccess) return DSR_ERR_LAUNCH;
    const dim3 dgrid((unsigned)(a.rows * kDrawSplit));
    if (a.dtype == DSR_BF16) {
      if (vec) hipLaunchKernelGGL((k_verify_draw<DSR_BF16, true>), dgrid, dim3(kStatThreads), 0, s, a, L);
      else hipLaunchKernelGGL((k_verify_draw<DSR_BF16, false>), dgrid, dim3(kStatThreads), 0, s, a, L);
    } else if (a.dtype == DSR_F32) {
      if (vec) hipLaunchKernelGGL((k_verify_draw<DSR_F32, true>), dgrid, dim3(kStatThreads), 0, s, a, L);
      else hipLaunchKernelGGL((k_verify_draw<DSR_F32, false>), dgrid, dim3(kStatThreads), 0, s, a, L);
    } else {
      if (vec) hipLaunchKernelGGL((k_verify_draw<DSR_F64, true>), dgrid, dim3(kStatThreads), 0, s, a, L);
      else hipLaunchKernelGGL((k_verify_draw<DSR_F64, false>), dgrid, dim3(kStatThreads), 0, s, a, L);
    }
    if (hipGetLastError() != hipSuccess) return DSR_ERR_LAUNCH;
    hipLaunchKernelGGL(k_verify_finish, dim3((unsigned)a.rows), dim3(64), 0, s, a, L);
  }
  return launched();
}

// From three 32-row blocks (65 rows) on, a workgroup takes 256 columns: each
// staged hidden chunk then serves twice the weight (at 160 rows x dim 5,120 x
// vocab 129,280: 331 us against 378 us with 128-column workgroups).
#ifndef DSR_HEAD_CB2_MIN_BLOCKS
#define DSR_HEAD_CB2_MIN_BLOCKS 3
#endif
#ifndef DSR_HEAD_CB2_MIN_BLOCKS_RECORDS
#define DSR_HEAD_CB2_MIN_BLOCKS_RECORDS DSR_HEAD_CB2_MIN_BLOCKS
#endif

template <int NB>
static void head_launch(const dsr_head_args_t& a, hipStream_t s) {
  const dim3 block(kHeadThreads);
  if (NB >= (a.parts ? DSR_HEAD_CB2_MIN_BLOCKS_RECORDS : DSR_HEAD_CB2_MIN_BLOCKS) && a.vocab % (2 * kHeadTile) == 0) {
    const dim3 grid((unsigned)(a.vocab / (2 * kHeadTile)));
    if (a.parts) hipLaunchKernelGGL((k_vocab_head<NB, 2, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_vocab_head<NB, 2, false>), grid, block, 0, s, a);
    return;
  }
  const dim3 grid((unsigned)(a.vocab / kHeadTile));
  if (a.parts) hipLaunchKernelGGL((k_vocab_head<NB, 1, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((k_vocab_head<NB, 1, false>), grid, block, 0, s, a);
}

extern "C" {

int32_t dsr_verify_drafts(const dsr_verify_args_t* args, void* stream) {
  if (!args) return DSR_ERR_ARG;
  return verify_launch(*args, nullptr, nullptr, stream);
}

int32_t dsr_verify_drafts_head(const dsr_verify_args_t* args, const dsr_head_part_t* target_parts,
                               const dsr_head_part_t* draft_parts, void* stream) {
  if (!args || !target_parts || (args->K > 0 && !draft_parts)) return DSR_ERR_ARG;
  const dsr_verify_args_t& a = *args;
  if (a.dtype != DSR_F32 || a.vocab % kHeadTile != 0 || a.ld != a.vocab || ((uintptr_t)target_parts & 7u) ||
      ((uintptr_t)draft_parts & 7u))
    return DSR_ERR_ARG;
  return verify_launch(a, target_parts, draft_parts, stream);
}

int32_t dsr_vocab_head(const dsr_head_args_t* args, void* stream) {
  if (!args) return DSR_ERR_ARG;
  const dsr_head_args_t& a = *args;
  if (!a.hidden || !a.weight || !a.logits || a.rows < 0 || a.rows > DSR_HEAD_MAX_ROWS || a.dim < kHeadDimStep ||
      a.dim % kHeadDimStep != 0 || a.vocab < kHeadTile || a.vocab % kHeadTile != 0 || a.vocab > DSR_MAX_VOCAB ||
      a.reserved != 0 || (a.policy && a.rows_per_policy < 1) || ((uintptr_t)a.hidden & 15u) ||
      ((uintptr_t)a.weight & 15u) || ((uintptr_t)a.logits & 15u) || ((uintptr_t)a.parts & 7u))
    return DSR_ERR_ARG;
  if (a.rows == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  switch ((a.rows + 31) / 32) {
    case 1: head_launch<1>(a, s); break;
    case 2: head_launch<2>(a, s); break;
    case 3: head_launch<3>(a, s); break;
    case 4: head_launch<4>(a, s); break;
    case 5: head_launch<5>(a, s); break;
    case 6: head_launch<6>(a, s); break;
    case 7: head_launch<7>(a, s); break;
    default: head_launch<8>(a, s); break;
  }
  return launched();
}

size_t dsr_verify_probs_workspace_bytes(int64_t rows, int32_t K) {
  if (rows < 0 || K < 0 || K > DSR_MAX_DRAFTS) return 0;
  return vprobs_ws_bytes(rows, K);
}

int32_t dsr_verify_probs(const dsr_verify_probs_args_t* args, void* stream) {
  if (!args) return DSR_ERR_ARG;
  const dsr_verify_probs_args_t& a = *args;
  if (!a.target || (a.K > 0 && (!a.draft || !a.draft_ids || (!a.u_accept && !a.rng_accept))) ||
      (!a.u_target && !a.rng_target) || !a.output_limit || !a.out_accepted || !a.out_ids || !a.out_count ||
      !a.out_pending || !a.out_stop || !a.out_used_accept || !a.out_used_target || !a.out_status || a.K < 0 ||
      a.K > DSR_MAX_DRAFTS || a.rows < 0 || a.vocab < 1 || a.vocab > DSR_MAX_VOCAB || a.reserved != 0 ||
      (a.eos_off && !a.eos_ids))
    return DSR_ERR_ARG;
  const int64_t slots = 2 * (int64_t)a.K + 1;
  if (a.rows * slots * kVpBuffers > INT_MAX) return DSR_ERR_ARG;
  if (!a.workspace || a.workspace_bytes < dsr_verify_probs_workspace_bytes(a.rows, a.K) ||
      ((uintptr_t)a.workspace & 7u))
    return DSR_ERR_WORKSPACE;
  if (a.rows == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  const VpLayout L = vprobs_layout(a.workspace, a.rows, a.K);
  hipLaunchKernelGGL(k_vprobs_stats, dim3((unsigned)(a.rows * slots * kVpBuffers)), dim3(kNpBufThreads), 0, s, a, L);
  if (hipGetLastError() != hipSuccess) return DSR_ERR_LAUNCH;
  hipLaunchKernelGGL(k_vprobs_chain, dim3((unsigned)a.rows), dim3(64), 0, s, a, L);
  if (hipGetLastError() != hipSuccess) return DSR_ERR_LAUNCH;
  hipLaunchKernelGGL(k_vprobs_draw, dim3((unsigned)(a.rows * kVpBuffers)), dim3(kNpBufThreads), 0, s, a, L);
  if (hipGetLastError() != hipSuccess) return DSR_ERR_LAUNCH;
  hipLaunchKernelGGL(k_vprobs_finish, dim3((unsigned)a.rows), dim3(64), 0, s, a, L);
  return launched();
}

int32_t dsr_prob_stats(const double* p, int64_t n, double* out_sum, int32_t* out_i32, void* stream) {
  if (!p || !out_sum || !out_i32 || n < 1 || n > DSR_MAX_VOCAB) return DSR_ERR_ARG;
  hipLaunchKernelGGL(k_prob_stats, dim3(1), dim3(kThreads), 0, (hipStream_t)stream, p, n, out_sum, out_i32);
  return launched();
}

int32_t dsr_prob_stats_rows(const double* const* rows, int32_t count, int64_t n, double* out, void* stream) {
  if (!rows || !out || count < 0 || count > DSR_STATS_MAX_ROWS || n < 1 || n > DSR_MAX_VOCAB) return DSR_ERR_ARG;
  if (count == 0) return 0;
  StatsRows r{};
  for (int i = 0; i < count; ++i) {
    if (!rows[i]) return DSR_ERR_ARG;
    r.p[i] = rows[i];
  }
  hipLaunchKernelGGL(k_prob_stats_rows, dim3((unsigned)count), dim3(kThreads), 0, (hipStream_t)stream, r, n, out);
  return launched();
}

int32_t dsr_prob_categorical(const double* p, int64_t n, double u, int32_t* out_i32, void* stream) {
  if (!p || !out_i32 || n < 1 || n > DSR_MAX_VOCAB || !(u >= 0.0 && u < 1.0)) return DSR_ERR_ARG;
  hipLaunchKernelGGL(k_prob_categorical, dim3(1), dim3(kThreads), 0, (hipStream_t)stream, p, n, u, out_i32);
  return launched();
}

int32_t dsr_prob_correction(const double* p, const double* q, int64_t n, double* out, int32_t* out_i32,
                            void* stream) {
  if (!p || !q || !out || !out_i32 || n < 1 || n > DSR_MAX_VOCAB) return DSR_ERR_ARG;
  hipLaunchKernelGGL(k_prob_correction, dim3(1), dim3(kThreads), 0, (hipStream_t)stream, p, q, n, out, out_i32);
  return launched();
}

int32_t dsr_prob_accept(const double* p, const double* q, int64_t n, int32_t x, double u, int32_t* out_i32,
                        void* stream) {
  if (!p || !q || !out_i32 || n < 1 || n > DSR_MAX_VOCAB || x < 0 || x >= n) return DSR_ERR_ARG;
  hipLaunchKernelGGL(k_prob_accept, dim3(1), dim3(64), 0, (hipStream_t)stream, p, q, x, u, out_i32);
  return launched();
}

int32_t dsr_rows_finite(const float* x, int64_t rows, int64_t n, int64_t ld, int32_t* out, void* stream) {
  if (!x || !out || rows < 0 || n < 1 || ld < n) return DSR_ERR_ARG;
  if (rows == 0) return 0;
  const int64_t chunks = (n + kFiniteChunk - 1) / kFiniteChunk;
  if (chunks > INT_MAX || rows * chunks > INT_MAX) return DSR_ERR_ARG;
  hipLaunchKernelGGL(k_rows_finite, dim3((unsigned)(rows * chunks)), dim3(kFiniteThreads), 0, (hipStream_t)stream, x,
                     n, ld, (int)chunks, out);
  return launched();
}

// Host scan of a count vector in one read-only pass, skipping blocks of 64
// zeros (an OR the compiler vectorises).
extern "C++" template <class T>
static int32_t count_scan(const T* c, int64_t n, int64_t* support, int64_t* out3) {
  int64_t k = 0, mx = 0;
  uint64_t total = 0;  // wraps as NumPy's int64 sum does
  int neg = 0;
  auto visit = [&](int64_t i) {
    const T v = c[i];
    if (v < 0) {
      neg = 1;
    } else if (v > 0) {
      support[k++] = i;
      total += (uint64_t)v;
      if ((int64_t)v > mx) mx = (int64_t)v;
    }
  };
  int64_t i = 0;
  for (; i + 64 <= n; i += 64) {
    T o = 0;
    for (int j = 0; j < 64; ++j) o |= c[i + j];
    if (o == 0) continue;
    for (int j = 0; j < 64; ++j) visit(i + j);
  }
  for (; i < n; ++i) visit(i);
  out3[0] = k;
  out3[1] = (int64_t)total;
  out3[2] = mx;
  return neg;
}

int32_t dsr_count_scan(const void* counts, int32_t width, int64_t n, int64_t* support, int64_t* out3) {
  if ((!counts && n > 0) || !support || !out3 || n < 0 || (width != 4 && width != 8)) return DSR_ERR_ARG;
  return width == 4 ? count_scan((const int32_t*)counts, n, support, out3)
                    : count_scan((const int64_t*)counts, n, support, out3);
}

int32_t dsr_history_from_dense(const int32_t* counts, const int32_t* generated, int64_t rows, int64_t vocab,
                               int64_t ld, int64_t* out_off, int32_t* out_ids, int32_t* out_count,
                               int32_t* out_gen, int64_t cap, int32_t* out_status, void* stream) {
  if ((!counts && rows > 0) || !out_off || (!out_status && rows > 0) || rows < 0 || rows > INT_MAX || vocab < 1 ||
      vocab > DSR_MAX_VOCAB ||
      ld < vocab || cap < 0 || (cap > 0 && (!out_ids || !out_count || !out_gen)))
    return DSR_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  HistDenseArgs h{counts, generated, rows, vocab, ld, cap, out_off, out_ids, out_count, out_gen, out_status};
  if (rows > 0) {
    hipLaunchKernelGGL(k_history_dense<false>, dim3((unsigned)rows), dim3(kThreads), 0, s, h);
    if (hipGetLastError() != hipSuccess) return DSR_ERR_LAUNCH;
  }
  hipLaunchKernelGGL(k_history_offsets, dim3(1), dim3(kThreads), 0, s, out_off, rows);
  if (rows > 0) {
    if (hipGetLastError() != hipSuccess) return DSR_ERR_LAUNCH;
    hipLaunchKernelGGL(k_history_dense<true>, dim3((unsigned)rows), dim3(kThreads), 0, s, h);
  }
  return launched();
}

int32_t dsr_history_append(const int64_t* off, const int32_t* ids, const int32_t* count, const int32_t* gen,
                           const int32_t* tokens, const int64_t* tok_off, const int64_t* gen_from, int64_t rows,
                           int64_t vocab, int64_t* out_off, int32_t* out_ids, int32_t* out_count, int32_t* out_gen,
                           int64_t cap, int32_t* out_status, void* stream) {
  if ((off && (!ids || !count || !gen)) || ((!tokens || !tok_off || !out_status) && rows > 0) || !out_off || rows < 0 ||
      rows > INT_MAX || vocab < 1 || vocab > DSR_MAX_VOCAB || cap < 0 ||
      (cap > 0 && (!out_ids || !out_count || !out_gen)))
    return DSR_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  HistAppendArgs h{off, ids, count, gen, tokens, tok_off, gen_from, rows, vocab, cap,
                   out_off, out_ids, out_count, out_gen, out_status};
  if (rows > 0) {
    hipLaunchKernelGGL(k_history_append<false>, dim3((unsigned)rows), dim3(kThreads), 0, s, h);
    if (hipGetLastError() != hipSuccess) return DSR_ERR_LAUNCH;
  }
  hipLaunchKernelGGL(k_history_offsets, dim3(1), dim3(kThreads), 0, s, out_off, rows);
  if (rows > 0) {
    if (hipGetLastError() != hipSuccess) return DSR_ERR_LAUNCH;
    if (gen_from)
      hipLaunchKernelGGL(HIP_KERNEL_NAME(k_history_append<true, false>), dim3((unsigned)rows), dim3(kThreads), 0, s, h);
    else
      hipLaunchKernelGGL(HIP_KERNEL_NAME(k_history_append<true, true>), dim3((unsigned)rows), dim3(kThreads), 0, s, h);
  }
  return launched();
}

}  // extern "C"
