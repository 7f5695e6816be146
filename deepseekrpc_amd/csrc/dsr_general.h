// The exact per-row sampling pipeline over a float64 workspace row.
//
// One workgroup owns one row.  The row's adjusted logits live in a float64
// workspace row W[0, V); each stage is one strided, coalesced pass over W in
// which every thread keeps kUnroll independent loads in flight (a pass with
// one load in flight per thread is latency-bound, not bandwidth-bound).
// This path accepts every input the reference accepts (any vocabulary size,
// bf16 / f32 / f64 logits, penalties, bias, masks, any top-k / min-p / top-p),
// so it is the fallback for rows the register-resident fast path does not
// take.  The stages follow SamplingPolicy.probabilities (sampling.py:48-106)
// in order and keep its float64 arithmetic; selection uses 11-bit radix
// passes over order-preserving keys instead of the reference's two stable
// argsorts (:90, :98).  Passes are fused where the reference's values allow
// it: the row maximum and its first index come out of the pass that writes
// the adjusted logits, the top-k mask is applied inside the exp pass, min-p
// inside the first normalisation (max(r) is 1 / sum, since the maximum's
// exp is exactly 1), and each normalisation carries the sum of what it
// wrote, so no pass exists only to sum.
#pragma once

#include "dsr_common.h"
#include "dsr_wave.h"

namespace dsr {

struct RowSpec {
  const void* logits;      // row base
  int dtype;
  int64_t V;
  dsr_policy_t pol;
  const int32_t* pen_ids;  // row's sparse history table (or null)
  const int32_t* pen_count;
  const int32_t* pen_gen;
  int64_t pen_n;
  const int32_t* prefix;   // extra tokens counted once each in count and generated count
  int prefix_n;
  const int32_t* bias_ids;
  const double* bias_val;
  int64_t bias_n;
  const uint32_t* allow;   // row's allow bitmask (or null)
  double* W;               // workspace row
  uint32_t* kept_bits;     // optional output: finite after top-k
  int64_t kept_words;
  float* probs_f32;        // optional outputs: the final distribution
  double* probs_f64;
};

constexpr int kRadixBits = 11;
constexpr int kBins = 1 << kRadixBits;  // two per thread
static_assert(kBins == 2 * kThreads, "radix selection assumes two bins per thread");
constexpr int kRadixPasses = 6;         // 5 x 11 bits + 9 bits = 64

struct GenShared {
  BlockScratch b;
  unsigned int hist[kBins];
  unsigned long long hmass[kBins];
  int sel_bin;
  long long sel_above;
  long long sel_count;
  long long bc[4];
};

constexpr int kUnroll = 8;

// Strided pass over [0, n): thread t visits t, t + kThreads, ... in increasing
// order (so per-thread accumulations keep one fixed order), kUnroll elements
// at a time with all of their loads issued before the first use.
template <class T, class Load, class Body>
__device__ __forceinline__ void row_pass(int64_t n, Load load, Body body) {
  for (int64_t b = threadIdx.x; b < n; b += (int64_t)kUnroll * kThreads) {
    T x[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = b + (int64_t)u * kThreads;
      x[u] = i < n ? load(i) : T();
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = b + (int64_t)u * kThreads;
      if (i < n) body(i, x[u]);
    }
  }
}

// The same over one contiguous range [lo, hi), in index order.
template <class T, class Load, class Body>
__device__ __forceinline__ void slice_pass(int64_t lo, int64_t hi, Load load, Body body) {
  for (int64_t b = lo; b < hi; b += kUnroll) {
    T x[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) x[u] = b + u < hi ? load(b + u) : T();
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (b + u < hi) body(b + u, x[u]);
  }
}

__device__ __forceinline__ bool allowed_bit(const uint32_t* allow, int64_t i) {
  return allow == nullptr || ((allow[i >> 5] >> (i & 31)) & 1u);
}

// Contiguous per-thread slice, used where index order matters.
__device__ __forceinline__ void slice_of(int64_t t, int64_t V, int64_t& lo, int64_t& hi) {
  const int64_t ch = (V + kThreads - 1) / kThreads;
  lo = t * ch;
  hi = lo + ch < V ? lo + ch : V;
  if (lo > V) lo = V;
}
__device__ __forceinline__ void thread_slice(int64_t V, int64_t& lo, int64_t& hi) { slice_of(threadIdx.x, V, lo, hi); }

__device__ __forceinline__ uint64_t raw_bits(double x) { return (uint64_t)__double_as_longlong(x); }

// Histogram adds merged per thread while consecutive adds hit one bin, and
// per wave at the end when every pending lane shares a bin: the first radix
// digits of a row are nearly constant, and unmerged LDS atomics on one
// address serialise.
template <class T>
struct RunAdd {
  int bin = -1;
  T n = 0;
  __device__ __forceinline__ void add(T* h, int b, T c) {
    if (b != bin) {
      if (n) atomicAdd(&h[bin], n);
      bin = b;
      n = 0;
    }
    n += c;
  }
  // Every lane of the wave calls.
  __device__ __forceinline__ void flush(T* h) {
    const unsigned long long act = __ballot(n != 0);
    if (act == 0) return;
    const int b0 = __shfl(bin, __ffsll((long long)act) - 1);
    if (__ballot(n != 0 && bin != b0) == 0) {
      const T s = wave_sum(n);
      if (lane_id() == 0) atomicAdd(&h[b0], s);
    } else if (n) {
      atomicAdd(&h[bin], n);
    }
    n = 0;
    bin = -1;
  }
};

// bins[] ranked from the top (largest digit first): the bin where the running
// total reaches rem (1-based), or -1, the total of the bins above it, and
// counts[] of that bin (the token count when bins[] holds masses).  Thread t
// holds bins kBins-1-2t and kBins-2-2t.  Every thread calls.
template <class T>
__device__ int select_from_top(const T* bins, long long rem, GenShared& sh, long long& above,
                               const unsigned int* counts, long long& count) {
  const int t = threadIdx.x;
  const int b0 = kBins - 1 - 2 * t, b1 = b0 - 1;
  const long long c0 = (long long)bins[b0], c1 = (long long)bins[b1];
  if (t == 0) sh.sel_bin = -1;  // ordered before the writes below by the scan's barrier
  long long total;
  const long long ex = block_exclusive_scan_i64(c0 + c1, sh.b, total);
  if (ex < rem && rem <= ex + c0) {
    sh.sel_bin = b0;
    sh.sel_above = ex;
    sh.sel_count = counts[b0];
  } else if (ex + c0 < rem && rem <= ex + c0 + c1) {
    sh.sel_bin = b1;
    sh.sel_above = ex + c0;
    sh.sel_count = counts[b1];
  }
  __syncthreads();
  const int b = sh.sel_bin;
  above = sh.sel_above;
  count = sh.sel_count;
  __syncthreads();
  return b;
}

__device__ __forceinline__ int radix_shift(int pass) { return pass < kRadixPasses - 1 ? 64 - kRadixBits * (pass + 1) : 0; }
__device__ __forceinline__ uint64_t radix_mask(int pass) {
  return pass < kRadixPasses - 1 ? (uint64_t)(kBins - 1) : (1ull << (64 - kRadixBits * (kRadixPasses - 1))) - 1;
}

// Index of the need-th (1-based, in index order) element with keyfn(W[i]) == key.
// Slices are counted per thread; wave 0 then walks the owning slice together.
template <class KeyFn>
__device__ int64_t nth_equal_index(const double* W, int64_t V, uint64_t key, long long need, KeyFn keyfn,
                                   GenShared& sh) {
  if (need <= 0) return -1;
  int64_t lo, hi;
  thread_slice(V, lo, hi);
  long long cnt = 0;
  slice_pass<double>(lo, hi, [&](int64_t i) { return W[i]; }, [&](int64_t, double x) { cnt += keyfn(x) == key; });
  if (threadIdx.x == 0) {
    sh.bc[0] = -1;
    sh.bc[2] = -1;
  }
  long long total;
  const long long base = block_exclusive_scan_i64(cnt, sh.b, total);
  if (base < need && need <= base + cnt) {
    sh.bc[0] = threadIdx.x;
    sh.bc[1] = need - base;
  }
  __syncthreads();
  if (wave_id() == 0 && sh.bc[0] >= 0) {
    const int l = lane_id();
    long long left = sh.bc[1];
    int64_t olo, ohi;
    slice_of(sh.bc[0], V, olo, ohi);
    for (int64_t s = olo; s < ohi; s += 128) {
      const int64_t e0 = s + 2 * l, e1 = e0 + 1;
      const bool m0 = e0 < ohi && keyfn(W[e0]) == key;
      const bool m1 = e1 < ohi && keyfn(W[e1]) == key;
      const uint32_t c = (uint32_t)m0 + (uint32_t)m1;
      const uint32_t incl = wave_scan_dpp(c);
      const uint32_t excl = incl - c;
      const bool hit = (long long)excl < left && left <= (long long)incl;
      const unsigned long long hb = __ballot(hit);
      if (hb) {
        if (hit) sh.bc[2] = (m0 && (long long)excl + 1 == left) ? e0 : e1;
        break;
      }
      left -= (long long)lane_value(incl, 63);
    }
  }
  __syncthreads();
  const int64_t r = sh.bc[2];
  __syncthreads();
  return r;
}

// Radix select of the k-th largest element (1-based, ties counted) and its
// tie group's cut: the first k elements in (key desc, index asc) order are
// those with key > kth, and those with key == kth and index <= cut.  A pass
// whose selected bin is taken whole ends the search: kth is then the bin's
// smallest key and its whole tie group is kept (cut = INT64_MAX).
__device__ void radix_top_k(const double* W, int64_t V, long long k, GenShared& sh, uint64_t& kth, int64_t& cut) {
  uint64_t prefix = 0, pmask = 0;
  long long rem = k;
  for (int pass = 0; pass < kRadixPasses; ++pass) {
    const int shift = radix_shift(pass);
    const uint64_t dm = radix_mask(pass);
    for (int b = threadIdx.x; b < kBins; b += kThreads) sh.hist[b] = 0;
    __syncthreads();
    RunAdd<unsigned int> ra;
    row_pass<double>(
        V, [&](int64_t i) { return W[i]; },
        [&](int64_t, double x) {
          const uint64_t key = order_key(x);
          if ((key & pmask) == prefix) ra.add(sh.hist, (int)((key >> shift) & dm), 1u);
        });
    ra.flush(sh.hist);
    __syncthreads();
    long long above, cb;
    const int b = select_from_top(sh.hist, rem, sh, above, sh.hist, cb);
    rem -= above;
    prefix |= (uint64_t)(b < 0 ? 0 : b) << shift;
    pmask |= dm << shift;
    if (b >= 0 && cb == rem) {
      cut = INT64_MAX;
      if (pass == kRadixPasses - 1) {
        kth = prefix;
        return;
      }
      long long mn = LLONG_MAX;  // smallest key of the bin, sign bit flipped so it orders as signed
      row_pass<double>(
          V, [&](int64_t i) { return W[i]; },
          [&](int64_t, double x) {
            const uint64_t key = order_key(x);
            const long long sk = (long long)(key ^ 0x8000000000000000ull);
            if ((key & pmask) == prefix && sk < mn) mn = sk;
          });
      kth = (uint64_t)block_min_i64(mn, sh.b) ^ 0x8000000000000000ull;
      return;
    }
  }
  kth = prefix;
  cut = nth_equal_index(W, V, kth, rem, [](double x) { return order_key(x); }, sh);
}

// Radix search over probability mass.  W holds r >= 0; ranks run (r desc,
// index asc).  Finds the bit pattern of r at L, the first ranked element
// whose inclusive cumulative mass reaches `top_p`.  Masses are summed as
// 60-bit fixed point (order-independent, so deterministic); the caller
// re-derives the decision exactly in float64.  A pass whose selected bin
// holds one element ends the search (L is that element).  Returns false if
// the whole mass stays below top_p.
__device__ bool radix_mass_crossing(const double* W, int64_t V, double top_p, GenShared& sh, uint64_t& lbits) {
  long long tgt = (long long)(top_p * 0x1p60);
  if (tgt == 0) tgt = 1;  // top_p == 0: the first ranked element is L
  uint64_t prefix = 0, pmask = 0;
  long long above = 0;
  for (int pass = 0; pass < kRadixPasses; ++pass) {
    const int shift = radix_shift(pass);
    const uint64_t dm = radix_mask(pass);
    for (int b = threadIdx.x; b < kBins; b += kThreads) {
      sh.hmass[b] = 0;
      sh.hist[b] = 0;
    }
    __syncthreads();
    RunAdd<unsigned long long> ra;
    RunAdd<unsigned int> rc;
    row_pass<double>(
        V, [&](int64_t i) { return W[i]; },
        [&](int64_t, double x) {
          if (x > 0.0) {
            const uint64_t key = raw_bits(x);
            if ((key & pmask) == prefix) {
              const int d = (int)((key >> shift) & dm);
              ra.add(sh.hmass, d, (unsigned long long)(x * 0x1p60));
              rc.add(sh.hist, d, 1u);
            }
          }
        });
    ra.flush(sh.hmass);
    rc.flush(sh.hist);
    __syncthreads();
    long long ab, cb;
    const int b = select_from_top(sh.hmass, tgt - above, sh, ab, sh.hist, cb);
    if (b < 0) return false;
    above += ab;
    prefix |= (uint64_t)b << shift;
    pmask |= dm << shift;
    if (cb == 1 && pass < kRadixPasses - 1) {
      long long mx = 0;  // the bin's one positive element
      row_pass<double>(
          V, [&](int64_t i) { return W[i]; },
          [&](int64_t, double x) {
            const uint64_t key = raw_bits(x);
            if (x > 0.0 && (key & pmask) == prefix) mx = (long long)key;
          });
      lbits = (uint64_t)block_max_i64(mx, sh.b);
      return true;
    }
  }
  lbits = prefix;
  return true;
}


// Wave 0 of the workgroup finishes a CDF search inside one contiguous slice
// [lo, hi): the first element whose running sum (from `base`) exceeds thr.
// Two elements per lane, one wave scan per 128 elements.  `margin` is set
// when the decision sits within tol of a boundary, or when rounding left no
// crossing inside the slice (the last positive element is taken).
template <class WF>
__device__ void wave_slice_cdf(WF wf, int64_t lo, int64_t hi, double base, double thr, double tol, int64_t& tok,
                               int& margin) {
  const int l = lane_id();
  double c = base;
  int64_t last = -1;
  for (int64_t s = lo; s < hi; s += 128) {
    const int64_t e0 = s + 2 * l, e1 = e0 + 1;
    const double w0 = e0 < hi ? wf(e0) : 0.0, w1 = e1 < hi ? wf(e1) : 0.0;
    const double pr = w0 + w1;
    const double incl = wave_scan_dpp(pr);
    double excl = __shfl_up(incl, 1);
    if (l == 0) excl = 0.0;
    const double b0 = c + excl;  // running sum before e0
    const double c0 = b0 + w0;
    const double c1 = c0 + w1;
    const bool x0 = w0 > 0.0 && c0 > thr, x1 = w1 > 0.0 && c1 > thr;
    const unsigned long long cross = __ballot(x0 || x1);
    if (cross) {
      const int f = __ffsll((long long)cross) - 1;
      const int64_t t = x0 ? e0 : e1;
      const double cv = x0 ? c0 : c1;
      const double before = x0 ? b0 : (w0 > 0.0 ? c0 : b0);
      const int m = (cv - thr <= tol || (before > 0.0 && thr - before <= tol)) ? 1 : 0;
      tok = (int64_t)__shfl((long long)t, f);
      margin = __shfl(m, f);
      return;
    }
    const unsigned long long pb = __ballot(w0 > 0.0 || w1 > 0.0);
    if (pb) {
      const int g = 63 - __clzll((long long)pb);
      last = (int64_t)__shfl((long long)(w1 > 0.0 ? e1 : e0), g);
    }
    c = c + lane_value(incl, 63);
  }
  tok = last;
  margin = 1;
}

// categorical's CDF search (sampling.py:126-128) over weights wf(i) >= 0: the
// first index whose running sum exceeds u times the total, in index order.
// Per-thread contiguous slices are summed, scanned across the workgroup, and
// wave 0 walks the slice that holds the crossing.
template <class WF>
__device__ int64_t cdf_search_fn(int64_t V, WF wf, double u, long long npos, GenShared& sh, unsigned& flags) {
  int64_t lo, hi;
  thread_slice(V, lo, hi);
  double part = 0.0;
  slice_pass<double>(lo, hi, wf, [&](int64_t, double w) { part += w; });
  double total;
  const double base = block_exclusive_scan_f64(part, sh.b, total);
  const double thr = u * total;
  const long long cand = (part > 0.0 && base <= thr) ? (long long)threadIdx.x : -1;
  const long long owner = block_max_i64(cand, sh.b);
  if ((long long)threadIdx.x == owner) sh.bc[0] = __double_as_longlong(base);
  __syncthreads();
  if (wave_id() == 0 && owner >= 0) {
    int64_t olo, ohi;
    slice_of(owner, V, olo, ohi);
    const double tol = ((double)npos + 16.0) * 0x1p-51 * total;
    int64_t tok;
    int margin;
    wave_slice_cdf(wf, olo, ohi, __longlong_as_double(sh.bc[0]), thr, tol, tok, margin);
    if (lane_id() == 0) {
      sh.bc[1] = tok;
      sh.bc[2] = margin;
    }
  }
  __syncthreads();
  const int64_t tok = owner >= 0 ? (int64_t)sh.bc[1] : -1;
  if (owner < 0 || sh.bc[2]) flags |= DSR_FLAG_MARGIN;
  __syncthreads();
  return tok;
}

__device__ int64_t cdf_search(const double* W, int64_t V, double u, long long npos, GenShared& sh, unsigned& flags) {
  return cdf_search_fn(V, [&](int64_t i) { return W[i]; }, u, npos, sh, flags);
}

// Row maximum and the first index holding it (each thread visits its indices
// in increasing order, so a strict comparison keeps the first), plus whether
// any value is finite.
struct RowMax {
  double m = -INFINITY;
  long long first = LLONG_MAX;
  int fin = 0;
  __device__ __forceinline__ void add(int64_t i, double x) {
    if (x > m) {
      m = x;
      first = i;
    }
    fin |= isfinite(x) ? 1 : 0;
  }
};

// Adjusted logits: float64 copy, penalties, bias, mask (sampling.py:49-81).
// Returns a status code; on DSR_OK W holds the adjusted logits, M their
// maximum and `first` the first index holding it.
__device__ int adjust_logits(const RowSpec& r, GenShared& sh, double& M, long long& first) {
  const int64_t V = r.V;
  double* W = r.W;
  int bad = 0;
  RowMax st;
  struct LX {
    double x;
    uint32_t w;
  };
  row_pass<LX>(
      V, [&](int64_t i) { return LX{load_logit(r.logits, r.dtype, i), r.allow ? r.allow[i >> 5] : ~0u}; },
      [&](int64_t i, LX v) {
        double x = v.x;
        if (x != x || x == INFINITY) bad = 1;
        if (!((v.w >> (i & 31)) & 1u)) x = -INFINITY;  // masking first is equivalent: -inf is a fixed point below
        W[i] = x;
        st.add(i, x);
      });
  if (block_or(bad, sh.b)) return DSR_E_LOGITS;

  const dsr_policy_t& p = r.pol;
  const bool touched = r.pen_n > 0 || r.prefix_n > 0 || r.bias_n > 0;
  if (r.pen_n > 0 || r.prefix_n > 0) {
    // Validate the table (sampling.py:55-58,62-65) with the prefix tokens added.
    long long csum = 0;
    int bad = 0;  // 3: prefix token out of range, 2: counts, 1: generated counts
    for (int64_t e = threadIdx.x; e < r.pen_n; e += kThreads) {
      int32_t id = r.pen_ids[e];
      long long c = r.pen_count[e], g = r.pen_gen[e];
      int b = 0;
      if (id < 0 || id >= V || (e > 0 && r.pen_ids[e - 1] >= id) || c < 0) b = 2;
      for (int q = 0; q < r.prefix_n; ++q) {
        if (r.prefix[q] == id) {
          ++c;
          ++g;
        }
      }
      if (c > DSR_MAX_COUNT) b = 2;
      if (b == 0 && (g < 0 || g > c)) b = 1;
      bad = b > bad ? b : bad;
      csum += c;
    }
    if (threadIdx.x == 0) {
      for (int q = 0; q < r.prefix_n; ++q) {
        if (r.prefix[q] < 0 || r.prefix[q] >= V) bad = 3;
      }
    }
    if (threadIdx.x < r.prefix_n) {
      // Prefix tokens absent from the table contribute to the total once each.
      int32_t id = r.prefix[threadIdx.x];
      int64_t lo = 0, hi = r.pen_n;
      while (lo < hi) {
        int64_t mid = (lo + hi) >> 1;
        if (r.pen_ids[mid] < id) lo = mid + 1; else hi = mid;
      }
      if (!(lo < r.pen_n && r.pen_ids[lo] == id)) csum += 1;
    }
    const long long worst = block_max_i64(bad, sh.b);
    csum = block_sum_i64(csum, sh.b);
    if (worst == 3) return DSR_E_TOKEN;
    if (worst == 2 || csum > DSR_MAX_COUNT) return DSR_E_COUNTS;
    if (worst == 1) return DSR_E_GENERATED;

    // Repetition on count > 0, then one subtraction of presence*(g>0) + frequency*g
    // (sampling.py:59-66).  Ids are unique, so the scatter is race-free.
    for (int64_t e = threadIdx.x; e < r.pen_n; e += kThreads) {
      int32_t id = r.pen_ids[e];
      long long c = r.pen_count[e], g = r.pen_gen[e];
      for (int q = 0; q < r.prefix_n; ++q) {
        if (r.prefix[q] == id) {
          ++c;
          ++g;
        }
      }
      double x = W[id];
      if (c > 0) x = x >= 0.0 ? x / p.repetition_penalty : x * p.repetition_penalty;
      double pen = p.presence_penalty * (g > 0 ? 1.0 : 0.0) + p.frequency_penalty * (double)g;
      W[id] = x - pen;
    }
    if (threadIdx.x < r.prefix_n) {
      const int q = threadIdx.x;
      int32_t id = r.prefix[q];
      bool first_q = true;
      for (int j = 0; j < q; ++j) first_q = first_q && r.prefix[j] != id;
      int64_t lo = 0, hi = r.pen_n;
      while (lo < hi) {
        int64_t mid = (lo + hi) >> 1;
        if (r.pen_ids[mid] < id) lo = mid + 1; else hi = mid;
      }
      bool in_table = lo < r.pen_n && r.pen_ids[lo] == id;
      if (first_q && !in_table) {
        long long c = 0;
        for (int j = 0; j < r.prefix_n; ++j) c += r.prefix[j] == id;
        double x = W[id];
        x = x >= 0.0 ? x / p.repetition_penalty : x * p.repetition_penalty;
        double pen = p.presence_penalty * 1.0 + p.frequency_penalty * (double)c;
        W[id] = x - pen;
      }
    }
    __syncthreads();
  }
  if (r.bias_n > 0) {
    int bad_b = 0;
    for (int64_t e = threadIdx.x; e < r.bias_n; e += kThreads) {
      int32_t id = r.bias_ids[e];
      double b = r.bias_val[e];
      if (id < 0 || id >= V || (e > 0 && r.bias_ids[e - 1] >= id) || !(b >= -100.0 && b <= 100.0)) bad_b = 1;
    }
    if (block_or(bad_b, sh.b)) return DSR_E_BIAS;
    for (int64_t e = threadIdx.x; e < r.bias_n; e += kThreads) W[r.bias_ids[e]] += r.bias_val[e];
    __syncthreads();
  }
  if (touched) {
    st = RowMax();
    row_pass<double>(V, [&](int64_t i) { return W[i]; }, [&](int64_t i, double x) { st.add(i, x); });
  }
  if (!block_or(st.fin, sh.b)) return DSR_E_MASKED;
  M = block_max(st.m, sh.b);
  first = block_min_i64(st.m == M ? st.first : LLONG_MAX, sh.b);
  return DSR_OK;
}

// Kept-token bits after top-k (1 = finite after step 9 of sampling.py:89-91).
// A wave covers 64 consecutive tokens per round, so each ballot is two whole words.
__device__ void write_kept_bits(const double* W, int64_t V, bool topk, uint64_t kth, int64_t cut, uint32_t* bits,
                                int64_t words) {
  for (int64_t base = 0; base < V; base += (int64_t)kUnroll * kThreads) {
    double z[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + (int64_t)u * kThreads + threadIdx.x;
      z[u] = i < V ? W[i] : -(double)INFINITY;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + (int64_t)u * kThreads + threadIdx.x;
      bool f = z[u] > -(double)INFINITY;
      if (topk) {
        const uint64_t key = order_key(z[u]);
        f = f && (key > kth || (key == kth && i <= cut));
      }
      const unsigned long long m = __ballot(f);
      const int64_t w0 = (base + (int64_t)u * kThreads + 64 * wave_id()) >> 5;
      if (lane_id() == 0 && w0 < words) bits[w0] = (uint32_t)m;
      if (lane_id() == 0 && w0 + 1 < words) bits[w0 + 1] = (uint32_t)(m >> 32);
    }
  }
}

struct DistOut {
  int64_t onehot;   // greedy argmax, or -1
  long long npos;   // positive entries of the final distribution
  long long first;  // first positive index
};

struct IdentityMap {
  __device__ __forceinline__ int64_t operator()(int64_t i) const { return i; }
};

// The top-p tie group at the crossing value rt (sampling.py:97-102): A is the
// mass of the n_above tokens above rt, n_tie tokens equal rt.  Tie member j
// (index order) has exclusive prefix A + j*rt; it is kept while that prefix
// is below top_p, and rank 0 always.  Returns the members kept; `close` is
// set when a float64 prefix over this many terms could round across top_p.
__device__ __forceinline__ long long top_p_tie_keep(double A, long long n_above, long long n_tie, double rt,
                                                    double top_p, bool& close) {
  long long keep = 0;
  {
    double q = ceil((top_p - A) / rt);
    keep = q <= 0.0 ? 0 : (q >= (double)n_tie ? n_tie : (long long)q);
    while (keep > 0 && A + (double)(keep - 1) * rt >= top_p) --keep;
    while (keep < n_tie && A + (double)keep * rt < top_p) ++keep;
  }
  if (n_above == 0 && keep == 0) keep = 1;
  // Rounding band of a float64 prefix over this many terms.
  const double tol = ((double)(n_above + keep) + 16.0) * 0x1p-51;
  close = fabs(A + (double)keep * rt - top_p) <= tol;                 // first removed
  if (keep >= 1 && n_above + keep > 1)
    close = close || fabs(A + (double)(keep - 1) * rt - top_p) <= tol;  // last kept
  if (keep == 0 && n_above > 0) close = true;                          // crossing above this group
  if (keep == n_tie && A + (double)n_tie * rt < top_p) close = true;   // crossing below it
  return keep;
}

// Steps 10-13 (sampling.py:92-106) over W[0, n), which holds s = (v - max) / T
// and the top-k decision (`kth`, `cut` from radix_top_k).  Position j of W is
// token map(j), positions in token order, so index-order ties and the CDF keep
// the reference's order.  `vocab` sizes the rounding band of a sum over the
// whole row.  `s1_row`, when not NaN, is the sum of exp(s) over the whole
// row (W then holds only part of the row's tokens, and the rest are removed
// by min-p or top-p).  On DSR_OK, W holds the final probabilities (also
// written to the optional outputs).
template <class Map>
__device__ __forceinline__ int filter_tail(const RowSpec& r, double* W, int64_t n, int64_t vocab, bool topk,
                                           uint64_t kth, int64_t cut, GenShared& sh, unsigned& flags, DistOut& out,
                                           Map map, double s1_row = __longlong_as_double(0x7FF8000000000000ll)) {
  const dsr_policy_t& p = r.pol;
  auto ldW = [&](int64_t i) { return W[i]; };
  double acc = 0.0;  // sampling.py:92-93; removed tokens are exp(-inf) = 0
  row_pass<double>(n, ldW, [&](int64_t i, double z) {
    bool keep = z > -(double)INFINITY;
    if (topk) {
      const uint64_t key = order_key(z);
      keep = keep && (key > kth || (key == kth && i <= cut));
    }
    double e = 0.0;
    if (keep) e = exp(z);
    W[i] = e;
    acc += e;
  });
  const double s1_own = block_sum(acc, sh.b);
  const double s1 = s1_row == s1_row ? s1_row : s1_own;

  double cur = 0.0;  // sum of what the last pass wrote
  if (p.min_p != 0.0) {  // sampling.py:94-96
    // max(r) = 1 / s1: the maximum's exp is exactly 1 and division is monotone.
    const double cut_p = p.min_p * (1.0 / s1);
    const double tol = cut_p * 0x1p-49;
    int close = 0;
    double acc2 = 0.0;
    row_pass<double>(n, ldW, [&](int64_t i, double e) {
      double x = e / s1;
      if (x > 0.0 && fabs(x - cut_p) <= tol) close = 1;
      if (x < cut_p) x = 0.0;
      W[i] = x;
      acc2 += x;
    });
    if (block_or(close, sh.b)) flags |= DSR_FLAG_MARGIN;
    const double s2 = block_sum(acc2, sh.b);
    row_pass<double>(n, ldW, [&](int64_t i, double x) {
      x = x / s2;
      W[i] = x;
      cur += x;
    });
  } else {
    row_pass<double>(n, ldW, [&](int64_t i, double e) {
      const double x = e / s1;
      W[i] = x;
      cur += x;
    });
  }
  __syncthreads();

  if (p.top_p < 1.0) {  // sampling.py:97-102
    uint64_t lbits;
    if (radix_mass_crossing(W, n, p.top_p, sh, lbits)) {
      const double rt = __longlong_as_double((long long)lbits);
      double a = 0.0;
      long long n_above = 0, n_tie = 0;
      row_pass<double>(n, ldW, [&](int64_t, double x) {
        a += x > rt ? x : 0.0;
        n_above += x > rt ? 1 : 0;
        n_tie += x == rt ? 1 : 0;
      });
      const double A = block_sum(a, sh.b);
      n_above = block_sum_i64(n_above, sh.b);
      n_tie = block_sum_i64(n_tie, sh.b);
      bool close;
      const long long keep = top_p_tie_keep(A, n_above, n_tie, rt, p.top_p, close);
      if (close) flags |= DSR_FLAG_MARGIN;
      const int64_t cutp = nth_equal_index(W, n, lbits, keep, [](double x) { return raw_bits(x); }, sh);
      cur = 0.0;
      row_pass<double>(n, ldW, [&](int64_t i, double x) {
        if (x < rt || (x == rt && i > cutp)) {
          x = 0.0;
          W[i] = 0.0;
        }
        cur += x;
      });
      __syncthreads();
    } else {
      // The whole mass stays below top_p: nothing is removed.
      const double tot = block_sum(cur, sh.b);
      if (fabs(tot - p.top_p) <= ((double)vocab + 16.0) * 0x1p-51) flags |= DSR_FLAG_MARGIN;
    }
  }

  const double total = block_sum(cur, sh.b);  // sampling.py:103-106
  if (!(total > 0.0) || !isfinite(total)) return DSR_E_NO_MASS;
  long long npos = 0, fpos = LLONG_MAX;
  row_pass<double>(n, ldW, [&](int64_t i, double x) {
    x = x / total;
    W[i] = x;
    if (r.probs_f32) r.probs_f32[map(i)] = (float)x;
    if (r.probs_f64) r.probs_f64[map(i)] = x;
    if (x > 0.0) {
      ++npos;
      if (i < fpos) fpos = i;
    }
  });
  out.npos = block_sum_i64(npos, sh.b);
  const long long f = block_min_i64(fpos, sh.b);
  out.first = f == LLONG_MAX ? f : (long long)map(f);
  return DSR_OK;
}

// Full distribution (sampling.py:48-106).  On DSR_OK, W holds the final
// probabilities (also written to the optional outputs).
__device__ __forceinline__ int general_distribution(const RowSpec& r, GenShared& sh, unsigned& flags, DistOut& out) {
  out.onehot = -1;
  out.npos = 0;
  out.first = -1;
  if (!policy_ok(r.pol)) return DSR_E_POLICY;
  double M;
  long long amax;
  int st = adjust_logits(r, sh, M, amax);
  if (st != DSR_OK) return st;
  const int64_t V = r.V;
  double* W = r.W;
  const dsr_policy_t& p = r.pol;
  auto ldW = [&](int64_t i) { return W[i]; };

  if (p.temperature == 0.0) {  // sampling.py:82-85: first index of the maximum
    out.onehot = amax;
    out.npos = 1;
    out.first = amax;
    row_pass<int>(
        V, [&](int64_t) { return 0; },
        [&](int64_t i, int) {
          const double x = i == amax ? 1.0 : 0.0;
          W[i] = x;
          if (r.probs_f32) r.probs_f32[i] = (float)x;
          if (r.probs_f64) r.probs_f64[i] = x;
        });
    if (r.kept_bits) {
      // A greedy row keeps the argmax alone.
      for (int64_t w = threadIdx.x; w < r.kept_words; w += kThreads) r.kept_bits[w] = 0;
      __syncthreads();
      if (threadIdx.x == 0) r.kept_bits[amax >> 5] = 1u << (amax & 31);
    }
    __syncthreads();
    return DSR_OK;
  }
  if (M == INFINITY) return DSR_E_NO_MASS;  // inf - inf: the reference's sum turns NaN

  const double T = p.temperature;
  row_pass<double>(V, ldW, [&](int64_t i, double x) { W[i] = (x - M) / T; });  // sampling.py:86-88, true division
  __syncthreads();

  const bool topk = p.top_k > 0 && p.top_k < V;  // sampling.py:89-91
  uint64_t kth = 0;
  int64_t cut = -1;
  if (topk) {
    radix_top_k(W, V, p.top_k, sh, kth, cut);
  }
  if (r.kept_bits) write_kept_bits(W, V, topk, kth, cut, r.kept_bits, r.kept_words);

  return filter_tail(r, W, V, V, topk, kth, cut, sh, flags, out, IdentityMap());
}

}  // namespace dsr
