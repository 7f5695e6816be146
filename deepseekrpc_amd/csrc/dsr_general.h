// The exact per-row sampling pipeline over a float64 workspace row.
//
// One workgroup owns one row.  The row's adjusted logits live in a float64
// workspace row W[0, V); each stage is one strided, coalesced pass over W.
// This path accepts every input the reference accepts (any vocabulary size,
// bf16 / f32 / f64 logits, penalties, bias, masks, any top-k / min-p / top-p),
// so it is the fallback for rows the register-resident fast path does not
// take.  The stages follow SamplingPolicy.probabilities (sampling.py:48-106)
// in order; selection uses radix passes over order-preserving keys instead of
// the reference's two stable argsorts (:90, :98).
#pragma once

#include "dsr_common.h"

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
};

struct GenShared {
  BlockScratch b;
  unsigned int hist[256];
  unsigned long long hmass[256];
  int sel_bin;
  unsigned int sel_above_cnt;
  unsigned long long sel_above_mass;
};

// Strided loop over [0, V): consecutive threads touch consecutive elements.
#define DSR_FOR_ROW(i, V) for (int64_t i = threadIdx.x; i < (V); i += kThreads)

__device__ __forceinline__ bool allowed_bit(const uint32_t* allow, int64_t i) {
  return allow == nullptr || ((allow[i >> 5] >> (i & 31)) & 1u);
}

// Contiguous per-thread slice, used where index order matters.
__device__ __forceinline__ void thread_slice(int64_t V, int64_t& lo, int64_t& hi) {
  int64_t ch = (V + kThreads - 1) / kThreads;
  lo = (int64_t)threadIdx.x * ch;
  hi = lo + ch < V ? lo + ch : V;
  if (lo > V) lo = V;
}

// Index of the need-th (1-based, in index order) element with keyfn(W[i]) == key.
template <class KeyFn>
__device__ int64_t nth_equal_index(const double* W, int64_t V, uint64_t key, long long need, KeyFn keyfn,
                                   GenShared& sh) {
  if (need <= 0) return -1;
  int64_t lo, hi;
  thread_slice(V, lo, hi);
  long long cnt = 0;
  for (int64_t i = lo; i < hi; ++i) cnt += keyfn(W[i]) == key;
  long long total;
  long long base = block_exclusive_scan_i64(cnt, sh.b, total);
  if (base < need && need <= base + cnt) {
    long long left = need - base;
    for (int64_t i = lo; i < hi; ++i) {
      if (keyfn(W[i]) == key && --left == 0) {
        sh.b.bcast_i[0] = i;
        break;
      }
    }
  }
  __syncthreads();
  int64_t r = sh.b.bcast_i[0];
  __syncthreads();
  return r;
}

// Radix select: key of the k-th largest element (1-based, ties counted) and
// `need`, how many elements carrying that key are ranked within the first k.
__device__ void radix_kth_largest(const double* W, int64_t V, long long k, GenShared& sh, uint64_t& kth,
                                  long long& need) {
  uint64_t prefix = 0, pmask = 0;
  long long rem = k;
  for (int shift = 56; shift >= 0; shift -= 8) {
    for (int b = threadIdx.x; b < 256; b += kThreads) sh.hist[b] = 0;
    __syncthreads();
    DSR_FOR_ROW(i, V) {
      uint64_t key = order_key(W[i]);
      if ((key & pmask) == prefix) atomicAdd(&sh.hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      const int l = threadIdx.x;
      unsigned c[4];
      for (int j = 0; j < 4; ++j) c[j] = sh.hist[4 * l + j];
      unsigned lsum = c[0] + c[1] + c[2] + c[3];
      unsigned suf = lsum;
      for (int o = 1; o < 64; o <<= 1) {
        unsigned y = __shfl_down(suf, o);
        if (l + o < 64) suf += y;
      }
      long long above = (long long)(suf - lsum);
      for (int j = 3; j >= 0; --j) {
        if (above < rem && rem <= above + (long long)c[j]) {
          sh.sel_bin = 4 * l + j;
          sh.sel_above_cnt = (unsigned)above;
        }
        above += c[j];
      }
    }
    __syncthreads();
    rem -= (long long)sh.sel_above_cnt;
    prefix |= (uint64_t)sh.sel_bin << shift;
    pmask |= 0xFFull << shift;
    __syncthreads();
  }
  kth = prefix;
  need = rem;
}

// Radix search over probability mass.  W holds r >= 0; ranks run (r desc,
// index asc).  Finds the bit pattern of r at L, the first ranked element
// whose inclusive cumulative mass reaches `top_p`.  Masses are summed as
// 60-bit fixed point (order-independent, so deterministic); the caller
// re-derives the decision exactly in float64.  Returns false if the whole
// mass stays below top_p.
__device__ bool radix_mass_crossing(const double* W, int64_t V, double top_p, GenShared& sh, uint64_t& lbits) {
  unsigned long long tgt = (unsigned long long)(top_p * 0x1p60);
  if (tgt == 0) tgt = 1;  // top_p == 0: the first ranked element is L
  uint64_t prefix = 0, pmask = 0;
  unsigned long long above = 0;
  for (int shift = 56; shift >= 0; shift -= 8) {
    for (int b = threadIdx.x; b < 256; b += kThreads) sh.hmass[b] = 0;
    if (threadIdx.x == 0) sh.sel_bin = -1;
    __syncthreads();
    DSR_FOR_ROW(i, V) {
      double x = W[i];
      if (x > 0.0) {
        uint64_t key = (uint64_t)__double_as_longlong(x);
        if ((key & pmask) == prefix)
          atomicAdd(&sh.hmass[(key >> shift) & 255u], (unsigned long long)(x * 0x1p60));
      }
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      const int l = threadIdx.x;
      unsigned long long m[4];
      for (int j = 0; j < 4; ++j) m[j] = sh.hmass[4 * l + j];
      unsigned long long lsum = m[0] + m[1] + m[2] + m[3];
      unsigned long long suf = lsum;
      for (int o = 1; o < 64; o <<= 1) {
        unsigned long long y = __shfl_down(suf, o);
        if (l + o < 64) suf += y;
      }
      unsigned long long excl = above + (suf - lsum);
      for (int j = 3; j >= 0; --j) {
        if (excl < tgt && tgt <= excl + m[j]) {
          sh.sel_bin = 4 * l + j;
          sh.sel_above_mass = excl;
        }
        excl += m[j];
      }
    }
    __syncthreads();
    int b = sh.sel_bin;
    unsigned long long ab = sh.sel_above_mass;
    __syncthreads();
    if (b < 0) return false;
    above = ab;
    prefix |= (uint64_t)b << shift;
    pmask |= 0xFFull << shift;
  }
  lbits = prefix;
  return true;
}

__device__ __forceinline__ uint64_t raw_bits(double x) { return (uint64_t)__double_as_longlong(x); }

// Writes one bit per token (1 = W[i] finite) into `bits`.  A wave covers 64
// consecutive tokens per iteration, so each ballot is two whole words.
__device__ void write_finite_bits(const double* W, int64_t V, uint32_t* bits, int64_t words) {
  for (int64_t base = 0; base < V; base += kThreads) {
    int64_t i = base + threadIdx.x;
    bool f = i < V && isfinite(W[i]);
    unsigned long long m = __ballot(f);
    int64_t w0 = (base + 64 * wave_id()) >> 5;
    if (lane_id() == 0 && w0 < words) bits[w0] = (uint32_t)m;
    if (lane_id() == 0 && w0 + 1 < words) bits[w0 + 1] = (uint32_t)(m >> 32);
  }
}

// Adjusted logits: float64 copy, penalties, bias, mask (sampling.py:49-81).
// Returns a status code; on DSR_OK W holds the adjusted logits.
__device__ int adjust_logits(const RowSpec& r, GenShared& sh) {
  const int64_t V = r.V;
  double* W = r.W;
  int bad = 0;
  DSR_FOR_ROW(i, V) {
    double x = load_logit(r.logits, r.dtype, i);
    if (x != x || x == INFINITY) bad = 1;
    if (!allowed_bit(r.allow, i)) x = -INFINITY;  // masking first is equivalent: -inf is a fixed point below
    W[i] = x;
  }
  if (block_or(bad, sh.b)) return DSR_E_LOGITS;

  const dsr_policy_t& p = r.pol;
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
      bool first = true;
      for (int j = 0; j < q; ++j) first = first && r.prefix[j] != id;
      int64_t lo = 0, hi = r.pen_n;
      while (lo < hi) {
        int64_t mid = (lo + hi) >> 1;
        if (r.pen_ids[mid] < id) lo = mid + 1; else hi = mid;
      }
      bool in_table = lo < r.pen_n && r.pen_ids[lo] == id;
      if (first && !in_table) {
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
  int fin = 0;
  DSR_FOR_ROW(i, V) fin |= isfinite(W[i]) ? 1 : 0;
  if (!block_or(fin, sh.b)) return DSR_E_MASKED;
  return DSR_OK;
}

// Full distribution (sampling.py:48-106).  On DSR_OK, W holds the final
// probabilities; `onehot` is the greedy argmax (or -1).
__device__ int general_distribution(const RowSpec& r, GenShared& sh, unsigned& flags, int64_t& onehot) {
  onehot = -1;
  if (!policy_ok(r.pol)) return DSR_E_POLICY;
  int st = adjust_logits(r, sh);
  if (st != DSR_OK) return st;
  const int64_t V = r.V;
  double* W = r.W;
  const dsr_policy_t& p = r.pol;

  double m = -INFINITY;
  DSR_FOR_ROW(i, V) m = W[i] > m ? W[i] : m;
  const double M = block_max(m, sh.b);

  if (p.temperature == 0.0) {  // sampling.py:82-85: first index of the maximum
    long long first = LLONG_MAX;
    DSR_FOR_ROW(i, V) if (W[i] == M && i < first) first = i;
    onehot = block_min_i64(first, sh.b);
    DSR_FOR_ROW(i, V) W[i] = i == onehot ? 1.0 : 0.0;
    if (r.kept_bits) {
      // A greedy row keeps the argmax alone.
      for (int64_t w = threadIdx.x; w < r.kept_words; w += kThreads) r.kept_bits[w] = 0;
      __syncthreads();
      if (threadIdx.x == 0) r.kept_bits[onehot >> 5] = 1u << (onehot & 31);
    }
    __syncthreads();
    return DSR_OK;
  }
  if (M == INFINITY) return DSR_E_NO_MASS;  // inf - inf: the reference's sum turns NaN

  DSR_FOR_ROW(i, V) W[i] = (W[i] - M) / p.temperature;  // sampling.py:86-88, true division
  __syncthreads();

  if (p.top_k > 0 && p.top_k < V) {  // sampling.py:89-91
    uint64_t kth;
    long long need;
    radix_kth_largest(W, V, p.top_k, sh, kth, need);
    int64_t cut = nth_equal_index(W, V, kth, need, [](double x) { return order_key(x); }, sh);
    DSR_FOR_ROW(i, V) {
      uint64_t key = order_key(W[i]);
      if (key < kth || (key == kth && i > cut)) W[i] = -INFINITY;
    }
    __syncthreads();
  }
  if (r.kept_bits) write_finite_bits(W, V, r.kept_bits, r.kept_words);

  double acc = 0.0;  // sampling.py:92-93
  DSR_FOR_ROW(i, V) {
    double e = exp(W[i]);
    W[i] = e;
    acc += e;
  }
  const double s1 = block_sum(acc, sh.b);
  DSR_FOR_ROW(i, V) W[i] = W[i] / s1;
  __syncthreads();

  if (p.min_p != 0.0) {  // sampling.py:94-96
    double rm = -INFINITY;
    DSR_FOR_ROW(i, V) rm = W[i] > rm ? W[i] : rm;
    const double cut = p.min_p * block_max(rm, sh.b);
    const double tol = cut * 0x1p-49;
    int close = 0;
    double acc2 = 0.0;
    DSR_FOR_ROW(i, V) {
      double x = W[i];
      if (x > 0.0 && fabs(x - cut) <= tol) close = 1;
      if (x < cut) x = 0.0;
      W[i] = x;
      acc2 += x;
    }
    if (block_or(close, sh.b)) flags |= DSR_FLAG_MARGIN;
    const double s2 = block_sum(acc2, sh.b);
    DSR_FOR_ROW(i, V) W[i] = W[i] / s2;
    __syncthreads();
  }

  if (p.top_p < 1.0) {  // sampling.py:97-102
    uint64_t lbits;
    if (radix_mass_crossing(W, V, p.top_p, sh, lbits)) {
      const double rt = __longlong_as_double((long long)lbits);
      double a = 0.0;
      long long n_above = 0, n_tie = 0;
      DSR_FOR_ROW(i, V) {
        double x = W[i];
        if (x > rt) {
          a += x;
          ++n_above;
        } else if (x == rt) {
          ++n_tie;
        }
      }
      const double A = block_sum(a, sh.b);
      n_above = block_sum_i64(n_above, sh.b);
      n_tie = block_sum_i64(n_tie, sh.b);
      // Tie member j (index order) has exclusive prefix A + j*rt; it is kept
      // while that prefix is below top_p, and rank 0 always (sampling.py:99-102).
      long long keep = 0;
      {
        double q = ceil((p.top_p - A) / rt);
        keep = q <= 0.0 ? 0 : (q >= (double)n_tie ? n_tie : (long long)q);
        while (keep > 0 && A + (double)(keep - 1) * rt >= p.top_p) --keep;
        while (keep < n_tie && A + (double)keep * rt < p.top_p) ++keep;
      }
      if (n_above == 0 && keep == 0) keep = 1;
      // Rounding band of a float64 prefix over this many terms.
      const double tol = ((double)(n_above + keep) + 16.0) * 0x1p-51;
      bool close = fabs(A + (double)keep * rt - p.top_p) <= tol;           // first removed
      if (keep >= 1 && n_above + keep > 1)
        close = close || fabs(A + (double)(keep - 1) * rt - p.top_p) <= tol;  // last kept
      if (keep == 0 && n_above > 0) close = true;                          // crossing above this group
      if (keep == n_tie && A + (double)n_tie * rt < p.top_p) close = true;  // crossing below it
      if (close) flags |= DSR_FLAG_MARGIN;
      const uint64_t tkey = lbits;
      int64_t cut = nth_equal_index(W, V, tkey, keep, [](double x) { return raw_bits(x); }, sh);
      DSR_FOR_ROW(i, V) {
        double x = W[i];
        if (x < rt || (x == rt && i > cut)) W[i] = 0.0;
      }
      __syncthreads();
    } else {
      // The whole mass stays below top_p: nothing is removed.
      double tot = 0.0;
      DSR_FOR_ROW(i, V) tot += W[i];
      tot = block_sum(tot, sh.b);
      if (fabs(tot - p.top_p) <= ((double)V + 16.0) * 0x1p-51) flags |= DSR_FLAG_MARGIN;
    }
  }

  double acc3 = 0.0;  // sampling.py:103-106
  DSR_FOR_ROW(i, V) acc3 += W[i];
  const double total = block_sum(acc3, sh.b);
  if (!(total > 0.0) || !isfinite(total)) return DSR_E_NO_MASS;
  DSR_FOR_ROW(i, V) W[i] = W[i] / total;
  __syncthreads();
  return DSR_OK;
}

// categorical's CDF search (sampling.py:126-128): the first index whose
// running sum exceeds u times the total, in index order.
__device__ int64_t cdf_search(const double* W, int64_t V, double u, long long npos, GenShared& sh,
                              unsigned& flags) {
  int64_t lo, hi;
  thread_slice(V, lo, hi);
  double part = 0.0;
  for (int64_t i = lo; i < hi; ++i) part += W[i];
  double total;
  const double base = block_exclusive_scan_f64(part, sh.b, total);
  const double thr = u * total;
  long long cand = (part > 0.0 && base <= thr) ? (long long)threadIdx.x : -1;
  const long long owner = block_max_i64(cand, sh.b);
  if ((long long)threadIdx.x == owner) {
    double c = base, before = base;
    int64_t tok = -1, last = -1;
    for (int64_t i = lo; i < hi; ++i) {
      double w = W[i];
      if (w > 0.0) {
        before = c;
        c += w;
        last = i;
        if (c > thr) {
          tok = i;
          break;
        }
      }
    }
    const double tol = ((double)npos + 16.0) * 0x1p-51 * total;
    int margin = 0;
    if (tok < 0) {
      tok = last;
      margin = 1;
    } else if (c - thr <= tol || (before > 0.0 && thr - before <= tol)) {
      margin = 1;
    }
    sh.b.bcast_i[0] = tok;
    sh.b.bcast_i[1] = margin;
  }
  __syncthreads();
  const int64_t tok = sh.b.bcast_i[0];
  if (sh.b.bcast_i[1]) flags |= DSR_FLAG_MARGIN;
  __syncthreads();
  return tok;
}

// Number of positive entries and the first positive index.
__device__ void positive_support(const double* W, int64_t V, GenShared& sh, long long& npos, long long& first) {
  long long n = 0, f = LLONG_MAX;
  DSR_FOR_ROW(i, V) {
    if (W[i] > 0.0) {
      ++n;
      if (i < f) f = i;
    }
  }
  npos = block_sum_i64(n, sh.b);
  first = block_min_i64(f, sh.b);
}

}  // namespace dsr
