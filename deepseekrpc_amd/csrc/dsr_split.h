// Split-row path: rows that the register-resident bf16 paths do not take
// (float32 / float64 logits, or bf16 rows those paths cannot load), with or
// without a token history and a logit bias, that carry a top-k filter
// (1 <= k <= 1024), are greedy, or carry top-p / min-p without top-k (those
// are decided from the row's 512 largest values when the kept set provably
// lies among them); and rows with no filter at all and no history or bias,
// decided from the slices' sums (split_no_filter).
//
// One workgroup walking a whole row through the general path's passes uses
// one CU of 256; a small batch (one fp32 row per call is the reference's own
// calling pattern, sampling.py:108-128) then waits on that CU alone.  Here the
// row is cut into S contiguous slices, one workgroup each:
//
//   k_split_select  reads its slice once (logits, allow bits, the history
//                   and bias entries that fall in it), validates it, applies
//                   the penalties and bias, and keeps the slice's k largest values (ranked by value,
//                   then index) by 11-bit radix passes over registers, in
//                   index order, at slice s * k of a candidate list in the
//                   row's workspace.  It also zeroes the slice's probability
//                   and kept-bit outputs.
//   k_split_finish  one workgroup per row runs steps 8-13 of
//                   SamplingPolicy.probabilities (sampling.py:86-106) over
//                   the <= 8,192 candidates instead of the V tokens (and over
//                   the <= 1,024 that survive top-k from there on), then the
//                   categorical draw (sampling.py:108-128).
//
// Why the candidates decide the row: s = (v - max) / T is non-decreasing in
// v, so a token that is not among its slice's k largest values has s at most
// t, the s of the slice's smallest kept value; and t is at most s_k, the
// row's k-th largest s (the slice alone holds k values with s >= t).  If
// t < s_k, no token outside the candidates survives top-k.  If t == s_k,
// rounding may have merged distinct values into the k-th s, whose tie group
// the reference cuts by index (sampling.py:89-91 argsort is stable); the
// candidates cannot settle that, and the row goes to the general path in the
// same workgroup, as do rows with NaN / +inf logits or no finite logit (the
// general path reports their status in the reference's order).
#pragma once

#include "dsr_general.h"

namespace dsr {

constexpr int kSplitCap = 8192;                  // candidates per row
constexpr int kSplitMaxK = 1024;
constexpr int kSplitMinSlice = kThreads;         // tokens per slice, at least
constexpr int kSplitPer = 16;                    // tokens per thread, at most
constexpr int kSplitMaxSlices = 128;
constexpr int kSplitMinSlices = 8;
constexpr int kSplitTarget = 32;                 // slices a one-row call aims for (see split_max_slices)
constexpr int64_t kSplitMinVocab = 16384;        // the candidate area must fit the row's workspace
constexpr int kHandSplit = 7;                    // reason: a slice's last candidate ties the k-th value
constexpr int kHandMass = 8;                     // reason: top-p / min-p keep tokens beyond the candidates
constexpr int kSplitNoTopK = 512;                // candidates kept for a row without top-k

constexpr int kSliceBad = 1;     // NaN or +inf in the slice
constexpr int kSliceFinite = 2;  // a finite value in the slice
constexpr int kSliceTrunc = 4;   // the slice holds more than k tokens
constexpr int kSliceOdd = 8;     // the selection did not come to k tokens (never expected)

struct SplitSlice {
  long long vmin;  // order key of the smallest kept value, sign bit flipped (so it orders as signed)
  int flags;
  int count;
  double smax;     // rows without top-k: the slice's largest value (-inf if none is finite)
  double ssum;     // and the sum of exp((v - smax) / T) over its tokens
};

// Per-row candidate area, at the start of the row's workspace row.
constexpr size_t kSplitIdsOff = (size_t)kSplitCap * 8;   // values (float64), then token ids (int32)
constexpr size_t kSplitRecOff = (size_t)kSplitCap * 12;  // then one SplitSlice per slice
constexpr size_t kSplitBytes = kSplitRecOff + (size_t)kSplitMaxSlices * sizeof(SplitSlice);
static_assert(kSplitBytes <= (size_t)kSplitMinVocab * 8, "candidate area exceeds the smallest workspace row");
static_assert((int64_t)kSplitMinSlices * kSplitPer * kThreads >= DSR_MAX_VOCAB, "slices too short for the vocabulary");

// Slice budget per row.  More slices shorten the first launch but lengthen
// the finishing workgroup's passes over S * k candidates; for a one-row call
// with k = 50 (V = 129,280) 32 slices measured fastest (43.8 us, against 48.2
// at 128 and 46.4 at 16), and batches share the same total.
static inline int split_max_slices(int64_t rows) {
  const int64_t s = kSplitTarget / (rows > 0 ? rows : 1);
  return (int)(s < kSplitMinSlices ? kSplitMinSlices : (s > kSplitMaxSlices ? kSplitMaxSlices : s));
}

// The first launch's grid (rows x slices workgroups of kThreads) must stay
// below 2^32 work-items; larger batches take the general path.
static inline bool split_path_eligible(const dsr_sample_args_t& a) {
  return a.vocab >= kSplitMinVocab && a.rows > 0 &&
         a.rows * (int64_t)split_max_slices(a.rows) * kThreads < ((int64_t)1 << 32);
}

struct SplitGeom {
  int k;        // values kept per slice
  int S;        // slices
  int64_t len;  // tokens per slice (a multiple of 64; the last slice may be shorter)
  bool nok;     // a row without top-k (top-p and / or min-p decide it, or no filter at all)
  bool nof;     // a row with no filter at all: no candidates, only the slices' sums
};

// The row carries neither history entries nor bias entries.
__device__ __forceinline__ bool row_plain(const dsr_sample_args_t& a, int64_t row) {
  return (a.pen_off == nullptr || a.pen_off[row + 1] - a.pen_off[row] <= 0) &&
         (a.bias_off == nullptr || a.bias_off[row + 1] - a.bias_off[row] <= 0);
}

// Both launches derive the same geometry from the policy.  With S <= 8192 / k
// the list holds at most 8,192 candidates; each slice holds at least k tokens,
// so every slice but the last contributes exactly k.
__device__ __forceinline__ bool split_geom(const dsr_policy_t& p, int64_t V, int smax, bool plain, SplitGeom& g) {
  if (!policy_ok(p)) return false;
  int k;
  g.nok = false;
  g.nof = false;
  if (p.temperature == 0.0) {
    k = 1;  // greedy: only the first maximum matters (sampling.py:82-85)
  } else if (p.top_k >= 1 && p.top_k <= kSplitMaxK && p.top_k < V) {
    k = p.top_k;
  } else if ((p.top_k == 0 || p.top_k >= V) && (p.top_p < 1.0 || p.min_p != 0.0)) {
    k = kSplitNoTopK;  // the row's largest values, if top-p / min-p keep no more
    g.nok = true;
  } else if ((p.top_k == 0 || p.top_k >= V) && plain) {
    k = kSplitNoTopK;  // no filter (the default policy, sampling.py:30-33): slice sums only
    g.nok = true;
    g.nof = true;
  } else {
    return false;
  }
  int s = kSplitCap / k;
  if (s > smax) s = smax;
  int64_t len = (V + s - 1) / s;
  len = (len + 63) & ~(int64_t)63;
  if (len < kSplitMinSlice) len = kSplitMinSlice;
  g.k = k;
  g.len = len;
  g.S = (int)((V + len - 1) / len);
  return true;
}

__device__ __forceinline__ double key_value(uint64_t key) {
  const uint64_t b = (key >> 63) ? (key & 0x7FFFFFFFFFFFFFFFull) : ~key;
  return __longlong_as_double((long long)b);
}

// The next representable logit above (or below) v in the row's input type;
// NaN for bf16 (whose rows then take the general path on any such tie).
__device__ __forceinline__ double next_input_value(double v, int dtype, bool up) {
  if (dtype == DSR_F64) return nextafter(v, up ? (double)INFINITY : -(double)INFINITY);
  if (dtype == DSR_F32) return (double)nextafterf((float)v, up ? INFINITY : -INFINITY);
  return __longlong_as_double(0x7FF8000000000000ll);
}

// Stage one: grid rows * smax, blockIdx.x = row * smax + slice.
__global__ __launch_bounds__(kThreads) void k_split_select(dsr_sample_args_t a, int smax) {
  __shared__ GenShared sh;
  __shared__ int32_t emap[kSplitPer * kThreads];  // slice position -> history entry, or -1
  __shared__ uint16_t bmap[kSplitPer * kThreads];  // slice position -> bias entry - first entry, or 0xFFFF
  const int64_t row = blockIdx.x / (unsigned)smax;
  const int s = (int)(blockIdx.x % (unsigned)smax);
  const int64_t V = a.vocab;
  const dsr_policy_t pol = a.policy[row];
  SplitGeom g;
  if (!split_geom(pol, V, smax, row_plain(a, row), g) || s >= g.S) return;
  const int64_t lo = (int64_t)s * g.len;
  const int64_t hi = lo + g.len < V ? lo + g.len : V;
  const int64_t len = hi - lo;
  char* ws = (char*)((double*)a.workspace + row * ws_stride(V));
  double* Wc = (double*)ws;
  int32_t* Ic = (int32_t*)(ws + kSplitIdsOff);
  SplitSlice* rec = (SplitSlice*)(ws + kSplitRecOff);

  // The slice's outputs start at zero; the finishing launch writes the kept tokens.
  if (a.out_probs_f32)
    for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads) a.out_probs_f32[row * a.probs_ld + i] = 0.0f;
  if (a.out_probs_f64)
    for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads) a.out_probs_f64[row * a.probs_ld + i] = 0.0;
  if (a.out_kept_bits)
    for (int64_t w = (lo >> 5) + threadIdx.x; w < ((hi + 31) >> 5); w += kThreads) a.out_kept_bits[row * a.kept_ld + w] = 0u;

  // Thread t holds the contiguous tokens [lo + t*E, lo + (t+1)*E), so one scan of
  // per-thread counts places the kept tokens in index order.
  const size_t esz = a.dtype == DSR_BF16 ? 2 : (a.dtype == DSR_F32 ? 4 : 8);
  const void* base = (const char*)a.logits + (size_t)row * (size_t)a.ld * esz;
  const uint32_t* allow = a.allow_bits ? a.allow_bits + row * a.allow_ld : nullptr;
  const int E = (int)((len + kThreads - 1) / kThreads);
  const int64_t t0 = lo + (int64_t)threadIdx.x * E;
  double v[kSplitPer];
  uint64_t key[kSplitPer];
  unsigned valid = 0;
  int bad = 0, fin = 0;
#pragma unroll
  for (int j = 0; j < kSplitPer; ++j) {
    const int64_t i = t0 + j;
    const bool in = j < E && i < hi;
    v[j] = in ? load_logit(base, a.dtype, i) : -(double)INFINITY;
    if (in) valid |= 1u << j;
  }
#pragma unroll
  for (int j = 0; j < kSplitPer; ++j) {
    const int64_t i = t0 + j;
    double x = v[j];
    if ((valid >> j) & 1u) {
      if (x != x || x == INFINITY) bad = 1;
      if (allow && !((allow[i >> 5] >> (i & 31)) & 1u)) x = -(double)INFINITY;  // sampling.py:75-79
    }
    v[j] = x;
  }

  // Repetition / presence / frequency penalties (sampling.py:59-66) from the
  // row's history table, in the general path's float64 operation order
  // (masking first is equivalent: -inf is a fixed point of both steps).
  // Slice 0 checks the whole table with the general path's rules
  // (sampling.py:55-58,62-65); a table it would reject hands the row over,
  // and the general path reports the status.  Each slice finds its entries by
  // counting the (sorted) ids below its bounds.
  int64_t pen_n = 0;
  const int32_t *pid = nullptr, *pcnt = nullptr, *pgen = nullptr;
  if (a.pen_off) {
    const int64_t o = a.pen_off[row];
    pen_n = a.pen_off[row + 1] - o;
    pid = a.pen_ids + o;
    pcnt = a.pen_count + o;
    pgen = a.pen_gen + o;
  }
  if (pen_n > V) {
    bad = 1;  // more entries than tokens: not a valid table
  } else if (pen_n > 0) {
    long long below = 0;  // entries with id < lo (low half) and id < hi (high half)
    long long csum = 0;
    int tbad = 0;
    for (int64_t e = threadIdx.x; e < pen_n; e += kThreads) {
      const int32_t id = pid[e];
      below += (id < lo ? 1ll : 0ll) + (id < hi ? (1ll << 32) : 0ll);
      if (s == 0) {
        const long long c = pcnt[e], gg = pgen[e];
        if (id < 0 || id >= V || (e > 0 && pid[e - 1] >= id) || c < 0 || c > DSR_MAX_COUNT || gg < 0 || gg > c)
          tbad = 1;
        csum += c;
      }
    }
    below = block_sum_i64(below, sh.b);
    if (s == 0) {
      const long long tb = block_or(tbad, sh.b);
      csum = block_sum_i64(csum, sh.b);
      if (tb || csum > DSR_MAX_COUNT) bad = 1;
    }
    const int64_t e0 = below & 0xFFFFFFFFll, e1 = below >> 32;
    for (int64_t q = threadIdx.x; q < len; q += kThreads) emap[q] = -1;
    __syncthreads();
    for (int64_t e = e0 + threadIdx.x; e < e1; e += kThreads) {
      const int32_t id = pid[e];
      if (id >= lo && id < hi) emap[id - lo] = (int32_t)e;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSplitPer; ++j) {
      if ((valid >> j) & 1u) {
        const int32_t e = emap[t0 + j - lo];
        if (e >= 0) {
          const long long c = pcnt[e], gg = pgen[e];
          double x = v[j];
          if (c > 0) x = x >= 0.0 ? x / pol.repetition_penalty : x * pol.repetition_penalty;
          const double pen = pol.presence_penalty * (gg > 0 ? 1.0 : 0.0) + pol.frequency_penalty * (double)gg;
          v[j] = x - pen;
        }
      }
    }
  }

  // Logit bias (sampling.py:69-74), added after the penalties as the general
  // path does; slice 0 checks the whole sorted list with that path's rules.
  int64_t bias_n = 0;
  const int32_t* bid = nullptr;
  const double* bval = nullptr;
  if (a.bias_off) {
    const int64_t o = a.bias_off[row];
    bias_n = a.bias_off[row + 1] - o;
    bid = a.bias_ids + o;
    bval = a.bias_val + o;
  }
  if (bias_n > V) {
    bad = 1;  // more entries than tokens: not a valid list
  } else if (bias_n > 0) {
    long long below = 0;
    int bbad = 0;
    for (int64_t e = threadIdx.x; e < bias_n; e += kThreads) {
      const int32_t id = bid[e];
      below += (id < lo ? 1ll : 0ll) + (id < hi ? (1ll << 32) : 0ll);
      if (s == 0) {
        const double b = bval[e];
        if (id < 0 || id >= V || (e > 0 && bid[e - 1] >= id) || !(b >= -100.0 && b <= 100.0)) bbad = 1;
      }
    }
    below = block_sum_i64(below, sh.b);
    if (s == 0 && block_or(bbad, sh.b)) bad = 1;
    const int64_t e0 = below & 0xFFFFFFFFll, e1 = below >> 32;
    for (int64_t q = threadIdx.x; q < len; q += kThreads) bmap[q] = 0xFFFF;
    __syncthreads();
    for (int64_t e = e0 + threadIdx.x; e < e1; e += kThreads) {
      const int32_t id = bid[e];
      if (id >= lo && id < hi && e - e0 < 0xFFFF) bmap[id - lo] = (uint16_t)(e - e0);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSplitPer; ++j) {
      if ((valid >> j) & 1u) {
        const uint16_t q = bmap[t0 + j - lo];
        if (q != 0xFFFF) v[j] += bval[e0 + q];
      }
    }
  }
  // A row without top-k: the slice's maximum and sum of exp((v - max) / T),
  // from which the finishing launch forms the row's sum; every finite token
  // survives top-k, so its kept bit is set here.
  double vmax = -(double)INFINITY, ssum = 0.0;
  if (g.nok) {
    double m = -(double)INFINITY;
#pragma unroll
    for (int j = 0; j < kSplitPer; ++j)
      if (((valid >> j) & 1u) && v[j] > m) m = v[j];
    vmax = block_max(m, sh.b);
    double acc = 0.0;
    if (vmax > -(double)INFINITY) {
#pragma unroll
      for (int j = 0; j < kSplitPer; ++j)
        if (((valid >> j) & 1u) && v[j] > -(double)INFINITY) acc += exp((v[j] - vmax) / pol.temperature);
    }
    ssum = block_sum(acc, sh.b);
    if (a.out_kept_bits) {
      uint32_t* bits = a.out_kept_bits + row * a.kept_ld;
      int64_t w = -1;
      uint32_t mask = 0;
#pragma unroll
      for (int j = 0; j < kSplitPer; ++j) {
        const int64_t i = t0 + j;
        if (((valid >> j) & 1u) && isfinite(v[j])) {
          if ((i >> 5) != w) {
            if (mask) atomicOr(&bits[w], mask);
            w = i >> 5;
            mask = 0;
          }
          mask |= 1u << (i & 31);
        }
      }
      if (mask) atomicOr(&bits[w], mask);
    }
  }
#pragma unroll
  for (int j = 0; j < kSplitPer; ++j) {
    if ((valid >> j) & 1u) fin |= isfinite(v[j]) ? 1 : 0;
    key[j] = order_key(v[j]);
  }

  // A row with no filter keeps no candidates.
  const bool trunc = !g.nof && len > g.k;
  long long total = 0, mn = LLONG_MAX;
  const long long expect = g.nof ? 0 : (trunc ? g.k : len);
  if (!g.nof) {
    // Radix selection of the slice's k largest keys.  A pass whose selected bin
    // is taken whole ends the search; a tie group split by the last pass keeps
    // its lowest indices.
    uint64_t prefix = 0, pmask = 0;
    long long rem = g.k;
    bool whole = true;
    if (trunc) {
      for (int pass = 0; pass < kRadixPasses; ++pass) {
        const int shift = radix_shift(pass);
        const uint64_t dm = radix_mask(pass);
        for (int b = threadIdx.x; b < kBins; b += kThreads) sh.hist[b] = 0;
        __syncthreads();
  #pragma unroll
        for (int j = 0; j < kSplitPer; ++j)
          if (((valid >> j) & 1u) && (key[j] & pmask) == prefix) atomicAdd(&sh.hist[(key[j] >> shift) & dm], 1u);
        __syncthreads();
        long long above, cb;
        const int b = select_from_top(sh.hist, rem, sh, above, sh.hist, cb);
        if (b < 0) cb = -1;
        rem -= above;
        prefix |= (uint64_t)(b < 0 ? 0 : b) << shift;
        pmask |= dm << shift;
        if (cb == rem) break;
        if (pass == kRadixPasses - 1) whole = false;
      }
    }
    long long tb = 0;
    if (trunc && !whole) {
      int ties = 0;
  #pragma unroll
      for (int j = 0; j < kSplitPer; ++j) ties += ((valid >> j) & 1u) && key[j] == prefix;
      long long tt;
      tb = block_exclusive_scan_i64(ties, sh.b, tt);
    }
    unsigned selm = 0;
    int cnt = 0;
  #pragma unroll
    for (int j = 0; j < kSplitPer; ++j) {
      bool sel = (valid >> j) & 1u;
      if (trunc) {
        const uint64_t km = key[j] & pmask;
        if (whole) {
          sel = sel && km >= prefix;
        } else {
          const bool tie = sel && km == prefix;
          sel = sel && (km > prefix || (tie && tb < rem));
          tb += tie ? 1 : 0;
        }
      }
      if (sel) {
        selm |= 1u << j;
        ++cnt;
      }
    }
    const long long pos = block_exclusive_scan_i64(cnt, sh.b, total);
    long long q = pos;
  #pragma unroll
    for (int j = 0; j < kSplitPer; ++j) {
      if ((selm >> j) & 1u) {
        if (q < expect) {
          Wc[(int64_t)s * g.k + q] = v[j];
          Ic[(int64_t)s * g.k + q] = (int32_t)(t0 + j);
        }
        ++q;
        const long long sk = (long long)(key[j] ^ 0x8000000000000000ull);
        mn = sk < mn ? sk : mn;
      }
    }
    mn = block_min_i64(mn, sh.b);
  }
  const long long bf = block_reduce((long long)(bad | (fin << 1)), sh.b.i64, 0ll, OpOr());
  bad = (int)(bf & 1);
  fin = (int)((bf >> 1) & 1);
  if (threadIdx.x == 0) {
    SplitSlice r;
    r.smax = vmax;
    r.ssum = ssum;
    r.vmin = mn;
    r.flags = (bad ? kSliceBad : 0) | (fin ? kSliceFinite : 0) | (trunc ? kSliceTrunc : 0) |
              (total != expect ? kSliceOdd : 0);
    r.count = (int)total;
    rec[s] = r;
  }
}

// Stage two over the candidate list.  Returns a row status when the
// candidates decide the row (kz then holds the final probabilities of the n
// kept tokens in index order, kid their token ids), or -1 with the reason in
// `why` when the general path must.  Wc is LDS for kSplitCap values.
__device__ __forceinline__ int split_distribution(const RowSpec& r, const SplitGeom& g, GenShared& sh, double* Wc,
                                                  double* kz, int32_t* kid, unsigned& flags, DistOut& out, int64_t& n,
                                                  int& why) {
  char* ws = (char*)r.W;
  const int32_t* Ic = (const int32_t*)(ws + kSplitIdsOff);
  const SplitSlice* rec = (const SplitSlice*)(ws + kSplitRecOff);
  out.onehot = -1;
  out.npos = 0;
  out.first = -1;
  const long long f = block_reduce((int)threadIdx.x < g.S ? (long long)rec[threadIdx.x].flags : 0ll, sh.b.i64, 0ll, OpOr());
  const bool odd = f & kSliceOdd, bad = f & kSliceBad, fin = f & kSliceFinite;
  if (odd) {
    why = kHandSplit;
    return -1;
  }
  if (bad || !fin) {
    why = kHandInvalid;
    return -1;
  }
  const int64_t last = r.V - (int64_t)(g.S - 1) * g.len;
  n = (int64_t)(g.S - 1) * g.k + (last < g.k ? last : g.k);
  // The candidates' values move to LDS (Wc, kSplitCap doubles): every pass
  // below re-reads them.  Candidates are in index order, so their first
  // maximum is the row's.
  const double* cand = (const double*)ws;
  RowMax mx;
  row_pass<double>(n, [&](int64_t j) { return cand[j]; }, [&](int64_t j, double x) {
    Wc[j] = x;
    mx.add(j, x);
  });
  auto ldW = [&](int64_t j) { return Wc[j]; };
  const double M = block_max(mx.m, sh.b);
  const long long fj = block_min_i64(mx.m == M ? mx.first : LLONG_MAX, sh.b);
  if (!(fj >= 0 && fj < n && M > -(double)INFINITY)) {  // not reached: a slice with a finite value keeps its maximum
    why = kHandSplit;
    return -1;
  }
  const dsr_policy_t& p = r.pol;
  if (p.temperature == 0.0) {  // sampling.py:82-85
    const int64_t first = Ic[fj];
    out.onehot = first;
    out.npos = 1;
    out.first = first;
    if (threadIdx.x == 0) {
      if (r.probs_f32) r.probs_f32[first] = 1.0f;
      if (r.probs_f64) r.probs_f64[first] = 1.0;
      if (r.kept_bits) r.kept_bits[first >> 5] = 1u << (first & 31);
    }
    __syncthreads();
    return DSR_OK;
  }
  const double T = p.temperature;
  row_pass<double>(n, ldW, [&](int64_t j, double x) { Wc[j] = (x - M) / T; });  // sampling.py:86-88
  __syncthreads();
  if (!(g.k < n)) {  // not reached: S >= 2 gives more than k candidates
    why = kHandSplit;
    return -1;
  }
  // A row without top-k: the row's sum of exp(s), from the slices' sums.
  double s1_row = __longlong_as_double(0x7FF8000000000000ll);
  if (g.nok) {
    double term = 0.0;
    if ((int)threadIdx.x < g.S) {
      const SplitSlice q = rec[threadIdx.x];
      if (q.smax > -(double)INFINITY) term = q.ssum * exp((q.smax - M) / T);
    }
    s1_row = block_sum(term, sh.b);
  }
  uint64_t kth;
  int64_t cut;
  radix_top_k(Wc, n, g.k, sh, kth, cut);
  const double sk = key_value(kth);
  // A truncated slice whose smallest kept value v maps onto s_k may have left
  // out tokens of the k-th tie group.  When v's neighbours in the input type
  // map strictly below and above s_k, that group's members in the slice are
  // exactly its tokens equal to v, and the ones left out follow the slice's
  // kept ones in index order: the candidates decide the row unless the cut
  // passes the slice's last kept member.
  int amb = 0, eq = 0;
  if ((int)threadIdx.x < g.S) {
    const SplitSlice q = rec[threadIdx.x];
    if (q.flags & kSliceTrunc) {
      const double v = key_value((uint64_t)q.vmin ^ 0x8000000000000000ull);
      const double t = (v - M) / T;
      if (!(t <= sk)) {
        amb = 1;  // not reached: t <= s_k
      } else if (t == sk) {
        eq = 1;
        // Penalised or biased values are float64, off the input type's grid.
        const int vt = (r.pen_n > 0 || r.bias_n > 0) ? DSR_F64 : r.dtype;
        const double dn = next_input_value(v, vt, false), up = next_input_value(v, vt, true);
        if (!(v > -(double)INFINITY && (dn - M) / T < sk && (up - M) / T > sk)) amb = 1;
      }
    }
  }
  if (block_or(amb, sh.b)) {
    why = kHandSplit;
    return -1;
  }
  if (block_or(eq, sh.b)) {
    int* last = (int*)sh.hist;  // per slice: the last candidate position holding s_k
    if ((int)threadIdx.x < g.S) last[threadIdx.x] = -1;
    __syncthreads();
    row_pass<double>(n, ldW, [&](int64_t j, double z) {
      if (order_key(z) == kth) atomicMax(&last[j / g.k], (int)j);
    });
    __syncthreads();
    // A tie group kept whole (cut = INT64_MAX) ends at its last candidate.
    const int64_t c = cut != INT64_MAX ? cut
                                       : block_max_i64((int)threadIdx.x < g.S ? (long long)last[threadIdx.x] : -1, sh.b);
    if (eq && last[threadIdx.x] < c) amb = 1;
    if (block_or(amb, sh.b)) {
      why = kHandSplit;
      return -1;
    }
  }
  // The k tokens that survive top-k (sampling.py:89-91) move to LDS in index
  // order, with their kept bits set (the slices zeroed the words); steps
  // 10-13 and the draw then run over them alone.
  auto kept = [&](int64_t j, double z) {
    const uint64_t key = order_key(z);
    return z > -(double)INFINITY && (key > kth || (key == kth && j <= cut));
  };
  int64_t lo, hi;
  slice_of(threadIdx.x, n, lo, hi);
  long long cnt = 0;
  for (int64_t j = lo; j < hi; ++j) cnt += kept(j, Wc[j]) ? 1 : 0;
  long long nk;
  long long pos = block_exclusive_scan_i64(cnt, sh.b, nk);
  if (nk > kSplitMaxK) {  // not reached: top-k keeps k tokens
    why = kHandSplit;
    return -1;
  }
  for (int64_t j = lo; j < hi; ++j) {
    const double z = Wc[j];
    if (kept(j, z)) {
      const int32_t i = Ic[j];
      kz[pos] = z;
      kid[pos] = i;
      ++pos;
      if (r.kept_bits && !g.nok) atomicOr(&r.kept_bits[i >> 5], 1u << (i & 31));
    }
  }
  __syncthreads();
  n = nk;
  if (g.nok) {
    // Every token outside the candidates has exp(s) <= exp(s_k).  With min-p,
    // all of them must fall below min_p * max (max(r) = 1 / sum, sampling.py:
    // 94-96); without it, the candidates' own mass must reach top_p
    // (sampling.py:97-102).  Both with a margin far above the rounding band.
    int ok;
    if (p.min_p != 0.0) {
      ok = exp(sk) < p.min_p * (1.0 - 0x1p-40);
    } else {
      double e = 0.0;
      for (int64_t j = threadIdx.x; j < nk; j += kThreads) e += exp(kz[j]);
      const double mass = block_sum(e, sh.b) / s1_row;
      ok = mass >= p.top_p * (1.0 + 0x1p-40) + 0x1p-50;
    }
    if (!ok) {
      why = kHandMass;
      return -1;
    }
  }
  return filter_tail(r, kz, nk, r.V, false, 0, -1, sh, flags, out, [kid](int64_t j) { return (int64_t)kid[j]; },
                     s1_row);
}

// A row with no filter (top-k, top-p and min-p all off): the final
// distribution is exp((v - max) / T) / sum over the whole row (sampling.py:
// 86-93; the second normalisation, :103-106, divides by a sum that the first
// made 1 up to rounding).  The row's maximum and sum come from the slices.
// One coalesced pass over the row recomputes each probability from its logit,
// writes it, and sums it per wave (each wave owns a contiguous range); the
// draw finds the wave range that holds u * total, sums that range in
// contiguous per-thread chunks and walks one chunk, as the general path's CDF
// search walks its per-thread ranges (sampling.py:108-128).  Returns false, with
// the reason in `why`, when the general path must decide the row.
template <bool RNG>
__device__ __forceinline__ bool split_no_filter(const dsr_sample_args_t& a, int64_t row, const RowSpec& r,
                                                const SplitGeom& g, GenShared& sh, int& why) {
  const SplitSlice* rec = (const SplitSlice*)((const char*)r.W + kSplitRecOff);
  const bool mine = (int)threadIdx.x < g.S;
  const long long f = block_reduce(mine ? (long long)rec[threadIdx.x].flags : 0ll, sh.b.i64, 0ll, OpOr());
  if ((f & kSliceBad) || !(f & kSliceFinite)) {
    why = kHandInvalid;
    return false;
  }
  const double T = r.pol.temperature;
  const double M = block_max(mine ? rec[threadIdx.x].smax : -(double)INFINITY, sh.b);
  double term = 0.0;
  if (mine && rec[threadIdx.x].smax > -(double)INFINITY)
    term = rec[threadIdx.x].ssum * exp((rec[threadIdx.x].smax - M) / T);
  const double s1 = block_sum(term, sh.b);
  const int64_t V = r.V;
  auto pf = [&](int64_t i) -> double {
    double x = load_logit(r.logits, r.dtype, i);
    if (r.allow && !((r.allow[i >> 5] >> (i & 31)) & 1u)) x = -(double)INFINITY;
    return exp((x - M) / T) / s1;
  };
  // Level 1: wave w owns the contiguous range [w*cw, (w+1)*cw), read 64
  // tokens at a time (coalesced); it writes the probabilities and sums them.
  const int64_t cw = (V + kWaves - 1) / kWaves;
  const int64_t wlo = (int64_t)wave_id() * cw < V ? (int64_t)wave_id() * cw : V;
  const int64_t whi = wlo + cw < V ? wlo + cw : V;
  double part = 0.0;
  long long np = 0, fp = LLONG_MAX;
  for (int64_t b = wlo; b < whi; b += 64 * kUnroll) {
    double q[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const int64_t i = b + 64 * k + lane_id();
      q[k] = i < whi ? pf(i) : 0.0;
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const int64_t i = b + 64 * k + lane_id();
      if (i < whi) {
        if (r.probs_f32) r.probs_f32[i] = (float)q[k];
        if (r.probs_f64) r.probs_f64[i] = q[k];
        part += q[k];
        if (q[k] > 0.0) {
          ++np;
          if (i < fp) fp = i;
        }
      }
    }
  }
  const double wsum = wave_sum(part);
  double total;
  // Wave totals in wave order: each wave's lane 0 contributes its total.
  const double wbase = block_exclusive_scan_f64(lane_id() == 0 ? wsum : 0.0, sh.b, total);
  const long long npos = block_sum_i64(np, sh.b);
  const long long first = block_min_i64(fp, sh.b);
  if (!(total > 0.0) || !isfinite(total) || npos < 1) {  // not reached: the maximum's exp is 1
    why = kHandInvalid;
    return false;
  }
  int st = DSR_OK;
  int64_t token = -1;
  int consumed = 0;
  unsigned flags = DSR_FLAG_SPLIT;
  if (has_draws<RNG>(a)) {
    if (npos == 1) {
      token = first;  // sampling.py:120-122: no uniform is drawn
    } else {
      uint64_t next[4];
      const double u = RNG ? pcg64_random(a.rng_state + 4 * row, next) : a.uniforms[row];
      if (!(u >= 0.0 && u < 1.0)) {
        st = DSR_E_UNIFORM;
      } else {
        const double thr = u * total;
        // The wave whose range holds the crossing: the last with mass whose base is <= thr.
        const long long wc = (lane_id() == 0 && wsum > 0.0 && wbase <= thr) ? (long long)wave_id() : -1;
        const long long ow = block_max_i64(wc, sh.b);
        if (lane_id() == 0 && (long long)wave_id() == ow) sh.bc[3] = __double_as_longlong(wbase);
        __syncthreads();
        int64_t tok = -1;
        int margin = 1;
        if (ow >= 0) {
          // Level 2: that range in contiguous per-thread chunks, then one walk.
          const double ob = __longlong_as_double(sh.bc[3]);
          const int64_t rlo = ow * cw, rhi = rlo + cw < V ? rlo + cw : V;
          const int64_t ch = (rhi - rlo + kThreads - 1) / kThreads;
          const int64_t clo = rlo + (int64_t)threadIdx.x * ch < rhi ? rlo + (int64_t)threadIdx.x * ch : rhi;
          const int64_t chi = clo + ch < rhi ? clo + ch : rhi;
          double cp = 0.0;
          slice_pass<double>(clo, chi, pf, [&](int64_t, double q) { cp += q; });
          double rt;
          const double cb = ob + block_exclusive_scan_f64(cp, sh.b, rt);
          const long long cc = (cp > 0.0 && cb <= thr) ? (long long)threadIdx.x : -1;
          const long long owner = block_max_i64(cc, sh.b);
          if ((long long)threadIdx.x == owner) sh.bc[0] = __double_as_longlong(cb);
          __syncthreads();
          if (wave_id() == 0 && owner >= 0) {
            const int64_t olo = rlo + owner * ch < rhi ? rlo + owner * ch : rhi;
            const int64_t ohi = olo + ch < rhi ? olo + ch : rhi;
            const double tol = ((double)npos + 16.0) * 0x1p-51 * total;
            int64_t t;
            int m;
            wave_slice_cdf(pf, olo, ohi, __longlong_as_double(sh.bc[0]), thr, tol, t, m);
            if (lane_id() == 0) {
              sh.bc[1] = t;
              sh.bc[2] = m;
            }
          }
          __syncthreads();
          if (owner >= 0) {
            tok = (int64_t)sh.bc[1];
            margin = (int)sh.bc[2];
          }
        }
        token = tok;
        if (tok < 0 || margin) flags |= DSR_FLAG_MARGIN;
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
  return true;
}

}  // namespace dsr
