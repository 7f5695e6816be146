// One-workgroup top-k path for FP32 rows (gfx950, wave64).
//
// The reference's terminal stage hands sampling FP32 rows (terminal_sampling.py
// :16-27); SamplingPolicy.probabilities then keeps the row's top_k largest
// values (sampling.py:89-91) before its exp, min-p and top-p steps.  For a
// row with 1 <= top_k <= 1,024 (or a greedy row) and no history or bias, one
// 1024-thread workgroup decides it from the few hundred tokens that can
// survive top-k:
//
//   * pass 1 reads the row once with coalesced 16-byte loads (wave w owns
//     quads [w*QW, (w+1)*QW), lane l takes quad w*QW + 64j + l at slot j;
//     two groups of four slots in flight) and keeps, per lane, the top 16
//     bits of the order key of each quad's largest allowed finite value (two
//     to a register), with the row's maximum, its first index and validity;
//   * tau, the 16-bit key prefix of the k-th largest maximum over pairs of a
//     lane's quads, comes from two histograms by distance to the row
//     maximum's prefix (coarse, then fine; one per wave, scanned by one
//     wave).  The pairs partition the row, and a subset's k-th largest value
//     never exceeds the row's, so every token that survives top-k, its tie
//     group included, has a key of at least tau << 16;
//   * pass 2 lists the quads whose maximum reaches tau from the prefixes in
//     registers, reads only those again, and lists their tokens at or above
//     tau in index order, per wave, in LDS;
//   * the list, as float64 z = (v - max) / T, is sorted by (z desc, index
//     asc) with a bucket sort (f32_sorted_tail); top-k, exp, min-p, top-p
//     and the normalisation then run over sorted positions, one per thread,
//     and the kept tokens return to index order for the categorical draw.  A
//     bucket too full to rank sends the list through radix_top_k and
//     filter_tail instead.
//
// Rows with NaN / +inf values, no allowed finite value, fewer allowed finite
// values than k, or more listed tokens than the list holds go to the general
// path in the same workgroup (reason in flags bits 4-7).
#pragma once

#include "dsr_fast.h"
#include "dsr_general.h"
#include "dsr_split.h"
#include "dsr_topk.h"

namespace dsr {

constexpr int kF32Slots = 32;                    // quads (16 bytes) per lane: rows of up to 131,072 values
constexpr int kF32MaxVocab = kF32Slots * 4 * kThreads;
constexpr int kF32Cap = 4096;                    // listed tokens per row
constexpr int kF32WaveCap = kF32Cap / kWaves;    // per wave
constexpr int kF32Bins = 256;

constexpr int kTailBins = 2048;       // buckets of the candidate sort
constexpr int kTailBucketMax = 256;   // members a bucket may hold (ranking inside one is quadratic)
constexpr int kTailFallback = -2;     // f32_sorted_tail: the radix route must decide the row

struct F32Lists {
  union alignas(16) {
    uint32_t hist[kWaves][kF32Bins];             // per-wave radix histograms, then pass 2's quad lists
    struct {
      uint32_t bins[kTailBins];                  // candidate sort: bucket counts, starts, ends
      double xs[kSplitMaxK];                     // probabilities by sorted position
    } srt;
  };
  union {
    float lv[kWaves][kF32WaveCap];               // listed values, per wave in index order
    int32_t sp[kF32Cap];                         // candidate sort: list position by sorted position
  };
  union {
    int32_t li[kWaves][kF32WaveCap];             // their token indices
    int32_t pos[kF32Cap];                        // candidate sort: sorted position by list position
  };
  double cz[kF32Cap];                            // the list, row-wide: (v - max) / T in index order
  int32_t cid[kF32Cap];
  double kz[kSplitMaxK];                         // kept tokens, index order
  int32_t kid[kSplitMaxK];
  int32_t wn[kWaves];                            // listed tokens per wave (or more than the cap)
  int32_t pick[4];                               // selected radix bins and counts
};

// A batch the one-workgroup FP32 kernel takes: FP32 rows, 16-byte aligned,
// no history or bias, and the caller's word that every row is greedy or has
// 1 <= top_k <= 1,024 (a row that is not is still decided exactly, by the
// general path in its workgroup).
static inline bool f32_path_eligible(const dsr_sample_args_t& a) {
  return a.dtype == DSR_F32 && (a.hints & DSR_HINT_TOPK_ALL) && !a.pen_off && !a.bias_off && a.rows > 0 &&
         a.rows <= (1 << 24) &&  // the probability fill's grid: rows x 32 chunks
         a.vocab <= kF32MaxVocab && a.vocab % 4 == 0 && a.ld % 4 == 0 && ((uintptr_t)a.logits & 15u) == 0;
}

struct F32Shared {
  GenShared gen;  // the finishing steps' scratch, and the general path's if the row falls back
  F32Lists t;
};

// Order key of an FP32 value as an unsigned 32-bit integer (larger value,
// larger key; -0 and +0 equal), or 0 for a token that cannot be kept
// (disallowed or -inf; NaN / +inf are reported separately).
__device__ __forceinline__ uint32_t f32_key(uint32_t bits, bool allowed) {
  if ((bits & 0x7FFFFFFFu) == 0u) bits = 0u;
  const uint32_t k = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return (allowed && bits != 0xFF800000u) ? k : 0u;
}

__device__ __forceinline__ bool f32_bad(uint32_t bits) {
  return (bits & 0x7F800000u) == 0x7F800000u && bits != 0xFF800000u;  // NaN or +inf
}

// The radix bin of the rem-th largest counted key: the largest b with
// sum(hist[b..255]) >= rem, counts summed over the waves' histograms; sets
// above = sum(hist[b+1..255]).  Returns -1 if fewer than rem keys were
// counted.  Every thread calls it after the barrier that completes the
// histograms; wave 0 scans them (lane l owns bins 4l..4l+3) and one barrier
// publishes the bin, after which the histograms may be written again.
__device__ __forceinline__ int f32_pick(F32Lists& t, long long rem, long long& above) {
  if (wave_id() == 0) {
    const int lane = lane_id();
    uint32_t c[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const uint4 h = *reinterpret_cast<const uint4*>(&t.hist[w][4 * lane]);
      c[0] += h.x;
      c[1] += h.y;
      c[2] += h.z;
      c[3] += h.w;
    }
    const uint32_t mine = c[0] + c[1] + c[2] + c[3];
    const uint32_t incl = wave_scan_dpp(mine);  // bins 0 .. 4l+3
    const uint32_t total = lane_value(incl, 63);
    long long a = (long long)(total - incl);   // keys in bins above 4l+3
    if (lane == 0 && (long long)total < rem) t.pick[0] = -1;
    if (a < rem && rem <= a + (long long)mine) {
      int b = 4 * lane + 3;
#pragma unroll
      for (int e = 3; e > 0; --e) {
        if (a + (long long)c[e] >= rem) break;
        a += c[e];
        --b;
      }
      t.pick[0] = b;
      t.pick[1] = (int)a;
    }
  }
  __syncthreads();
  const int r = t.pick[0];
  above = r >= 0 ? t.pick[1] : 0;
  return r;
}

// Order key of (float)z: rounding to nearest is monotone, and equal z give
// equal keys, so buckets by it order the candidates coarsely and keep each
// tie group of z in one bucket.
__device__ __forceinline__ uint32_t z_key32(double z) { return f32_key(__float_as_uint((float)z), true); }

// Bucket width in key units: 2,048 buckets span one binade of |z| (z <= 0,
// so a key is ~bits(|z|) there), from the list's smallest z up; the z
// closer to zero (the row maximum's own 0 among them) share the top bucket.
constexpr int kTailShift = 12;

// Steps 9-13 (sampling.py:89-106) over the candidate list t.cz / t.cid
// (nc entries, index order, every token that can survive top-k among them).
// The list is sorted by (z desc, index asc), the reference's ranking: a
// counting sort into 2,048 buckets of 1/2,048 binade of |z| up from the
// list's smallest z (the candidates of a top-k cluster there), then each
// member ranked inside its bucket.  In that order top-k
// keeps the first k, the probabilities do not increase, min-p and top-p cut a
// prefix, and the top-p crossing is a prefix scan of fixed-point masses
// (the same crossing radix_mass_crossing finds).  The float64 steps and
// their rounding-band flags follow filter_tail.  Returns a status (kz / kid
// then hold the n kept tokens' probabilities in index order), or
// kTailFallback, with nothing written, for a bucket too full to rank.
__device__ __forceinline__ int f32_sorted_tail(const RowSpec& r, F32Lists& t, GenShared& sh, int64_t nc, long long k, int64_t V,
                               unsigned& flags, DistOut& out, int64_t& n) {
  const int tid = threadIdx.x;
  const dsr_policy_t& p = r.pol;
  constexpr int kPer = kF32Cap / kThreads;
  uint32_t* bins = t.srt.bins;
  uint32_t pz[kPer], bk[kPer], at[kPer];
  uint32_t lo = 0xFFFFFFFFu;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int c = tid + u * kThreads;
    pz[u] = c < nc ? z_key32(t.cz[c]) : 0xFFFFFFFFu;
    lo = min(lo, pz[u]);
  }
  bins[tid] = 0u;
  bins[tid + kThreads] = 0u;
  const uint32_t zlo = (uint32_t)block_min_i64((long long)lo, sh.b);  // its barriers order the clearing
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    if (tid + u * kThreads < nc) {
      bk[u] = min((pz[u] - zlo) >> kTailShift, (uint32_t)(kTailBins - 1));
      atomicAdd(&bins[bk[u]], 1u);
    }
  }
  __syncthreads();
  // Bucket starts, highest bucket first: thread t owns buckets 2047 - 2t and 2046 - 2t.
  {
    const int b0 = kTailBins - 1 - 2 * tid, b1 = b0 - 1;
    const uint32_t c0 = bins[b0], c1 = bins[b1];
    long long tot;
    const long long ex = block_exclusive_scan_i64((long long)(c0 + c1), sh.b, tot);
    bins[b0] = (uint32_t)ex;
    bins[b1] = (uint32_t)ex + c0;
    if (block_or(c0 > (uint32_t)kTailBucketMax || c1 > (uint32_t)kTailBucketMax, sh.b)) return kTailFallback;
  }
  // Arrival order inside each bucket; the bucket's start becomes its end.
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int c = tid + u * kThreads;
    if (c < nc) t.sp[atomicAdd(&bins[bk[u]], 1u)] = c;
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int c = tid + u * kThreads;
    if (c < nc) {
      const uint32_t s0 = bk[u] == (uint32_t)(kTailBins - 1) ? 0u : bins[bk[u] + 1], s1 = bins[bk[u]];
      const uint64_t key = order_key(t.cz[c]);
      uint32_t rank = 0u;
      for (uint32_t q = s0; q < s1; ++q) {
        const int o = t.sp[q];
        const uint64_t ko = order_key(t.cz[o]);
        rank += (ko > key || (ko == key && o < c)) ? 1u : 0u;
      }
      at[u] = s0 + rank;
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int c = tid + u * kThreads;
    if (c < nc) {
      t.sp[at[u]] = c;
      t.pos[c] = (int32_t)at[u];
    }
  }
  __syncthreads();

  // Top-k (sampling.py:89-91): sorted positions below k whose z is finite
  // (-inf sorts last).  Thread t holds sorted position t.
  const bool in = tid < k && tid < nc;
  const int cme = in ? t.sp[tid] : 0;
  const double z = in ? t.cz[cme] : -(double)INFINITY;
  const bool kept = z > -(double)INFINITY;
  const int32_t tok = kept ? t.cid[cme] : 0;
  if (kept && r.kept_bits) atomicOr(&r.kept_bits[tok >> 5], 1u << (tok & 31));
  const long long nk = block_sum_i64(kept ? 1 : 0, sh.b);

  // sampling.py:92-96
  const double e = kept ? exp(z) : 0.0;
  const double s1 = block_sum(e, sh.b);
  double x;
  if (p.min_p != 0.0) {
    // max(r) = 1 / s1: the maximum's exp is exactly 1 and division is monotone.
    const double cut_p = p.min_p * (1.0 / s1);
    const double tol = cut_p * 0x1p-49;
    x = e / s1;
    const int close = (x > 0.0 && fabs(x - cut_p) <= tol) ? 1 : 0;
    if (x < cut_p) x = 0.0;
    if (block_or(close, sh.b)) flags |= DSR_FLAG_MARGIN;
    const double s2 = block_sum(x, sh.b);
    x = x / s2;
  } else {
    x = e / s1;
  }

  if (p.top_p < 1.0) {  // sampling.py:97-102
    long long tgt = (long long)(p.top_p * 0x1p60);
    if (tgt == 0) tgt = 1;  // top_p == 0: the first ranked element is the crossing
    const long long fx = x > 0.0 ? (long long)(x * 0x1p60) : 0ll;
    if (tid < kSplitMaxK) t.srt.xs[tid] = x;
    if (tid == 0) sh.bc[0] = -1;
    long long ftot;
    const long long fex = block_exclusive_scan_i64(fx, sh.b, ftot);
    if (ftot >= tgt) {
      if (fx > 0 && fex < tgt && fex + fx >= tgt) sh.bc[0] = tid;  // one thread: the crossing
      __syncthreads();
      const double rt = t.srt.xs[sh.bc[0]];
      const double A = block_sum(x > rt ? x : 0.0, sh.b);
      const long long both = block_sum_i64((x > rt ? (1ll << 20) : 0ll) + (x == rt ? 1ll : 0ll), sh.b);
      const long long n_above = both >> 20, n_tie = both & ((1ll << 20) - 1);
      bool close;
      const long long keep = top_p_tie_keep(A, n_above, n_tie, rt, p.top_p, close);
      if (close) flags |= DSR_FLAG_MARGIN;
      // The keep-th member of the tie group in index order: the group holds
      // sorted positions [n_above, n_above + n_tie), in index order when it
      // is one value of z (else several z round to one probability).
      int cutc = -1;
      if (keep > 0) {
        const int f = (int)n_above, l = f + (int)n_tie - 1;
        if (t.cz[t.sp[f]] == t.cz[t.sp[l]]) {
          cutc = t.sp[f + (int)keep - 1];
        } else {
          if (tid >= f && tid <= l) {
            int rank = 0;
            for (int q = f; q <= l; ++q) rank += t.sp[q] < cme ? 1 : 0;
            if (rank == (int)keep - 1) sh.bc[1] = cme;
          }
          __syncthreads();
          cutc = (int)sh.bc[1];
        }
      }
      if (x < rt || (x == rt && cme > cutc)) x = 0.0;
    } else {
      // The whole mass stays below top_p: nothing is removed.
      const double tot = block_sum(x, sh.b);
      if (fabs(tot - p.top_p) <= ((double)V + 16.0) * 0x1p-51) flags |= DSR_FLAG_MARGIN;
    }
  }

  const double total = block_sum(x, sh.b);  // sampling.py:103-106
  if (!(total > 0.0) || !isfinite(total)) return DSR_E_NO_MASS;
  x = x / total;
  if (kept) {
    if (r.probs_f32) r.probs_f32[tok] = (float)x;
    if (r.probs_f64) r.probs_f64[tok] = x;
  }
  if (tid < kSplitMaxK) t.srt.xs[tid] = x;
  out.npos = block_sum_i64(x > 0.0 ? 1 : 0, sh.b);
  const long long fpos = block_min_i64(x > 0.0 ? (long long)cme : LLONG_MAX, sh.b);
  out.first = fpos == LLONG_MAX ? fpos : (long long)t.cid[fpos];

  // The kept tokens in index order (sorted positions below nk).
  int64_t jlo, jhi;
  slice_of(tid, nc, jlo, jhi);
  long long cnt = 0;
  for (int64_t j = jlo; j < jhi; ++j) cnt += t.pos[j] < nk ? 1 : 0;
  long long nkk;
  long long w = block_exclusive_scan_i64(cnt, sh.b, nkk);
  for (int64_t j = jlo; j < jhi; ++j) {
    const int ps = t.pos[j];
    if (ps < nk) {
      t.kz[w] = t.srt.xs[ps];
      t.kid[w] = t.cid[j];
      ++w;
    }
  }
  __syncthreads();
  n = nk;
  return DSR_OK;
}

// The 16-bit prefix of the k-th largest of the 16-bit key prefixes that the
// workgroup's threads hold (NV each, val(0 .. NV-1); 0 is not counted), D
// the largest of them; 0 when fewer than k are counted.  By distance d = D -
// prefix: a coarse histogram of d / 8 over d < 2,048 (sixteen binades below a
// positive maximum), then a fine one of d % 8 inside the selected coarse bin.
// Few lanes of a wave share a bin either way, so the LDS atomics rarely
// serialise; by top byte of the key instead, most prefixes of a row share a
// handful of bins and a wave's atomics would hit one address.  Rows with
// fewer than k prefixes inside that distance take two 8-bit radix passes
// over the whole prefix instead.  Each wave counts into its own histogram,
// cleared by itself.  Every thread calls it.
template <int NV, class Val>
__device__ __forceinline__ uint32_t f32_tau16(F32Lists& t, int wave, int lane, uint32_t D, long long k, Val val) {
  auto clear_hist = [&]() {
    *reinterpret_cast<uint4*>(&t.hist[wave][4 * lane]) = make_uint4(0u, 0u, 0u, 0u);
    wave_lds_sync();
  };
  uint32_t tau16 = 0u;
  {
    long long rem = k;
    uint32_t cbin = 0u;  // selected coarse bin (d / 8)
    for (int pass = 0; pass < 2; ++pass) {
      clear_hist();
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const uint32_t x = val(i);
        const uint32_t d = D - x;  // x <= D
        if (pass == 0) {
          if (x != 0u && d < 8u * kF32Bins) atomicAdd(&t.hist[wave][kF32Bins - 1 - (d >> 3)], 1u);
        } else {
          if (x != 0u && (d >> 3) == cbin) atomicAdd(&t.hist[wave][kF32Bins - 1 - (d & 7u)], 1u);
        }
      }
      __syncthreads();
      long long above;
      const int b = f32_pick(t, rem, above);  // uniform
      if (b < 0) break;  // fewer than k inside the distance (pass 0 only)
      rem -= above;
      if (pass == 0) cbin = (uint32_t)(kF32Bins - 1 - b);
      else tau16 = D - (8u * cbin + (uint32_t)(kF32Bins - 1 - b));
    }
  }
  if (tau16 == 0u) {
    uint32_t prefix = 0u;
    long long rem = k;
    for (int pass = 0; pass < 2; ++pass) {
      const int shift = pass == 0 ? 24 : 16;
      clear_hist();
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const uint32_t x = val(i) << 16;
        const bool cnt = x != 0u && (pass == 0 || (x >> 24) == (prefix >> 24));
        if (cnt) atomicAdd(&t.hist[wave][(x >> shift) & 0xFFu], 1u);
      }
      __syncthreads();
      long long above;
      const int b = f32_pick(t, rem, above);
      if (b < 0) return 0u;  // fewer than k counted
      rem -= above;
      prefix |= (uint32_t)b << shift;
    }
    tau16 = prefix >> 16;
  }
  return tau16;
}

constexpr int kDecided = -4;      // f32_list_finish: the row's outputs are written
constexpr int kWaveTailMax = 64;  // lists a single wave finishes (one candidate per lane)

// Steps 9-13 and the draw (sampling.py:89-128) for a list of at most 64
// candidates (t.cz / t.cid, nc entries, index order), by wave 0 alone with
// one candidate per lane: the steps, float64 arithmetic and rounding-band
// flags of f32_sorted_tail and finish_row, with wave reductions in place of
// workgroup ones.  The candidates are ranked by (z desc, list position asc),
// the reference's order, by comparing every pair.  Writes the row's outputs.
__device__ __forceinline__ void f32_wave_tail(const dsr_sample_args_t& a, int64_t row, const RowSpec& r, F32Lists& t,
                                              int nc, long long k, int64_t V, unsigned flags) {
  if (wave_id() != 0) return;
  const int l = lane_id();
  const dsr_policy_t& p = r.pol;
  const bool have = l < nc;
  const double z0 = have ? t.cz[l] : -(double)INFINITY;
  const unsigned long long key = have ? (unsigned long long)order_key(z0) : 0ull;
  int rank = 0;
  for (int j = 0; j < nc; ++j) {  // uniform
    const unsigned long long kj = lane_value(key, j);
    rank += (kj > key || (kj == key && j < l)) ? 1 : 0;
  }
  if (have) {
    t.srt.xs[rank] = z0;
    t.sp[rank] = l;
  }
  wave_lds_sync();
  // Lane l holds sorted position l: top-k (sampling.py:89-91) keeps the
  // first k with finite z.
  const double z = have ? t.srt.xs[l] : -(double)INFINITY;
  const int c = have ? t.sp[l] : 0;  // list position
  const bool kept = have && l < k && z > -(double)INFINITY;
  const int32_t tok = kept ? t.cid[c] : 0;
  if (kept && r.kept_bits) atomicOr(&r.kept_bits[tok >> 5], 1u << (tok & 31));

  // sampling.py:92-96
  const double e = kept ? exp(z) : 0.0;
  const double s1 = wave_sum(e);
  double x;
  if (p.min_p != 0.0) {
    const double cut_p = p.min_p * (1.0 / s1);
    const double tol = cut_p * 0x1p-49;
    x = e / s1;
    const bool close = x > 0.0 && fabs(x - cut_p) <= tol;
    if (x < cut_p) x = 0.0;
    if (__ballot(close)) flags |= DSR_FLAG_MARGIN;
    const double s2 = wave_sum(x);
    x = x / s2;
  } else {
    x = e / s1;
  }
  if (p.top_p < 1.0) {  // sampling.py:97-102, as f32_sorted_tail
    long long tgt = (long long)(p.top_p * 0x1p60);
    if (tgt == 0) tgt = 1;
    const long long fx = x > 0.0 ? (long long)(x * 0x1p60) : 0ll;
    const long long incl = wave_scan_dpp(fx);
    const long long fex = incl - fx;
    if (lane_value(incl, 63) >= tgt) {
      const unsigned long long hit = __ballot(fx > 0 && fex < tgt && fex + fx >= tgt);
      const double rt = lane_value(x, __ffsll((long long)hit) - 1);
      const double A = wave_sum(x > rt ? x : 0.0);
      const long long n_above = __popcll(__ballot(x > rt)), n_tie = __popcll(__ballot(x == rt));
      bool close;
      const long long keep = top_p_tie_keep(A, n_above, n_tie, rt, p.top_p, close);
      if (close) flags |= DSR_FLAG_MARGIN;
      int cutc = -1;
      if (keep > 0) {
        const int f = (int)n_above, lst = f + (int)n_tie - 1;
        if (lane_value(z, f) == lane_value(z, lst)) {
          cutc = (int)lane_value((uint32_t)c, f + (int)keep - 1);
        } else {  // several z round to one probability: rank the group by list position
          int rk = 0;
          for (int q = f; q <= lst; ++q) rk += (int)lane_value((uint32_t)c, q) < c ? 1 : 0;
          const unsigned long long hb = __ballot(l >= f && l <= lst && rk == (int)keep - 1);
          cutc = (int)lane_value((uint32_t)c, __ffsll((long long)hb) - 1);
        }
      }
      if (x < rt || (x == rt && c > cutc)) x = 0.0;
    } else {
      // The whole mass stays below top_p: nothing is removed.
      const double tot = wave_sum(x);
      if (fabs(tot - p.top_p) <= ((double)V + 16.0) * 0x1p-51) flags |= DSR_FLAG_MARGIN;
    }
  }

  const double total = wave_sum(x);  // sampling.py:103-106
  int st = (total > 0.0 && isfinite(total)) ? DSR_OK : DSR_E_NO_MASS;
  int64_t token = -1;
  int consumed = 0;
  if (st == DSR_OK) {
    x = x / total;
    if (kept) {
      if (r.probs_f32) r.probs_f32[tok] = (float)x;
      if (r.probs_f64) r.probs_f64[tok] = x;
    }
    // The final probabilities by list position (index order) for the draw.
    if (have) t.cz[c] = kept ? x : 0.0;
    wave_lds_sync();
    const double w = have ? t.cz[l] : 0.0;
    const long long npos = __popcll(__ballot(w > 0.0));
    const unsigned long long pos_l = __ballot(w > 0.0);
    if (a.rng_state || a.uniforms) {
      if (npos == 1) {
        token = t.cid[__ffsll((long long)pos_l) - 1];  // sampling.py:120-122: no uniform is drawn
      } else {
        uint64_t next[4];
        const double u = a.rng_state ? pcg64_random(a.rng_state + 4 * row, next) : a.uniforms[row];
        if (!(u >= 0.0 && u < 1.0)) {
          st = DSR_E_UNIFORM;
        } else {
          // categorical (sampling.py:126-128): the first index whose running
          // sum exceeds u times the total, in index order.
          const double tot2 = wave_sum(w);
          const double thr = u * tot2;
          const double tol = ((double)npos + 16.0) * 0x1p-51 * tot2;
          const double cv = wave_scan_dpp(w), before = cv - w;
          const unsigned long long cross = __ballot(w > 0.0 && cv > thr);
          int owner;
          if (cross) {
            owner = __ffsll((long long)cross) - 1;
            const double cvo = lane_value(cv, owner), bo = lane_value(before, owner);
            if (cvo - thr <= tol || (bo > 0.0 && thr - bo <= tol)) flags |= DSR_FLAG_MARGIN;
          } else {  // rounding left no crossing: the last positive entry
            owner = 63 - __clzll((long long)pos_l);
            flags |= DSR_FLAG_MARGIN;
          }
          token = t.cid[owner];
          consumed = 1;
        }
        if (a.rng_state && l == 0) store_rng(a, row, next);
      }
    }
  }
  if (l == 0) {
    a.out_token[row] = st == DSR_OK ? (int32_t)token : -1;
    a.out_consumed[row] = (uint8_t)(st == DSR_OK ? consumed : 0);
    a.out_status[row] = st;
    if (a.out_flags) a.out_flags[row] = (uint8_t)flags;
  }
}

// From the per-wave token lists (t.lv / t.li, wn entries in this wave) to
// the row's decision: the row-wide list as float64 z = (v - max) / T, then
// f32_sorted_tail, or radix_top_k and filter_tail when a bucket is too full.
__device__ __forceinline__ int f32_list_finish(const dsr_sample_args_t& a, int64_t row, const RowSpec& r,
                                               F32Shared& shu, int wave, int lane, int wn, double M, long long k,
                                               int64_t V, unsigned& flags, DistOut& out, int64_t& n, int& why) {
  F32Lists& t = shu.t;
  GenShared& sh = shu.gen;
  const int tid = threadIdx.x;
  const dsr_policy_t& p = r.pol;
  if (lane == 0) t.wn[wave] = wn;
  __syncthreads();
  int base = 0, total = 0, over = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int c = t.wn[w];
    over |= c > kF32WaveCap ? 1 : 0;
    if (w < wave) base += c;
    total += c;
  }
  if (over) {
    why = kHandCapacity;
    return -1;
  }
  // The row-wide list in index order, as float64 (v - max) / T
  // (sampling.py:86-88, true division).
  const double T = p.temperature;
  for (int i = lane; i < wn; i += 64) {
    t.cz[base + i] = ((double)t.lv[wave][i] - M) / T;
    t.cid[base + i] = t.li[wave][i];
  }
  __syncthreads();
  const int64_t nc = total;
  if (nc <= kWaveTailMax) {
    f32_wave_tail(a, row, r, t, (int)nc, k, V, flags);
    return kDecided;
  }

  const int st = f32_sorted_tail(r, t, sh, nc, k, V, flags, out, n);
  if (st != kTailFallback) return st;

  // ---- a bucket too full to rank: radix top-k over the list
  // (sampling.py:89-91), the kept tokens in index order, and filter_tail.
  uint64_t kth = 0;
  int64_t cut = INT64_MAX;
  if (k < nc) radix_top_k(t.cz, nc, k, sh, kth, cut);
  auto kept = [&](int64_t j, double z) {
    const uint64_t key = order_key(z);
    return z > -(double)INFINITY && (key > kth || (key == kth && j <= cut));
  };
  int64_t lo, hi;
  slice_of(tid, nc, lo, hi);
  long long cnt = 0;
  for (int64_t j = lo; j < hi; ++j) cnt += kept(j, t.cz[j]) ? 1 : 0;
  long long nk;
  long long pos = block_exclusive_scan_i64(cnt, sh.b, nk);
  if (nk > kSplitMaxK || nk < 1) {  // not reached: top-k keeps k tokens, the maximum among them
    why = kHandCapacity;
    return -1;
  }
  for (int64_t j = lo; j < hi; ++j) {
    const double z = t.cz[j];
    if (kept(j, z)) {
      const int32_t i = t.cid[j];
      t.kz[pos] = z;
      t.kid[pos] = i;
      ++pos;
      if (r.kept_bits) atomicOr(&r.kept_bits[i >> 5], 1u << (i & 31));
    }
  }
  __syncthreads();
  n = nk;
  const int32_t* kid = t.kid;
  return filter_tail(r, t.kz, nk, V, false, 0, -1, sh, flags, out, [kid](int64_t j) { return (int64_t)kid[j]; });
}

// Returns a status when the row is decided (kz / kid then hold the n final
// probabilities and their tokens, in index order), or -1 with the reason in
// `why` when the general path must decide it.
__device__ __forceinline__ int f32_distribution(const dsr_sample_args_t& a, int64_t row, const RowSpec& r,
                                                F32Shared& shu, unsigned& flags, DistOut& out, int64_t& n, int& why) {
  F32Lists& t = shu.t;
  GenShared& sh = shu.gen;
  const int tid = threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int64_t V = a.vocab;
  const uint32_t Q = (uint32_t)(V >> 2);
  const uint32_t QW = (Q + kWaves - 1) / kWaves;
  const dsr_policy_t& p = r.pol;
  out.onehot = -1;
  out.npos = 0;
  out.first = -1;
  if (!policy_ok(p)) {
    why = kHandPolicy;
    return -1;
  }
  if (p.temperature != 0.0 && !(p.top_k >= 1 && p.top_k <= kSplitMaxK && p.top_k < V)) {
    why = kHandTopK;
    return -1;
  }
  const long long k = p.temperature == 0.0 ? 1 : p.top_k;

  const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const float*)a.logits + row * a.ld), (short)0, (int)(V * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t mrs = __builtin_amdgcn_make_buffer_rsrc(
      a.allow_bits ? (void*)(a.allow_bits + row * a.allow_ld) : (void*)&kAllowAll, (short)0,
      a.allow_bits ? (int)(((V + 31) >> 5) * 4) : 0, 0x00020000);
  // The quad of slot j for lane `ln`, or an offset past every buffer (reads
  // 0) for slots past this wave's range.  Each pass derives its quads from
  // its own copy of the lane id (laundered through an empty asm), so the
  // compiler does not keep the first pass's 32 addresses alive for the
  // second, which spills.
  auto quad_at = [&](int j, uint32_t ln) -> uint32_t {
    const uint32_t cw = (uint32_t)j * 64u + ln;
    return cw < QW ? (uint32_t)wave * QW + cw : 0x0FFFFFFFu;
  };
  uint32_t ln1 = (uint32_t)lane;
  asm volatile("" : "+v"(ln1));
  auto quad_of = [&](int j) -> uint32_t { return quad_at(j, ln1); };
  // Allow nibble of quad q (4 tokens); all allowed without a mask.
  // The mask word holding quad q's bits, loaded without a branch (a load
  // inside one makes its use wait for every load in flight); without a
  // mask the descriptor's extent is 0 and the load reads 0.  nib4 takes the
  // quad's nibble once the word has landed.
  const uint32_t fill = a.allow_bits ? 0u : 0xFFFFFFFFu;
  auto allow4 = [&](uint32_t q) -> uint32_t {
    return __builtin_amdgcn_raw_buffer_load_b32(mrs, (int)(q < Q ? (q >> 3) * 4u : 0x7FFFFFF0u), 0, 0);
  };
  auto nib4 = [&](uint32_t word, uint32_t q) -> uint32_t { return ((word | fill) >> ((q & 7u) * 4u)) & 0xFu; };
  auto load4 = [&](uint32_t q) -> uint4 {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rrs, (int)(q < Q ? q * 16u : 0x7FFFFFF0u), 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
  };

  // ---- pass 1: quad maxima, the row maximum and its first index, validity.
  // The row's kept bits start at zero below (its probability row was cleared
  // by k_zero_probs before this launch); the finishing steps write the kept
  // tokens.
  uint32_t qp[kF32Slots / 2];  // 16-bit key prefixes of the quad maxima, slot j in half j & 1 of word j / 2
  uint32_t kmax = 0u;
  uint32_t imax = 0xFFFFFFFFu;  // index of this lane's first maximum (rows hold < 2^31 values)
  uint32_t bad = 0u;
  // Groups of four slots, two groups in flight: group g + 1's loads are
  // issued before group g is reduced.
  uint4 v[2][4];
  uint32_t m[2][4];
  auto issue = [&](int g) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v[g & 1][u] = load4(quad_of(4 * g + u));
      m[g & 1][u] = allow4(quad_of(4 * g + u));
    }
  };
  issue(0);
#pragma unroll
  for (int g = 0; g < kF32Slots / 4; ++g) {
    // A scheduling fence per group: left to itself the compiler hoists all
    // 32 loads and spills.
    __builtin_amdgcn_sched_barrier(0);
    if (g + 1 < kF32Slots / 4) issue(g + 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = 4 * g + u;
      const uint32_t q = quad_of(j);
      const uint4 x = v[g & 1][u];
      const uint32_t w4[4] = {x.x, x.y, x.z, x.w};
      // Disallowed tokens (and the zeros read past the row) become -inf;
      // the quad's maximum and its key, then the first element holding it
      // only when it raises this lane's maximum (keys treat -0 as +0, as
      // == does).
      const uint32_t nib = q < Q ? nib4(m[g & 1][u], q) : 0u;
      float f[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bad |= __builtin_isfpclass(__uint_as_float(w4[e]), 0x0203) ? 1u : 0u;  // NaN or +inf
        const uint32_t am = (uint32_t)((int32_t)(nib << (31 - e)) >> 31);
        f[e] = __uint_as_float((w4[e] & am) | (0xFF800000u & ~am));
      }
      const float mx = fmaxf(fmaxf(f[0], f[1]), fmaxf(f[2], f[3]));
      const uint32_t qm = f32_key(__float_as_uint(mx), true);
      // A lane's quads come in increasing index order: a strict comparison
      // keeps the first maximum.
      if (qm > kmax) {
        const uint32_t qe = f[0] == mx ? 0u : (f[1] == mx ? 1u : (f[2] == mx ? 2u : 3u));
        imax = 4u * q + qe;
        kmax = qm;
      }
      if (j & 1) qp[j >> 1] |= (qm >> 16) << 16; else qp[j >> 1] = qm >> 16;
      // Pin this slot's results here: left to itself the compiler sinks the
      // key computations to their uses and keeps the loaded quads live,
      // which spills (and a spill reload waits for every outstanding load).
      asm volatile("" : "+v"(qp[j >> 1]), "+v"(kmax), "+v"(imax), "+v"(bad));
    }
  }
  if (r.kept_bits)
    for (int64_t w = tid; w < r.kept_words; w += kThreads) r.kept_bits[w] = 0u;
  // One reduction for the row maximum's key (high word), its first index
  // (low word, complemented, so that the larger is the first) and validity
  // (all ones; no finite key reaches 0xFFFFFFFF).  The sign bit is flipped
  // so that the signed maximum orders the words as unsigned.
  const uint64_t mine = bad ? ~0ull : (((uint64_t)kmax << 32) | (uint64_t)(~imax));
  const uint64_t top = (uint64_t)block_max_i64((long long)(mine ^ 0x8000000000000000ull), sh.b) ^ 0x8000000000000000ull;
  if (top == ~0ull) {
    why = kHandInvalid;
    return -1;
  }
  const uint32_t K = (uint32_t)(top >> 32);
  if (K == 0u) {  // no allowed finite value
    why = kHandInvalid;
    return -1;
  }
  const int64_t first = (int64_t)(~(uint32_t)top);
  // The row maximum as a value: the key's inverse (K >= 2^31 for v >= 0).
  const uint32_t kb = (K & 0x80000000u) ? (K & 0x7FFFFFFFu) : ~K;
  const double M = (double)__uint_as_float(kb);

  if (p.temperature == 0.0) {  // sampling.py:82-85: the first index of the maximum
    out.onehot = first;
    out.npos = 1;
    out.first = first;
    if (tid == 0) {
      if (r.probs_f32) r.probs_f32[first] = 1.0f;
      if (r.probs_f64) r.probs_f64[first] = 1.0;
    }
    __syncthreads();  // the zeroing above is ordered before the kept bit
    if (tid == 0 && r.kept_bits) r.kept_bits[first >> 5] = 1u << (first & 31);
    n = 0;
    return DSR_OK;
  }

  // ---- tau: the 16-bit prefix of the k-th largest maximum over pairs of
  // quads (slots 2i and 2i + 1 of a lane; counted keys > 0).  The pairs
  // partition the row, so this is a lower bound for the k-th largest token
  // too.
  auto pair16 = [&](int i) -> uint32_t { return max(qp[i] & 0xFFFFu, qp[i] >> 16); };
  const uint32_t tau16 = f32_tau16<kF32Slots / 2>(t, wave, lane, K >> 16, k, pair16);
  if (tau16 == 0u) {  // fewer allowed finite pairs than k
    why = kHandCapacity;
    return -1;
  }
  const uint32_t tau = tau16 << 16;

  // ---- pass 2: the tokens with key >= tau, per wave in index order.  The
  // quads whose maximum reaches tau are listed first (slot-major, so in
  // index order) from the prefixes in registers, and only those are read
  // again, 64 to a load round.  A wave lists at most kF32WaveCap quads
  // (each holds a token to list); more overflow the token list too.
  uint32_t* ql = t.hist[wave];  // the histograms are no longer read (f32_pick ends on a barrier)
  auto slot16 = [&](int j) -> uint32_t { return (qp[j >> 1] >> (16 * (j & 1))) & 0xFFFFu; };
  uint32_t ln2 = (uint32_t)lane;
  asm volatile("" : "+v"(ln2));
  int nq = 0;  // uniform
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int j = 0; j < kF32Slots; ++j) {
    const uint32_t x = slot16(j);
    const bool need = x != 0u && x >= tau16;
    const uint64_t bal = __ballot(need);
    const int pos = nq + __popcll(bal & below);
    if (need && pos < kF32WaveCap) ql[pos] = quad_at(j, ln2);
    nq += __popcll(bal);
  }
  wave_lds_sync();
  int wn = 0;  // this wave's listed tokens (uniform)
  if (nq > kF32WaveCap) {
    wn = kF32WaveCap + 1;
  } else {
    constexpr int kRounds = kF32WaveCap / 64;
    const int rounds = (nq + 63) >> 6;
    uint4 v[kRounds];
    uint32_t m[kRounds], qq[kRounds];
#pragma unroll
    for (int u = 0; u < kRounds; ++u) {
      const int i = u * 64 + lane;
      qq[u] = i < nq ? ql[i] : 0x0FFFFFFFu;
      if (u < rounds) {
        v[u] = load4(qq[u]);
        m[u] = allow4(qq[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < kRounds; ++u) {
      if (u < rounds) {
        const uint32_t q = qq[u];
        const uint32_t w4[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
        const uint32_t nib = nib4(m[u], q);
        uint32_t sel = 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (q < Q && f32_key(w4[e], (nib >> e) & 1u) >= tau) sel |= 1u << e;
        const uint32_t c = (uint32_t)__popc(sel);
        const uint32_t incl = wave_scan_dpp(c);
        int pos = wn + (int)(incl - c);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if ((sel >> e) & 1u) {
            if (pos < kF32WaveCap) {
              t.lv[wave][pos] = __uint_as_float(w4[e]);
              t.li[wave][pos] = (int32_t)(4 * q + (uint32_t)e);
            }
            ++pos;
          }
        }
        wn += (int)lane_value(incl, 63);
      }
    }
  }
  return f32_list_finish(a, row, r, shu, wave, lane, wn, M, k, V, flags, out, n, why);
}


// ---------------------------------------------------------------------------
// Rows whose logits came from dsr_vocab_head, with its per-tile records
// (the tile's maximum and first column holding it, and flags): the records
// stand in for pass 1.  tau is the 16-bit prefix of the k-th largest tile
// maximum (the tiles partition the row, so it bounds the k-th largest token
// from below), and only the tiles whose maximum reaches it are read.  A row
// with fewer than k finite tiles, or more than kF32HeadMaxTiles tiles to
// read, returns kHeadFull: the full front end (pass 1 over the row) then
// decides it in the same workgroup.  The allow mask is not in the records,
// so masked batches never come here.

constexpr int kF32HeadTile = 128;      // columns per record (DSR_HEAD_TILE)
constexpr int kF32HeadMaxTiles = 256;  // tiles a row may read again: a fifth of a 129,280-token row
constexpr int kHeadFull = -3;

static inline bool f32_head_eligible(const dsr_sample_args_t& a) {
  return f32_path_eligible(a) && !a.allow_bits && a.vocab % kF32HeadTile == 0 && a.vocab / kF32HeadTile <= kThreads;
}

__device__ __forceinline__ int f32_distribution_head(const dsr_sample_args_t& a, int64_t row,
                                                     const dsr_head_part_t* parts, const RowSpec& r, F32Shared& shu,
                                                     unsigned& flags, DistOut& out, int64_t& n, int& why) {
  F32Lists& t = shu.t;
  GenShared& sh = shu.gen;
  const int tid = threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int64_t V = a.vocab;
  const int NT = (int)(V / kF32HeadTile);
  const dsr_policy_t& p = r.pol;
  out.onehot = -1;
  out.npos = 0;
  out.first = -1;
  if (!policy_ok(p)) {
    why = kHandPolicy;
    return -1;
  }
  if (p.temperature != 0.0 && !(p.top_k >= 1 && p.top_k <= kSplitMaxK && p.top_k < V)) {
    why = kHandTopK;
    return -1;
  }
  const long long k = p.temperature == 0.0 ? 1 : p.top_k;

  // Thread t holds tile t's record: its maximum's key (0 without a finite
  // value), the maximum's first index, and NaN / +inf.
  uint32_t key = 0u, fidx = 0xFFFFFFFFu, bad = 0u;
  if (tid < NT) {
    const dsr_head_part_t pt = parts[row * NT + tid];
    const uint32_t info = (uint32_t)pt.info, col = info >> 8;
    bad = info & 1u;
    if ((info & 2u) && col < (uint32_t)kF32HeadTile) {
      key = f32_key(__float_as_uint(pt.max), true);
      fidx = (uint32_t)tid * kF32HeadTile + col;
    }
  }
  if (r.kept_bits)
    for (int64_t w = tid; w < r.kept_words; w += kThreads) r.kept_bits[w] = 0u;
  const uint64_t mine = bad ? ~0ull : (((uint64_t)key << 32) | (uint64_t)(~fidx));
  const uint64_t top = (uint64_t)block_max_i64((long long)(mine ^ 0x8000000000000000ull), sh.b) ^ 0x8000000000000000ull;
  if (top == ~0ull) {
    why = kHandInvalid;
    return -1;
  }
  const uint32_t K = (uint32_t)(top >> 32);
  if (K == 0u) {  // no finite value
    why = kHandInvalid;
    return -1;
  }
  const int64_t first = (int64_t)(~(uint32_t)top);
  const uint32_t kb = (K & 0x80000000u) ? (K & 0x7FFFFFFFu) : ~K;
  const double M = (double)__uint_as_float(kb);
  if (p.temperature == 0.0) {  // sampling.py:82-85: the first index of the maximum
    out.onehot = first;
    out.npos = 1;
    out.first = first;
    if (tid == 0) {
      if (r.probs_f32) r.probs_f32[first] = 1.0f;
      if (r.probs_f64) r.probs_f64[first] = 1.0;
    }
    __syncthreads();  // the zeroing above is ordered before the kept bit
    if (tid == 0 && r.kept_bits) r.kept_bits[first >> 5] = 1u << (first & 31);
    n = 0;
    return DSR_OK;
  }

  const uint32_t tau16 = f32_tau16<1>(t, wave, lane, K >> 16, k, [&](int) { return key >> 16; });
  if (tau16 == 0u) return kHeadFull;  // fewer finite tiles than k
  const uint32_t tau = tau16 << 16;

  // The tiles to read, per wave in index order (wave w holds tiles 64w ..).
  const bool need = key != 0u && (key >> 16) >= tau16;
  const uint64_t bal = __ballot(need);
  const int nt = __popcll(bal);  // uniform
  uint32_t* ql = t.hist[wave];  // the histograms are no longer read (f32_pick ends on a barrier)
  if (need) ql[__popcll(bal & ((1ull << lane) - 1ull))] = (uint32_t)tid;
  if (lane == 0) ql[kF32Bins - 1] = (uint32_t)nt;  // past the wave's (at most 64) tiles
  __syncthreads();
  int tiles = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) tiles += (int)t.hist[w][kF32Bins - 1];
  if (tiles > kF32HeadMaxTiles) return kHeadFull;  // uniform

  // Two tiles per round (lanes 0-31 and 32-63, a quad each), eight rounds in
  // flight; tokens at or above tau listed per wave in index order.
  const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const float*)a.logits + row * a.ld), (short)0, (int)(V * 4), 0x00020000);
  constexpr int kBatch = 8;
  int wn = 0;  // this wave's listed tokens (uniform)
  const int rounds = (nt + 1) >> 1;
  for (int r0 = 0; r0 < rounds; r0 += kBatch) {
    uint4 v[kBatch];
    uint32_t qv[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int slot = 2 * (r0 + u) + (lane >> 5);
      qv[u] = slot < nt ? ql[slot] * (kF32HeadTile / 4) + (uint32_t)(lane & 31) : 0x0FFFFFFFu;
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(
          rrs, (int)(qv[u] < (uint32_t)(V >> 2) ? qv[u] * 16u : 0x7FFFFFF0u), 0, 0);
      v[u] = make_uint4(x[0], x[1], x[2], x[3]);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (r0 + u < rounds) {  // uniform
        const uint32_t q = qv[u];
        const uint32_t w4[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
        uint32_t sel = 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (q < (uint32_t)(V >> 2) && f32_key(w4[e], true) >= tau) sel |= 1u << e;
        const uint32_t c = (uint32_t)__popc(sel);
        const uint32_t incl = wave_scan_dpp(c);
        int pos = wn + (int)(incl - c);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if ((sel >> e) & 1u) {
            if (pos < kF32WaveCap) {
              t.lv[wave][pos] = __uint_as_float(w4[e]);
              t.li[wave][pos] = (int32_t)(4 * q + (uint32_t)e);
            }
            ++pos;
          }
        }
        wn += (int)lane_value(incl, 63);
      }
    }
  }
  return f32_list_finish(a, row, r, shu, wave, lane, wn, M, k, V, flags, out, n, why);
}
}  // namespace dsr
