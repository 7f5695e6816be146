// Device history tables (gfx950): the reference's dense `counts` /
// `generated_counts` pair (history.py:46-47,92,136-137; sampling.py:54-66)
// kept on the device as the sparse CSR table dsr_sample_rows reads: per row,
// strictly increasing token ids with their count and generated count.
//
// Two builders, each three launches on the caller's stream (no allocation,
// no synchronisation):
//   1. a count pass, one 1024-thread workgroup per row: validates the row and
//      writes its entry count to out_off[row + 1] and its status;
//   2. k_history_offsets turns those counts into offsets in place (one
//      workgroup; out_off[rows] is the total);
//   3. the write pass repeats the count pass's work and writes the entries,
//      or nothing at all when the total exceeds the caller's capacity.
//
// dsr_history_from_dense compacts dense count vectors (np.flatnonzero of
// counts > 0) with the reference's validation.  dsr_history_append adds
// tokens to a table as np.add.at does (history.py:136-137; the tentative
// prefix of terminal_sampling.py:129-133): the row's new tokens mark a
// presence bitmap of the vocabulary in LDS next to a bitmap of the row's old
// ids.  Per-word rank bases of the old ids, of the new ids and of the new ids
// the table lacks give, for any id, its rank in the merged row (old ids
// below it plus absent new ids below it), its old entry and its slot in a
// count table indexed by rank among the new ids, which carries each new id's
// multiplicity and generated multiplicity (16 bits each).  In the write pass
// a wave takes 64 consecutive words of the union of the two bitmaps and
// writes their entries 64 consecutive entries per store.
#pragma once

#include "dsr_wave.h"

namespace dsr {

constexpr int kHistWords = (DSR_MAX_VOCAB + 31) / 32;  // 4040 bitmap words
constexpr int kMaxAppend = DSR_MAX_APPEND;            // new tokens per row and call
static_assert(4 * kThreads >= kHistWords, "four bitmap words per thread");
static_assert(kMaxAppend < 65536, "multiplicities are packed in 16 bits");
constexpr int kTokPer = kMaxAppend / kThreads;  // a row's new tokens held per thread
static_assert(kTokPer * kThreads == kMaxAppend, "new tokens split evenly over the threads");

struct HistAppendArgs {
  const int64_t* off;   // [rows + 1] or null: empty input table
  const int32_t* ids;
  const int32_t* count;
  const int32_t* gen;
  const int32_t* tokens;
  const int64_t* tok_off;   // [rows + 1]
  const int64_t* gen_from;  // [rows] or null: every new token is generated
  int64_t rows, vocab, cap;
  int64_t* out_off;
  int32_t* out_ids;
  int32_t* out_count;
  int32_t* out_gen;
  int32_t* out_status;
};

struct HistDenseArgs {
  const int32_t* counts;     // [rows, ld]
  const int32_t* generated;  // [rows, ld] or null: generated counts = counts
  int64_t rows, vocab, ld, cap;
  int64_t* out_off;
  int32_t* out_ids;
  int32_t* out_count;
  int32_t* out_gen;
  int32_t* out_status;
};

constexpr int kHistGroups = (kHistWords + 63) / 64;  // groups of 64 bitmap words (one wave's stretch)
static_assert(kMaxAppend < 65536, "new-id ranks and multiplicities fit 16 bits");

// The write pass: both bitmaps, each word's rank base among the new ids,
// each 64-word group's base among the old ids and among the new ids the
// table lacks, and the new ids' multiplicities by rank.  ALLGEN (every new
// token generated) needs the multiplicity alone, two to a word: at 74 KB two
// such workgroups fit on a CU; with separate generated counts (106 KB) one.
template <bool ALLGEN>
struct HistAppendShared {
  uint32_t nb[kHistWords];       // new ids present
  uint32_t ob[kHistWords];       // old ids present
  uint16_t nbase[kHistWords];    // new ids below the word
  uint32_t gob[kHistGroups];     // old ids below the group
  uint32_t gub[kHistGroups];     // new ids absent from the table, below the group
  uint32_t cnt[ALLGEN ? kMaxAppend / 2 : kMaxAppend];  // by rank: ALLGEN 16-bit pairs, else mult | gen << 16
  int bad;
  SyncSlots sync;
};

// The count pass needs only the two bitmaps (33 KB).
struct HistCountShared {
  uint32_t nb[kHistWords];
  uint32_t ob[kHistWords];
  int bad;
  SyncSlots sync;
};

template <bool WRITE, bool ALLGEN> struct HistSharedOf { using T = HistCountShared; };
template <bool ALLGEN> struct HistSharedOf<true, ALLGEN> { using T = HistAppendShared<ALLGEN>; };

__device__ __forceinline__ uint32_t bits_below(uint32_t w, uint32_t b) { return __popc(w & ((1u << b) - 1u)); }

// One row of dsr_history_append.  WRITE = false: validate and count the
// merged row; WRITE = true: write it at out_off[row] (rows the count pass
// rejected, and every row when the total exceeds cap, write nothing).
// ALLGEN (no gen_from): every new token counts as generated.
template <bool WRITE, bool ALLGEN = false>
__global__ __launch_bounds__(kThreads) void k_history_append(HistAppendArgs a) {
  __shared__ typename HistSharedOf<WRITE, ALLGEN>::T sh;
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t V = a.vocab;
  const int words = (int)((V + 31) >> 5);
  BlockSync bs(sh.sync);
  const int64_t o0 = a.off ? a.off[row] : 0, o1 = a.off ? a.off[row + 1] : 0;
  const int64_t t0 = a.tok_off[row], t1 = a.tok_off[row + 1];
  const int64_t m = t1 - t0;
  const int64_t gf = a.gen_from ? a.gen_from[row] : 0;  // new tokens at positions >= gf are generated
  if (WRITE) {
    if (a.out_status[row] != DSR_OK || a.out_off[a.rows] > a.cap) return;  // uniform
  } else {
    int st = DSR_OK;
    if (m < 0 || m > kMaxAppend) st = DSR_E_APPEND;
    else if (o1 < o0 || o1 - o0 > V) st = DSR_E_HISTORY;
    if (st != DSR_OK) {
      if (tid == 0) {
        a.out_status[row] = st;
        a.out_off[row + 1] = 0;
      }
      return;
    }
  }
  // The row's new tokens, all loaded before any is used (their loads overlap
  // the set-up below): token q of this thread is at position tid + q * kThreads
  // of the row's tokens.  A row of more than kMaxAppend tokens was rejected
  // above; this reads inside [t0, t1) whatever m is.
  int32_t tk[kTokPer];
#pragma unroll
  for (int q = 0; q < kTokPer; ++q) {
    const int64_t i = (int64_t)tid + (int64_t)q * kThreads;
    tk[q] = i < m ? a.tokens[t0 + i] : 0;
  }
  for (int w = tid; w < words; w += kThreads) {
    sh.nb[w] = 0u;
    sh.ob[w] = 0u;
  }
  if constexpr (WRITE) {
    const int64_t cw = ALLGEN ? (m + 1) / 2 : m;  // count words in use
    for (int64_t i = tid; i < cw; i += kThreads) sh.cnt[i] = 0u;
  }
  if (tid == 0) sh.bad = 0;
  lds_barrier();
  // Old ids: strictly increasing, in range, 1 <= count <= DSR_MAX_COUNT, 0 <= gen <= count.
  for (int64_t e = o0 + tid; e < o1; e += kThreads) {
    const int32_t id = a.ids[e], c = a.count[e], g = a.gen[e];
    const bool ok = id >= 0 && id < V && (e == o0 || a.ids[e - 1] < id) && c >= 1 && c <= DSR_MAX_COUNT && g >= 0 &&
                    g <= c;
    if (ok) atomicOr(&sh.ob[id >> 5], 1u << (id & 31));
    else sh.bad = 1;
  }
#pragma unroll
  for (int q = 0; q < kTokPer; ++q) {
    if ((int64_t)tid + (int64_t)q * kThreads < m) {
      if (tk[q] >= 0 && tk[q] < V) atomicOr(&sh.nb[tk[q] >> 5], 1u << (tk[q] & 31));
      else sh.bad = 1;
    }
  }
  lds_barrier();
  if (sh.bad) {  // uniform: read after the barrier
    if (!WRITE && tid == 0) {
      a.out_status[row] = DSR_E_HISTORY;
      a.out_off[row + 1] = 0;
    }
    return;
  }
  // Rank bases per word; thread t holds words 4t .. 4t + 3, so thread order
  // is word order.  New and absent-new counts share one packed scan (each
  // total is at most kMaxAppend < 2^16).
  uint32_t nw[4], ow[4], pn = 0, pu = 0;
  long long po = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int w = 4 * tid + q;
    nw[q] = w < words ? sh.nb[w] : 0u;
    ow[q] = w < words ? sh.ob[w] : 0u;
    pn += __popc(nw[q]);
    pu += __popc(nw[q] & ~ow[q]);
    po += __popc(ow[q]);
  }
  long long n_old;
  uint32_t bex, btot;
  const long long oex = bs.scan2(po, pn | (pu << 16), n_old, bex, btot);
  if constexpr (!WRITE) {
    if (tid == 0) {
      a.out_status[row] = DSR_OK;
      a.out_off[row + 1] = n_old + (long long)(btot >> 16);
    }
    return;
  } else {
    {
      // Thread t holds words 4t .. 4t + 3; the group of 64 words starting at
      // word 4t takes thread t's bases when t is a multiple of 16.
      uint32_t nb0 = bex & 0xFFFFu, ub0 = bex >> 16, ob0 = (uint32_t)oex;
      if ((tid & 15) == 0 && 4 * tid < words) {
        sh.gob[tid >> 4] = ob0;
        sh.gub[tid >> 4] = ub0;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int w = 4 * tid + q;
        if (w < words) sh.nbase[w] = (uint16_t)nb0;
        nb0 += __popc(nw[q]);
      }
    }
    lds_barrier();
    // Multiplicities of the new ids (and of their generated occurrences).
#pragma unroll
    for (int q = 0; q < kTokPer; ++q) {
      const int64_t i = (int64_t)tid + (int64_t)q * kThreads;
      if (i < m) {
        const uint32_t t = (uint32_t)tk[q], w = t >> 5, b = t & 31u;
        const uint32_t r = (uint32_t)sh.nbase[w] + bits_below(sh.nb[w], b);
        if constexpr (ALLGEN) atomicAdd(&sh.cnt[r >> 1], 1u << (16u * (r & 1u)));
        else atomicAdd(&sh.cnt[r], i >= gf ? 0x10001u : 1u);
      }
    }
    lds_barrier();
    // The merged row is the union of both bitmaps in id order.  Wave w takes
    // the groups of 64 consecutive words g0 = 64 w, 64 (w + 16), ...; the
    // group's entries are contiguous in the output from word g0's rank in the
    // merged row (old ids below it plus absent new ids below it), word s of the
    // group holding entries [ex_s, ex_s + popc) of them.  The wave writes them
    // 64 at a time with lane l taking entry i = i0 + l, so every store covers
    // 64 consecutive entries: the word holding entry i is the last lane s with
    // ex_s <= i (a binary search over the lanes), its id is that word's
    // (i - ex_s)-th set bit.  An old id's entry is its rank in the old bitmap;
    // a new id's multiplicities are at its rank in the new bitmap.
    const int lane = lane_id(), wave = wave_id();
    const int64_t base = a.out_off[row];
    for (int g0 = wave * 64; g0 < words; g0 += kWaves * 64) {  // uniform over the wave
      const int w = g0 + lane, G = g0 >> 6;
      uint32_t nwv = 0u, owv = 0u, nbw = 0u;
      if (w < words) {
        nwv = sh.nb[w];
        owv = sh.ob[w];
        nbw = sh.nbase[w];
      }
      const uint32_t po = (uint32_t)__popc(owv);
      const uint32_t obw = sh.gob[G] + wave_scan_dpp(po) - po;  // old ids below this lane's word
      const uint32_t uw = nwv | owv;
      const uint32_t n = (uint32_t)__popc(uw);
      const uint32_t ex = wave_scan_dpp(n) - n;
      const uint32_t total = lane_value(ex + n, 63);
      const int64_t p0 = base + (int64_t)sh.gob[G] + (int64_t)sh.gub[G];  // word g0's rank in the merged row
      for (uint32_t i0 = 0; i0 < total; i0 += 64) {  // uniform: every lane takes part in the shuffles
        const uint32_t i = i0 + (uint32_t)lane;
        int s = 0;
#pragma unroll
        for (int step = 32; step >= 1; step >>= 1)  // s + step <= 63 at every step
          if ((uint32_t)__shfl((int)ex, s + step) <= i) s += step;
        const uint32_t k = i - (uint32_t)__shfl((int)ex, s);
        const uint32_t u = (uint32_t)__shfl((int)uw, s);
        const uint32_t nws = (uint32_t)__shfl((int)nwv, s), ows = (uint32_t)__shfl((int)owv, s);
        const uint32_t nbs = (uint32_t)__shfl((int)nbw, s), obs = (uint32_t)__shfl((int)obw, s);
        uint32_t b = 0, kk = k;  // the k-th set bit of u, by halves
#pragma unroll
        for (uint32_t h = 16; h >= 1; h >>= 1) {
          const uint32_t c = (uint32_t)__popc((u >> b) & ((1u << h) - 1u));
          if (kk >= c) {
            b += h;
            kk -= c;
          }
        }
        if (i < total) {
          int32_t c = 0, g = 0;
          if ((ows >> b) & 1u) {
            const int64_t e = o0 + obs + bits_below(ows, b);
            c = a.count[e];
            g = a.gen[e];
          }
          if ((nws >> b) & 1u) {
            const uint32_t r = nbs + bits_below(nws, b);
            if constexpr (ALLGEN) {
              const int32_t add = (int32_t)((sh.cnt[r >> 1] >> (16u * (r & 1u))) & 0xFFFFu);
              c += add;
              g += add;
            } else {
              const uint32_t add = sh.cnt[r];
              c += (int32_t)(add & 0xFFFFu);
              g += (int32_t)(add >> 16);
            }
          }
          const int64_t p = p0 + i;
          a.out_ids[p] = 32 * (g0 + s) + (int32_t)b;
          a.out_count[p] = c;
          a.out_gen[p] = g;
        }
      }
    }
  }
}

// One row of dsr_history_from_dense.  The count pass validates as
// sampling.py:54-58 then :62-65 do (DSR_E_COUNTS before DSR_E_GENERATED) and
// counts the nonzero entries; the write pass compacts them in index order:
// wave w owns ids [w * seg, (w + 1) * seg), counts its nonzero entries, and
// after one barrier writes them from its base (ballot ranks per 64 ids).
template <bool WRITE>
__global__ __launch_bounds__(kThreads) void k_history_dense(HistDenseArgs a) {
  __shared__ SyncSlots sync;
  __shared__ uint32_t wn[kWaves];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t V = a.vocab;
  const int32_t* C = a.counts + row * a.ld;
  const int32_t* G = a.generated ? a.generated + row * a.ld : C;
  BlockSync bs(sync);
  if (!WRITE) {
    uint32_t bad = 0, nnz = 0;
    long long sum = 0;
    for (int64_t i = tid; i < V; i += kThreads) {
      const int32_t c = C[i], g = G[i];
      if (c < 0 || c > DSR_MAX_COUNT) bad |= 1u;
      if (g < 0 || g > c) bad |= 2u;
      sum += c < 0 ? 0 : (c > DSR_MAX_COUNT ? DSR_MAX_COUNT + 1 : c);
      nnz += c > 0;
    }
    const uint32_t bad_any = bs.reduce(bad, 0u, [](uint32_t p, uint32_t q) { return p | q; });
    const long long total = bs.sum(sum);
    const uint32_t n = bs.sum(nnz);
    if (tid == 0) {
      const int st = ((bad_any & 1u) || total > DSR_MAX_COUNT) ? DSR_E_COUNTS : ((bad_any & 2u) ? DSR_E_GENERATED : DSR_OK);
      a.out_status[row] = st;
      a.out_off[row + 1] = st == DSR_OK ? (int64_t)n : 0;
    }
    return;
  }
  if (a.out_status[row] != DSR_OK || a.out_off[a.rows] > a.cap) return;  // uniform
  const int lane = lane_id(), wave = wave_id();
  const int64_t seg = ((V + kWaves - 1) / kWaves + 63) & ~(int64_t)63;
  const int64_t lo = (int64_t)wave * seg, hi = lo + seg < V ? lo + seg : V;
  uint32_t mine = 0;
  for (int64_t i = lo + lane; i - lane < hi; i += 64) mine += (uint32_t)__popcll(__ballot(i < hi && C[i] > 0));
  if (lane == 0) wn[wave] = mine;
  lds_barrier();
  int64_t pos = a.out_off[row];
  for (int w = 0; w < wave; ++w) pos += wn[w];
  for (int64_t i = lo + lane; i - lane < hi; i += 64) {
    int32_t c = 0;
    if (i < hi) c = C[i];
    const unsigned long long b = __ballot(c > 0);
    if (c > 0) {
      const int64_t p = pos + lanes_below(b);
      a.out_ids[p] = (int32_t)i;
      a.out_count[p] = c;
      a.out_gen[p] = G[i];
    }
    pos += __popcll(b);
  }
}

// Entry counts at off[1 .. rows] -> offsets in place; off[0] = 0.  One
// workgroup; thread t sums a contiguous run of rows.
__global__ __launch_bounds__(kThreads) void k_history_offsets(int64_t* off, int64_t rows) {
  __shared__ SyncSlots sync;
  BlockSync bs(sync);
  const int tid = threadIdx.x;
  const int64_t per = (rows + kThreads - 1) / kThreads;
  const int64_t lo = 1 + (int64_t)tid * per, hi = lo + per < rows + 1 ? lo + per : rows + 1;
  long long s = 0;
  for (int64_t i = lo; i < hi; ++i) s += off[i];
  long long total;
  long long run = bs.scan(s, total);
  for (int64_t i = lo; i < hi; ++i) {
    run += off[i];
    off[i] = run;
  }
  if (tid == 0) off[0] = 0;
}

}  // namespace dsr
