// Register-resident fast path for bf16 rows (gfx950, wave64, no MFMA).
//
// One 1024-thread workgroup owns one row of up to 131,072 bf16 logits.  The
// row is read from HBM exactly once, by raw buffer loads of 16 bytes issued
// all up front, straight into VGPRs (16 x uint4 per thread: 256 KB per row
// across the workgroup), and turned into order-preserving 16-bit keys with
// the allow mask and the NaN/+inf check fused into that pass, which overlaps
// the loads still in flight (the staging barrier orders LDS only).  Wave w
// owns the contiguous chunk range [w*CW, (w+1)*CW) of 8-token chunks; lane l
// of it takes chunk w*CW + 64*j + l at step j, so every load instruction
// reads a contiguous 1 KB and the row's index order is (wave, j, lane, elem).
//
// Selection works on chunks first, so per-element work stays off the
// 129k-token row:
//   * a 12-bit radix histogram of the 16,160 chunk maxima gives tau, the low
//     edge of the bin that holds the k-th largest chunk maximum: at least k
//     chunks (hence k tokens) reach tau, and only about k more do;
//   * those chunks are compacted, whole and in index order, into LDS with
//     one ballot per register slot;
//   * a 12-bit and a 4-bit radix pass over the tokens of that short list give
//     the exact k-th key; its tie group is resolved by index (lowest first),
//     as the reference's stable argsort does (sampling.py:89-91), and one
//     packed scan gives both tie ranks and the kept tokens' positions;
//   * the k <= 1024 kept tokens then sit one per thread: float64
//     (v - max) / T, exp, sums, min-p, top-p (radix passes over probability
//     mass in fixed point, then exact float64 tie arithmetic) and the
//     index-order CDF search of categorical (sampling.py:92-128).
// Workgroup reductions use DPP inside waves and cost one barrier each.
//
// The path is exact only where bf16 key order equals the reference's float64
// order; each row checks that at its decision boundaries (no +-0 boundary,
// neighbouring bf16 values keep distinct (v - max) / T and probabilities) and
// otherwise hands the row to the general path in the same workgroup, as it
// does for rows with penalties, bias, no top-k, k > 1024 or too many
// boundary chunks.
#pragma once

#include "dsr_general.h"
#include "dsr_wave.h"

namespace dsr {

constexpr int kFastChunks = 16;                                         // 16-byte chunks per thread
constexpr int64_t kFastMaxVocab = (int64_t)kThreads * kFastChunks * 8;  // 131072
constexpr int kChunkCap = 2048;                                         // compacted chunk list
constexpr int kFastMaxK = kThreads;                                     // one kept token per thread
constexpr int kBins = 4096;                                             // 12-bit radix digit

// Why a row is handed to the general path (reported in out_flags bits 4-7).
constexpr int kHandPolicy = 1;     // controls out of bounds (the general path reports it)
constexpr int kHandTopK = 2;       // no top-k, or k > 1024, or k >= vocabulary
constexpr int kHandZero = 3;       // a decision boundary sits at +-0
constexpr int kHandCapacity = 4;   // more than kChunkCap chunks reach tau
constexpr int kHandOrder = 5;      // bf16 key order may differ from float64 order at a boundary

struct FastLists {
  union {
    struct {
      uint32_t lut[256][4];                // allow byte -> four 2 x 16-bit lane masks
      uint32_t allow[kFastMaxVocab / 32];  // the row's allow bitmask
    } stage;                               // pass 1 only
    struct {
      uint4 keys[kChunkCap];               // chunks reaching tau, index order
      uint32_t id[kChunkCap];
    } list;
  };
  uint32_t hist[2][kBins];                 // 12-bit counts: chunk maxima, then list tokens
  unsigned long long mass[kBins];          // 12-bit fixed-point probability mass
  uint32_t sub[16];                        // 4-bit second digit
  unsigned long long submass[16];
  uint16_t kkey[kFastMaxK];                // kept tokens, index order
  uint32_t kidx[kFastMaxK];
  int sel[4];
  long long sel_mass;
  double bcast_d;
  int bcast_i[2];
  SyncSlots sync;
};

struct FastShared {
  union {
    GenShared gen;  // reused by the general path when a row falls back
    FastLists f;
  };
};

typedef unsigned short dsr_us2 __attribute__((ext_vector_type(2)));
typedef short dsr_s2 __attribute__((ext_vector_type(2)));

// Two bf16 -> two order-preserving 16-bit keys (larger value, larger key).
__device__ __forceinline__ uint32_t bf16x2_keys(uint32_t x) {
  dsr_s2 v = __builtin_bit_cast(dsr_s2, x);
  dsr_s2 sg = v >> (short)15;
  return x ^ (__builtin_bit_cast(uint32_t, sg) | 0x80008000u);
}

__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(dsr_us2, a),
                                                                __builtin_bit_cast(dsr_us2, b)));
}

__device__ __forceinline__ uint32_t pk_min_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(dsr_us2, a),
                                                                __builtin_bit_cast(dsr_us2, b)));
}

__device__ __forceinline__ double bf16_key_value(uint32_t key) {
  const uint32_t raw = (key & 0x8000u) ? (key ^ 0x8000u) : (key ^ 0xFFFFu);
  return (double)__uint_as_float(raw << 16);
}

constexpr uint32_t kKeyNegInf = 0x007Fu;   // key of -inf; masked tokens get key 0
constexpr uint32_t kKeyPosInf = 0xFF80u;
constexpr uint32_t kKeyNegZero = 0x7FFFu;
constexpr uint32_t kKeyPosZero = 0x8000u;

__device__ __forceinline__ bool zero_key(uint32_t k) { return k == kKeyNegZero || k == kKeyPosZero; }

__device__ __forceinline__ uint32_t key_at(const uint4& v, int e) {
  const uint32_t w = e < 4 ? (e < 2 ? v.x : v.y) : (e < 6 ? v.z : v.w);
  return (w >> (16 * (e & 1))) & 0xFFFFu;
}

__device__ __forceinline__ uint32_t lanes_below(unsigned long long b) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
}

static inline bool fast_path_eligible(const dsr_sample_args_t& a) {
  return a.dtype == DSR_BF16 && a.vocab >= 8 && a.vocab <= kFastMaxVocab && (a.vocab & 7) == 0 && (a.ld & 7) == 0 &&
         ((uintptr_t)a.logits & 15u) == 0 && a.pen_off == nullptr && a.bias_off == nullptr;
}

// Writes the row's decision (token may be -1 with no draw).
__device__ __forceinline__ void fast_write_result(const dsr_sample_args_t& a, int64_t row, int st, int64_t token,
                                                  int consumed, unsigned flags) {
  a.out_token[row] = st == DSR_OK ? (int32_t)token : -1;
  a.out_consumed[row] = (uint8_t)(st == DSR_OK ? consumed : 0);
  a.out_status[row] = st;
  if (a.out_flags) a.out_flags[row] = (uint8_t)flags;
}

// Zero the optional dense outputs of a row before the kept tokens are scattered.
__device__ __forceinline__ void fast_clear_outputs(const dsr_sample_args_t& a, int64_t row) {
  const int64_t V = a.vocab;
  if (a.out_probs_f32) {
    float* o = a.out_probs_f32 + row * a.probs_ld;
    for (int64_t i = threadIdx.x; i < V; i += kThreads) o[i] = 0.0f;
  }
  if (a.out_probs_f64) {
    double* o = a.out_probs_f64 + row * a.probs_ld;
    for (int64_t i = threadIdx.x; i < V; i += kThreads) o[i] = 0.0;
  }
  if (a.out_kept_bits) {
    uint32_t* o = a.out_kept_bits + row * a.kept_ld;
    const int64_t words = (V + 31) >> 5;
    for (int64_t i = threadIdx.x; i < words; i += kThreads) o[i] = 0u;
  }
  __syncthreads();
}

__device__ __forceinline__ void fast_scatter(const dsr_sample_args_t& a, int64_t row, int64_t idx, double p) {
  if (a.out_probs_f32) a.out_probs_f32[row * a.probs_ld + idx] = (float)p;
  if (a.out_probs_f64) a.out_probs_f64[row * a.probs_ld + idx] = p;
  if (a.out_kept_bits) atomicOr(&a.out_kept_bits[row * a.kept_ld + (idx >> 5)], 1u << (idx & 31));
}

// Over 4096 counting bins held 4 per thread (scanned from the top), finds the
// bin where the count first reaches `rem`: sel[0] = bin, sel[1] = count above.
__device__ __forceinline__ void select_count_bin(const uint32_t* hist, uint32_t rem, FastLists& sh, BlockSync& bs) {
  const int rt = kThreads - 1 - (int)threadIdx.x;
  const uint4 c = *(const uint4*)(hist + 4 * rt);
  uint32_t total;
  uint32_t above = bs.scan(c.x + c.y + c.z + c.w, total);
  const uint32_t cc[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int j = 3; j >= 0; --j) {
    if (above < rem && rem <= above + cc[j]) {
      sh.sel[0] = 4 * rt + j;
      sh.sel[1] = (int)above;
    }
    above += cc[j];
  }
  lds_barrier();
}

// The same for fixed-point mass; sel[0] = -1 if the mass never reaches tgt.
__device__ __forceinline__ void select_mass_bin(const unsigned long long* m, unsigned long long tgt, FastLists& sh,
                                                BlockSync& bs) {
  const int rt = kThreads - 1 - (int)threadIdx.x;
  unsigned long long c[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) c[j] = m[4 * rt + j];
  if (threadIdx.x == 0) sh.sel[0] = -1;  // ordered before the writes below by the scan's barrier
  long long total;
  unsigned long long above = (unsigned long long)bs.scan((long long)(c[0] + c[1] + c[2] + c[3]), total);
#pragma unroll
  for (int j = 3; j >= 0; --j) {
    if (above < tgt && tgt <= above + c[j]) {
      sh.sel[0] = 4 * rt + j;
      sh.sel_mass = (long long)above;
    }
    above += c[j];
  }
  lds_barrier();
}

// Returns 0 if the row was decided here, else the reason it is handed to the
// general path (kHand*).
__device__ int fast_sample_row(const dsr_sample_args_t& a, int64_t row, FastShared& shu) {
  FastLists& sh = shu.f;
  const dsr_policy_t pol = a.policy[row];
  const bool greedy = pol.temperature == 0.0;
  const int64_t V = a.vocab;
  if (!policy_ok(pol)) return kHandPolicy;
  if (!greedy && !(pol.top_k >= 1 && pol.top_k <= kFastMaxK && pol.top_k < V)) return kHandTopK;

  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const uint32_t C = (uint32_t)(V >> 3);
  const uint32_t CW = (C + kWaves - 1) / kWaves;
  const uint16_t* lrow = (const uint16_t*)a.logits + row * a.ld;
  const uint32_t* mrow = a.allow_bits ? a.allow_bits + row * a.allow_ld : nullptr;
  BlockSync bs(sh.sync);

  // ---- one HBM pass: every load of the row is issued up front, as raw
  // buffer loads over the row (32-bit offsets; out-of-range reads return 0).
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)lrow, (short)0, (int)(V * 2), 0x00020000);
  uint4 d[kFastChunks];
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j) {
    const uint32_t cw = (uint32_t)j * 64u + (uint32_t)lane;
    const uint32_t off = cw < CW ? (wave * CW + cw) * 16u : 0x7FFFFFF0u;  // chunks of the next wave read as 0
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)off, 0, 0);
    d[j] = make_uint4(v[0], v[1], v[2], v[3]);
  }
  // While the row streams in: stage the allow bitmask (one byte per 8-token
  // chunk) and the mask lookup table, and clear the histograms.
  const int64_t mwords = (V + 31) >> 5;
  if (mrow) {
    for (int64_t i = tid; i < mwords; i += kThreads) sh.stage.allow[i] = mrow[i];
  }
  {
    const uint32_t m = (uint32_t)tid >> 2, q = (uint32_t)tid & 3u;
    sh.stage.lut[m][q] = (((m >> (2 * q)) & 1u) ? 0x0000FFFFu : 0u) | (((m >> (2 * q + 1)) & 1u) ? 0xFFFF0000u : 0u);
  }
  for (int j = tid; j < 2 * kBins; j += kThreads) (&sh.hist[0][0])[j] = 0u;
  for (int j = tid; j < kBins; j += kThreads) sh.mass[j] = 0ull;
  if (tid < 16) {
    sh.sub[tid] = 0u;
    sh.submass[tid] = 0ull;
  }
  lds_barrier();  // LDS only: the row's loads keep streaming
  const uint8_t* mbytes = (const uint8_t*)sh.stage.allow;

  // ---- keys, mask, NaN/+inf check, chunk maxima (pass 1, as chunks arrive).
  uint32_t rmax = 0u, rmin = 0xFFFFFFFFu, cmx[kFastChunks / 2];
  uint32_t tmax = 0u;
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j) {
    // Keep each chunk's mask lookup next to its use: hoisting all sixteen
    // 16-byte lookups would need 64 more VGPRs than the row leaves free.
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t cw = (uint32_t)j * 64u + (uint32_t)lane;
    const uint32_t c = wave * CW + cw;  // < 16384: always inside the staged bitmask
    const uint32_t staged = mbytes[c];  // read unconditionally; selected below without a branch
    const uint32_t mbyte = (cw < CW && c < C) ? (mrow ? staged : 0xFFu) : 0u;
    const uint4 lm = *(const uint4*)sh.stage.lut[mbyte];
    uint32_t w[4] = {d[j].x, d[j].y, d[j].z, d[j].w};
    const uint32_t m4[4] = {lm.x, lm.y, lm.z, lm.w};
    uint32_t cm = 0u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t k = bf16x2_keys(w[q]);
      rmax = pk_max_u16(rmax, k);
      rmin = pk_min_u16(rmin, k);
      w[q] = k & m4[q];
      cm = pk_max_u16(cm, w[q]);
    }
    d[j] = make_uint4(w[0], w[1], w[2], w[3]);
    const uint32_t cmj = max(cm & 0xFFFFu, cm >> 16);
    if (j & 1) cmx[j >> 1] |= cmj << 16; else cmx[j >> 1] = cmj;
    tmax = max(tmax, cmj);
  }
  const long long bad = max(rmax & 0xFFFFu, rmax >> 16) >= kKeyPosInf || min(rmin & 0xFFFFu, rmin >> 16) < kKeyNegInf;
  // One reduction carries both the row maximum and the NaN/+inf flag, so no
  // branch separates pass 1 from the uses of its masked keys.
  const long long red = bs.max((long long)tmax | (bad << 32));
  if (red >> 32) {
    if (tid == 0) fast_write_result(a, row, DSR_E_LOGITS, -1, 0, 0);
    return 0;
  }
  const uint32_t Mkey = (uint32_t)red;
  if (Mkey <= kKeyNegInf) {
    if (tid == 0) fast_write_result(a, row, DSR_E_MASKED, -1, 0, 0);
    return 0;
  }
  if (zero_key(Mkey)) return kHandZero;  // +0 and -0 tie in value but not in key

  // ---- tau: low edge of the 12-bit bin holding the k-th largest chunk maximum.
  const uint32_t k = greedy ? 1u : (uint32_t)pol.top_k;
  uint32_t tau = Mkey;
  if (!greedy) {
#pragma unroll
    for (int j = 0; j < kFastChunks; ++j) atomicAdd(&sh.hist[0][((cmx[j >> 1] >> (16 * (j & 1))) & 0xFFFFu) >> 4], 1u);
    lds_barrier();
    select_count_bin(sh.hist[0], k, sh, bs);
    tau = (uint32_t)sh.sel[0] << 4;
  }

  // ---- compact the chunks whose maximum reaches tau, whole, in index order.
  uint32_t wn = 0;
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j)
    wn += (uint32_t)__popcll(__ballot(((cmx[j >> 1] >> (16 * (j & 1))) & 0xFFFFu) >= tau));
  uint32_t nlist;
  uint32_t lpos = lane_value(bs.scan(lane == 0 ? wn : 0u, nlist), 0);
  if (nlist > (uint32_t)kChunkCap) return kHandCapacity;  // uniform
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j) {
    const bool q = ((cmx[j >> 1] >> (16 * (j & 1))) & 0xFFFFu) >= tau;
    const unsigned long long b = __ballot(q);
    if (q) {
      const uint32_t p = lpos + lanes_below(b);
      sh.list.keys[p] = d[j];
      sh.list.id[p] = wave * CW + (uint32_t)j * 64u + (uint32_t)lane;
    }
    lpos += (uint32_t)__popcll(b);
  }
  lds_barrier();

  if (greedy) {  // sampling.py:82-85: the first listed chunk holds the first maximum
    if (tid == 0) {
      const uint4 v = sh.list.keys[0];
      int e = 0;
      while (e < 7 && key_at(v, e) != Mkey) ++e;
      sh.bcast_i[0] = (int)(8u * sh.list.id[0]) + e;
    }
    lds_barrier();
    const int64_t tok = sh.bcast_i[0];
    if (a.out_probs_f32 || a.out_probs_f64 || a.out_kept_bits) {
      fast_clear_outputs(a, row);
      if (tid == 0) fast_scatter(a, row, tok, 1.0);
    }
    if (tid == 0) fast_write_result(a, row, DSR_OK, a.uniforms ? tok : -1, 0, 0);
    return 0;
  }

  // ---- exact top-k over the listed tokens: 12-bit then 4-bit radix digit.
  // Thread t holds list chunks 2t and 2t+1 (index order is thread order).
  uint4 lv[2];
  uint32_t lid[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const uint32_t li = 2u * (uint32_t)tid + c;
    const bool ok = li < nlist;
    lv[c] = ok ? sh.list.keys[li] : make_uint4(0u, 0u, 0u, 0u);  // masked keys: below any tau
    lid[c] = ok ? sh.list.id[li] : 0u;
  }
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t key = key_at(lv[c], e);
      if (key >= tau) atomicAdd(&sh.hist[1][key >> 4], 1u);
    }
  lds_barrier();
  select_count_bin(sh.hist[1], k, sh, bs);
  const uint32_t b1 = (uint32_t)sh.sel[0], rem1 = k - (uint32_t)sh.sel[1];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t key = key_at(lv[c], e);
      if (key >= tau && (key >> 4) == b1) atomicAdd(&sh.sub[key & 15u], 1u);
    }
  lds_barrier();
  uint32_t bkey = 0, need = 0;
  {
    uint32_t above = 0;
    for (int j = 15; j >= 0; --j) {  // every thread reads the 16 counts and selects
      const uint32_t c = sh.sub[j];
      if (above < rem1 && rem1 <= above + c) {
        bkey = (b1 << 4) | (uint32_t)j;
        need = rem1 - above;  // boundary-key tokens kept, lowest index first
      }
      above += c;
    }
  }
  // One scan of (tokens above the boundary, boundary ties) per thread gives
  // every thread its tie rank and the position of its kept tokens.
  uint32_t n_up = 0, n_eq = 0;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t key = key_at(lv[c], e);
      n_up += key > bkey;
      n_eq += key == bkey;
    }
  uint32_t ptot;
  const uint32_t pex = bs.scan(n_up | (n_eq << 16), ptot);
  uint32_t tr = pex >> 16;                        // ties before this thread
  uint32_t kb = (pex & 0xFFFFu) + min(tr, need);  // kept tokens before this thread
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t key = key_at(lv[c], e);
      bool keep = key > bkey;
      if (key == bkey) keep = tr++ < need;
      if (keep && kb < (uint32_t)kFastMaxK) {
        sh.kkey[kb] = (uint16_t)key;
        sh.kidx[kb] = 8u * lid[c] + e;
        ++kb;
      }
    }
  const uint32_t ktot = (ptot & 0xFFFFu) + min(ptot >> 16, need);
  // Boundary certificate: the bf16 neighbours of the k-th value must stay
  // distinct after (v - max) / T, so key order and the reference's float64
  // order agree on which boundary tokens tie (resolved by index).
  const double T = pol.temperature;
  const double M = bf16_key_value(Mkey);
  if (tid == 0) {
    int ok = ktot == k;
    if (bkey > kKeyNegInf) {
      if (zero_key(bkey)) {
        ok = 0;
      } else {
        const double sb = (bf16_key_value(bkey) - M) / T;
        const double sp = bkey - 1 > kKeyNegInf ? (bf16_key_value(bkey - 1) - M) / T : -INFINITY;
        const double sn = bkey + 1 < kKeyPosInf ? (bf16_key_value(bkey + 1) - M) / T : INFINITY;
        ok = ok && sp < sb && sb < sn;
      }
    }
    sh.bcast_i[0] = ok;
  }
  lds_barrier();
  if (!sh.bcast_i[0]) return kHandOrder;

  // ---- one kept token per thread: softmax, min-p, top-p, categorical.
  const bool have = tid < (int)k;
  const uint32_t key = have ? sh.kkey[tid] : 0u;
  const int64_t idx = have ? (int64_t)sh.kidx[tid] : 0;
  const bool fin = have && key > kKeyNegInf;
  unsigned flags = 0;
  double r = fin ? exp((bf16_key_value(key) - M) / T) : 0.0;  // sampling.py:86-92
  const double s1 = bs.sum(r);
  r = r / s1;                                                  // :93
  double s2 = 0.0;                                             // min-p renormaliser (0: off)
  bool minp_close = false;
  if (pol.min_p != 0.0) {                                      // :94-96
    const double cut = pol.min_p * (1.0 / s1);                 // the maximum is exp(0) / s1
    minp_close = r > 0.0 && fabs(r - cut) <= cut * 0x1p-49;
    if (r < cut) r = 0.0;
    s2 = bs.sum(r);
    r = r / s2;
  }
  if (pol.top_p < 1.0) {                                       // :97-102
    unsigned long long tgt = (unsigned long long)(pol.top_p * 0x1p60);
    if (tgt == 0) tgt = 1;
    const unsigned long long fx = (unsigned long long)(r * 0x1p60);
    if (r > 0.0) atomicAdd(&sh.mass[key >> 4], fx);
    lds_barrier();
    select_mass_bin(sh.mass, tgt, sh, bs);
    const int m1 = sh.sel[0];
    uint32_t lkey = 0;
    bool found = false;
    if (m1 >= 0) {
      const unsigned long long above1 = (unsigned long long)sh.sel_mass;
      if (r > 0.0 && (int)(key >> 4) == m1) atomicAdd(&sh.submass[key & 15u], fx);
      lds_barrier();
      unsigned long long excl = above1;
      for (int j = 15; j >= 0; --j) {
        const unsigned long long c = sh.submass[j];
        if (!found && excl < tgt && tgt <= excl + c) {
          lkey = ((uint32_t)m1 << 4) | (uint32_t)j;
          found = true;
        }
        excl += c;
      }
    }
    if (!found) {
      // The whole mass stays below top_p: nothing is removed.
      const double tot = bs.sum(r);
      if (fabs(tot - pol.top_p) <= ((double)k + 16.0) * 0x1p-51) flags |= DSR_FLAG_MARGIN;
    } else {
      if (zero_key(lkey)) return kHandZero;
      if (tid == 0) {
        // Tie members share one probability rt.  Key order must equal
        // probability order next to the boundary: its bf16 neighbours, taken
        // through the same arithmetic, must not collapse onto rt (else the
        // row is handed over); one within a few ulps is a rounding-band
        // decision.
        double rt = exp((bf16_key_value(lkey) - M) / T) / s1;
        if (s2 != 0.0) rt = rt / s2;
        int ok = 1, near = 0;
        for (int side = -1; side <= 1; side += 2) {
          const uint32_t nk = lkey + side;
          if (nk <= kKeyNegInf || nk >= kKeyPosInf || zero_key(nk)) continue;
          double rn = exp((bf16_key_value(nk) - M) / T) / s1;
          if (s2 != 0.0) rn = rn / s2;
          ok = ok && rn != rt;
          near = near || fabs(rn - rt) <= rt * 0x1p-50;
        }
        sh.bcast_d = rt;
        sh.bcast_i[0] = ok;
        sh.bcast_i[1] = near;
      }
      const bool pos = r > 0.0;
      const double A = bs.sum(pos && key > lkey ? r : 0.0);  // its barrier publishes thread 0's values
      const double rt = sh.bcast_d;
      if (!sh.bcast_i[0]) return kHandOrder;
      if (sh.bcast_i[1]) flags |= DSR_FLAG_MARGIN;
      uint32_t cnt_tot;
      const uint32_t cex = bs.scan((uint32_t)(pos && key > lkey) | ((uint32_t)(pos && key == lkey) << 16), cnt_tot);
      const long long trank = cex >> 16;
      const long long n_above = cnt_tot & 0xFFFFu, n_tie = cnt_tot >> 16;
      long long keep;
      {
        const double q = ceil((pol.top_p - A) / rt);
        keep = q <= 0.0 ? 0 : (q >= (double)n_tie ? n_tie : (long long)q);
        while (keep > 0 && A + (double)(keep - 1) * rt >= pol.top_p) --keep;
        while (keep < n_tie && A + (double)keep * rt < pol.top_p) ++keep;
      }
      if (n_above == 0 && keep == 0) keep = 1;
      const double tol = ((double)(n_above + keep) + 16.0) * 0x1p-51;
      bool close = fabs(A + (double)keep * rt - pol.top_p) <= tol;
      if (keep >= 1 && n_above + keep > 1) close = close || fabs(A + (double)(keep - 1) * rt - pol.top_p) <= tol;
      if (keep == 0 && n_above > 0) close = true;
      if (keep == n_tie && A + (double)n_tie * rt < pol.top_p) close = true;
      if (close) flags |= DSR_FLAG_MARGIN;
      if (key < lkey || (key == lkey && trank >= keep)) r = 0.0;
    }
  }

  // ---- categorical (sampling.py:103-128): the CDF in index order, its
  // total, the number of positive tokens and any min-p rounding-band flag.
  const bool pos = r > 0.0;
  double ctot;
  const double ex = bs.scan(r, ctot);
  const long long pos_info = bs.sum((long long)pos | ((long long)(minp_close ? 1 : 0) << 40));
  const long long npos = pos_info & 0xFFFFFFFFll;
  if (pos_info >> 40) flags |= DSR_FLAG_MARGIN;
  if (!(ctot > 0.0) || !isfinite(ctot)) {
    if (tid == 0) fast_write_result(a, row, DSR_E_NO_MASS, -1, 0, flags);
    return 0;
  }
  const double p = r / ctot;
  if (a.out_probs_f32 || a.out_probs_f64 || a.out_kept_bits) {
    fast_clear_outputs(a, row);
    if (fin) fast_scatter(a, row, idx, p);
  }
  if (!a.uniforms) {
    if (tid == 0) fast_write_result(a, row, DSR_OK, -1, 0, flags);
    return 0;
  }
  if (npos == 1) {  // no uniform is drawn (sampling.py:120-122)
    if (pos) fast_write_result(a, row, DSR_OK, idx, 0, flags);
    return 0;
  }
  const double u = a.uniforms[row];
  if (!(u >= 0.0 && u < 1.0)) {
    if (tid == 0) fast_write_result(a, row, DSR_E_UNIFORM, -1, 0, flags);
    return 0;
  }
  const double thr = u * ctot;
  const double inc = ex + r;
  // First thread whose inclusive prefix exceeds u * total (thread order is index order).
  const long long owner = bs.min(pos && inc > thr ? (long long)tid : LLONG_MAX);
  if (owner == LLONG_MAX) {
    // Rounding left u * total above every prefix: the last positive token.
    const long long last = bs.max(pos ? (long long)tid : -1ll);
    if (tid == last) fast_write_result(a, row, DSR_OK, idx, 1, flags | DSR_FLAG_MARGIN);
    return 0;
  }
  if (tid == owner) {
    const double tol = ((double)npos + 16.0) * 0x1p-51 * ctot;
    if (inc - thr <= tol || (ex > 0.0 && thr - ex <= tol)) flags |= DSR_FLAG_MARGIN;
    fast_write_result(a, row, DSR_OK, idx, 1, flags);
  }
  return 0;
}

}  // namespace dsr
