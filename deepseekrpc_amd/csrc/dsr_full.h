// Register-resident full-vocabulary path for bf16 rows with history
// penalties and no top-k (gfx950, wave64).
//
// Rows that keep the whole vocabulary (top_k 0 or >= V) cannot be cut to a
// short candidate list the way the top-k fast path cuts them, and rows with
// a token history carry float64 values that are not bf16.  This path keeps
// the row in VGPRs exactly as the fast path loads it (one HBM read, 16 x 16
// bytes per thread) and splits it in two:
//   * tokens the history touches (sampling.py:59-66) leave the registers:
//     their float64 adjusted values are computed once, from a gather of their
//     logits, into the row's workspace, beside their fixed-point mass and the
//     bf16 key of the largest bf16 value not above them;
//   * every other token is an exact bf16 value, so its mass depends on its
//     16-bit key alone: one LDS histogram of key counts (two 16-bit counts
//     per word, 128 KB) replaces per-token work for the totals and the top-p
//     boundary, and a mass table indexed by (binade, mantissa) replaces the
//     per-token exp in the CDF pass.
// Masses are 45-bit fixed point, floor-free round-to-nearest of
// exp((v - max) / T) (the table-driven float64 exp of dsr_common.h), so
// every sum is exact and order-independent; decisions inside their rounding
// band are reported with DSR_FLAG_MARGIN, and rows whose boundary order the
// keys cannot certify are handed to the general path (reason in flags).
//
// Steps: (1) loads and the history's penalised-token bitmap; pass 1 over the
// arriving chunks drops masked and penalised tokens from the key set and
// checks for NaN/+inf; (2) the row maximum over keys and penalised values;
// greedy rows end here; (3) the key-count histogram; (4) per 64-key block,
// the masses of the present keys (thread t owns block t); penalised masses
// are added to the block of their floor key; (5) the top-p boundary: the
// block, then the key (one wave), then inside the boundary key's bucket the
// penalised values above its bf16 value and its tie group, resolved by value
// and by index as the reference's stable sort does (sampling.py:97-102);
// (6) the categorical draw (:118-128): per-wave kept mass, then the wave
// holding u * total walks its chunks in index order.
#pragma once

#include "dsr_fast.h"

namespace dsr {

constexpr int kFxBits = 45;                       // fixed-point mass scale 2^45 (sums < 2^62)
constexpr int kLutBinades = 32;                   // per sign
constexpr int kLutSize = 2 * kLutBinades * 128;   // 8192 keys
constexpr int kPenItems = 64;                     // penalised values resolved exactly at the boundary
constexpr int kPenPre = 16;                       // history ids per thread fetched ahead of the row

struct PenItem {
  double v;
  long long fx;
  int32_t id;
  int16_t key;  // floor key
  int16_t pos;  // positive mass
};

static inline bool full_path_eligible(const dsr_sample_args_t& a) {
  return a.dtype == DSR_BF16 && a.vocab >= 8 && a.vocab <= kFastMaxVocab && (a.vocab & 7) == 0 && (a.ld & 7) == 0 &&
         ((uintptr_t)a.logits & 15u) == 0 && a.bias_off == nullptr;
}

struct FullShared {
  union {
    uint32_t cnt[32768];  // key counts, key k in bits 16*(k&1) of word k>>1
    struct {
      double lut[kLutSize];          // kept mass by (sign, binade, mantissa); 0 when not kept
      long long pm[kLutSize];        // penalised fixed-point masses of the walking wave's tokens
    } cdf;
  } big;
  union {
    struct {
      uint32_t pbits[kFastMaxVocab / 32];  // penalised tokens
      uint32_t lut[256][4];                // allow byte -> disallowed masks
    } p1;
    struct {
      long long bm[1024];  // mass per 64-key block
      uint32_t bp[1024];   // positive tokens per block
    } blk;
  } mid;
  PenItem items[kPenItems];
  long long kmass[64];
  uint32_t kpos[64];
  long long wtot[kWaves];
  double etab[64];
  SyncSlots sync;
  long long bc_l[4];
  int bc_i[8];
  int nitems;
};

__device__ __forceinline__ long long to_fx(double e) {
  // e in [0, 1]: e * 2^45 + 2^52 holds round(e * 2^45) in its low mantissa bits.
  const double y = e * 0x1p45 + 0x1p52;
  return (long long)(__double_as_longlong(y) & ((1ll << 52) - 1));
}

__device__ __forceinline__ uint32_t value_key(uint32_t bf) {
  return (bf & 0x8000u) ? (bf ^ 0xFFFFu) : (bf | 0x8000u);
}

// Key of the largest bf16 value not above v (v finite).
__device__ __forceinline__ uint32_t floor_key(double v) {
  const float f = (float)v;
  uint32_t b = __float_as_uint(f);
  if ((double)f > v) {  // step one float down: f is finite and above v
    if (f > 0.0f) b -= 1u;
    else if (f == 0.0f) b = 0x80000001u;
    else b += 1u;
  }
  uint32_t hb = b >> 16;
  if ((b & 0x80000000u) && (b & 0xFFFFu)) hb += 1u;  // truncation moved a negative value up
  return value_key(hb & 0xFFFFu);
}

// Mass-table slot of a key, or -1 outside the table's binades.
__device__ __forceinline__ int lut_slot(uint32_t key, int epos, int eneg) {
  if (key & 0x8000u) {
    const uint32_t bits = key ^ 0x8000u;
    const int s = epos - (int)(bits >> 7);
    return (s >= 0 && s < kLutBinades) ? s * 128 + (int)(bits & 127u) : -1;
  }
  const uint32_t bits = key ^ 0x7FFFu;  // magnitude bits of the negative value
  const int s = eneg - (int)(bits >> 7);
  return (s >= 0 && s < kLutBinades) ? kLutBinades * 128 + s * 128 + (int)(bits & 127u) : -1;
}

// Workgroup-uniform values into scalar registers (they stay out of the
// VGPRs the row occupies).
__device__ __forceinline__ uint32_t uni(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); }
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ long long uni(long long x) {
  const uint32_t lo = uni((uint32_t)x), hi = uni((uint32_t)((unsigned long long)x >> 32));
  return (long long)(((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double uni(double x) { return __longlong_as_double(uni((long long)__double_as_longlong(x))); }

// Whether history entry e of a row changes its token (count or generated count positive).
__device__ __forceinline__ bool pen_touches(long long c, long long g) { return c > 0 || g > 0; }

// Returns 0 if the row was decided here, else the reason it is handed to the general path.
__device__ __forceinline__ int full_sample_row(const dsr_sample_args_t& a, int64_t row, FullShared& sh) {
  const int tid = threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int64_t V = a.vocab;
  const uint32_t C = (uint32_t)(V >> 3);
  const uint32_t CW = (C + kWaves - 1) / kWaves;
  BlockSync bs(sh.sync);

  // ---- loads, smallest first so that waiting for them never waits for the
  // row: the exp table constants, the policy and history bounds (scalar),
  // the first kPenPre history ids per thread, then the row and its allow
  // bytes as raw buffer loads, as the fast path issues them.
  const dsr_policy_t pol = a.policy[row];
  const int64_t o0 = a.pen_off ? a.pen_off[row] : 0;
  const int64_t pn = a.pen_off ? a.pen_off[row + 1] - o0 : 0;
  const double etv = kExp2Frac[lane];
  int32_t pid[kPenPre];
#pragma unroll
  for (int i = 0; i < kPenPre; ++i) {
    const int64_t e = tid + (int64_t)i * kThreads;
    pid[i] = e < pn ? a.pen_ids[o0 + e] : -1;
  }
  const __amdgpu_buffer_rsrc_t mrs = __builtin_amdgcn_make_buffer_rsrc(
      a.allow_bits ? (void*)(a.allow_bits + row * a.allow_ld) : (void*)&kAllowAll, (short)0, (int)C, 0x00020000);
  const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint16_t*)a.logits + row * a.ld), (short)0, (int)(V * 2), 0x00020000);
  uint32_t mb[kFastChunks];
  uint4 d[kFastChunks];
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j) {
    const uint32_t cw = (uint32_t)j * 64u + (uint32_t)lane;
    const uint32_t c = (uint32_t)wave * CW + cw;
    const bool mine = cw < CW;
    mb[j] = __builtin_amdgcn_raw_buffer_load_b8(mrs, (int)(mine ? c : 0x7FFFFFF0u), 0, 0);
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rrs, (int)(mine ? c * 16u : 0x7FFFFFF0u), 0, 0);
    d[j] = make_uint4(v[0], v[1], v[2], v[3]);
  }
  __builtin_amdgcn_sched_barrier(0);
  if (!policy_ok(pol)) return kHandPolicy;
  if (pol.top_k != 0 && pol.top_k < V) return kHandTopK;  // a top-k cut with history: the general path
  const bool greedy = pol.temperature == 0.0;
  if (pn < 0 || 2 * pn > (int64_t)((V + 31) & ~31)) return kHandCapacity;  // workspace holds 2 words per entry
  double* Wv = (double*)a.workspace + row * ((V + 31) & ~(int64_t)31);    // adjusted values
  long long* Wp = (long long*)(Wv + pn);                                     // mass | floor key << 48

  // ---- LDS set-up while the row streams in: mask table, bitmap, key counts,
  // exp table; then the penalised-token bitmap from the prefetched ids (ids
  // out of range are left to the validity check after pass 1).
  {
    const uint32_t m = (uint32_t)tid >> 2, q = (uint32_t)tid & 3u;
    sh.mid.p1.lut[m][q] = (((m >> (2 * q)) & 1u) ? 0u : 0x0000FFFFu) | (((m >> (2 * q + 1)) & 1u) ? 0u : 0xFFFF0000u);
    uint4* zb = (uint4*)sh.mid.p1.pbits;
    zb[tid] = make_uint4(0u, 0u, 0u, 0u);
    uint4* zc = (uint4*)sh.big.cnt;
#pragma unroll
    for (int i = 0; i < 8; ++i) zc[tid + i * kThreads] = make_uint4(0u, 0u, 0u, 0u);
    if (tid < 64) sh.etab[tid] = etv;
  }
  lds_barrier();
#pragma unroll
  for (int i = 0; i < kPenPre; ++i)
    if (pid[i] >= 0 && pid[i] < V) atomicOr(&sh.mid.p1.pbits[pid[i] >> 5], 1u << (pid[i] & 31));
  for (int64_t e = tid + (int64_t)kPenPre * kThreads; e < pn; e += kThreads) {  // long histories
    const int32_t id = a.pen_ids[o0 + e];
    if (id >= 0 && id < V) atomicOr(&sh.mid.p1.pbits[id >> 5], 1u << (id & 31));
  }
  lds_barrier();

  // ---- pass 1, chunk by chunk as the loads land: keys, with masked and
  // penalised tokens set to key 0; raw NaN/+inf check; key max and min.
  uint32_t vmax_s = 0x80008000u, vmax_u = 0u, kmax = 0u, kmin = 0xFFFFFFFFu;
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j) {
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t c = (uint32_t)wave * CW + (uint32_t)j * 64u + (uint32_t)lane;
    const uint32_t cc = c < C ? c : C - 1u;  // chunks past the row are masked by their zero allow byte
    const uint32_t pb = (sh.mid.p1.pbits[cc >> 2] >> ((cc & 3u) * 8u)) & 0xFFu;
    const uint4 lm = *(const uint4*)sh.mid.p1.lut[(mb[j] & ~pb) & 0xFFu];
    uint32_t w[4] = {d[j].x, d[j].y, d[j].z, d[j].w};
    const uint32_t m4[4] = {lm.x, lm.y, lm.z, lm.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      vmax_s = pk_max_i16(vmax_s, w[q]);
      vmax_u = pk_max_u16(vmax_u, w[q]);
      const uint32_t k = bf16x2_keys(w[q] | m4[q]);  // excluded -> key 0
      kmax = pk_max_u16(kmax, k);
      kmin = pk_min_u16(kmin, k | m4[q]);            // excluded -> 0xFFFF, neutral for the minimum
      w[q] = k;
    }
    d[j] = make_uint4(w[0], w[1], w[2], w[3]);
  }
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j) asm volatile("" : "+v"(d[j].x), "+v"(d[j].y), "+v"(d[j].z), "+v"(d[j].w));
  asm volatile("" : "+v"(vmax_s), "+v"(vmax_u), "+v"(kmax), "+v"(kmin));
  __builtin_amdgcn_sched_barrier(0);

  // History validity (the general path reports any error in the reference's
  // order) and the penalised values (sampling.py:59-66, then the mask
  // :75-79) into the workspace.
  int bad = 0;
  long long csum = 0;
  double pmax = -INFINITY;
  long long pfirst = LLONG_MAX;
  const uint32_t* allow = a.allow_bits ? a.allow_bits + row * a.allow_ld : nullptr;
  for (int64_t e = tid; e < pn; e += kThreads) {
    const int32_t id = a.pen_ids[o0 + e];
    const long long c = a.pen_count[o0 + e], g = a.pen_gen[o0 + e];
    const bool ok = id >= 0 && id < V && (e == 0 || a.pen_ids[o0 + e - 1] < id) && c >= 0 && c <= DSR_MAX_COUNT &&
                    g >= 0 && g <= c;
    bad |= ok ? 0 : 1;
    csum += c;
    double v = -INFINITY;
    if (ok) {
      const uint32_t raw = ((const uint16_t*)a.logits)[row * a.ld + id];
      double x = (double)__uint_as_float(raw << 16);
      if (c > 0) x = x >= 0.0 ? x / pol.repetition_penalty : x * pol.repetition_penalty;
      const double pen = pol.presence_penalty * (g > 0 ? 1.0 : 0.0) + pol.frequency_penalty * (double)g;
      v = x - pen;
      if (!allowed_bit(allow, id)) v = -INFINITY;
      if (v != v) v = -INFINITY;  // NaN logits are caught by the raw check below
      if (v > pmax) {  // ids increase with e: the first holder of the maximum stays
        pmax = v;
        pfirst = id;
      }
    }
    Wv[e] = v;
  }

  // ---- row maximum over keys and penalised values; invalid rows hand over.
  const uint32_t kmx = max(kmax & 0xFFFFu, kmax >> 16), kmn = min(kmin & 0xFFFFu, kmin >> 16);
  const uint32_t badv = (max((int)(short)(vmax_s & 0xFFFFu), (int)(short)(vmax_s >> 16)) >= 0x7F80 ||
                         max(vmax_u & 0xFFFFu, vmax_u >> 16) >= 0xFF81u || bad) ? 1u : 0u;
  const uint32_t red = bs.max((kmx << 1) | badv);
  const uint32_t Mk = red >> 1;
  const long long csum_all = bs.sum(csum);
  if ((red & 1u) || csum_all > DSR_MAX_COUNT) return kHandInvalid;
  const uint32_t Kmin = bs.min(kmn);
  const double PM = bs.reduce(pmax, -(double)INFINITY, OpMax());
  const double Mv = Mk > kKeyNegInf ? bf16_key_value(Mk) : -(double)INFINITY;
  const double M = Mv > PM ? Mv : PM;
  if (!(M > -(double)INFINITY)) return kHandInvalid;  // every token masked or -inf: reported by the general path
  const double T = pol.temperature;
  const double* etab = sh.etab;
  const bool dense = a.out_probs_f32 || a.out_probs_f64 || a.out_kept_bits;

  // First index holding the maximum (sampling.py:82-85); +-0 maxima hand over.
  auto first_of_max = [&]() -> long long {
    long long f = LLONG_MAX;
    if (Mv == M) {
#pragma unroll
      for (int j = kFastChunks - 1; j >= 0; --j) {
        const uint32_t c = (uint32_t)wave * CW + (uint32_t)j * 64u + (uint32_t)lane;
#pragma unroll
        for (int e = 7; e >= 0; --e)
          if (key_at(d[j], e) == Mk) f = 8ll * c + e;
      }
    }
    if (PM == M && pfirst < f) f = pfirst;
    return bs.min(f);
  };
  if (greedy) {
    if (M == 0.0) return kHandZero;
    const long long tok = first_of_max();
    if (dense) {
      fast_clear_outputs(a, row);
      if (tid == 0) fast_scatter(a, row, tok, 1.0);
    }
    if (tid == 0) fast_write_result(a, row, DSR_OK, a.uniforms ? tok : -1, 0, 0);
    return 0;
  }
  unsigned flags = 0;

  // ---- key-count histogram of the register-resident tokens.
  uint32_t nlive = 0;
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t k = key_at(d[j], e);
      if (k > kKeyNegInf) {
        atomicAdd(&sh.big.cnt[k >> 1], 1u << ((k & 1u) << 4));
        ++nlive;
      }
    }
  }
  lds_barrier();

  // ---- masses of the present keys, per 64-key block (thread t owns block t),
  // with min-p (sampling.py:94-96: r < min_p * max(r), and max(r) is 1 / sum).
  const double min_p = pol.min_p;
  auto mass_of = [&](double v) {
    double e = exp_nonpos((v - M) / T, etab);  // (v - max) / T as the reference divides
    if (e < min_p) e = 0.0;
    return e;
  };
  int close = 0;
  {
    long long bmass = 0;
    uint32_t bpos = 0, bcount = 0;
    const uint4* cw4 = (const uint4*)&sh.big.cnt[32 * tid];
#pragma unroll 1
    for (int i = 0; i < 8; ++i) {
      const uint4 q = cw4[i];
      const uint32_t ws[4] = {q.x, q.y, q.z, q.w};
#pragma unroll 1
      for (int h = 0; h < 8; ++h) {
        const uint32_t wq = h < 4 ? (h < 2 ? ws[0] : ws[1]) : (h < 6 ? ws[2] : ws[3]);
        const uint32_t c = (wq >> (16 * (h & 1))) & 0xFFFFu;
        if (c) {
          const uint32_t k = 64u * (uint32_t)tid + 8u * (uint32_t)i + (uint32_t)h;
          const double e0 = exp_nonpos((bf16_key_value(k) - M) / T, etab);
          if (min_p != 0.0 && e0 > 0.0 && fabs(e0 - min_p) <= min_p * 0x1p-48) close = 1;
          const double e = e0 < min_p ? 0.0 : e0;
          bmass += (long long)c * to_fx(e);
          bpos += e > 0.0 ? c : 0u;
          bcount += c;
        }
      }
    }
    sh.mid.blk.bm[tid] = bmass;
    sh.mid.blk.bp[tid] = bpos;
    const uint32_t chk = bs.sum(bcount) ^ bs.sum(nlive);  // a 16-bit count that wrapped shows here
    if (chk) return kHandCapacity;
  }
  // Penalised tokens: mass, floor key, added to their block.
  for (int64_t e = tid; e < pn; e += kThreads) {
    const double v = Wv[e];
    long long packed = 0;
    if (v > -(double)INFINITY) {
      const double m0 = exp_nonpos((v - M) / T, etab);
      if (min_p != 0.0 && m0 > 0.0 && fabs(m0 - min_p) <= min_p * 0x1p-48) close = 1;
      const double m = m0 < min_p ? 0.0 : m0;
      const long long fx = to_fx(m);
      const uint32_t kb = floor_key(v);
      atomicAdd((unsigned long long*)&sh.mid.blk.bm[kb >> 6], (unsigned long long)fx);
      if (m > 0.0) atomicAdd(&sh.mid.blk.bp[kb >> 6], 1u);
      packed = fx | (m > 0.0 ? (1ll << 47) : 0ll) | ((long long)kb << 48);
    }
    Wp[e] = packed;
  }
  lds_barrier();
  if (bs.max((uint32_t)close)) flags |= DSR_FLAG_MARGIN;

  // ---- total mass and, with top-p, the boundary (sampling.py:97-102):
  // blocks in descending key order, thread t holding block 1023 - t.
  const long long bmt = sh.mid.blk.bm[1023 - tid];
  const uint32_t bpt = sh.mid.blk.bp[1023 - tid];
  if (tid == 0) sh.bc_i[0] = -1;  // ordered before the crossing's write by the scan's barrier
  long long S;
  uint32_t pex, ptot;
  const long long run = bs.scan2(bmt, bpt, S, pex, ptot);
  uint32_t L = 0;           // boundary key; 0: nothing removed by top-p
  long long keep = 0;       // boundary tie members kept, lowest index first
  long long cut_idx = -1;   // index of the last kept tie member when the group is split
  long long Sk = S;         // kept mass
  uint32_t npos_k = ptot;   // kept tokens with positive mass
  int nkept_items = 0;      // penalised values kept inside the boundary bucket (sorted first)
  if (pol.top_p < 1.0) {
    const double P = pol.top_p * (double)S;
    long long tgt = (long long)P;
    tgt = tgt < 1 ? 1 : (tgt > S ? S : tgt);
    if (run < tgt && tgt <= run + bmt) {
      sh.bc_i[0] = 1023 - tid;
      sh.bc_l[0] = run;
      sh.bc_i[1] = (int)pex;
    }
    if (tid < 64) {
      sh.kmass[tid] = 0;
      sh.kpos[tid] = 0;
    }
    if (tid == 0) sh.nitems = 0;
    lds_barrier();
    const int B = sh.bc_i[0];
    if (B < 0) return kHandCapacity;  // unreachable: the running mass reaches tgt <= S
    const long long AB = sh.bc_l[0];
    const uint32_t posAB = (uint32_t)sh.bc_i[1];
    for (int64_t e = tid; e < pn; e += kThreads) {
      const long long pk = Wp[e];
      const uint32_t kb = (uint32_t)((unsigned long long)pk >> 48);
      if (pk != 0 && (int)(kb >> 6) == B) {
        atomicAdd((unsigned long long*)&sh.kmass[kb & 63u], (unsigned long long)(pk & ((1ll << 47) - 1)));
        if ((pk >> 47) & 1) atomicAdd(&sh.kpos[kb & 63u], 1u);
      }
    }
    lds_barrier();
    if (wave == 0) {  // keys of block B, descending, one per lane
      const uint32_t k = 64u * (uint32_t)B + 63u - (uint32_t)lane;
      const uint32_t c = (sh.big.cnt[k >> 1] >> ((k & 1u) << 4)) & 0xFFFFu;
      const double e = (c && k > kKeyNegInf) ? mass_of(bf16_key_value(k)) : 0.0;
      const long long fk = to_fx(e);
      const long long mk = (long long)c * fk + sh.kmass[k & 63u];
      const uint32_t pk = (e > 0.0 ? c : 0u) + sh.kpos[k & 63u];
      const long long incl = wave_scan_dpp(mk);
      const uint32_t pincl = wave_scan_dpp(pk);
      const long long ex = AB + incl - mk;
      if (ex < tgt && tgt <= ex + mk) {
        sh.bc_i[2] = (int)k;
        sh.bc_l[1] = ex;                          // mass above bucket k
        sh.bc_i[3] = (int)(posAB + pincl - pk);   // positive tokens above bucket k
        sh.bc_i[4] = (int)c;                      // tie group size
        sh.bc_l[2] = fk;                          // tie member mass
        sh.bc_i[5] = e > 0.0 ? 1 : 0;
      }
    }
    lds_barrier();
    L = uni((uint32_t)sh.bc_i[2]);
    const long long AL = sh.bc_l[1];
    const uint32_t posAL = (uint32_t)sh.bc_i[3];
    const long long n_tie = sh.bc_i[4];
    const long long mt = sh.bc_l[2];
    const int tie_pos = sh.bc_i[5];
    // Penalised values in the boundary bucket and its two neighbours.
    for (int64_t e = tid; e < pn; e += kThreads) {
      const long long pk = Wp[e];
      const uint32_t kb = (uint32_t)((unsigned long long)pk >> 48);
      if (pk != 0 && kb + 1u >= L && kb <= L + 1u) {
        const int slot = atomicAdd(&sh.nitems, 1);
        if (slot < kPenItems) {
          PenItem it;
          it.v = Wv[e];
          it.fx = pk & ((1ll << 47) - 1);
          it.id = a.pen_ids[o0 + e];
          it.key = (int16_t)kb;
          it.pos = (int16_t)((pk >> 47) & 1);
          sh.items[slot] = it;
        }
      }
    }
    lds_barrier();
    const int nit = sh.nitems;
    if (nit > kPenItems) return kHandCapacity;
    // Sort the items (value descending, index ascending: the stable sort's
    // order), then walk the boundary bucket: penalised values above the bf16
    // value first, then the tie group.  One thread decides; every ordering
    // the keys cannot certify hands the row over.
    if (wave == 0) {
      PenItem mine;
      int rank = 0;
      if (lane < nit) {
        mine = sh.items[lane];
        for (int q = 0; q < nit; ++q) {
          const PenItem o = sh.items[q];
          rank += (o.v > mine.v || (o.v == mine.v && o.id < mine.id)) ? 1 : 0;
        }
      }
      __builtin_amdgcn_wave_barrier();
      if (lane < nit) sh.items[rank] = mine;  // every lane read before any writes (one wave, in order)
    }
    lds_barrier();
    if (tid == 0) {
      const double vL = bf16_key_value(L);
      int hand = (zero_key(L) && n_tie > 0) ? kHandZero : 0;
      // Distinct values around the boundary must keep (v - max) / T at least
      // 2^-40 apart, so the reference's float64 masses order them as the
      // values do; a penalised value equal to a bf16 group's value would join
      // that tie group, which this path does not resolve.
      double prev = INFINITY;
      int ii = 0;
      for (int dk = 1; dk >= -1 && !hand; --dk) {
        const uint32_t kk = L + (uint32_t)dk;
        if (kk == 0u || kk > 0xFFFFu) continue;
        const uint32_t ck = (sh.big.cnt[kk >> 1] >> ((kk & 1u) << 4)) & 0xFFFFu;
        const double vk = bf16_key_value(kk);
        while (ii < nit && (uint16_t)sh.items[ii].key > kk) ++ii;  // items sort by value, hence by bucket
        while (!hand && ii < nit && (uint16_t)sh.items[ii].key == kk) {
          const double v = sh.items[ii].v;
          if (ck > 0 && v == vk) hand = kHandOrder;
          if (v != prev && prev != INFINITY && !((prev - v) / T >= 0x1p-40)) hand = kHandOrder;
          prev = v;
          ++ii;
        }
        if (ck > 0 && kk > kKeyNegInf && kk < kKeyPosInf) {
          if (prev != INFINITY && !((prev - vk) / T >= 0x1p-40)) hand = kHandOrder;
          prev = vk;
        }
      }
      // The walk: items of bucket L, in order.
      long long cum = AL;
      bool removed = false;
      int nk = 0, nk_pos = 0, first_item = -1;
      long long ex_last = -1, ex_first_removed = -1;
      for (int q = 0; q < nit && !hand; ++q) {
        if ((uint16_t)sh.items[q].key != L) continue;
        if (first_item < 0) first_item = q;
        const long long ex = cum;
        if (!removed && ((double)ex < P || ex == 0)) {
          cum += sh.items[q].fx;
          ++nk;
          nk_pos += sh.items[q].pos;
          ex_last = ex;
        } else if (!removed) {
          removed = true;
          ex_first_removed = ex;
        }
      }
      long long kp = 0;
      if (!removed) {
        if (n_tie > 0 && mt > 0) {
          double q = ceil((P - (double)cum) / (double)mt);
          kp = q <= 0.0 ? 0 : (q >= (double)n_tie ? n_tie : (long long)q);
          while (kp > 0 && (double)(cum + (kp - 1) * mt) >= P) --kp;
          while (kp < n_tie && (double)(cum + kp * mt) < P) ++kp;
          if (cum == 0 && kp == 0) kp = 1;  // the first token is never removed
        } else if (n_tie > 0) {
          kp = n_tie;  // zero-mass members: kept or not, they carry nothing
        }
      }
      const long long nab = (long long)posAL + nk;  // tokens ranked above the tie group
      const double tol = ((double)(nab + kp) + 16.0) * 0x1p-50 * (double)S + (double)(nab + n_tie + 2);
      bool near = false;
      if (removed) {
        near = fabs((double)ex_first_removed - P) <= tol || (ex_last >= 0 && fabs((double)ex_last - P) <= tol);
      } else if (n_tie > 0) {
        near = fabs((double)(cum + kp * mt) - P) <= tol;
        if (kp >= 1 && nab + kp > 1) near = near || fabs((double)(cum + (kp - 1) * mt) - P) <= tol;
        if (kp == n_tie && (double)(cum + n_tie * mt) < P) near = true;
      } else {
        near = (ex_last >= 0 && fabs((double)ex_last - P) <= tol) || fabs((double)cum - P) <= tol;
      }
      if (kp == 0 && !removed && nab > 0 && n_tie > 0) near = true;
      (void)first_item;
      sh.bc_i[6] = hand;
      sh.bc_i[7] = nk | (near ? 0x10000 : 0);
      sh.bc_l[3] = kp;
      sh.bc_l[0] = cum + kp * mt;  // kept mass up to the boundary
      sh.bc_l[2] = (long long)posAL + nk_pos + (tie_pos ? kp : 0);
    }
    lds_barrier();
    if (sh.bc_i[6]) return sh.bc_i[6];
    nkept_items = uni(sh.bc_i[7] & 0xFFFF);
    if (sh.bc_i[7] & 0x10000) flags |= DSR_FLAG_MARGIN;
    keep = uni(sh.bc_l[3]);
    Sk = uni(sh.bc_l[0]);
    npos_k = uni((uint32_t)sh.bc_l[2]);
    // A split tie group: the index of its keep-th member, in index order
    // (wave, register slot, lane, element).
    if (keep > 0 && keep < n_tie) {
      uint32_t before = 0;  // ties in this wave before the current slot
      long long found = -1;
      uint32_t tw[kFastChunks];
      uint32_t wsum = 0;
#pragma unroll
      for (int j = 0; j < kFastChunks; ++j) {
        uint32_t t = 0;
#pragma unroll 1
        for (int e = 0; e < 8; ++e) t += key_at(d[j], e) == L ? 1u : 0u;
        tw[j] = t;
        wsum += lane_value(wave_scan_dpp(t), 63);
      }
      if (lane == 0) sh.wtot[wave] = wsum;
      lds_barrier();
      uint32_t base = 0;
      for (int w = 0; w < wave; ++w) base += (uint32_t)sh.wtot[w];
#pragma unroll
      for (int j = 0; j < kFastChunks; ++j) {
        const uint32_t incl = wave_scan_dpp(tw[j]);
        uint32_t r = base + before + incl - tw[j];
        const uint32_t c = (uint32_t)wave * CW + (uint32_t)j * 64u + (uint32_t)lane;
#pragma unroll 1
        for (int e = 0; e < 8; ++e) {
          if (key_at(d[j], e) == L) {
            if ((long long)r == keep - 1) found = 8ll * c + e;
            ++r;
          }
        }
        before += lane_value(incl, 63);
      }
      if (found >= 0) sh.bc_l[1] = found;
      lds_barrier();
      cut_idx = uni(sh.bc_l[1]);
    }
  }

  // ---- categorical (sampling.py:103-128) on the kept masses.
  if (Sk <= 0) {
    if (tid == 0) fast_write_result(a, row, DSR_E_NO_MASS, -1, 0, flags);
    return 0;
  }
  // Kept penalised values of the boundary bucket: the first nkept_items of
  // its items in sorted order.
  auto pen_kept = [&](uint32_t kb, int32_t id) {
    if (L == 0u || kb > L) return true;
    if (kb < L) return false;
    for (int q = 0, seen = 0; q < sh.nitems && q < kPenItems; ++q) {
      if ((uint16_t)sh.items[q].key != L) continue;
      if (seen++ >= nkept_items) return false;
      if (sh.items[q].id == id) return true;
    }
    return false;
  };
  auto unpen_kept = [&](uint32_t k, long long idx) {
    return k > kKeyNegInf && (L == 0u || k > L || (k == L && (keep >= 1) && (cut_idx < 0 || idx <= cut_idx)));
  };
  // Mass table over the kept keys' top 32 binades per sign.  Values too
  // small to move v - max (|v| < ulp(max) / 2) all have the mass of 0; a kept
  // key in neither hands the row over.
  const int epos = uni((Mk & 0x8000u) ? (int)((Mk ^ 0x8000u) >> 7) : -1);
  const uint32_t kneg = L ? L : Kmin;  // most negative kept value's key
  const int eneg = uni((kneg < 0x8000u && kneg > kKeyNegInf) ? (int)((kneg ^ 0x7FFFu) >> 7) : -1);
  const double tiny = uni(M != 0.0 ? ldexp(1.0, ilogb(M) - 53) : 0.0);
  const double e_zero = uni(mass_of(0.0));
  lds_barrier();  // every read of the key counts is done
  for (int i = tid; i < kLutSize; i += kThreads) {
    const int half = i / (kLutBinades * 128), s = (i / 128) % kLutBinades, mant = i & 127;
    const int ex = (half ? eneg : epos) - s;
    double m = 0.0;
    if (ex >= 0) {
      const uint32_t bits = ((uint32_t)ex << 7) | (uint32_t)mant;
      const uint32_t k = half ? (bits ^ 0x7FFFu) : (bits | 0x8000u);
      if (k > kKeyNegInf && k < kKeyPosInf && k <= Mk && (L == 0u || k >= L)) m = mass_of(bf16_key_value(k));
    }
    sh.big.cdf.lut[i] = m;
  }
  if (tid < kWaves) sh.wtot[tid] = 0;
  lds_barrier();
  // Mass of a register-resident token (0 when not kept); `miss` when its key
  // is outside the table.
  auto unpen_e = [&](uint32_t k, long long idx, int& miss) -> double {
    if (!unpen_kept(k, idx)) return 0.0;
    const int sl = lut_slot(k, epos, eneg);
    if (sl >= 0) return sh.big.cdf.lut[sl];
    if (fabs(bf16_key_value(k)) < tiny) return e_zero;
    miss = 1;
    return 0.0;
  };
  // Kept mass per wave (index order is wave-major).
  {
    long long acc = 0;
    int miss = 0;
#pragma unroll
    for (int j = 0; j < kFastChunks; ++j) {
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t c = (uint32_t)wave * CW + (uint32_t)j * 64u + (uint32_t)lane;
#pragma unroll 1
      for (int e = 0; e < 8; ++e) acc += to_fx(unpen_e(key_at(d[j], e), 8ll * c + e, miss));
    }
    acc = wave_reduce_dpp(acc, OpSum());
    if (lane == 0) atomicAdd((unsigned long long*)&sh.wtot[wave], (unsigned long long)acc);
    for (int64_t e = tid; e < pn; e += kThreads) {
      const long long pk = Wp[e];
      if (pk == 0) continue;
      const uint32_t kb = (uint32_t)((unsigned long long)pk >> 48);
      const int32_t id = a.pen_ids[o0 + e];
      if (pen_kept(kb, id)) {
        const int w = (int)((uint32_t)(id >> 3) / CW);
        atomicAdd((unsigned long long*)&sh.wtot[w], (unsigned long long)(pk & ((1ll << 47) - 1)));
      }
    }
    if (bs.max((uint32_t)miss)) return kHandCapacity;
  }
  lds_barrier();
  if (tid == 0) {
    long long base = 0;
    for (int w = 0; w < kWaves; ++w) base += sh.wtot[w];
    sh.bc_l[1] = base;
  }
  lds_barrier();
  if (sh.bc_l[1] != Sk) return kHandCapacity;  // the per-wave masses must add up to the kept total
  if (dense) {
    // Kept probabilities mass / kept total in float64 (from the masses, not
    // the fixed-point sums), zero elsewhere; kept bits mark every finite
    // token (no top-k on this path).
    fast_clear_outputs(a, row);
    const double Sd = (double)Sk * 0x1p-45;
#pragma unroll
    for (int j = 0; j < kFastChunks; ++j) {
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t c = (uint32_t)wave * CW + (uint32_t)j * 64u + (uint32_t)lane;
#pragma unroll 1
      for (int e = 0; e < 8; ++e) {
        const uint32_t k = key_at(d[j], e);
        if (k > kKeyNegInf) {
          int miss = 0;
          fast_scatter(a, row, 8ll * c + e, unpen_e(k, 8ll * c + e, miss) / Sd);
        }
      }
    }
    for (int64_t e = tid; e < pn; e += kThreads) {
      const double v = Wv[e];
      if (!(v > -(double)INFINITY)) continue;
      const long long pk = Wp[e];
      const int32_t id = a.pen_ids[o0 + e];
      const double p = pen_kept((uint32_t)((unsigned long long)pk >> 48), id) ? mass_of(v) / Sd : 0.0;
      fast_scatter(a, row, id, p);
    }
  }
  if (!a.uniforms) {
    if (tid == 0) fast_write_result(a, row, DSR_OK, -1, 0, flags);
    return 0;
  }
  if (npos_k == 1) {  // sampling.py:120-122: the single positive token is the maximum; no uniform
    if (M == 0.0) return kHandZero;
    const long long tok = first_of_max();
    if (tid == 0) fast_write_result(a, row, DSR_OK, tok, 0, flags);
    return 0;
  }
  const double u = a.uniforms[row];
  if (!(u >= 0.0 && u < 1.0)) {
    if (tid == 0) fast_write_result(a, row, DSR_E_UNIFORM, -1, 0, flags);
    return 0;
  }
  const double thr_d = u * (double)Sk;
  long long thr = (long long)thr_d;
  if (thr >= Sk) {
    thr = Sk - 1;
    flags |= DSR_FLAG_MARGIN;
  }
  // The wave holding thr, and the mass before it.
  if (tid == 0) {
    long long base = 0, obase = 0;
    int ow = -1;
    for (int w = 0; w < kWaves; ++w) {
      if (ow < 0 && thr < base + sh.wtot[w]) {
        ow = w;
        obase = base;
      }
      base += sh.wtot[w];
    }
    sh.bc_i[0] = ow;
    sh.bc_l[0] = obase;
  }
  lds_barrier();
  const int ow = sh.bc_i[0];
  if (ow < 0) return kHandCapacity;  // unreachable: thr < Sk
  const long long obase = sh.bc_l[0];
  // Penalised masses of that wave's tokens, by token offset.
  const int64_t wlo = (int64_t)ow * CW * 8;
  for (int i = tid; i < kLutSize; i += kThreads) sh.big.cdf.pm[i] = 0;
  lds_barrier();
  for (int64_t e = tid; e < pn; e += kThreads) {
    const long long pk = Wp[e];
    if (pk == 0) continue;
    const int32_t id = a.pen_ids[o0 + e];
    const int64_t off = (int64_t)id - wlo;
    if (off >= 0 && off < (int64_t)CW * 8 && pen_kept((uint32_t)((unsigned long long)pk >> 48), id))
      sh.big.cdf.pm[off] = pk & ((1ll << 47) - 1);
  }
  lds_barrier();
  // That wave walks its chunks in index order (slot, lane, element).
  if (wave == ow) {
    long long runw = obase;
    long long tok = -1;
#pragma unroll
    for (int j = 0; j < kFastChunks; ++j) {
      __builtin_amdgcn_sched_barrier(0);
      if (tok < 0) {  // uniform over the wave
        const uint32_t cw = (uint32_t)j * 64u + (uint32_t)lane;
        const uint32_t c = (uint32_t)wave * CW + cw;
        int miss = 0;
        long long cm = 0;
#pragma unroll 1
        for (int e = 0; e < 8; ++e) {
          cm += to_fx(unpen_e(key_at(d[j], e), 8ll * c + e, miss));
          if (cw < CW) cm += sh.big.cdf.pm[8 * cw + e];
        }
        const long long incl = wave_scan_dpp(cm);
        const long long ex = runw + incl - cm;
        const bool hit = cm > 0 && ex <= thr && thr < ex + cm;
        const unsigned long long hb = __ballot(hit);
        if (hb) {
          long long t = -1;
          if (hit) {
            long long x = ex, tex = 0, tfx = 0;
#pragma unroll 1
            for (int e = 0; e < 8; ++e) {
              long long f = to_fx(unpen_e(key_at(d[j], e), 8ll * c + e, miss));
              if (cw < CW) f += sh.big.cdf.pm[8 * cw + e];
              if (t < 0 && f > 0 && x <= thr && thr < x + f) {
                t = 8ll * c + e;
                tex = x;
                tfx = f;
              }
              x += f;
            }
            const double tol = ((double)npos_k + 16.0) * 0x1p-50 * (double)Sk + (double)npos_k + 2.0;
            unsigned fl = flags;
            if ((double)(tex + tfx) - thr_d <= tol || (tex > 0 && thr_d - (double)tex <= tol)) fl |= DSR_FLAG_MARGIN;
            fast_write_result(a, row, DSR_OK, t, 1, fl);
          }
          tok = __shfl(t, __ffsll((long long)hb) - 1);
        }
        runw += lane_value(incl, 63);
      }
    }
    if (lane == 0) sh.bc_i[1] = tok < 0 ? 1 : 0;
  }
  lds_barrier();
  return sh.bc_i[1] ? kHandCapacity : 0;  // unreachable: the crossing lies in the wave found above
}

}  // namespace dsr
