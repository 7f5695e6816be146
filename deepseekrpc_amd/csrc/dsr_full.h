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
// Steps: (1) loads, issued in rounds, and the history's penalised-token
// bitmap; pass 1 over the arriving chunks drops masked and penalised tokens
// from the key set, fills the key-count histogram and checks for NaN/+inf;
// (2) the row maximum over keys and penalised values; greedy rows end here;
// (3) per 64-key block, the masses of the present keys; penalised masses
// are added to the block of their floor key; (4) the top-p boundary: the
// block, then the key (one wave), then inside the boundary key's bucket the
// penalised values above its bf16 value and its tie group, resolved by value
// and by index as the reference's stable sort does (sampling.py:97-102);
// (5) the categorical draw (:118-128): per-wave kept mass, then the wave
// holding u * total walks its chunks in index order.
#pragma once

#include "dsr_fast.h"

namespace dsr {

constexpr int kFxBits = 45;                       // fixed-point mass scale 2^45 (sums < 2^62)
constexpr int kLutBinades = 32;                   // per sign
constexpr int kLutSize = 2 * kLutBinades * 128;   // 8192 keys
constexpr int kPenItems = 64;                     // penalised values resolved exactly at the boundary
constexpr int kPenPre = 8;                        // history ids per thread fetched ahead of the row

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

constexpr int kLutSlots = 64;  // binade slots of the mass table; slot 0 stays zero

struct FullShared {
  union {
    uint32_t cnt[32768];               // key counts, key k in bits 16*(k&1) of word k>>1
    long long lut[kLutSlots * 128];    // kept fixed-point mass by (binade slot, mantissa)
  } big;
  union {
    struct {
      uint32_t pbits[kFastMaxVocab / 32];  // tokens kept in registers: allowed, untouched by the history
      uint32_t lut[256][4];                // allow byte -> disallowed masks
    } p1;
    struct {
      long long bm[1024];  // mass per 64-key block
      uint32_t bp[1024];   // positive tokens per block
      uint32_t bc[1024];   // register-resident tokens per block
    } blk;
    struct {
      long long pe[512];    // kept penalised mass by element of the crossing slot's 64 chunks
      long long pen[64];    // kept penalised mass per chunk of that slot
    } cm;
  } mid;
  uint16_t boff[512];         // binade -> mass-table slot (0: none)
  uint16_t bslot[kLutSlots];  // slot -> binade
  PenItem items[kPenItems];
  long long kmass[64];
  uint32_t kpos[64];
  long long wtot[kWaves];
  uint32_t wtie[kWaves];      // tie members of a split boundary group per wave
  uint32_t tslot[kWaves][kFastChunks];  // ... and per (wave, register slot)
  int cut_w, cut_j, cut_r;    // wave, slot and rank within the slot of the last kept member
  int32_t elo[kWaves + 1];    // first history entry whose token lies at or after wave w's chunks; elo[16] = pn
  long long smass[kWaves][kFastChunks];  // kept register-resident mass per (wave, register slot)
  long long spen[kWaves][kFastChunks];   // kept penalised mass per (wave, register slot)
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

// Element e of a chunk for a runtime e.  It selects between two computed
// 64-bit halves, never between the chunk's words themselves: a select between
// the words of an array element is folded into a dynamically indexed load,
// which moves the whole register array to scratch memory.
__device__ __forceinline__ uint32_t key_at_rt(const uint4& v, int e) {
  const uint64_t lo = ((uint64_t)v.y << 32) | v.x, hi = ((uint64_t)v.w << 32) | v.z;
  return (uint32_t)((e < 4 ? lo : hi) >> (16 * (e & 3))) & 0xFFFFu;
}

// Bit e set when element e of the chunk holds key L.
__device__ __forceinline__ uint32_t key_bits(const uint4& v, uint32_t L) {
  const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
  uint32_t m = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    m |= ((w4[q] & 0xFFFFu) == L ? 1u : 0u) << (2 * q) | ((w4[q] >> 16) == L ? 1u : 0u) << (2 * q + 1);
  return m;
}

constexpr int kPenBatch = 4;  // history entries per thread whose loads are in flight together

// Visits this thread's history entries e = first + kThreads * i in batches of
// kPenBatch: fetch(e) for the whole batch first (fetch(-1) for entries past
// the end must not load), so the batch's global loads are in flight together
// and the loop waits once per batch instead of once per entry; then
// body(e, fetched) in entry order.
template <int NB = kPenBatch, class F, class B>
__device__ __forceinline__ void pen_batches(int64_t pn, int64_t first, F fetch, B body) {
  for (int64_t base = first; base < pn; base += (int64_t)NB * kThreads) {
    decltype(fetch((int64_t)0)) x[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int64_t e = base + (int64_t)i * kThreads;
      x[i] = fetch(e < pn ? e : (int64_t)-1);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int64_t e = base + (int64_t)i * kThreads;
      if (e < pn) body(e, x[i]);
    }
  }
}

struct PenPk {  // a history entry's packed mass word and token id
  long long pk;
  int32_t id;
};

struct PenVal {  // a history entry's adjusted value and token id
  double v;
  int32_t id;
};

// Whether history entry e of a row changes its token (count or generated count positive).
__device__ __forceinline__ bool pen_touches(long long c, long long g) { return c > 0 || g > 0; }

// Returns 0 if the row was decided here, else the reason it is handed to the general path.
template <bool RNG>
__device__ __forceinline__ int full_sample_row(const dsr_sample_args_t& a, int64_t row, FullShared& sh) {
  const int tid = threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int64_t V = a.vocab;
  const uint32_t C = (uint32_t)(V >> 3);
  const uint32_t CW = (C + kWaves - 1) / kWaves;
  BlockSync bs(sh.sync);

  // ---- loads, smallest first so that waiting for them never waits for the
  // row: the allow words (4 per thread), the policy and history bounds
  // (scalar), the first kPenPre history ids per thread, then the row as raw
  // buffer loads, as the fast path issues them.
  const dsr_policy_t pol = a.policy[row];
  const int64_t o0 = a.pen_off ? a.pen_off[row] : 0;
  const int64_t pn = a.pen_off ? a.pen_off[row + 1] - o0 : 0;
  const uint32_t nwords = (uint32_t)((V + 31) >> 5);
  uint32_t aw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = (uint32_t)tid + (uint32_t)i * kThreads;
    aw[i] = (a.allow_bits && w < nwords) ? a.allow_bits[row * a.allow_ld + w] : 0xFFFFFFFFu;
  }
  const double etv = kExp2Frac[lane];
  // The row's uniform or PCG64 state, read with the small loads: the draw at
  // the end then waits for no memory round trip.
  uint64_t st_pre[4] = {0ull, 0ull, 0ull, 0ull};
  double u_pre = 0.0;
  if (RNG) {
#pragma unroll
    for (int i = 0; i < 4; ++i) st_pre[i] = a.rng_state[4 * row + i];
  } else if (a.uniforms) {
    u_pre = a.uniforms[row];
  }
  int32_t pid[kPenPre];
#pragma unroll
  for (int i = 0; i < kPenPre; ++i) {
    const int64_t e = tid + (int64_t)i * kThreads;
    pid[i] = e < pn ? a.pen_ids[o0 + e] : -1;
  }
  const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint16_t*)a.logits + row * a.ld), (short)0, (int)(V * 2), 0x00020000);
  // Every wave's small loads enter the CU's memory pipeline before any
  // wave's row loads: the LDS set-up below waits only for them, and the
  // first pass then takes each slot as it lands instead of starting after
  // the whole row (a wave's small loads would otherwise queue behind the
  // row loads of the waves issued before it).  No wait: a bare barrier at
  // workgroup-uniform control flow.
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  // The row's slots are issued in rounds (the first kAhead now, then one
  // per round with a barrier per round), as the top-k kernel issues them: a
  // wave whose next instruction is a load waits until the CU's memory
  // pipeline (about 40 KB in flight) takes it, so sixteen slots issued up
  // front would hold every wave in its loads until the row had nearly
  // landed, and the first pass could not start before then.
  uint4 d[kFastChunks];
  auto issue = [&](int j) {
    const uint32_t cw = (uint32_t)j * 64u + (uint32_t)lane;
    const uint32_t c = (uint32_t)wave * CW + cw;
    const bool mine = cw < CW;
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rrs, (int)(mine ? c * 16u : 0x7FFFFFF0u), 0, 0);
    d[j] = make_uint4(v[0], v[1], v[2], v[3]);
  };
  constexpr int kAhead = 4;
#pragma unroll
  for (int j = 0; j < kAhead; ++j) issue(j);
  __builtin_amdgcn_sched_barrier(0);
  if (!policy_ok(pol)) return kHandPolicy;
  if (pol.top_k != 0 && pol.top_k < V) return kHandTopK;  // a top-k cut with history: the general path
  const bool greedy = pol.temperature == 0.0;
  if (pn < 0 || 2 * pn > (int64_t)((V + 31) & ~31)) return kHandCapacity;  // workspace holds 2 words per entry
  double* Wv = (double*)a.workspace + row * ((V + 31) & ~(int64_t)31);    // adjusted values
  long long* Wp = (long long*)(Wv + pn);                                     // mass | floor key << 48

  // ---- LDS set-up while the row streams in: the mask table, the key
  // counts, the exp table and one bitmap of the tokens that stay in
  // registers (allowed and untouched by the history).  Ids out of range are
  // left to the validity check after pass 1.
  {
    const uint32_t m = (uint32_t)tid >> 2, q = (uint32_t)tid & 3u;
    sh.mid.p1.lut[m][q] = (((m >> (2 * q)) & 1u) ? 0u : 0x0000FFFFu) | (((m >> (2 * q + 1)) & 1u) ? 0u : 0xFFFF0000u);
#pragma unroll
    for (int i = 0; i < 4; ++i) sh.mid.p1.pbits[tid + i * kThreads] = aw[i];
    uint4* zc = (uint4*)sh.big.cnt;
#pragma unroll
    for (int i = 0; i < 8; ++i) zc[tid + i * kThreads] = make_uint4(0u, 0u, 0u, 0u);
    if (tid < 64) sh.etab[tid] = etv;
    if (tid <= kWaves) sh.elo[tid] = (int32_t)pn;
    if (tid < kWaves * kFastChunks) sh.spen[tid / kFastChunks][tid % kFastChunks] = 0;
  }
  lds_barrier();
#pragma unroll
  for (int i = 0; i < kPenPre; ++i)
    if (pid[i] >= 0 && pid[i] < V) atomicAnd(&sh.mid.p1.pbits[pid[i] >> 5], ~(1u << (pid[i] & 31)));
  pen_batches(  // long histories
      pn, tid + (int64_t)kPenPre * kThreads, [&](int64_t e) { return e >= 0 ? a.pen_ids[o0 + e] : -1; },
      [&](int64_t, int32_t id) {
        if (id >= 0 && id < V) atomicAnd(&sh.mid.p1.pbits[id >> 5], ~(1u << (id & 31)));
      });
  lds_barrier();

  // ---- pass 1, chunk by chunk as the loads land: keys, with masked and
  // penalised tokens set to keys below every value's (2 + lane: no LDS
  // atomic contention on them later); raw NaN/+inf check; key max and min.
  uint32_t vmax_s = 0x80008000u, vmax_u = 0u, kmax = 0u;
  const uint32_t dummy2 = (2u + (uint32_t)lane) * 0x00010001u;  // keys 2..65 hold no value
  auto pass1 = [&](int j) {
    const uint32_t cw = (uint32_t)j * 64u + (uint32_t)lane;
    const uint32_t c = (uint32_t)wave * CW + cw;
    // Slots past this wave's chunks or past the row were not loaded (they
    // read as +0.0) and stay masked; the read itself is not branched around.
    const bool live = cw < CW && c < C;
    const uint32_t cc = live ? c : 0u;
    const uint32_t stay = (sh.mid.p1.pbits[cc >> 2] >> ((cc & 3u) * 8u)) & (live ? 0xFFu : 0u);
    const uint4 lm = *(const uint4*)sh.mid.p1.lut[stay];
    uint32_t w[4] = {d[j].x, d[j].y, d[j].z, d[j].w};
    const uint32_t m4[4] = {lm.x, lm.y, lm.z, lm.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      vmax_s = pk_max_i16(vmax_s, w[q]);
      vmax_u = pk_max_u16(vmax_u, w[q]);
      const uint32_t k = bf16x2_keys(w[q] | m4[q]);  // excluded -> key 0
      kmax = pk_max_u16(kmax, k);
      w[q] = k | (m4[q] & dummy2);                   // excluded -> a per-lane key below the real ones
      // The key-count histogram of the register-resident tokens, filled while
      // the later slots stream in (excluded and dummy keys land below 128 and
      // are ignored from here on; greedy rows never read it).
      const uint32_t k0 = w[q] & 0xFFFFu, k1 = w[q] >> 16;
      atomicAdd(&sh.big.cnt[k0 >> 1], 1u << ((k0 & 1u) << 4));
      atomicAdd(&sh.big.cnt[k1 >> 1], 1u << ((k1 & 1u) << 4));
    }
    d[j] = make_uint4(w[0], w[1], w[2], w[3]);
  };
  // Round r issues slot r (r < 16) and runs the pass of slot r - kAhead.
  // The barriers keep the waves' issues in step (workgroup-uniform control
  // flow).  They carry no fence: the histogram's atomics are read only after
  // the fenced barrier of the row maximum.
#pragma unroll
  for (int r = kAhead; r < kFastChunks + kAhead; ++r) {
    if (r < kFastChunks) issue(r);
    __builtin_amdgcn_sched_barrier(0);
    pass1(r - kAhead);
    __builtin_amdgcn_sched_barrier(0);
    if (r + 1 < kFastChunks) __builtin_amdgcn_s_barrier();
  }
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j) asm volatile("" : "+v"(d[j].x), "+v"(d[j].y), "+v"(d[j].z), "+v"(d[j].w));
  asm volatile("" : "+v"(vmax_s), "+v"(vmax_u), "+v"(kmax));
  __builtin_amdgcn_sched_barrier(0);

  // History validity (the general path reports any error in the reference's
  // order) and the penalised values (sampling.py:59-66, then the mask
  // :75-79) into the workspace.
  int bad = 0;
  long long csum = 0;
  double pmax = -INFINITY;
  long long pfirst = LLONG_MAX;
  const uint32_t* allow = a.allow_bits ? a.allow_bits + row * a.allow_ld : nullptr;
  // kPenBatch entries per thread at a time: their ids, counts and the previous
  // ids are fetched together, then their logits are gathered together.
  for (int64_t base = tid; base < pn; base += (int64_t)kPenBatch * kThreads) {
    int32_t id[kPenBatch], prv[kPenBatch], c[kPenBatch], g[kPenBatch];
#pragma unroll
    for (int i = 0; i < kPenBatch; ++i) {
      const int64_t e = base + (int64_t)i * kThreads;
      const bool in = e < pn;
      id[i] = in ? a.pen_ids[o0 + e] : 0;
      prv[i] = (in && e > 0) ? a.pen_ids[o0 + e - 1] : INT_MIN;
      c[i] = in ? a.pen_count[o0 + e] : 0;
      g[i] = in ? a.pen_gen[o0 + e] : 0;
    }
    uint32_t raw[kPenBatch];
    bool ok[kPenBatch];
#pragma unroll
    for (int i = 0; i < kPenBatch; ++i) {
      const int64_t e = base + (int64_t)i * kThreads;
      ok[i] = e < pn && id[i] >= 0 && id[i] < V && prv[i] < id[i] && c[i] >= 0 && c[i] <= DSR_MAX_COUNT &&
              g[i] >= 0 && g[i] <= c[i];
      // Unbranched raw buffer loads (out of range reads 0), so that the
      // batch's gathers are in flight together.
      raw[i] = __builtin_amdgcn_raw_buffer_load_b16(rrs, ok[i] ? 2 * id[i] : 0x7FFFFFF0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kPenBatch; ++i) {
      const int64_t e = base + (int64_t)i * kThreads;
      if (e >= pn) continue;
      bad |= ok[i] ? 0 : 1;
      csum += c[i];
      {  // ids increase with e: this entry starts the run of every wave after its predecessor's, up to its own
        const int wv = id[i] < 0 ? -1 : (int)min((uint32_t)id[i] / 8u / CW, (uint32_t)kWaves - 1u);
        const int wp = prv[i] < 0 ? -1 : (int)min((uint32_t)prv[i] / 8u / CW, (uint32_t)kWaves - 1u);
        for (int w = wp + 1; w <= wv; ++w) sh.elo[w] = (int32_t)e;
      }
      double v = -INFINITY;
      if (ok[i]) {
        double x = (double)__uint_as_float(raw[i] << 16);
        if (c[i] > 0) x = x >= 0.0 ? x / pol.repetition_penalty : x * pol.repetition_penalty;
        const double pen = pol.presence_penalty * (g[i] > 0 ? 1.0 : 0.0) + pol.frequency_penalty * (double)g[i];
        v = x - pen;
        if (!allowed_bit(allow, id[i])) v = -INFINITY;
        if (v != v) v = -INFINITY;  // NaN logits are caught by the raw check below
        if (v > pmax) {  // ids increase with e: the first holder of the maximum stays
          pmax = v;
          pfirst = id[i];
        }
      }
      Wv[e] = v;
    }
  }

  // ---- row maximum over keys and penalised values; invalid rows hand over.
  const uint32_t kmx = max(kmax & 0xFFFFu, kmax >> 16);
  const uint32_t badv = (max((int)(short)(vmax_s & 0xFFFFu), (int)(short)(vmax_s >> 16)) >= 0x7F80 ||
                         max(vmax_u & 0xFFFFu, vmax_u >> 16) >= 0xFF81u || bad) ? 1u : 0u;
  // One barrier for the key maximum (with the invalid flag), one more for
  // the history's count total and value maximum when the row has a history
  // (pn is uniform).
  const uint32_t red = bs.max((kmx << 1) | badv);
  const uint32_t Mk = red >> 1;
  long long csum_all = 0;
  double PM = -(double)INFINITY;
  if (pn > 0) {
    csum_all = csum;
    PM = pmax;
    bs.sum_max(csum_all, PM);
  }
  if ((red & 1u) || csum_all > DSR_MAX_COUNT) return kHandInvalid;
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
    if (tid == 0) fast_write_result(a, row, DSR_OK, has_draws<RNG>(a) ? tok : -1, 0, 0);
    return 0;
  }
  unsigned flags = 0;

  // The key-count histogram was filled by the first pass.
  lds_barrier();

  // ---- masses of the present keys (sampling.py:86-96: exp((v - max) / T),
  // min-p keeping r >= min_p since max(r) = 1 / sum).  Thread t takes the
  // 8-key groups t + 1024 i, so dense key ranges spread over many threads;
  // the 8 groups of a 64-key block sit in 8 neighbouring lanes and are
  // summed by DPP.
  const double min_p = pol.min_p;
  auto mass_of = [&](double v) {
    double e = exp_nonpos((v - M) / T, etab);  // (v - max) / T divided as the reference divides
    if (e < min_p) e = 0.0;
    return e;
  };
  int close = 0;
  {
    uint32_t counted = 0;  // every register slot, dummy keys included
#pragma unroll 1
    for (int i = 0; i < 8; ++i) {
      const uint32_t g = (uint32_t)tid + 1024u * (uint32_t)i;
      const uint4 q4 = *(const uint4*)&sh.big.cnt[4u * g];
      counted += ((q4.x & 0xFFFFu) + (q4.x >> 16)) + ((q4.y & 0xFFFFu) + (q4.y >> 16)) +
                 ((q4.z & 0xFFFFu) + (q4.z >> 16)) + ((q4.w & 0xFFFFu) + (q4.w >> 16));
      long long gm = 0;
      uint32_t gp = 0, gc = 0;
      const bool any = (q4.x | q4.y | q4.z | q4.w) != 0u && g >= 16u;  // keys below 128 hold no value
      if (!__ballot(any)) {  // no key of the wave's 512 (most of them: the keys cluster)
        if ((tid & 7) == 0) {
          sh.mid.blk.bm[g >> 3] = 0;
          sh.mid.blk.bp[g >> 3] = 0u;
          sh.mid.blk.bc[g >> 3] = 0u;
        }
        continue;
      }
      if (any) {
#pragma unroll 1
        for (int h = 0; h < 8; ++h) {
          const uint32_t wq = h < 4 ? (h < 2 ? q4.x : q4.y) : (h < 6 ? q4.z : q4.w);
          const uint32_t c = (wq >> (16 * (h & 1))) & 0xFFFFu;
          if (c) {
            const double e0 = exp_nonpos((bf16_key_value(8u * g + (uint32_t)h) - M) / T, etab);
            if (min_p != 0.0 && e0 > 0.0 && fabs(e0 - min_p) <= min_p * 0x1p-48) close = 1;
            const double e = e0 < min_p ? 0.0 : e0;
            gm += (long long)c * to_fx(e);
            gp += e > 0.0 ? c : 0u;
            gc += c;
          }
        }
      }
      // Sum the 8 groups of block g >> 3 (lanes with equal tid >> 3).
      gm = gm + dpp_move<long long, 0xB1>(gm);
      gm = gm + dpp_move<long long, 0x4E>(gm);
      gm = gm + dpp_move<long long, 0x141>(gm);
      gp = gp + dpp_move<uint32_t, 0xB1>(gp);
      gp = gp + dpp_move<uint32_t, 0x4E>(gp);
      gp = gp + dpp_move<uint32_t, 0x141>(gp);
      gc = gc + dpp_move<uint32_t, 0xB1>(gc);
      gc = gc + dpp_move<uint32_t, 0x4E>(gc);
      gc = gc + dpp_move<uint32_t, 0x141>(gc);
      if ((tid & 7) == 0) {
        sh.mid.blk.bm[g >> 3] = gm;
        sh.mid.blk.bp[g >> 3] = gp;
        sh.mid.blk.bc[g >> 3] = gc;
      }
    }
    // The histogram holds one count per register slot (16 x 8 per thread), so a
    // 16-bit count that wrapped (more than 65,535 equal keys) shows in the total.
    if (bs.sum(counted) != (uint32_t)(kThreads * kFastChunks * 8)) return kHandCapacity;
  }
  // Kept penalised mass by the wave and register slot whose chunks hold the
  // token (the index-order CDF below works by wave, then slot).
  auto add_kept = [&](int32_t id, long long fx) {
    const uint32_t cid = (uint32_t)(id >> 3);
    const int w = (int)(cid / CW), js = (int)((cid - (uint32_t)w * CW) >> 6);
    atomicAdd((unsigned long long*)&sh.spen[w][js], (unsigned long long)fx);
  };
  const bool all_kept = !(pol.top_p < 1.0);  // no top-p: every positive mass stays
  // Penalised tokens: mass, floor key, added to the block of their floor key.
  pen_batches(pn, tid,
              [&](int64_t e) { return e >= 0 ? PenVal{Wv[e], a.pen_ids[o0 + e]} : PenVal{-(double)INFINITY, 0}; },
              [&](int64_t e, PenVal x) {
                const double v = x.v;
                long long packed = 0;
                if (v > -(double)INFINITY) {
                  const double m0 = exp_nonpos((v - M) / T, etab);
                  if (min_p != 0.0 && m0 > 0.0 && fabs(m0 - min_p) <= min_p * 0x1p-48) close = 1;
                  const double m = m0 < min_p ? 0.0 : m0;
                  const long long fx = to_fx(m);
                  const uint32_t kb = floor_key(v);
                  atomicAdd((unsigned long long*)&sh.mid.blk.bm[kb >> 6], (unsigned long long)fx);
                  if (m > 0.0) atomicAdd(&sh.mid.blk.bp[kb >> 6], 1u);
                  if (all_kept && fx > 0) add_kept(x.id, fx);
                  packed = fx | (m > 0.0 ? (1ll << 47) : 0ll) | ((long long)kb << 48);
                }
                Wp[e] = packed;
              });
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
  S = uni(S);
  uint32_t L = 0;          // boundary key; 0: nothing removed by top-p
  long long keep = 0;      // boundary tie members kept, lowest index first
  long long n_tie = 0;
  long long mtie = 0;      // fixed-point mass of one tie member
  long long cut_idx = -1;  // index of the last kept tie member when the group is split
  long long Sk = S;        // kept mass
  uint32_t npos_k = uni(ptot);
  int nkept_items = 0;     // penalised values kept inside the boundary bucket (first in sorted order)
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
    const int B = uni(sh.bc_i[0]);
    if (B < 0) return kHandCapacity;  // unreachable: the running mass reaches tgt <= S
    const long long AB = sh.bc_l[0];
    const uint32_t posAB = (uint32_t)sh.bc_i[1];
    pen_batches(pn, tid, [&](int64_t e) { return e >= 0 ? Wp[e] : 0ll; },
                [&](int64_t, long long pk) {
                  const uint32_t kb = (uint32_t)((unsigned long long)pk >> 48);
                  if (pk != 0 && (int)(kb >> 6) == B) {
                    atomicAdd((unsigned long long*)&sh.kmass[kb & 63u], (unsigned long long)(pk & ((1ll << 47) - 1)));
                    if ((pk >> 47) & 1) atomicAdd(&sh.kpos[kb & 63u], 1u);
                  }
                });
    lds_barrier();
    if (wave == 0) {  // keys of block B, descending, one per lane
      const uint32_t k = 64u * (uint32_t)B + 63u - (uint32_t)lane;
      const uint32_t c = k >= 128u ? (sh.big.cnt[k >> 1] >> ((k & 1u) << 4)) & 0xFFFFu : 0u;
      const double e = c ? mass_of(bf16_key_value(k)) : 0.0;
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
    n_tie = uni((long long)sh.bc_i[4]);
    mtie = uni(sh.bc_l[2]);
    const int tie_pos = sh.bc_i[5];
    // Penalised values in the boundary bucket and its two neighbours.
    // Entries above the boundary bucket are kept: their masses go to their
    // wave and slot here; the bucket's own entries once the walk below has
    // decided them.
    pen_batches(pn, tid, [&](int64_t e) { return e >= 0 ? PenPk{Wp[e], a.pen_ids[o0 + e]} : PenPk{0ll, 0}; },
                [&](int64_t e, PenPk x) {
      const long long pk = x.pk;
      const uint32_t kb = (uint32_t)((unsigned long long)pk >> 48);
      const long long fx = pk & ((1ll << 47) - 1);
      if (pk != 0 && kb > L && fx > 0) add_kept(x.id, fx);
      if (pk != 0 && kb + 1u >= L && kb <= L + 1u) {
        const int slot = atomicAdd(&sh.nitems, 1);
        if (slot < kPenItems) {
          PenItem it;
          it.v = Wv[e];
          it.fx = fx;
          it.id = x.id;
          it.key = (int16_t)kb;
          it.pos = (int16_t)((pk >> 47) & 1);
          sh.items[slot] = it;
        }
      }
    });
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
      if (lane < nit) sh.items[rank] = mine;  // every lane has read its item before any write (one wave)
    }
    lds_barrier();
    if (tid == 0) {
      int hand = (zero_key(L) && n_tie > 0) ? kHandZero : 0;
      // Distinct values around the boundary must keep (v - max) / T at least
      // 2^-40 apart, so the reference's float64 masses order them as the
      // values do; a penalised value equal to a bf16 group's value would join
      // that tie group, which this path does not resolve.
      double prev = INFINITY;
      int ii = 0;
      for (int dk = 1; dk >= -1 && !hand; --dk) {
        const uint32_t kk = L + (uint32_t)dk;
        if (kk < 128u || kk > 0xFFFFu) continue;
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
      // The walk: items of bucket L, in order, then its tie group.
      long long cum = AL;
      bool removed = false;
      int nk = 0, nk_pos = 0;
      long long ex_last = -1, ex_first_removed = -1;
      for (int q = 0; q < nit && !hand; ++q) {
        if ((uint16_t)sh.items[q].key != L) continue;
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
      if (!removed && n_tie > 0) {
        if (mtie > 0) {
          const double q = ceil((P - (double)cum) / (double)mtie);
          kp = q <= 0.0 ? 0 : (q >= (double)n_tie ? n_tie : (long long)q);
          while (kp > 0 && (double)(cum + (kp - 1) * mtie) >= P) --kp;
          while (kp < n_tie && (double)(cum + kp * mtie) < P) ++kp;
          if (cum == 0 && kp == 0) kp = 1;  // the first token is never removed
        } else {
          kp = n_tie;  // zero-mass members carry nothing either way
        }
      }
      const long long nab = (long long)posAL + nk;  // tokens ranked above the tie group
      const double tol = ((double)(nab + kp) + 16.0) * 0x1p-50 * (double)S + (double)(nab + n_tie + 2);
      bool near = false;
      if (removed) {
        near = fabs((double)ex_first_removed - P) <= tol || (ex_last >= 0 && fabs((double)ex_last - P) <= tol);
      } else if (n_tie > 0) {
        near = fabs((double)(cum + kp * mtie) - P) <= tol;
        if (kp >= 1 && nab + kp > 1) near = near || fabs((double)(cum + (kp - 1) * mtie) - P) <= tol;
        if (kp == n_tie && (double)(cum + n_tie * mtie) < P) near = true;
        if (kp == 0 && nab > 0) near = true;
      } else {
        near = (ex_last >= 0 && fabs((double)ex_last - P) <= tol) || fabs((double)cum - P) <= tol;
      }
      sh.bc_i[6] = hand;
      sh.bc_i[7] = nk | (near ? 0x10000 : 0);
      sh.bc_l[3] = kp;
      sh.bc_l[0] = cum + kp * mtie;  // kept mass
      sh.bc_l[2] = (long long)posAL + nk_pos + (tie_pos ? kp : 0);
    }
    lds_barrier();
    if (sh.bc_i[6]) return sh.bc_i[6];
    nkept_items = uni(sh.bc_i[7] & 0xFFFF);
    if (sh.bc_i[7] & 0x10000) flags |= DSR_FLAG_MARGIN;
    if (wave == 0) {  // the kept entries of the boundary bucket: the first nkept_items in sorted order
      const bool inb = lane < nit && (uint16_t)sh.items[lane].key == L;
      const unsigned long long mb = __ballot(inb);
      const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(mb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mb, 0u));
      if (inb && (int)rank < nkept_items && sh.items[lane].fx > 0) add_kept(sh.items[lane].id, sh.items[lane].fx);
    }
    keep = uni(sh.bc_l[3]);
    Sk = uni(sh.bc_l[0]);
    npos_k = uni((uint32_t)sh.bc_l[2]);
  }
  if (Sk <= 0) {
    if (tid == 0) fast_write_result(a, row, DSR_E_NO_MASS, -1, 0, flags);
    return 0;
  }
  // Tie members of a split boundary group are kept up to the keep-th in
  // index order (wave, register slot, lane, element): ties per wave, then
  // per slot, give each member its rank; cut_idx is the index of the last
  // kept member.
  const bool split = keep > 0 && keep < n_tie;
  if (split) {
    // A compare per element gives the wave-wide mask of the tie members at
    // that element of a register slot; member counts are scalar bit counts.
    uint32_t tslot[kFastChunks];  // members per register slot of this wave (uniform)
    uint32_t wsum = 0;
#pragma unroll
    for (int j = 0; j < kFastChunks; ++j) {
      uint32_t t = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) t += (uint32_t)__popcll(__ballot(key_at(d[j], e) == L));
      tslot[j] = t;
      wsum += t;
    }
    if (lane == 0) {
      sh.wtie[wave] = wsum;
#pragma unroll
      for (int j = 0; j < kFastChunks; ++j) sh.tslot[wave][j] = tslot[j];
    }
    lds_barrier();
    uint32_t base = 0;
    for (int w = 0; w < wave; ++w) base += sh.wtie[w];
    base = uni(base);
    // Only the wave holding the member of rank keep - 1 looks for it: the
    // slot from the slot counts, the lane from the members in lanes below
    // (chunk order within a slot is lane order), the element from its mask.
    const long long r0 = keep - 1 - (long long)base;
    if (r0 >= 0 && r0 < (long long)wsum) {
      uint32_t r = (uint32_t)r0;
      int js = 0;
#pragma unroll
      for (int j = 0; j < kFastChunks; ++j) {
        const bool here = js == j && r >= tslot[j];
        r -= here ? tslot[j] : 0u;
        js += here ? 1 : 0;
      }
      if (lane == 0) {
        sh.cut_w = wave;
        sh.cut_j = js;
        sh.cut_r = (int)r;
      }
      uint4 v = d[0];
#pragma unroll
      for (int j = 1; j < kFastChunks; ++j)
        if (js == j) v = d[j];
      uint32_t below = 0, m = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool hit = key_at(v, e) == L;
        const unsigned long long mk = __ballot(hit);
        below += __builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u));
        m |= (hit ? 1u : 0u) << e;
      }
      const uint32_t t = (uint32_t)__popc(m);
      if (below <= r && r < below + t) {
        const uint32_t fn = r - below;  // set bit fn of m
        uint32_t e = 0;
#pragma unroll
        for (int b = 0; b < 8; ++b) e += (uint32_t)__popc(m & ((2u << b) - 1u)) <= fn ? 1u : 0u;
        const uint32_t c = (uint32_t)wave * CW + (uint32_t)js * 64u + (uint32_t)lane;
        sh.bc_l[1] = 8ll * c + e;
      }
    }
    lds_barrier();
    cut_idx = uni(sh.bc_l[1]);
  }
  const int cut_w = split ? uni(sh.cut_w) : -1, cut_j = split ? uni(sh.cut_j) : 0;
  const int cut_r = split ? uni(sh.cut_r) : 0;

  // ---- mass table of the kept register-resident keys: every binade (128
  // keys) holding a kept key gets a slot of 128 fixed-point masses; absent
  // binades map to slot 0, all zero.  A split tie group's key stays 0 in the
  // table (its kept members are added by index).
  {
    const uint32_t b = (uint32_t)tid;  // binade, threads 0..511
    uint32_t present = 0;
    if (b < 512u && b >= 1u) {
      const uint32_t lo = 128u * b, hi = lo + 127u;
      const bool inr = lo <= Mk && (L == 0u || hi >= L);
      present = inr && (sh.mid.blk.bc[2u * b] + sh.mid.blk.bc[2u * b + 1u]) > 0u ? 1u : 0u;
    }
    uint32_t nbin;
    const uint32_t rank = bs.scan(present, nbin);
    if (nbin > (uint32_t)(kLutSlots - 1)) return kHandCapacity;  // more binades than the table holds
    if (b < 512u) sh.boff[b] = present ? (uint16_t)(1u + rank) : (uint16_t)0;
    if (present) sh.bslot[1u + rank] = (uint16_t)b;
  }
  lds_barrier();
  {
    const int slot = tid >> 4, m0 = (tid & 15) * 8;  // 8 table entries per thread
    const uint32_t nbin = bs.sum((uint32_t)(tid < 512 && sh.boff[tid] != 0 ? 1 : 0));
    const bool mine = slot >= 1 && (uint32_t)slot <= nbin;
    const uint32_t b = mine ? (uint32_t)sh.bslot[slot] : 0u;
    auto entry = [&](int i) -> long long {
      const uint32_t k = 128u * b + (uint32_t)(m0 + i);
      const uint32_t c = (sh.big.cnt[k >> 1] >> ((k & 1u) << 4)) & 0xFFFFu;
      const bool kept = k <= Mk && (L == 0u || k > L || (k == L && !split && keep > 0));
      return (mine && c && kept) ? to_fx(mass_of(bf16_key_value(k))) : 0ll;
    };
    // Two rounds of four: every count is read before the table overwrites it.
    long long f0 = entry(0), f1 = entry(1), f2 = entry(2), f3 = entry(3);
    const long long g0 = entry(4), g1 = entry(5), g2 = entry(6), g3 = entry(7);
    lds_barrier();
    long long* dst = &sh.big.lut[8 * tid];
    dst[0] = f0;
    dst[1] = f1;
    dst[2] = f2;
    dst[3] = f3;
    dst[4] = g0;
    dst[5] = g1;
    dst[6] = g2;
    dst[7] = g3;
  }
  lds_barrier();
  // Fixed-point kept mass of a register-resident key (split tie members excluded).
  auto key_fx = [&](uint32_t k) -> long long {
    return sh.big.lut[((uint32_t)sh.boff[k >> 7] << 7) | (k & 127u)];
  };
  // Index-order CDF: kept mass per (wave, register slot) -- slot j of wave w
  // is the 64 consecutive chunks w*CW + 64j .. 64j + 63 -- and per wave; then
  // the wave and slot holding u * total, and one lane of that slot walks its
  // chunk.  Tie members of a split group count up to cut_idx.
  auto chunk_mass = [&](const uint4& v, uint32_t c, bool ties) -> long long {
    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
    long long cm = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) cm += key_fx(w4[q] & 0xFFFFu) + key_fx(w4[q] >> 16);
    if (ties) {
      const long long lim = cut_idx - 8ll * c;
      const uint32_t m = key_bits(v, L);
      const uint32_t km = lim < 0 ? 0u : (lim >= 7 ? m : m & ((2u << lim) - 1u));
      cm += (long long)__popc(km) * mtie;
    }
    return cm;
  };
  {
    long long acc = 0;
#pragma unroll
    for (int j = 0; j < kFastChunks; ++j) {
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t c = (uint32_t)wave * CW + (uint32_t)j * 64u + (uint32_t)lane;
      long long sj = wave_reduce_dpp(chunk_mass(d[j], c, false), OpSum());
      if (split) {  // kept tie members of this slot: all before the cut, r + 1 in its slot, none after
        const long long t = (long long)sh.tslot[wave][j];
        const long long kt = wave < cut_w ? t : (wave > cut_w ? 0 : (j < cut_j ? t : (j == cut_j ? cut_r + 1 : 0)));
        sj += kt * mtie;
      }
      if (lane == 0) sh.smass[wave][j] = sj;
      acc += sj;
    }
    // The wave's total: its register-resident mass and its slots' penalised masses.
    const long long pw = wave_reduce_dpp(lane < kFastChunks ? sh.spen[wave][lane] : 0ll, OpSum());
    if (lane == 0) sh.wtot[wave] = acc + pw;
  }
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
  auto fetch_pk = [&](int64_t e) { return e >= 0 ? PenPk{Wp[e], a.pen_ids[o0 + e]} : PenPk{0ll, 0}; };
  // The crossing slot's per-chunk penalised masses start at zero (the
  // block sums sharing their LDS were last read before the mass table's
  // barrier).
  if (tid < 512) sh.mid.cm.pe[tid] = 0;
  if (tid < 64) sh.mid.cm.pen[tid] = 0;
  if (tid == 0) sh.bc_i[2] = 1;
  lds_barrier();
  // Every wave reads the 16 wave totals: their inclusive prefix on lanes 0..15.
  const long long wtl = lane < kWaves ? sh.wtot[lane] : 0ll;
  const long long wti = row_scan_dpp(wtl);
  if (lane_value(wti, kWaves - 1) != Sk) return kHandCapacity;  // the per-wave masses must add up to the kept total

  if (dense) {
    // Kept probabilities mass / kept total in float64 (recomputed, not the
    // fixed-point masses), zero elsewhere; kept bits mark every finite token
    // (no top-k on this path).
    fast_clear_outputs(a, row);
    const double Sd = (double)Sk * 0x1p-45;
#pragma unroll
    for (int j = 0; j < kFastChunks; ++j) {
      const uint32_t c = (uint32_t)wave * CW + (uint32_t)j * 64u + (uint32_t)lane;
#pragma unroll 1
      for (int e = 0; e < 8; ++e) {
        const uint32_t k = key_at_rt(d[j], e);
        if (k > kKeyNegInf) {
          const long long idx = 8ll * c + e;
          const bool kept = L == 0u || k > L || (k == L && keep > 0 && (!split || idx <= cut_idx));
          fast_scatter(a, row, idx, kept ? mass_of(bf16_key_value(k)) / Sd : 0.0);
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
  if (!has_draws<RNG>(a)) {
    if (tid == 0) fast_write_result(a, row, DSR_OK, -1, 0, flags);
    return 0;
  }
  if (npos_k == 1) {  // sampling.py:120-122: the single positive token is the maximum; no uniform
    if (M == 0.0) return kHandZero;
    const long long tok = first_of_max();
    if (tid == 0) fast_write_result(a, row, DSR_OK, tok, 0, flags);
    return 0;
  }
  uint64_t rng_next[4];
  const double u = RNG ? pcg64_random(st_pre, rng_next) : u_pre;
  if (!(u >= 0.0 && u < 1.0)) {
    if (tid == 0) fast_write_result(a, row, DSR_E_UNIFORM, -1, 0, flags);
    return 0;
  }
  const double thr_d = uni(u * (double)Sk);
  long long thr = uni((long long)thr_d);
  if (thr >= Sk) {
    thr = Sk - 1;
    flags |= DSR_FLAG_MARGIN;
  }
  flags = uni(flags);
  // The wave holding thr (the first whose inclusive total exceeds it), and
  // the mass before it.
  const unsigned long long owb = __ballot(lane < kWaves && thr < wti);
  if (!owb) return kHandCapacity;  // unreachable: thr < Sk
  const int ow = uni(__ffsll((long long)owb) - 1);
  const long long obase = uni(lane_value(wti - wtl, ow));
  // The register slot of that wave holding thr, from its 16 slot masses in
  // order (every wave finds the same one).
  int js;
  long long jbase;
  {
    const long long m = lane < kFastChunks ? sh.smass[ow][lane] + sh.spen[ow][lane] : 0ll;
    const long long incl = wave_scan_dpp(m);
    const long long ex = obase + incl - m;
    const unsigned long long hb = __ballot(m > 0 && ex <= thr && thr < ex + m);
    if (!hb) return kHandCapacity;  // unreachable: the crossing lies in the wave found above
    js = uni(__ffsll((long long)hb) - 1);
    jbase = uni(__shfl(ex, js));
  }
  const uint32_t cw0 = (uint32_t)ow * CW + (uint32_t)js * 64u;  // first chunk of that slot
  // Kept penalised masses of that slot's chunks, per chunk and per element
  // (only the run of entries whose tokens lie in the wave's chunks).
  // Each thread takes the entries of its own stride (e = tid mod kThreads),
  // whose packed words it wrote itself: no other thread's global stores are
  // read, so the LDS-only barriers above order everything this pass needs.
  const int64_t elo = sh.elo[ow], ehi = sh.elo[ow + 1];
  const int64_t first = elo + (((int64_t)tid - elo) % kThreads + kThreads) % kThreads;
  if (ehi > elo) {  // uniform
    pen_batches<1>(ehi, first, fetch_pk, [&](int64_t, PenPk x) {
      const uint32_t cid = (uint32_t)(x.id >> 3);
      if (x.pk != 0 && cid >= cw0 && cid < cw0 + 64u && cid < (uint32_t)(ow + 1) * CW &&
          pen_kept((uint32_t)((unsigned long long)x.pk >> 48), x.id)) {
        const long long fx = x.pk & ((1ll << 47) - 1);
        atomicAdd((unsigned long long*)&sh.mid.cm.pen[cid - cw0], (unsigned long long)fx);
        sh.mid.cm.pe[(cid - cw0) * 8u + (uint32_t)(x.id & 7)] = fx;  // one entry per token
      }
    });
    lds_barrier();
  }
  // The chunk of that slot holding thr (a scan over its 64 lanes), then that
  // lane walks its 8 tokens.
  if (wave == ow) {
    uint4 v = d[0];
#pragma unroll
    for (int j = 1; j < kFastChunks; ++j)
      if (js == j) v = d[j];
    const uint32_t cw = (uint32_t)js * 64u + (uint32_t)lane;
    const uint32_t c = (uint32_t)ow * CW + cw;
    const long long cm = cw < CW ? chunk_mass(v, c, split) + sh.mid.cm.pen[lane] : 0ll;
    const long long incl = wave_scan_dpp(cm);
    const long long ex = jbase + incl - cm;
    if (cm > 0 && ex <= thr && thr < ex + cm) {
      long long x = ex, tok = -1, tex = 0, tfx = 0;
#pragma unroll 1
      for (int e = 0; e < 8; ++e) {
        const uint32_t k = key_at_rt(v, e);
        const long long idx = 8ll * c + e;
        long long f = key_fx(k) + sh.mid.cm.pe[(uint32_t)lane * 8u + (uint32_t)e];
        if (split && k == L && idx <= cut_idx) f += mtie;
        if (tok < 0 && f > 0 && x <= thr && thr < x + f) {
          tok = idx;
          tex = x;
          tfx = f;
        }
        x += f;
      }
      const double tol = ((double)npos_k + 16.0) * 0x1p-50 * (double)Sk + (double)npos_k + 2.0;
      unsigned fl = flags;
      if ((double)(tex + tfx) - thr_d <= tol || (tex > 0 && thr_d - (double)tex <= tol)) fl |= DSR_FLAG_MARGIN;
      if (tok >= 0) fast_write_result(a, row, DSR_OK, tok, 1, fl);
      sh.bc_i[2] = tok < 0 ? 1 : 0;
    }
  }
  lds_barrier();
  // The row is decided: its advanced PCG64 state goes back (every thread read
  // the old one before the barriers above).
  if (RNG && tid == 0 && !sh.bc_i[2]) store_rng(a, row, rng_next);
  return sh.bc_i[2] ? kHandCapacity : 0;  // unreachable: thr lies inside the chunk found above
}

}  // namespace dsr
