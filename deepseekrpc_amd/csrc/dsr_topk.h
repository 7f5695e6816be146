// Streamed register-resident top-k path for bf16 rows (gfx950, wave64, no MFMA).
//
// One 1024-thread workgroup owns one row of up to 131,072 bf16 logits, read
// from HBM once as raw buffer loads straight into VGPRs (16 chunks of eight
// tokens per thread, every load issued up front; wave w owns chunks
// [w*CW, (w+1)*CW), lane l takes chunk w*CW + 64j + l at slot j, so index
// order is (wave, slot, lane, element)).  The row takes about 11 us to land
// when every CU streams its own row, and the sampling decision is a chain of
// dependent workgroup steps, so the chain is started while the row is still
// arriving:
//
//   * once slots 0..7 (the first half of each wave's range) have landed,
//     tau_lb is the k-th largest maximum over pairs of chunks of those slots,
//     taken from a histogram of 4-level bins.  A subset's k-th largest value
//     never exceeds the row's (k tokens of the subset reach it), so every
//     top-k token, boundary ties included, lies in a chunk whose maximum
//     reaches tau_lb;
//   * such chunks are listed whole, in index order, in their wave's LDS list, the
//     slots already landed at once and the rest slot by slot as they land; batches of
//     listed chunks feed an exact histogram of the keys at or above tau_lb (4,096
//     keys) and keep an 8-bit mask of their tokens that reach it;
//   * after the last slot: the row maximum, one scan of the histogram bins (count,
//     fixed-point mass of r = exp((v - max) / T) per key, tokens with r > 0) that
//     gives the top-k boundary key and its kept ties (sampling.py:89-91, lowest
//     indices first), the total mass and the top-p boundary (sampling.py:97-102)
//     with its tie group settled in float64 as the reference's exclusive prefix
//     rule; min-p keeps r >= min_p (sampling.py:94-96, max(result) = 1 / sum);
//   * one scan over the listed candidates in index order gives the CDF of
//     categorical (sampling.py:103-128); the thread whose interval holds
//     floor(u * total) walks its tokens to the draw.
//
// Masses are fixed point at 2^48 (every sum of up to 32,768 masses <= 1 fits in
// 64 bits), so all sums are exact and order-independent.  The path is exact
// where bf16 key order equals the reference's float64 order; each row checks
// that at its decision boundaries and otherwise hands the row to the general
// path in the same workgroup, as it does for invalid rows, a top-k the
// register path does not take, a top-k reaching zero or below, and list or key
// window overflow.  Decisions the reference's own rounding could tip are
// reported with DSR_FLAG_MARGIN.
#pragma once

#include "dsr_fast.h"

namespace dsr {

constexpr int kTkBound = 8;            // slots whose pair maxima give the lower bound (even, 6 to 12; 8 measured best)
constexpr uint32_t kTkRing = 128;      // candidate chunks waiting for a histogram round, per wave
constexpr uint32_t kTkTokCap = 512;    // candidate tokens per wave
constexpr int kTkWin = 4096;           // exact keys tracked from the lower bound up
constexpr int kTkCoarseWords = 4096;   // 8,192 bins of 4 positive levels, two 16-bit counts per word
constexpr double kTkFix = 0x1p48;      // fixed-point scale of the masses
constexpr unsigned long long kTkFixU = 1ull << 48;

struct TopkLists {
  uint32_t lut[256][4];                  // allow byte -> four 2 x 16-bit "disallowed" masks (every slot)
  uint32_t cnt[kTkWin];                  // candidate tokens by level - tau_lb
  union {
    uint32_t coarse[kTkCoarseWords];     // pair maxima of slots 0 .. kTkBound-1 by level / 4
    unsigned long long ftab[kTkWin];     // fixed-point mass by distance below the maximum
  };
  uint4 ring[kWaves][kTkRing];           // candidate chunks (masked bf16 bits) waiting for a histogram round
  uint16_t rid[kWaves][kTkRing];         // their chunk index in the wave's range
  uint32_t tok[kWaves][kTkTokCap];       // candidate tokens, index order per wave: level | index in range << 16
  double etab[64];                       // 2^(j/64) for exp_nonpos
  uint32_t polw[24];                     // the row's policy words, then its uniform or PCG64 state
  uint32_t wred[kWaves];                 // per wave: max key | flags << 16
  uint32_t wc[kWaves];                   // per wave: key count | positive count << 16, then boundary ties
  unsigned long long wm[kWaves];         // per wave: fixed-point mass, then kept mass off the boundary
  int lb;                                // tau_lb as a level
  uint32_t close_min;                    // smallest distance of a key inside the min-p rounding band
  unsigned long long ea[kWaves];         // per wave: kept mass off the boundary (CDF)
  uint32_t et[kWaves];                   // per wave: boundary ties | top-k boundary ties << 16 (CDF)
  int p_late;                            // top-p boundary checks: hand-over reason | margin << 8
  int p_dk, p_need, p_dl, p_keep, p_info;
  uint32_t p_close, p_npos;              // p_close: DSR_FLAG_MARGIN when a top-k mass sits in the min-p band
  unsigned long long p_C, p_fl;
  SyncSlots sync;
};

struct TopkShared {
  union {
    GenShared gen;  // reused by the general path when a row falls back
    TopkLists t;
  };
};

// Orders this wave's LDS writes before its later LDS reads (no workgroup barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Signed 16-bit level (the bf16 bit pattern) of element e of a listed chunk
// (words x, y, z, w).  Selects on values, then one 64-bit shift: a select
// between the vector's fields would be turned into an indexed load from a
// stack copy of it.
__device__ __forceinline__ int chunk_elem_level(uint32_t x, uint32_t y, uint32_t z, uint32_t w, int e) {
  const uint32_t lo = (e & 4) ? z : x, hi = (e & 4) ? w : y;
  const uint64_t h = ((uint64_t)hi << 32) | lo;
  return (int)(short)(uint16_t)(h >> (16 * (e & 3)));
}

// Returns 0 if the row was decided here, else the reason it is handed to the
// general path (kHand*).
template <bool RNG>
__device__ __forceinline__ int topk_sample_row(const dsr_sample_args_t& a, int64_t row, TopkShared& shu) {
  TopkLists& sh = shu.t;
  const int tid = threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int64_t V = a.vocab;
  const uint32_t C = (uint32_t)(V >> 3);
  const uint32_t CW = (C + kWaves - 1) / kWaves;
  BlockSync bs(sh.sync);

  // ---- loads are raw buffer loads (out-of-range reads return 0): one word
  // per thread of the policy (threads 0-13) and of the uniform or PCG64 state,
  // then per slot the chunk's allow byte and its 16 bytes of logits.
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a.policy + row), (short)0, (int)sizeof(dsr_policy_t), 0x00020000);
  const __amdgpu_buffer_rsrc_t urs = __builtin_amdgcn_make_buffer_rsrc(
      RNG ? (void*)(a.rng_state + 4 * row) : (a.uniforms ? (void*)(a.uniforms + row) : (void*)a.policy),
      (short)0, RNG ? 32 : (a.uniforms ? 8 : 0), 0x00020000);
  constexpr int kPolWords = (int)(sizeof(dsr_policy_t) / 4);
  // Wave 0 alone reads the policy words: a wave waiting for its first load
  // waits behind every load the waves before it issued.
  uint32_t pw = 0;
  double etv = 0.0;
  if (wave == 0) {
    pw = __builtin_amdgcn_raw_buffer_load_b32(prs, tid < kPolWords ? 4 * tid : 0x7FFFFFF0, 0, 0) |
         __builtin_amdgcn_raw_buffer_load_b32(
             urs, (tid >= kPolWords && tid < kPolWords + (RNG ? 8 : 2)) ? 4 * (tid - kPolWords) : 0x7FFFFFF0, 0, 0);
    const __amdgpu_buffer_rsrc_t ers =
        __builtin_amdgcn_make_buffer_rsrc((void*)kExp2Frac, (short)0, (int)sizeof(kExp2Frac), 0x00020000);
    const auto ev = __builtin_amdgcn_raw_buffer_load_b64(ers, 8 * lane, 0, 0);
    etv = __builtin_bit_cast(double, ((unsigned long long)(uint32_t)ev[1] << 32) | (uint32_t)ev[0]);
  }
  const __amdgpu_buffer_rsrc_t mrs = __builtin_amdgcn_make_buffer_rsrc(
      a.allow_bits ? (void*)(a.allow_bits + row * a.allow_ld) : (void*)&kAllowAll, (short)0, (int)C, 0x00020000);
  const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint16_t*)a.logits + row * a.ld), (short)0, (int)(V * 2), 0x00020000);
  uint32_t mb[kFastChunks];
  uint4 d[kFastChunks];
  auto issue = [&](int j) {
    const uint32_t cw = (uint32_t)j * 64u + (uint32_t)lane;
    const uint32_t c = (uint32_t)wave * CW + cw;
    const bool mine = cw < CW;  // chunks past this wave's range belong to the next wave: read as 0 (masked)
    mb[j] = __builtin_amdgcn_raw_buffer_load_b8(mrs, (int)(mine ? c : 0x7FFFFFF0u), 0, 2);
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rrs, (int)(mine ? c * 16u : 0x7FFFFFF0u), 0, 2);
    d[j] = make_uint4(v[0], v[1], v[2], v[3]);
  };

  // ---- pass 1 of a slot once it has landed.  Disallowed tokens become
  // 0xFFFF (a negative NaN pattern no valid input holds; level -1).  Chunk
  // maxima are taken as signed 16-bit integers of the bf16 bits ("levels"),
  // which order positive values exactly.
  uint32_t vmax_s = 0x80008000u, vmax_u = 0u, cmx[kFastChunks / 2];
  auto pass1 = [&](int j) {
    __builtin_amdgcn_sched_barrier(0);
    const uint4 lm = *(const uint4*)sh.lut[mb[j] & 0xFFu];
    uint32_t w[4] = {d[j].x, d[j].y, d[j].z, d[j].w};
    const uint32_t m4[4] = {lm.x, lm.y, lm.z, lm.w};
    uint32_t cm = 0x80008000u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      vmax_s = pk_max_i16(vmax_s, w[q]);  // +inf / +NaN: 0x7F80 and up
      vmax_u = pk_max_u16(vmax_u, w[q]);  // -NaN: 0xFF81 and up
      w[q] |= m4[q];
      cm = pk_max_i16(cm, w[q]);
    }
    d[j] = make_uint4(w[0], w[1], w[2], w[3]);
    const int cmj = max((int)(short)(cm & 0xFFFFu), (int)(short)(cm >> 16));
    if (j & 1) cmx[j >> 1] |= (uint32_t)cmj << 16; else cmx[j >> 1] = (uint32_t)cmj & 0xFFFFu;
    // Pin this slot's results here: left to itself the compiler sinks the
    // masking and the NaN maxima to their uses and keeps the raw and masked
    // row (and unpacked maxima) live together, which spills, and a spill
    // reload waits for every outstanding load of the row.
    asm volatile("" : "+v"(d[j].x), "+v"(d[j].y), "+v"(d[j].z), "+v"(d[j].w), "+v"(vmax_s), "+v"(vmax_u));
    if (j & 1) asm volatile("" : "+v"(cmx[j >> 1]));
    __builtin_amdgcn_sched_barrier(0);
  };

  // ---- the load schedule.  A CU keeps only about 40 KB of loads in flight;
  // a wave whose next instruction is a load waits until the memory pipeline
  // takes it, and the oldest wave issues first, so loads issued up front
  // would land wave by wave and keep every wave blocked in its loads until
  // the last ones were taken.  Instead the slots are issued in rounds, one
  // slot per wave and a barrier per round, so they land slot by slot for the
  // whole workgroup, and each round does the work of a slot issued four
  // rounds before (landed by then).  The lower bound tau_lb is taken from
  // slots 0 .. kTkBound-1 in the barriers of the three rounds after theirs.
#pragma unroll
  for (int j = 0; j < 4; ++j) issue(j);
  __builtin_amdgcn_sched_barrier(0);
  // While the first slots stream in: the mask lookup table, cleared histograms.
  {
    const uint32_t m = (uint32_t)tid >> 2, q = (uint32_t)tid & 3u;
    sh.lut[m][q] = (((m >> (2 * q)) & 1u) ? 0u : 0x0000FFFFu) | (((m >> (2 * q + 1)) & 1u) ? 0u : 0xFFFF0000u);
    ((uint4*)sh.cnt)[tid] = make_uint4(0u, 0u, 0u, 0u);     // 4,096 words
    ((uint4*)sh.coarse)[tid] = make_uint4(0u, 0u, 0u, 0u);  // 4,096 words
    if (tid == 0) {
      sh.close_min = 0xFFFFFFFFu;
      sh.p_late = 0;
    }
    if (tid < kWaves) {
      sh.ea[tid] = 0ull;
      sh.et[tid] = 0u;
    }
  }
  lds_barrier();
  if (wave == 0) {  // ordered by the next barrier
    if (tid < kPolWords + (RNG ? 8 : 2)) sh.polw[tid] = pw;
    sh.etab[lane] = etv;
  }
  // Round r issues slot r (r < 16) and runs pass 1 of slot r - 4.
  auto step = [&](int r) {
    if (r < kFastChunks) issue(r);
    __builtin_amdgcn_sched_barrier(0);
    pass1(r - 4);
  };
  step(4);
  lds_barrier();

  dsr_policy_t pol;
  double u;
  {
    uint32_t w[kPolWords + 2];
#pragma unroll
    for (int i = 0; i < kPolWords + 2; ++i) w[i] = (uint32_t)__builtin_amdgcn_readfirstlane((int)sh.polw[i]);
    __builtin_memcpy(&pol, w, sizeof(pol));
    u = __builtin_bit_cast(double, ((unsigned long long)w[kPolWords + 1] << 32) | w[kPolWords]);
  }
  const double T = pol.temperature;
  const int top_k = pol.top_k;
  const bool greedy = T == 0.0;
  // The order of these checks decides which launch owns a whole row when the
  // full-vocabulary kernel runs after this one (kModeDeferWhole).
  if (!(T >= 0.0 && T <= 100.0)) return kHandPolicy;
  if (whole_row(T, top_k, V)) {  // the next launch's row: end with no load of it outstanding
    __builtin_amdgcn_s_waitcnt(0);
    return kHandTopK;
  }
  if (!policy_ok(pol)) return kHandPolicy;
  const uint32_t k = greedy ? 1u : (uint32_t)top_k;

#pragma unroll
  for (int r = 5; r < kTkBound + 3; ++r) {
    step(r);
    lds_barrier();
  }
  step(kTkBound + 3);

  // ---- tau_lb: the k-th largest positive pair maximum of slots
  // 0 .. kTkBound-1, to 4 levels (its bin's lower edge).  Fewer than k
  // positive pair maxima hand the row over (a top-k reaching zero or below).
#pragma unroll
  for (int q = 0; q < kTkBound / 2; ++q) {
    const int gq = max((int)(short)(cmx[q] & 0xFFFFu), (int)(short)(cmx[q] >> 16));
    if (gq > 0) {
      const uint32_t b = (uint32_t)gq >> 2;  // < 8,192
      atomicAdd(&sh.coarse[b >> 1], 1u << (16u * (b & 1u)));
    }
  }
  lds_barrier();
  step(kTkBound + 4);
  uint32_t cc[8];
  {
    const uint4 w4 = ((const uint4*)sh.coarse)[1023 - tid];  // words 4092-4t .. 4095-4t: bins 8191-8t down to 8184-8t
    cc[0] = w4.w >> 16; cc[1] = w4.w & 0xFFFFu; cc[2] = w4.z >> 16; cc[3] = w4.z & 0xFFFFu;
    cc[4] = w4.y >> 16; cc[5] = w4.y & 0xFFFFu; cc[6] = w4.x >> 16; cc[7] = w4.x & 0xFFFFu;
  }
  uint32_t s8 = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) s8 += cc[i];
  uint32_t ptot;
  const uint32_t prun = bs.scan(s8, ptot);
  if (ptot < k) return kHandCapacity;  // uniform
  if (prun < k && k <= prun + s8) {
    uint32_t rr = prun;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (rr < k && k <= rr + cc[i]) sh.lb = (int)((8191u - 8u * (uint32_t)tid - (uint32_t)i) << 2);
      rr += cc[i];
    }
  }
  step(kTkBound + 5);
  lds_barrier();
  const int lb = __builtin_amdgcn_readfirstlane(sh.lb);
#pragma unroll
  for (int r = kTkBound + 6; r < kFastChunks; ++r) issue(r);
  __builtin_amdgcn_sched_barrier(0);

  // ---- candidate chunks (maximum >= tau_lb) pass, in index order, through a
  // 128-entry ring per wave; rounds of 64 of them feed the exact histogram of
  // the candidate keys and append the candidate tokens (level, index in the
  // wave's range) to the wave's token list, in index order.
  uint32_t wn = 0, hdone = 0, ntok = 0;  // wave-uniform
  auto hist = [&](uint32_t hend) {        // wave-uniform; hend - hdone <= kTkRing
    wave_lds_sync();
    for (uint32_t base = hdone; base < hend; base += 64u) {
      const uint32_t e = base + (uint32_t)lane;
      uint32_t m = 0, tb = 0;
      uint4 r4 = make_uint4(0u, 0u, 0u, 0u);
      if (e < hend) {
        r4 = sh.ring[wave][e & (kTkRing - 1u)];
        tb = 8u * (uint32_t)sh.rid[wave][e & (kTkRing - 1u)];
        // A candidate more than 4,095 keys above tau_lb is counted in the top
        // key's bin; the row maximum then lies above the window too, and the
        // row is handed over once that is known.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int off = chunk_elem_level(r4.x, r4.y, r4.z, r4.w, i) - lb;
          m |= (off >= 0 ? 1u : 0u) << i;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if ((m >> i) & 1u) atomicAdd(&sh.cnt[min(chunk_elem_level(r4.x, r4.y, r4.z, r4.w, i) - lb, kTkWin - 1)], 1u);
        }
      }
      const uint32_t n = (uint32_t)__popc(m);
      const uint32_t incl = wave_scan_dpp(n);
      uint32_t p = ntok + incl - n;
      while (m) {
        const int b = __builtin_ctz(m);
        m &= m - 1u;
        if (p < kTkTokCap)
          sh.tok[wave][p] = (uint32_t)(uint16_t)chunk_elem_level(r4.x, r4.y, r4.z, r4.w, b) | ((tb + (uint32_t)b) << 16);
        ++p;
      }
      ntok += lane_value(incl, 63);
    }
    hdone = hend;
  };
  // Before each call fewer than 64 ring entries wait, so a slot's (at most 64)
  // never overwrite one that waits.
  auto compact = [&](int j) {
    const bool q = chunk_level(cmx, j) >= lb;
    const unsigned long long b = __ballot(q);
    if (q) {
      const uint32_t p = (wn + lanes_below(b)) & (kTkRing - 1u);
      sh.ring[wave][p] = d[j];
      sh.rid[wave][p] = (uint16_t)((uint32_t)j * 64u + (uint32_t)lane);
    }
    wn += (uint32_t)__popcll(b);
    if (wn - hdone >= 64u) hist(hdone + 64u);
  };
#pragma unroll
  for (int j = 0; j < kTkBound + 2; ++j) compact(j);
#pragma unroll
  for (int j = kTkBound + 2; j < kFastChunks; ++j) {
    pass1(j);
    compact(j);
  }
  hist(wn);
  __builtin_amdgcn_sched_barrier(0);

  // ---- the row maximum and the flags of every wave.
  uint32_t mm = cmx[0];
#pragma unroll
  for (int i = 1; i < kFastChunks / 2; ++i) mm = pk_max_i16(mm, cmx[i]);
  const int tmax = max((int)(short)(mm & 0xFFFFu), (int)(short)(mm >> 16));
  const uint32_t bad = max((int)(short)(vmax_s & 0xFFFFu), (int)(short)(vmax_s >> 16)) >= 0x7F80 ||
                       max(vmax_u & 0xFFFFu, vmax_u >> 16) >= 0xFF81u;
  {
    const uint32_t wk = wave_reduce_dpp((uint32_t)(tmax + 0x8000), OpMax());
    const uint32_t wf = wave_reduce_dpp(bad, OpOr());
    if (lane == 0) sh.wred[wave] = wk | ((wf | (ntok > kTkTokCap ? 2u : 0u)) << 16);
  }
  lds_barrier();
  uint32_t Mkey, F;
  {
    const uint32_t y = lane < kWaves ? sh.wred[lane] : 0u;
    Mkey = lane_value(row_reduce(y & 0xFFFFu, OpMax()), 0);
    F = lane_value(row_reduce(y >> 16, OpOr()), 0);
  }
  if (F & 1u) return kHandInvalid;   // NaN / +inf: the general path reports it in the reference's order
  const int Mlev = (int)Mkey - 0x8000;  // at least k tokens reach tau_lb, so the maximum does
  const double M = bf16_key_value(Mkey);
  const int dM = Mlev - lb;
  if ((F & 2u) || dM >= kTkWin) return kHandCapacity;  // a token list or the key window overflowed

  // ---- this lane's candidate tokens: lane l of wave w holds tokens
  // G*l .. G*l+G-1 of its wave's list (G = ceil(count / 64) <= 8, the same in
  // the whole wave), so thread order is index order and every loop over a
  // lane's tokens stops at G.
  const uint32_t nt = ntok;  // <= kTkTokCap after the overflow check
  const uint32_t G = (nt + 63u) >> 6;
  const uint32_t t0 = G * (uint32_t)lane;
  uint32_t tk[8], ddv[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    tk[t] = 0u;
    ddv[t] = 0xFFFFFFFFu;
    if ((uint32_t)t < G) {  // wave-uniform
      if (t0 + t < nt) {
        tk[t] = sh.tok[wave][t0 + t];
        ddv[t] = (uint32_t)(Mlev - (int)(short)(uint16_t)(tk[t] & 0xFFFFu));
      }
    }
  }

  unsigned flags = 0;
  // Top-k boundary (distance dk below the maximum, `need` of its ties kept),
  // top-p boundary (dl <= dk, K of its ties kept), kept total, positive count.
  uint32_t dk = 0, need = 1, dl = 0, K = 1, npos = 1;
  unsigned long long Ct = kTkFixU, fxdl = kTkFixU;
  if (!greedy) {
    // ---- per key (thread t: distances 4t .. 4t+3 below the maximum): count,
    // r = exp((v - max) / T) (sampling.py:86-92; the division rounds as the
    // reference's, the exp is Tang's table-driven method, a few ulps from a
    // correctly rounded one, inside the decisions' tolerances) as fixed
    // point, and min-p, which keeps r >= min_p (:94-96).  Only the waves that
    // hold keys in range work; each publishes its totals.
    uint32_t c[4] = {0u, 0u, 0u, 0u};
    unsigned long long fx[4] = {0ull, 0ull, 0ull, 0ull};
    bool rp[4] = {false, false, false, false};
    const int nwb = dM / 256 + 1;  // waves holding keys in range
    if (wave < nwb) {
      double r[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int dd = 4 * tid + q;
        c[q] = dd <= dM ? sh.cnt[dM - dd] : 0u;
        // Clamped into range so that every lane's four exps run side by side.
        r[q] = exp_nonpos((bf16_key_value(Mkey - (uint32_t)min(dd, dM)) - M) / T, sh.etab);
      }
      unsigned long long msum = 0;
      uint32_t csum = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (!c[q]) continue;
        const int dd = 4 * tid + q;
        if (pol.min_p != 0.0) {
          if (r[q] > 0.0 && fabs(r[q] - pol.min_p) <= pol.min_p * 0x1p-48) atomicMin(&sh.close_min, (uint32_t)dd);
          if (r[q] < pol.min_p) r[q] = 0.0;
        }
        fx[q] = (unsigned long long)(r[q] * kTkFix);
        rp[q] = r[q] > 0.0;
        sh.ftab[dd] = fx[q];
        msum += (unsigned long long)c[q] * fx[q];
        csum += c[q] | ((rp[q] ? c[q] : 0u) << 16);
      }
      const unsigned long long wm = wave_reduce_dpp(msum, OpSum());
      const uint32_t wc = wave_reduce_dpp(csum, OpSum());
      if (lane == 0) {
        sh.wm[wave] = wm;
        sh.wc[wave] = wc;
      }
    }
    lds_barrier();
    // Totals of the waves (count | positive count << 16, mass), their
    // inclusive prefix in key order on lanes 0..15 of every wave.
    const uint32_t wcl = lane < nwb ? sh.wc[lane] : 0u;
    const unsigned long long wml = lane < nwb ? sh.wm[lane] : 0ull;
    const uint32_t wci = row_scan_dpp(wcl);
    const unsigned long long wmi = row_scan_dpp(wml);
    const unsigned long long bk = __ballot(lane < kWaves && (wci & 0xFFFFu) >= k);
    if (!bk) return kHandCapacity;  // uniform; at least k tokens reach tau_lb
    const int wk = __builtin_ctzll(bk);
    // This lane's keys: counts, masses and positive counts, cut at (cutd,
    // cutn) (key cutd keeps cutn tokens, keys beyond it none); exclusive
    // prefixes inside the wave plus the wave's base.
    auto lane_prefix = [&](uint32_t cutd, uint32_t cutn, uint32_t cbase, unsigned long long mbase, uint32_t* kc,
                           unsigned long long& mex, uint32_t& cex, uint32_t& pex, unsigned long long& msum,
                           uint32_t& csum) {
      uint32_t p4 = 0;
      csum = 0;
      msum = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t dd = 4u * (uint32_t)tid + q;
        kc[q] = dd < cutd ? c[q] : (dd == cutd ? cutn : 0u);
        csum += kc[q];
        p4 += rp[q] ? kc[q] : 0u;
        msum += (unsigned long long)kc[q] * fx[q];
      }
      const uint32_t cs = csum | (p4 << 16);
      const uint32_t ci = wave_scan_dpp(cs) - cs;
      mex = mbase + (wave_scan_dpp(msum) - msum);
      cex = (cbase & 0xFFFFu) + (ci & 0xFFFFu);
      pex = (cbase >> 16) + (ci >> 16);
    };
    if (wave == wk) {  // the wave holding the k-th token (sampling.py:89-91)
      uint32_t kc[4], cex, pex, csum;
      unsigned long long mex, msum;
      lane_prefix(0xFFFFFFFFu, 0u, lane_value(wci - wcl, wk), lane_value(wmi - wml, wk), kc, mex, cex, pex, msum, csum);
      if (cex < k && k <= cex + csum) {
        uint32_t rc = cex, rpc = pex, bdk = 0, bneed = 0, bpos = 0;
        unsigned long long rm = mex, bS = 0, bfx = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (rc < k && k <= rc + c[q]) {
            bdk = 4u * (uint32_t)tid + q;
            bneed = k - rc;
            bS = rm + (unsigned long long)bneed * fx[q];
            bpos = rpc + (rp[q] ? bneed : 0u);
            bfx = fx[q];
          }
          rc += c[q];
          rpc += rp[q] ? c[q] : 0u;
          rm += (unsigned long long)c[q] * fx[q];
        }
        // Boundary certificate: the bf16 neighbours of the k-th value stay
        // distinct after (v - max) / T, so key order and the reference's
        // float64 order agree on which boundary tokens tie (resolved by
        // index).  A neighbour within 2^40 of the maximum passes without
        // dividing: v - max is then exact and neighbours differ by more
        // than 2^-48 of it.
        const uint32_t bkey = Mkey - bdk;
        bool ok = !zero_key(bkey);
        if (ok && !(bf16_key_value(bkey - 1u) >= M * 0x1p-40)) {
          double s3[3];
#pragma unroll
          for (int i = 0; i < 3; ++i) {
            const uint32_t nk = bkey - 1u + (uint32_t)i;
            s3[i] = i == 0 ? -(double)INFINITY : (double)INFINITY;
            if (nk > kKeyNegInf && nk < kKeyPosInf) s3[i] = (bf16_key_value(nk) - M) / T;
          }
          ok = s3[0] < s3[1] && s3[1] < s3[2];
        }
        sh.p_dk = (int)bdk;
        sh.p_need = (int)bneed;
        sh.p_C = bS;
        sh.p_fl = bfx;
        sh.p_npos = bpos;
        sh.p_close = sh.close_min <= bdk ? DSR_FLAG_MARGIN : 0u;
        sh.p_info = ok ? 0 : kHandOrder;
      }
    }
    lds_barrier();
    if (const int info = __builtin_amdgcn_readfirstlane(sh.p_info)) return info;
    dk = (uint32_t)__builtin_amdgcn_readfirstlane(sh.p_dk);
    need = (uint32_t)__builtin_amdgcn_readfirstlane(sh.p_need);
    const unsigned long long S = sh.p_C;
    flags |= (unsigned)__builtin_amdgcn_readfirstlane((int)sh.p_close);
    dl = dk;
    K = need;
    Ct = S;
    fxdl = sh.p_fl;
    npos = (uint32_t)__builtin_amdgcn_readfirstlane((int)sh.p_npos);
    if (pol.top_p < 1.0) {  // sampling.py:97-102 on the top-k tokens' masses
      const double P = pol.top_p * (double)S;
      unsigned long long tgt = (unsigned long long)P;
      tgt = tgt < 1 ? 1 : (tgt > S ? S : tgt);  // S >= 2^48: the maximum's mass is exactly 1
      // Top-k totals of the waves: whole before the top-k boundary's wave,
      // the rest of S in it, nothing after.
      const unsigned long long cwm = lane < wk ? wml : (lane == wk ? S - lane_value(wmi - wml, wk) : 0ull);
      const unsigned long long cwi = row_scan_dpp(cwm);
      const int wl = __builtin_ctzll(__ballot(lane < kWaves && cwi >= tgt));
      // The boundary lane's values, kept for its checks after the barrier.
      bool mine = false;
      unsigned long long A = 0, rt = 0;
      uint32_t dlq = 0, n_above = 0, n_tie = 0;
      long long keep = 0;
      if (wave == wl) {  // the wave holding the top-p boundary
        uint32_t kc[4], cex, pex, csum;
        unsigned long long mex, msum;
        lane_prefix(dk, need, lane_value(wci - wcl, wl), lane_value(cwi - cwm, wl), kc, mex, cex, pex, msum, csum);
        mine = mex < tgt && tgt <= mex + msum;
        if (mine) {
          unsigned long long run = mex;
          uint32_t ce = cex;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const unsigned long long km = (unsigned long long)kc[q] * fx[q];
            if (run < tgt && tgt <= run + km) {
              dlq = 4u * (uint32_t)tid + q;
              A = run;
              n_above = ce;
              n_tie = kc[q];
              rt = fx[q];
            }
            run += km;
            ce += kc[q];
          }
          // Tie member i (index order) keeps iff A + i * rt < P (:98-101).
          if (n_tie == 1) {
            keep = (double)A < P ? 1 : 0;
          } else {
            keep = (long long)ceil((P - (double)A) / (double)rt);
            keep = keep < 0 ? 0 : (keep > (long long)n_tie ? (long long)n_tie : keep);
            while (keep > 0 && (double)(A + (unsigned long long)(keep - 1) * rt) >= P) --keep;
            while (keep < (long long)n_tie && (double)(A + (unsigned long long)keep * rt) < P) ++keep;
          }
          if (n_above == 0 && keep == 0) keep = 1;  // the first token is never removed
          sh.p_dl = (int)dlq;
          sh.p_keep = (int)keep;
          sh.p_C = A + (unsigned long long)keep * rt;
          sh.p_fl = rt;
          sh.p_npos = n_above + (uint32_t)keep;  // the boundary key holds mass, so every kept token has r > 0
        }
      }
      lds_barrier();
      if (mine) {
        // Checked while the other waves go on; read after the next barrier,
        // before anything is written.  The rounding band of the boundary
        // decision, and key order equal to mass order next to the boundary:
        // its bf16 neighbours keep (v - max) / T at least 2^-40 apart (always
        // so when the lower neighbour is at least 2^-24: its bf16 spacing is
        // then at least 2^-32 and T <= 100); ties with +-0 never pass.
        const unsigned long long uk = (unsigned long long)keep;
        const double tol = ((double)(n_above + uk) + 16.0) * 0x1p-51 * (double)S + (double)(n_above + n_tie + 2);
        bool near = fabs((double)(A + uk * rt) - P) <= tol;
        if (uk >= 1 && n_above + uk > 1) near = near || fabs((double)(A + (uk - 1) * rt) - P) <= tol;
        if (uk == 0 && n_above > 0) near = true;
        if (uk == n_tie && (double)(A + (unsigned long long)n_tie * rt) < P) near = true;
        const uint32_t lkey = Mkey - dlq;
        int hand = zero_key(lkey) ? kHandZero : 0;
        if (!hand && !(bf16_key_value(lkey - 1u) >= 0x1p-24)) {
          for (int side = -1; side <= 1 && !hand; side += 2) {
            const uint32_t nb = lkey + side;
            if (nb <= kKeyNegInf || nb >= kKeyPosInf || zero_key(nb)) continue;
            if (!(fabs(bf16_key_value(nb) - bf16_key_value(lkey)) / T >= 0x1p-40)) hand = kHandOrder;
          }
        }
        sh.p_late = hand | (near ? 0x100 : 0);
      }
      dl = (uint32_t)__builtin_amdgcn_readfirstlane(sh.p_dl);
      K = (uint32_t)__builtin_amdgcn_readfirstlane(sh.p_keep);
      Ct = sh.p_C;
      fxdl = sh.p_fl;
      npos = (uint32_t)__builtin_amdgcn_readfirstlane((int)sh.p_npos);
    }
  }

  // ---- categorical (sampling.py:103-128): each token's kept mass (boundary
  // ties aside) and its exclusive prefix inside the lane, the totals of every
  // wave, then the wave whose interval holds floor(u * total) finds the lane
  // and the token in it.  Boundary ties keep the lowest indices: a tie's rank
  // is the number of ties before it, and K of them are kept.
  unsigned long long fm[8], pm[8], At = 0;
  uint32_t pt[8], Tt = 0, Tk = 0;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    fm[t] = 0ull;
    if ((uint32_t)t < G) {  // wave-uniform; the read is unconditional so that all of them are in flight together
      const unsigned long long v = sh.ftab[ddv[t] < dl ? ddv[t] : 0u];
      fm[t] = ddv[t] < dl ? v : 0ull;
    }
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    pm[t] = At;
    pt[t] = Tt;
    if ((uint32_t)t < G) {
      At += fm[t];
      Tt += ddv[t] == dl;
      Tk += ddv[t] == dk;
    }
  }
  if (At) atomicAdd(&sh.ea[wave], At);
  if (Tt | Tk) atomicAdd(&sh.et[wave], Tt | (Tk << 16));
  // The draw's threshold, ahead of the barrier.
  const bool draws = has_draws<RNG>(a);
  unsigned long long thr = 0;
  double thr_d = 0.0;
  int consumed = 0, ust = DSR_OK;
  uint64_t rng_next[4];
  if (draws && npos > 1) {  // exactly one positive token: no uniform is drawn (sampling.py:120-122)
    if (RNG) {  // the row's PCG64 state, staged in LDS with the policy words
      uint64_t st4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st4[i] = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)sh.polw[kPolWords + 2 * i]) |
                 ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)sh.polw[kPolWords + 2 * i + 1]) << 32);
      u = pcg64_random(st4, rng_next);
    }
    if (!(u >= 0.0 && u < 1.0)) {
      ust = DSR_E_UNIFORM;
    } else {
      // First token whose CDF value exceeds u * total: with integer CDF
      // values the token whose interval [ex, ex + fx) holds floor(u * total);
      // if rounding leaves u * total at the total, the last positive token.
      thr_d = u * (double)Ct;
      thr = (unsigned long long)thr_d;
      if (thr >= Ct) {
        thr = Ct - 1;
        flags |= DSR_FLAG_MARGIN;
      }
      consumed = 1;
    }
  }
  const double tol = ((double)npos + 16.0) * 0x1p-51 * (double)Ct + (double)npos + 2.0;
  lds_barrier();
  {
    const int late = __builtin_amdgcn_readfirstlane(sh.p_late);
    if (late & 0xFF) return late & 0xFF;
    if (late & 0x100) flags |= DSR_FLAG_MARGIN;
  }
  // Wave bases (strict mass, boundary ties, top-k boundary ties) on lanes 0..15.
  const unsigned long long wal = lane < kWaves ? sh.ea[lane] : 0ull;
  const uint32_t wtl = lane < kWaves ? sh.et[lane] : 0u;
  const unsigned long long wai = row_scan_dpp(wal);
  const uint32_t wti = row_scan_dpp(wtl);
  const int64_t tok0 = 8 * (int64_t)wave * (int64_t)CW;  // row index of the wave's first token

  const bool dense = a.out_probs_f32 || a.out_probs_f64 || a.out_kept_bits;
  if (dense) {
    const uint32_t pq = wave_scan_dpp(Tt | (Tk << 16)) - (Tt | (Tk << 16));  // ties before this lane in its wave
    const uint32_t wb = lane_value(wti - wtl, wave);
    fast_clear_outputs(a, row);
    uint32_t tl = (wb & 0xFFFFu) + (pq & 0xFFFFu), tq = (wb >> 16) + (pq >> 16);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      if ((uint32_t)t >= G || t0 + t >= nt) continue;
      const int lvl = (int)(short)(uint16_t)(tk[t] & 0xFFFFu);
      const uint32_t dd = ddv[t];
      const bool topk = dd < dk || (dd == dk && tq < need);
      const bool kept = dd < dl || (dd == dl && tl < K);
      tq += dd == dk;
      tl += dd == dl;
      if (!topk) continue;
      double p = 1.0;  // greedy: the first maximum alone
      if (!greedy) {
        double r = 0.0;
        if (kept) {
          r = exp_nonpos((bf16_key_value((uint32_t)(lvl + 0x8000)) - M) / T, sh.etab);
          if (pol.min_p != 0.0 && r < pol.min_p) r = 0.0;
        }
        p = r / ((double)Ct * 0x1p-48);
      }
      fast_scatter(a, row, tok0 + (int64_t)(tk[t] >> 16), p);
    }
  }
  if (!draws || ust != DSR_OK) {
    if (tid == 0) fast_write_result(a, row, ust, -1, 0, flags);
    return 0;
  }
  if (RNG && consumed && tid == 0) store_rng(a, row, rng_next);  // the row is decided here
  // Each wave's interval [start, end) of the CDF: its strict mass plus its
  // kept boundary ties, after the waves before it.
  const uint32_t tb_l = (wti - wtl) & 0xFFFFu;
  const unsigned long long ws_l = (wai - wal) + (unsigned long long)min(tb_l, K) * fxdl;
  const unsigned long long we_l = wai + (unsigned long long)min(tb_l + (wtl & 0xFFFFu), K) * fxdl;
  const unsigned long long bo = __ballot(lane < kWaves && ws_l <= thr && thr < we_l && we_l > ws_l);
  if (wave == (bo ? __builtin_ctzll(bo) : -1)) {  // the wave whose interval holds thr
    const uint32_t tw = (wti - wtl) & 0xFFFFu;   // boundary ties before this wave
    const unsigned long long aw = lane_value(wai - wal, wave);
    const uint32_t tbw = lane_value(tw, wave);
    const unsigned long long aex = aw + (wave_scan_dpp(At) - At);
    const uint32_t tex = tbw + (wave_scan_dpp(Tt) - Tt);
    const unsigned long long ext = aex + (unsigned long long)min(tex, K) * fxdl;
    const unsigned long long kept_t = At + (unsigned long long)(min(tex + Tt, K) - min(tex, K)) * fxdl;
    if (kept_t > 0 && ext <= thr && thr < ext + kept_t) {
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        if ((uint32_t)t >= G) break;
        const uint32_t rank = tex + pt[t];
        const unsigned long long ex = aex + pm[t] + (unsigned long long)min(rank, K) * fxdl;
        const unsigned long long f = ddv[t] == dl ? (rank < K ? fxdl : 0ull) : fm[t];
        if (f > 0 && ex <= thr && thr < ex + f) {
          if (consumed && ((double)(ex + f) - thr_d <= tol || (ex > 0 && thr_d - (double)ex <= tol)))
            flags |= DSR_FLAG_MARGIN;
          fast_write_result(a, row, DSR_OK, tok0 + (int64_t)(tk[t] >> 16), consumed, flags);
        }
      }
    }
  }
  return 0;
}

}  // namespace dsr
