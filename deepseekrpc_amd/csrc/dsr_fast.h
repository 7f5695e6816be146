// Register-resident fast path for bf16 rows (gfx950, wave64, no MFMA).
//
// One 1024-thread workgroup owns one row of up to 131,072 bf16 logits.  The
// row is read from HBM exactly once: the allow bitmask is fetched first, then
// every 16-byte load of the row is issued up front, as raw buffer loads
// straight into VGPRs (16 x uint4 per thread, 256 KB per row across the
// workgroup).  Pass 1 turns each chunk into order-preserving 16-bit keys as
// it arrives, with the allow mask and the NaN/+inf check fused in, so it runs
// under the loads still in flight (the staging barrier orders LDS only).
// Wave w owns the contiguous chunk range [w*CW, (w+1)*CW) of 8-token chunks;
// lane l of it takes chunk w*CW + 64*j + l at step j, so every load
// instruction reads a contiguous 1 KB and the row's index order is
// (wave, j, lane, element).
//
// The path is VALU-issue bound once the row is in registers, so everything
// after pass 1 works on few tokens, few waves and few barriers:
//   * keys are tracked as distances below the row maximum; a histogram of
//     the 4,096 group maxima (a group is 4 chunks of one thread) over the
//     4,096 keys below the maximum gives tau, the k-th largest group maximum:
//     at least k tokens reach tau, and only the chunks whose maximum reaches
//     it are compacted, whole and in index order, into LDS (one ballot per
//     register slot);
//   * an exact-key histogram of the listed tokens gives the k-th key; its
//     tie group is resolved by index (lowest first), as the reference's
//     stable argsort does (sampling.py:89-91), and one packed scan gives both
//     tie ranks and the kept tokens' positions;
//   * the k <= 1024 kept tokens then sit one per thread: float64
//     r = exp((v - max) / T) (sampling.py:86-92); min-p and top-p are decided
//     on these unnormalised masses (the maximum is exp(0) = 1, so min-p keeps
//     r >= min_p, and top-p compares prefix mass with top_p times the total);
//     the top-p boundary key comes from a fixed-point mass histogram, its tie
//     group is settled in exact float64 arithmetic;
//   * one wave finishes with the index-order CDF search of categorical
//     (sampling.py:103-128).
//
// The path is exact only where bf16 key order equals the reference's float64
// order; each row checks that at its decision boundaries (no +-0 boundary,
// neighbouring bf16 values keep distinct (v - max) / T and masses) and
// otherwise hands the row to the general path in the same workgroup, as it
// does for rows with penalties, bias, no top-k, k > 1024, too many boundary
// chunks or a k-th group maximum more than 4,095 keys below the maximum.
// Decisions that the reference's own rounding could tip (min-p, top-p and
// CDF comparisons within a few ulps) are reported with DSR_FLAG_MARGIN.
#pragma once

#include "dsr_general.h"
#include "dsr_wave.h"

namespace dsr {

constexpr int kFastChunks = 16;                                         // 16-byte chunks per thread
constexpr int64_t kFastMaxVocab = (int64_t)kThreads * kFastChunks * 8;  // 131072
constexpr int kChunkCap = 2048;                                         // compacted chunk list
constexpr int kFastMaxK = kThreads;                                     // one kept token per thread
constexpr uint32_t kWindow = 4096;                                      // keys tracked below the maximum

// Why a row is handed to the general path (reported in out_flags bits 4-7).
constexpr int kHandPolicy = 1;     // controls out of bounds (the general path reports it)
constexpr int kHandTopK = 2;       // no top-k, or k > 1024, or k >= vocabulary
constexpr int kHandZero = 3;       // a decision boundary sits at +-0
constexpr int kHandCapacity = 4;   // too many chunks reach tau, or tau lies outside the key window
constexpr int kHandOrder = 5;      // bf16 key order may differ from float64 order at a boundary
constexpr int kHandInvalid = 6;    // invalid or fully masked logits (reported in the reference's order)

// Launch modes the host writes into dsr_sample_args_t.hints of the kernel's
// copy of the arguments (the caller's DSR_HINT_* bits are not passed on).
constexpr uint32_t kModeDeferWhole = 1u << 8;  // top-k register kernel: leave whole rows untouched
constexpr uint32_t kModeOnlyWhole = 1u << 9;   // full-vocabulary kernel: decide whole rows only

// A whole row: sampled (0 < T <= 100) without a top-k the register kernel
// takes, so its filters keep the whole vocabulary or a top-k above 1024.  In
// a call that launches both bf16 kernels, the top-k register kernel leaves
// exactly these rows (its kHandTopK hand-over) to the full-vocabulary kernel,
// which decides exactly these rows.
__host__ __device__ __forceinline__ bool whole_row(double T, int top_k, int64_t V) {
  return T > 0.0 && T <= 100.0 && !(top_k >= 1 && top_k <= kFastMaxK && top_k < V);
}

struct FastLists {
  union {
    uint32_t lut[256][4];                  // allow byte -> four 2 x 16-bit "disallowed" masks (pass 1)
    struct {
      uint4 raw[kChunkCap];                // chunks reaching tau (masked bf16 bits), index order
      uint32_t id[kChunkCap];
    } list;
  };
  uint32_t cnt[2][kWindow];                // counts by distance below the maximum key
  long long mass[kWindow];                 // fixed-point mass by distance below the maximum key
  uint16_t kkey[kFastMaxK];                // kept tokens, index order
  uint32_t kidx[kFastMaxK];
  uint32_t wn[kWaves];
  uint32_t polw[24];                       // the row's policy words, then its uniform or PCG64 state
  long long sel_above;
  int sel;
  int bc_i[2];
  double bc_d[2];
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

typedef short dsr_i16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_max_i16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(dsr_i16x2, a),
                                                                __builtin_bit_cast(dsr_i16x2, b)));
}

// Chunk maxima are held as signed 16-bit "levels": level = key - 0x8000, so a
// positive bf16 value's level is its own bit pattern.
__device__ __forceinline__ int chunk_level(const uint32_t* cmx, int j) {
  return (int)(short)(uint16_t)(cmx[j >> 1] >> (16 * (j & 1)));
}

// All-allowed bitmask read in place of a row's allow bits when there are none.
struct AllowAll {
  uint8_t b[kFastMaxVocab / 8];
  constexpr AllowAll() : b() {
    for (int i = 0; i < kFastMaxVocab / 8; ++i) b[i] = 0xFF;
  }
};
__device__ const AllowAll kAllowAll;

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

// Exclusive prefix of one wave-uniform count per wave, and the total.
__device__ __forceinline__ uint32_t wave_offset(uint32_t wn, uint32_t* slot, uint32_t& total) {
  if (lane_id() == 0) slot[wave_id()] = wn;
  lds_barrier();
  const uint32_t y = lane_id() < kWaves ? slot[lane_id()] : 0u;
  const uint32_t incl = row_scan_dpp(y);
  total = lane_value(incl, kWaves - 1);
  return lane_value(incl - y, wave_id());
}

template <class T> struct Bins4;
template <> struct Bins4<uint32_t> {
  static __device__ __forceinline__ void load(const uint32_t* p, uint32_t* c) {
    const uint4 v = *(const uint4*)p;
    c[0] = v.x; c[1] = v.y; c[2] = v.z; c[3] = v.w;
  }
};
template <> struct Bins4<long long> {
  static __device__ __forceinline__ void load(const long long* p, long long* c) {
    const longlong2 a = ((const longlong2*)p)[0], b = ((const longlong2*)p)[1];
    c[0] = a.x; c[1] = a.y; c[2] = b.x; c[3] = b.y;
  }
};

// bins[0..kWindow) hold counts (or fixed-point mass) by distance below the
// maximum key, largest key first.  Returns the first bin where the running
// total reaches `rem` (-1 if the whole window stays below it) and the total
// before that bin.  Thread t takes bins 4t .. 4t+3: one workgroup scan, then
// the thread holding the crossing publishes it.  Every thread calls.
template <class T>
__device__ int select_bin(const T* bins, T rem, FastLists& sh, BlockSync& bs, T& above) {
  const int t = threadIdx.x;
  T c[4];
  Bins4<T>::load(bins + 4 * t, c);
  if (t == 0) sh.sel = -1;  // the scan's barrier orders this before the writes below
  T total;
  T run = bs.scan((c[0] + c[1]) + (c[2] + c[3]), total);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (run < rem && rem <= run + c[j]) {
      sh.sel = 4 * t + j;
      sh.sel_above = (long long)run;
    }
    run += c[j];
  }
  lds_barrier();
  above = (T)sh.sel_above;
  return sh.sel;
}

// Returns 0 if the row was decided here, else the reason it is handed to the
// general path (kHand*).
template <bool RNG>
__device__ __forceinline__ int fast_sample_row(const dsr_sample_args_t& a, int64_t row, FastShared& shu) {
  FastLists& sh = shu.f;
  const int tid = threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int64_t V = a.vocab;
  const uint32_t C = (uint32_t)(V >> 3);
  const uint32_t CW = (C + kWaves - 1) / kWaves;
  BlockSync bs(sh.sync);

  // ---- one HBM pass, every load issued up front in the order it is used,
  // as raw buffer loads (vector memory, so the waits stay in issue order;
  // out-of-range reads return 0): first one word per thread of the policy
  // (threads 0-13) and of the uniform (threads 14-15), parked in LDS by the
  // set-up below (waiting for them never waits for the row), then for each
  // register slot j the chunk's allow byte and its 16 bytes of logits.
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(a.policy + row), (short)0, (int)sizeof(dsr_policy_t), 0x00020000);
  const __amdgpu_buffer_rsrc_t urs = __builtin_amdgcn_make_buffer_rsrc(
      RNG ? (void*)(a.rng_state + 4 * row) : (a.uniforms ? (void*)(a.uniforms + row) : (void*)a.policy),
      (short)0, RNG ? 32 : (a.uniforms ? 8 : 0), 0x00020000);
  constexpr int kPolWords = (int)(sizeof(dsr_policy_t) / 4);
  const uint32_t pw = __builtin_amdgcn_raw_buffer_load_b32(prs, tid < kPolWords ? 4 * tid : 0x7FFFFFF0, 0, 0) |
                      __builtin_amdgcn_raw_buffer_load_b32(
                          urs, (tid >= kPolWords && tid < kPolWords + (RNG ? 8 : 2)) ? 4 * (tid - kPolWords) : 0x7FFFFFF0,
                          0, 0);
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
    const bool mine = cw < CW;  // chunks past this wave's range belong to the next wave: read as 0
    // Non-temporal (cache policy bit 2): each byte is read once.
    mb[j] = __builtin_amdgcn_raw_buffer_load_b8(mrs, (int)(mine ? c : 0x7FFFFFF0u), 0, 2);
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rrs, (int)(mine ? c * 16u : 0x7FFFFFF0u), 0, 2);
    d[j] = make_uint4(v[0], v[1], v[2], v[3]);
  }
  __builtin_amdgcn_sched_barrier(0);
  // While the row streams in: the mask lookup table (allow byte -> per-lane
  // "disallowed" masks) and cleared histograms.
  {
    const uint32_t m = (uint32_t)tid >> 2, q = (uint32_t)tid & 3u;
    sh.lut[m][q] = (((m >> (2 * q)) & 1u) ? 0u : 0x0000FFFFu) | (((m >> (2 * q + 1)) & 1u) ? 0u : 0xFFFF0000u);
    uint4* z = (uint4*)&sh.cnt[0][0];  // 2 x 4096 words of counts
#pragma unroll
    for (int i = 0; i < 2; ++i) z[tid + i * kThreads] = make_uint4(0u, 0u, 0u, 0u);
    uint4* zm = (uint4*)&sh.mass[0];   // 4096 x 8 bytes of mass
#pragma unroll
    for (int i = 0; i < 2; ++i) zm[tid + i * kThreads] = make_uint4(0u, 0u, 0u, 0u);
    if (tid < kPolWords + (RNG ? 8 : 2)) sh.polw[tid] = pw;
  }
  lds_barrier();  // LDS only: the row's loads keep streaming

  // ---- pass 1, chunk by chunk as the loads land.  Disallowed tokens become
  // 0xFFFF (a negative NaN pattern no valid input holds; its key is 0).
  // Chunk maxima are taken as signed 16-bit integers of the bf16 bits, which
  // orders positive values exactly; rows whose top-k reaches zero or below
  // redo the maxima with full keys (below).
  uint32_t vmax_s = 0x80008000u, vmax_u = 0u, cmx[kFastChunks / 2];
  int g[4] = {-32768, -32768, -32768, -32768};
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j) {
    // Keep each chunk's mask lookup next to its use: hoisting all sixteen
    // 16-byte lookups would need 64 more VGPRs than the row leaves free.
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
    g[j >> 2] = max(g[j >> 2], cmj);
  }
  // Pin pass 1 here: without these the compiler sinks it below the policy
  // branches, after every load has landed, and the whole row stays live twice.
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j) asm volatile("" : "+v"(d[j].x), "+v"(d[j].y), "+v"(d[j].z), "+v"(d[j].w));
#pragma unroll
  for (int i = 0; i < kFastChunks / 2; ++i) asm volatile("" : "+v"(cmx[i]));
  asm volatile("" : "+v"(g[0]), "+v"(g[1]), "+v"(g[2]), "+v"(g[3]), "+v"(vmax_s), "+v"(vmax_u));
  const int gmax = max(max(g[0], g[1]), max(g[2], g[3]));
  __builtin_amdgcn_sched_barrier(0);
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
  if (!(T >= 0.0 && T <= 100.0)) return kHandPolicy;
  if (whole_row(T, top_k, V)) return kHandTopK;

  const uint32_t bad = max((int)(short)(vmax_s & 0xFFFFu), (int)(short)(vmax_s >> 16)) >= 0x7F80 ||
                       max(vmax_u & 0xFFFFu, vmax_u >> 16) >= 0xFF81u;
  // One reduction carries the row maximum (as a key) and the NaN/+inf flag.
  const uint32_t red = bs.max((uint32_t)(gmax + 0x8000) | (bad << 16));
  // Invalid logits: the general path reports them after the policy checks,
  // in the reference's order.
  if (red >> 16) return kHandInvalid;
  const uint32_t k = greedy ? 1u : (uint32_t)top_k;
  int Ms = (int)(red & 0xFFFFu) - 0x8000;  // the row maximum's level
  bool full = Ms <= 0;                     // no positive value: signed maxima do not order this row
  int tau = Ms;                            // level every top-k token reaches
  if (!full && !greedy) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t dd = (uint32_t)(Ms - g[q]);
      if (g[q] > 0 && dd < kWindow) atomicAdd(&sh.cnt[0][dd], 1u);
    }
    lds_barrier();
    uint32_t above;
    const int b = select_bin(sh.cnt[0], k, sh, bs, above);
    if (b >= 0) tau = Ms - b; else full = true;  // fewer than k positive group maxima in the window
  }
  if (full) {
    // Rare: redo the maxima with full order keys (level = key - 0x8000).
#pragma unroll
    for (int q = 0; q < 4; ++q) g[q] = -32768;
#pragma unroll
    for (int j = 0; j < kFastChunks; ++j) {
      uint32_t cm = 0u;
      cm = pk_max_u16(cm, bf16x2_keys(d[j].x));
      cm = pk_max_u16(cm, bf16x2_keys(d[j].y));
      cm = pk_max_u16(cm, bf16x2_keys(d[j].z));
      cm = pk_max_u16(cm, bf16x2_keys(d[j].w));
      const int cmj = (int)max(cm & 0xFFFFu, cm >> 16) - 0x8000;
      if (j & 1) cmx[j >> 1] |= (uint32_t)cmj << 16; else cmx[j >> 1] = (uint32_t)cmj & 0xFFFFu;
      g[j >> 2] = max(g[j >> 2], cmj);
    }
    const uint32_t Mk = bs.max((uint32_t)(max(max(g[0], g[1]), max(g[2], g[3])) + 0x8000));
    if (Mk <= kKeyNegInf) return kHandInvalid;  // every token masked: reported by the general path
    if (zero_key(Mk)) return kHandZero;  // +0 and -0 tie in value but not in key
    Ms = (int)Mk - 0x8000;
    tau = Ms;
    if (!greedy) {
      uint4* z = (uint4*)&sh.cnt[0][0];
      z[tid] = make_uint4(0u, 0u, 0u, 0u);
      lds_barrier();
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t dd = (uint32_t)(Ms - g[q]);
        if (g[q] > -32768 && dd < kWindow) atomicAdd(&sh.cnt[0][dd], 1u);
      }
      lds_barrier();
      uint32_t above;
      const int b = select_bin(sh.cnt[0], k, sh, bs, above);
      if (b < 0) return kHandCapacity;
      tau = Ms - b;
    }
  }
  const uint32_t Mkey = (uint32_t)(Ms + 0x8000);

  // ---- compact the chunks whose maximum reaches tau, whole, in index order.
  uint32_t wn = 0;
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j) wn += (uint32_t)__popcll(__ballot(chunk_level(cmx, j) >= tau));
  uint32_t nlist;
  uint32_t lpos = wave_offset(wn, sh.wn, nlist);
  if (nlist > (uint32_t)kChunkCap) return kHandCapacity;  // uniform
#pragma unroll
  for (int j = 0; j < kFastChunks; ++j) {
    const bool q = chunk_level(cmx, j) >= tau;
    const unsigned long long b = __ballot(q);
    if (q) {
      uint32_t p = lpos + lanes_below(b), pi = p;
      // Opaque copy: derived from p * 16, the word index would cost a 64-bit multiply-add.
      asm volatile("" : "+v"(pi));
      sh.list.raw[p] = d[j];
      sh.list.id[pi] = (uint32_t)wave * CW + (uint32_t)j * 64u + (uint32_t)lane;
    }
    lpos += (uint32_t)__popcll(b);
  }
  lds_barrier();

  if (!policy_ok(pol)) return kHandPolicy;

  if (greedy) {  // sampling.py:82-85: the first listed chunk holds the first maximum
    if (tid == 0) {
      const uint4 r4 = sh.list.raw[0];
      const uint4 v = make_uint4(bf16x2_keys(r4.x), bf16x2_keys(r4.y), bf16x2_keys(r4.z), bf16x2_keys(r4.w));
      int e = 0;
      while (e < 7 && key_at(v, e) != Mkey) ++e;
      sh.bc_i[0] = (int)(8u * sh.list.id[0]) + e;
    }
    lds_barrier();
    const int64_t tok = sh.bc_i[0];
    if (a.out_probs_f32 || a.out_probs_f64 || a.out_kept_bits) {
      fast_clear_outputs(a, row);
      if (tid == 0) fast_scatter(a, row, tok, 1.0);
    }
    if (tid == 0) fast_write_result(a, row, DSR_OK, has_draws<RNG>(a) ? tok : -1, 0, 0);
    return 0;
  }

  // ---- exact top-k over the listed tokens (exact-key histogram).  Thread t
  // holds list chunks 2t and 2t+1, so thread order is index order.
  const uint32_t Dtau = (uint32_t)(Ms - tau);
  const bool busy = (uint32_t)wave * 128u < nlist;  // uniform: this wave holds listed chunks
  uint4 lv[2];
  uint32_t lid[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const uint32_t li = 2u * (uint32_t)tid + c;
    const bool ok = li < nlist;
    const uint4 r4 = ok ? sh.list.raw[li] : make_uint4(0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu);
    lv[c] = make_uint4(bf16x2_keys(r4.x), bf16x2_keys(r4.y), bf16x2_keys(r4.z), bf16x2_keys(r4.w));
    lid[c] = ok ? sh.list.id[li] : 0u;
  }
  if (busy) {
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t dd = Mkey - key_at(lv[c], e);
        if (dd <= Dtau) atomicAdd(&sh.cnt[1][dd], 1u);
      }
  }
  lds_barrier();
  uint32_t above_k;
  const int dk_i = select_bin(sh.cnt[1], k, sh, bs, above_k);
  if (dk_i < 0) return kHandCapacity;  // unreachable: the list holds at least k tokens at or above tau
  const uint32_t dk = (uint32_t)dk_i;
  const uint32_t need = k - above_k;  // boundary-key tokens kept, lowest index first
  const uint32_t bkey = Mkey - dk;

  // One scan of (tokens above the boundary, boundary ties) per thread gives
  // every thread its tie rank and the position of its kept tokens.
  uint32_t n_up = 0, n_eq = 0;
  if (busy) {  // waves past the list hold no tokens
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t dd = Mkey - key_at(lv[c], e);
        n_up += dd < dk;
        n_eq += dd == dk;
      }
  }
  uint32_t ptot;
  const uint32_t pex = bs.scan(n_up | (n_eq << 16), ptot);
  if (busy) {
    uint32_t tr = pex >> 16;                        // ties before this thread
    uint32_t kb = (pex & 0xFFFFu) + min(tr, need);  // kept tokens before this thread
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t key = key_at(lv[c], e);
        const uint32_t dd = Mkey - key;
        bool keep = dd < dk;
        if (dd == dk) keep = tr++ < need;
        if (keep && kb < (uint32_t)kFastMaxK) {
          sh.kkey[kb] = (uint16_t)key;
          sh.kidx[kb] = 8u * lid[c] + e;
          ++kb;
        }
      }
  }
  const uint32_t ktot = (ptot & 0xFFFFu) + min(ptot >> 16, need);
  const double M = bf16_key_value(Mkey);
  // Boundary certificate: the bf16 neighbours of the k-th value must stay
  // distinct after (v - max) / T, so key order and the reference's float64
  // order agree on which boundary tokens tie (resolved by index).
  if (wave == 0) {
    const uint32_t nk = bkey - 1u + (uint32_t)lane;
    double s = lane == 0 ? -(double)INFINITY : (double)INFINITY;
    if (lane < 3 && nk > kKeyNegInf && nk < kKeyPosInf) s = (bf16_key_value(nk) - M) / T;
    const double s0 = lane_value(s, 0), s1 = lane_value(s, 1), s2 = lane_value(s, 2);
    if (lane == 0)
      sh.bc_i[0] = ktot == k && (bkey <= kKeyNegInf || (!zero_key(bkey) && s0 < s1 && s1 < s2));
  }
  lds_barrier();
  if (!sh.bc_i[0]) return kHandOrder;

  // ---- one kept token per thread: its unnormalised mass r = exp((v - max) / T)
  // (sampling.py:86-92; the maximum's mass is exactly 1) and min-p, which
  // keeps r >= min_p (:94-96: result < min_p * max(result) with
  // max(result) = 1 / sum).  Masses are summed as exact 64-bit fixed point,
  // fx = floor(r * 2^50) (k <= 1024 masses <= 1 stay below 2^61), so every
  // sum and prefix is order-independent and exact; the rounding this adds
  // (under one unit per token) is part of the decision margins below.
  const bool have = tid < (int)k;
  const uint32_t key = have ? (uint32_t)sh.kkey[tid] : 0u;
  const uint32_t idx = have ? sh.kidx[tid] : 0u;
  const bool fin = have && key > kKeyNegInf;
  double r = 0.0;
  if (fin) r = exp((bf16_key_value(key) - M) / T);
  bool close = false;
  if (pol.min_p != 0.0) {
    close = r > 0.0 && fabs(r - pol.min_p) <= pol.min_p * 0x1p-48;
    if (r < pol.min_p) r = 0.0;
  }
  long long fx = (long long)(r * 0x1p50);
  if (pol.top_p < 1.0 && fx > 0) atomicAdd((unsigned long long*)&sh.mass[Mkey - key], (unsigned long long)fx);
  unsigned flags = 0;
  if (pol.top_p < 1.0) {  // :97-102
    lds_barrier();  // the mass histogram is complete
    // One scan over the mass bins (largest key first) and the kept-token
    // counts per key gives the total S, hence the target P = top_p * S, and
    // each thread can test its own four bins for the first one whose running
    // mass reaches P: the boundary key.  Its thread settles the tie group.
    const int t = threadIdx.x;
    long long cm[4];
    uint32_t cc[4];
    Bins4<long long>::load(sh.mass + 4 * t, cm);
    {
      const uint4 c4 = *(const uint4*)(sh.cnt[1] + 4 * t);
      const uint32_t cw[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t d = 4u * (uint32_t)t + q;
        cc[q] = d < dk ? cw[q] : (d == dk ? need : 0u);  // kept tokens per key
      }
    }
    if (t == 0) sh.sel = -1;  // ordered before the crossing's write by the scan's barrier
    long long S;
    uint32_t cex, ctot;
    long long run = bs.scan2((cm[0] + cm[1]) + (cm[2] + cm[3]), (cc[0] + cc[1]) + (cc[2] + cc[3]), S, cex, ctot);
    const double P = pol.top_p * (double)S;
    long long tgt = (long long)P;
    tgt = tgt < 1 ? 1 : (tgt > S ? S : tgt);  // S >= 2^50: the maximum's mass is exactly 1
    if (run < tgt && tgt <= run + ((cm[0] + cm[1]) + (cm[2] + cm[3]))) {  // the crossing is in this thread's bins
      uint32_t dl = 0, n_tie = 0;
      long long A = 0, n_above = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (run < tgt && tgt <= run + cm[q]) {
          dl = 4u * (uint32_t)t + q;
          A = run;
          n_above = cex;
          n_tie = cc[q];
        }
        run += cm[q];
        cex += cc[q];
      }
      // Tie member i (index order) keeps iff A + i * rt < P (:98-101).  All
      // members carry the same fixed-point mass, so rt is the bin's mass over
      // its count.
      const uint32_t lkey = Mkey - dl;
      const long long rt = (long long)((unsigned long long)sh.mass[dl] / n_tie);
      long long keep = (long long)ceil((P - (double)A) / (double)rt);
      keep = keep < 0 ? 0 : (keep > (long long)n_tie ? (long long)n_tie : keep);
      while (keep > 0 && (double)(A + (keep - 1) * rt) >= P) --keep;
      while (keep < (long long)n_tie && (double)(A + keep * rt) < P) ++keep;
      if (n_above == 0 && keep == 0) keep = 1;  // the first token is never removed
      const double tol = ((double)(n_above + keep) + 16.0) * 0x1p-51 * (double)S + (double)(n_above + n_tie + 2);
      bool near = fabs((double)(A + keep * rt) - P) <= tol;
      if (keep >= 1 && n_above + keep > 1) near = near || fabs((double)(A + (keep - 1) * rt) - P) <= tol;
      if (keep == 0 && n_above > 0) near = true;
      if (keep == (long long)n_tie && (double)(A + (long long)n_tie * rt) < P) near = true;
      // Key order must equal mass order next to the boundary: its bf16
      // neighbours must keep (v - max) / T at least 2^-40 apart, so their
      // masses differ by far more than rounding; ties with +-0 never pass.
      int hand = zero_key(lkey) ? kHandZero : 0;
      for (int side = -1; side <= 1 && !hand; side += 2) {
        const uint32_t nk = lkey + side;
        if (nk <= kKeyNegInf || nk >= kKeyPosInf || zero_key(nk)) continue;
        if (!(fabs(bf16_key_value(nk) - bf16_key_value(lkey)) / T >= 0x1p-40)) hand = kHandOrder;
      }
      sh.sel = (int)lkey;
      sh.bc_i[0] = (int)keep;
      sh.bc_i[1] = hand | (near ? 0x100 : 0) | ((keep > 0 && keep < (long long)n_tie) ? 0x200 : 0);
    }
    lds_barrier();
    if (sh.sel < 0) return kHandCapacity;  // unreachable: the running mass reaches tgt <= S
    const uint32_t lkey = (uint32_t)sh.sel;
    const long long keep = sh.bc_i[0];
    const int info = sh.bc_i[1];
    if (info & 0xFF) return info & 0xFF;
    if (info & 0x100) flags |= DSR_FLAG_MARGIN;
    long long trank = 0;
    if (info & 0x200) {  // a partly kept tie group: ranks by index (thread order)
      uint32_t tt;
      trank = bs.scan((uint32_t)(fx > 0 && key == lkey), tt);
    }
    if (key < lkey || (key == lkey && trank >= keep)) {
      r = 0.0;
      fx = 0;
    }
  }

  // ---- categorical (sampling.py:103-128): the CDF in index order (thread
  // order) as an exact integer scan, the number of positive tokens and the
  // min-p rounding bands.
  const bool pos = r > 0.0;
  long long ctot;
  uint32_t tex, tally;
  const long long ex = bs.scan2(fx, (uint32_t)pos | ((uint32_t)close << 16), ctot, tex, tally);
  const uint32_t npos = tally & 0xFFFFu;
  if (tally >> 16) flags |= DSR_FLAG_MARGIN;
  const bool dense = a.out_probs_f32 || a.out_probs_f64 || a.out_kept_bits;
  if (dense) {
    fast_clear_outputs(a, row);
    if (fin && ctot > 0) fast_scatter(a, row, idx, r / ((double)ctot * 0x1p-50));
  }
  if (ctot <= 0) {
    if (tid == 0) fast_write_result(a, row, DSR_E_NO_MASS, -1, 0, flags);
    return 0;
  }
  if (!has_draws<RNG>(a)) {
    if (tid == 0) fast_write_result(a, row, DSR_OK, -1, 0, flags);
    return 0;
  }
  if (npos == 1) {  // no uniform is drawn (sampling.py:120-122)
    if (pos) fast_write_result(a, row, DSR_OK, idx, 0, flags);
    return 0;
  }
  uint64_t rng_next[4];
  if (RNG) {  // the row's PCG64 state, staged in LDS with the policy words
    uint64_t st4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      st4[i] = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)sh.polw[kPolWords + 2 * i]) |
               ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)sh.polw[kPolWords + 2 * i + 1]) << 32);
    u = pcg64_random(st4, rng_next);
  }
  if (!(u >= 0.0 && u < 1.0)) {
    if (tid == 0) fast_write_result(a, row, DSR_E_UNIFORM, -1, 0, flags);
    return 0;
  }
  // First token whose CDF value exceeds u * total (c_i / c_last > u): with
  // integer CDF values that is the token whose interval [ex, ex + fx) holds
  // floor(u * total).  If rounding leaves u * total at the total, the last
  // positive token (its interval ends at the total).
  const double thr_d = u * (double)ctot;
  long long thr = (long long)thr_d;
  if (thr >= ctot) {
    thr = ctot - 1;
    flags |= DSR_FLAG_MARGIN;
  }
  if (RNG && tid == 0) store_rng(a, row, rng_next);  // the row is decided here
  if (fx > 0 && ex <= thr && thr < ex + fx) {
    const double tol = ((double)npos + 16.0) * 0x1p-51 * (double)ctot + (double)npos + 2.0;
    if ((double)(ex + fx) - thr_d <= tol || (ex > 0 && thr_d - (double)ex <= tol)) flags |= DSR_FLAG_MARGIN;
    fast_write_result(a, row, DSR_OK, idx, 1, flags);
  }
  return 0;
}

}  // namespace dsr
