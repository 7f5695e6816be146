// Shared pieces of the register-resident bf16 kernels (gfx950, wave64, no
// MFMA): order-preserving 16-bit keys of bf16 values, packed 16-bit maxima,
// the reasons a row is handed to the general path, the launch modes of the
// two bf16 kernels, and the result writers.  The top-k kernel is in
// dsr_topk.h, the full-vocabulary kernel in dsr_full.h.
#pragma once

#include "dsr_general.h"
#include "dsr_wave.h"

namespace dsr {

constexpr int kFastChunks = 16;                                         // 16-byte chunks per thread
constexpr int64_t kFastMaxVocab = (int64_t)kThreads * kFastChunks * 8;  // 131072
constexpr int kFastMaxK = kThreads;                                     // largest top-k the register kernel takes

// Why a row is handed to the general path (reported in out_flags bits 4-7).
constexpr int kHandPolicy = 1;     // controls out of bounds (the general path reports it)
constexpr int kHandTopK = 2;       // no top-k, or k > 1024, or k >= vocabulary
constexpr int kHandZero = 3;       // a decision boundary sits at +-0
constexpr int kHandCapacity = 4;   // a top-k reaching zero or below, or a candidate list or key window overflow
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

}  // namespace dsr
