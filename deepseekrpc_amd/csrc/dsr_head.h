// Vocabulary projection with the verifier's row statistics in its epilogue:
// the sampling side of stage_graph.py:356-362 and :396, where the terminal
// stage computes logits = lm_head(norm(hidden)) in FP32, checks
// torch.isfinite(logits).all(), and hands the rows to the sampler, which
// reads every logit again for its maximum and softmax sum.
//
// k_vocab_head: logits[r, v] = sum_k hidden[r, k] * weight[v, k] for bf16
// hidden [rows, dim] and weight [vocab, dim], FP32 accumulation on the matrix
// cores (v_mfma_f32_32x32x16_bf16, A = 32 weight rows, B = 32 hidden rows).
// One workgroup of four waves owns 128 vocabulary columns and every hidden
// row; wave w multiplies its 32 columns (one operand block, loaded straight
// from HBM into registers, four 64-wide dim chunks in flight) by the hidden
// rows, which pass through LDS one 64-wide chunk at a time (double-buffered,
// shared by the four waves, fetched two chunks ahead).  Small register and
// LDS footprints keep two or three workgroups on each CU, so that their
// weight streams and barriers overlap.  At decode sizes the weight stream
// (vocab x dim x 2 bytes, read once) bounds the kernel.
//
// With a record buffer the epilogue also writes, for each (row, 128-column
// tile), a dsr_head_part_t: the tile's maximum, the first column holding it,
// NaN / +inf / -inf / finite flags and sum exp((v - max) / T) by ExpTerm at
// the row's temperature.  These are the verifier fast path's per-row shares
// (k_verify_stats computes the same quantities from the logits), so
// k_head_shares turns them into the verifier's statistics without another
// pass over the logits, and the finiteness check reads the flags.
#pragma once

#include "dsr_verify.h"

namespace dsr {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kHeadThreads = 256;               // four waves
constexpr int kHeadTile = DSR_HEAD_TILE;        // vocabulary columns per workgroup
constexpr int kHeadChunk = 64;                  // dim per LDS stage
constexpr int kHeadDimStep = 4 * kHeadChunk;    // dim is a multiple of this (the main loop's unrolling)
constexpr int kHeadStride = 72;                 // bf16 per staged hidden row: 144 B, rows 36 banks apart
static_assert(DSR_HEAD_MAX_ROWS == 8 * 32, "the dispatch instantiates one to eight 32-row blocks");
static_assert(kHeadTile == 4 * 32, "four waves of 32 columns");

template <int N> using HeadSlot = std::integral_constant<int, N>;

template <int NB, int CB>
union alignas(16) HeadShared {  // 16-byte aligned: the staged rows are read as b128
  __bf16 x[2][NB * 32][kHeadStride];  // hidden chunk, double-buffered
  struct {                            // epilogue, after the last chunk: [tile][wave][row]
    double s[CB][4][NB * 32];         // sum of exp((v - max) / T) over the wave's 32 columns
    float m[CB][4][NB * 32];          // maximum of the wave's 32 columns
    uint32_t f[CB][4][NB * 32];       // flags
    int32_t i[CB][4][NB * 32];        // first column holding the tile maximum
    float tm[CB][NB * 32];            // tile maximum
    uint32_t tf[CB][NB * 32];         // tile flags
  } r;
};

__device__ __forceinline__ double head_temperature(const dsr_head_args_t& a, int64_t row) {
  return a.policy ? a.policy[row / a.rows_per_policy].temperature : 0.0;
}

// One workgroup per CB 128-column tiles; NB = 32-row blocks of hidden rows
// (rows <= 32 NB; rows past `rows` never reach the logits or records).
// Wave w's column block b is columns 128 b + 32 w .. + 31 of the
// workgroup's span, so block b of the four waves is record tile b.
template <int NB, int CB, bool STATS>
__global__ __launch_bounds__(kHeadThreads, CB == 1 && NB <= 5 ? 2 : 1) void k_vocab_head(dsr_head_args_t a) {
  __shared__ HeadShared<NB, CB> sh;
  __shared__ double etab[64];
  __shared__ double temp[STATS ? NB * 32 : 1];  // each row's temperature
  const int t = threadIdx.x, l = t & 63, w = t >> 6, j = l & 31, h = l >> 5;
  const int64_t dim = a.dim, rows = a.rows;
  const int nc = (int)(dim / kHeadChunk);
  const int64_t v0 = (int64_t)blockIdx.x * (kHeadTile * CB);
  const __bf16* X = (const __bf16*)a.hidden;
  // This lane's weight operand row in block b: column v0 + 128 b + 32 w + j,
  // dim offset 8 h.
  const __bf16* wp = (const __bf16*)a.weight + (v0 + 32 * w + j) * dim + 8 * h;
  const int64_t wstep = (int64_t)kHeadTile * dim;

  bf16x8_t wr[4][CB][4];  // weight ring: chunk c in slot c % 4, [column block][16-wide dim step]
  // Hidden chunks in flight to LDS: chunk c in slot c % XL.  Four for the
  // 256-column workgroups with up to five row blocks (then the weight loads
  // of the last four steps stay in flight through each step's wait: 160 rows
  // x dim 5,120 x vocab 129,280 in 309-325 us against 331-368 us with two);
  // two otherwise, where more workgroups per CU share the latency.
  constexpr int XL = CB == 2 && NB <= 5 ? 4 : 2;
  bf16x8_t xr[XL][NB];
  f32x16_t acc[CB][NB];
#pragma unroll
  for (int b = 0; b < CB; ++b)
#pragma unroll
    for (int n = 0; n < NB; ++n) acc[b][n] = f32x16_t{};

  // Every load in the loop is unconditional, so that the compiler's wait
  // counts leave the weight loads of the next chunks in flight: chunk
  // indices past the end are clamped to the last chunk, and hidden rows past
  // `rows` read row rows - 1 (their products land in columns that are never
  // stored).
  auto load_w = [&](auto S, int c) __attribute__((always_inline)) {
    constexpr int s = decltype(S)::value;
    const int64_t off = (int64_t)min(c, nc - 1) * kHeadChunk;
#pragma unroll
    for (int b = 0; b < CB; ++b)
#pragma unroll
      for (int q = 0; q < 4; ++q) wr[s][b][q] = *(const bf16x8_t*)(wp + b * wstep + off + 16 * q);
  };
  // Thread t stages 16 bytes (segment t & 7) of hidden rows (t >> 3) + 32 p.
  auto load_x = [&](auto S, int c) __attribute__((always_inline)) {
    constexpr int s = decltype(S)::value;
    const int64_t off = (int64_t)min(c, nc - 1) * kHeadChunk + 8 * (t & 7);
#pragma unroll
    for (int p = 0; p < NB; ++p) {
      const int64_t r = min((int64_t)(t >> 3) + 32 * p, rows - 1);
      xr[s][p] = *(const bf16x8_t*)(X + r * dim + off);
    }
  };
  auto store_x = [&](auto S, int buf) __attribute__((always_inline)) {
    constexpr int s = decltype(S)::value;
#pragma unroll
    for (int p = 0; p < NB; ++p) *(bf16x8_t*)&sh.x[buf][(t >> 3) + 32 * p][8 * (t & 7)] = xr[s][p];
  };
  // The hidden operands of dim step q + 1 are read from LDS while the
  // products of step q run, so that LDS latency overlaps the matrix cores.
  auto compute = [&](auto S, int buf) __attribute__((always_inline)) {
    constexpr int s = decltype(S)::value;
    bf16x8_t xb[2][NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) xb[0][n] = *(const bf16x8_t*)&sh.x[buf][32 * n + j][8 * h];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q < 3) {
#pragma unroll
        for (int n = 0; n < NB; ++n) xb[(q + 1) & 1][n] = *(const bf16x8_t*)&sh.x[buf][32 * n + j][16 * (q + 1) + 8 * h];
      }
#pragma unroll
      for (int n = 0; n < NB; ++n)
#pragma unroll
        for (int b = 0; b < CB; ++b)
          acc[b][n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wr[s][b][q], xb[q & 1][n], acc[b][n], 0, 0, 0);
    }
    // Schedule: the first step's NB reads, then CB products and one read at
    // a time, so that every operand is read NB reads ahead of its use.
    __builtin_amdgcn_sched_group_barrier(0x100, NB, 0);
#pragma unroll
    for (int i = 0; i < 3 * NB; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, CB, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, CB * NB, 0);
  };
  // Chunk c: fetch hidden chunk c + XL, multiply chunk c, refill this
  // weight slot four chunks ahead, stage hidden chunk c + 1 (fetched XL - 1
  // steps earlier, so that waiting for it leaves the weight loads of the
  // last XL steps in flight).  The barrier ends every reader of buffer c & 1
  // before the next step overwrites it.  nc is a multiple of 4 (dim of 256).
  // The scheduling barriers keep this order of issue: the wait counts depend
  // on it.
  auto step = [&](auto S, int c) __attribute__((always_inline)) {
    constexpr int s = decltype(S)::value;
    load_x(HeadSlot<s % XL>{}, c + XL);
    __builtin_amdgcn_sched_barrier(0);
    compute(S, c & 1);
    __builtin_amdgcn_sched_barrier(0);
    load_w(S, c + 4);
    __builtin_amdgcn_sched_barrier(0);
    store_x(HeadSlot<(s + 1) % XL>{}, (c + 1) & 1);
    __syncthreads();
  };

  // The rows' temperatures first (the epilogue reads them from LDS), then
  // the steady state's order of issue (each hidden chunk before the weight
  // chunk of its step), so that the first steps' waits are the steady ones.
  double tr = 0.0;
  if (STATS && t < NB * 32 && t < rows) tr = head_temperature(a, t);
  if constexpr (XL == 4) {
    load_x(HeadSlot<0>{}, 0);
    load_w(HeadSlot<0>{}, 0);
    load_x(HeadSlot<1>{}, 1);
    load_w(HeadSlot<1>{}, 1);
    load_x(HeadSlot<2>{}, 2);
    load_w(HeadSlot<2>{}, 2);
    load_x(HeadSlot<3>{}, 3);
    load_w(HeadSlot<3>{}, 3);
  } else {
    load_w(HeadSlot<0>{}, 0);
    load_w(HeadSlot<1>{}, 1);
    load_x(HeadSlot<0>{}, 0);
    load_w(HeadSlot<2>{}, 2);
    load_x(HeadSlot<1>{}, 1);
    load_w(HeadSlot<3>{}, 3);
  }
  __builtin_amdgcn_sched_barrier(0);
  store_x(HeadSlot<0>{}, 0);
  if (STATS) {
    exp_table_init(etab);
    if (t < NB * 32) temp[t] = tr;
  }
  __syncthreads();
  for (int c = 0; c < nc; c += 4) {
    step(HeadSlot<0>{}, c);
    step(HeadSlot<1>{}, c + 1);
    step(HeadSlot<2>{}, c + 2);
    step(HeadSlot<3>{}, c + 3);
  }

  // acc[b][n] element e holds column v0 + 128 b + 32 w + 8 (e >> 2) + 4 h +
  // (e & 3) of hidden row 32 n + j.  Each (tile, row block) is copied from
  // the accumulators when it is used, so that only one block's values are
  // live outside them.  With records, three workgroup barriers in all: the
  // lanes' maxima and flags, the tile maxima, the lanes' first maximum column
  // and exp sum, then one thread per (tile, row) writes the record.
  float* out = a.logits;
#pragma unroll
  for (int b = 0; b < CB; ++b)
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      const int r = 32 * n + j;
      float v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = acc[b][n][e];
      if (r < rows) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4_t x4 = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
          *(f32x4_t*)(out + (int64_t)r * a.vocab + v0 + kHeadTile * b + 32 * w + 8 * q + 4 * h) = x4;
        }
      }
      if constexpr (STATS) {
        // Maximum (a float maximum passes over NaN; the flags report it) and flags.
        float m = -INFINITY;
        uint32_t fl = 0u;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float x = v[e];
          const bool nan = x != x;
          fl |= (nan || x == INFINITY) ? 1u : 0u;
          fl |= (!nan && fabsf(x) != INFINITY) ? 2u : 0u;
          fl |= x == -INFINITY ? 4u : 0u;
          m = fmaxf(m, x);
        }
        m = fmaxf(m, __shfl_xor(m, 32));
        fl |= __shfl_xor(fl, 32);
        if (h == 0) {
          sh.r.m[b][w][r] = m;
          sh.r.f[b][w][r] = fl;
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // keeps the next block's copies after this one
    }
  if constexpr (STATS) {
    __syncthreads();
    for (int x = t; x < CB * NB * 32; x += kHeadThreads) {
      const int b = x / (NB * 32), rr = x % (NB * 32);
      sh.r.tm[b][rr] = fmaxf(fmaxf(sh.r.m[b][0][rr], sh.r.m[b][1][rr]), fmaxf(sh.r.m[b][2][rr], sh.r.m[b][3][rr]));
      sh.r.tf[b][rr] = sh.r.f[b][0][rr] | sh.r.f[b][1][rr] | sh.r.f[b][2][rr] | sh.r.f[b][3][rr];
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < CB; ++b)
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const int r = 32 * n + j;
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = acc[b][n][e];
        // First column holding the maximum, and sum exp((v - max) / T).
        const float M = sh.r.tm[b][r];
        int first = INT_MAX;
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (v[e] == M) first = min(first, 32 * w + 8 * (e >> 2) + 4 * h + (e & 3));
        first = min(first, __shfl_xor(first, 32));
        double sum = 0.0;
        const double T = temp[r];  // 0 for rows past `rows`
        if (T > 0.0 && T <= 100.0 && fabsf(M) != INFINITY) {  // sampled rows with a finite maximum
          const ExpTerm term{(double)M, exp_scale(T), etab};
#pragma unroll
          for (int e = 0; e < 16; ++e) sum += term((double)v[e]);
        }
        sum += __shfl_xor(sum, 32);  // both lanes add the same two values
        if (h == 0) {
          sh.r.i[b][w][r] = first;
          sh.r.s[b][w][r] = sum;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    __syncthreads();
    const int64_t tiles = a.vocab / kHeadTile;
    for (int x = t; x < CB * rows; x += kHeadThreads) {
      const int b = x / (int)rows, rr = x % (int)rows;
      const int first = min(min(sh.r.i[b][0][rr], sh.r.i[b][1][rr]), min(sh.r.i[b][2][rr], sh.r.i[b][3][rr]));
      dsr_head_part_t p;
      p.sum = ((sh.r.s[b][0][rr] + sh.r.s[b][1][rr]) + sh.r.s[b][2][rr]) + sh.r.s[b][3][rr];
      p.max = sh.r.tm[b][rr];
      p.info = (int32_t)((sh.r.tf[b][rr] & 7u) | ((uint32_t)(first == INT_MAX ? 0xFFFFFF : first) << 8));
      a.parts[(int64_t)rr * tiles + (int64_t)blockIdx.x * CB + b] = p;
    }
  }
}

// The verifier's statistics from head records: one wave per distribution
// row of a fast request combines the row's tiles (maximum over the tiles
// holding a finite value, their sums rescaled by exp((m_t - M) / T), the
// first column of the maximum, the flags) into share 0 of the row's
// VerifyPart slots; the other shares are left empty, so k_verify_chain's
// combine_shares reads the row as one share.  Target slot j of request r is
// head row r (K + 1) + j of `tp`, draft slot K + 1 + j is row r K + j of `dp`.
__global__ __launch_bounds__(64) void k_head_shares(dsr_verify_args_t a, VerifyLayout L, const dsr_head_part_t* tp,
                                                    const dsr_head_part_t* dp) {
  __shared__ double etab[64];
  const int64_t rs = blockIdx.x;
  const int64_t row = rs / L.slots;
  const int slot = (int)(rs % L.slots);
  const int K = a.K;
  const int64_t tiles = a.vocab / kHeadTile;
  const dsr_head_part_t* src =
      slot <= K ? tp + (row * (K + 1) + slot) * tiles : dp + (row * K + (slot - K - 1)) * tiles;
  const int q = lane_id();
  // Every record first, unconditionally (indices past the row's tiles read
  // its last tile and are masked below), so that the loads, the policy read
  // and the table set-up share one round trip.
  constexpr int kPer = (DSR_MAX_VOCAB / kHeadTile + 63) / 64;
  dsr_head_part_t p[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) p[u] = src[min((int64_t)(q + 64 * u), tiles - 1)];
  exp_table_init(etab);
  __syncthreads();
  if (!verify_fast_row(a, L, row)) return;  // uniform over the wave
  const double T = policy_of(a, row).temperature;
#pragma unroll
  for (int u = 0; u < kPer; ++u)
    if (q + 64 * u >= tiles) p[u].info = 0;  // no flags: left out of every pass
  uint32_t fl = 0u;
  double M = -INFINITY;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    fl |= (uint32_t)p[u].info & 7u;
    if (p[u].info & 2) M = fmax(M, (double)p[u].max);
  }
  fl = wave_reduce_dpp(fl, [](uint32_t x, uint32_t y) { return x | y; });
  M = wave_reduce_dpp(M, OpMax());
  double s = 0.0;
  long long first = LLONG_MAX;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    if (!(p[u].info & 2)) continue;
    if (T != 0.0) s += p[u].sum * exp_nonpos(((double)p[u].max - M) / T, etab);
    if ((double)p[u].max == M)
      first = min(first, (long long)((q + 64 * u) * kHeadTile + ((uint32_t)p[u].info >> 8)));
  }
  s = wave_reduce_dpp(s, OpSum());
  first = wave_reduce_dpp(first, OpMin());
  if (q < kVerifySplit) {
    VerifyPart out;
    out.m = q == 0 ? M : -INFINITY;
    out.s = q == 0 ? s : 0.0;
    out.amax = q == 0 && first != LLONG_MAX ? (int32_t)first : -1;
    out.flags = q == 0 ? (int32_t)(fl & 3u) : 0;
    out.pad[0] = out.pad[1] = 0;
    L.part[rs * kVerifySplit + q] = out;
  }
}

}  // namespace dsr
