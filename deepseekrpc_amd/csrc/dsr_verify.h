// Exact sampled speculative verification (SamplingWork.verify -> verify_drafts,
// terminal_sampling.py:170-183, sampling.py:247-294), two paths.
//
// General path: every conditional distribution (targets 0..K, drafts 0..K-1,
// row j conditioned on the prefix draft_ids[:j], terminal_sampling.py:234-244)
// is built in full by general_distribution into a float64 workspace row, one
// workgroup each; one workgroup per request then runs the sequential accept
// chain and draws the replacement or bonus token from those rows.
//
// Fast path, for requests whose policy has no filter (top_k 0 or >= V,
// top_p 1, min_p 0) and that carry no history, bias or allow mask: such a
// distribution is exp((v - M) / T) / s1 followed by a renormalisation that
// only moves it by rounding, so each row is summarised by its maximum M, the
// first index holding it and s1 = sum exp((v - M) / T).  Those come out of
// one pass over the logits (an online maximum / rescaled sum per thread),
// split over kVerifySplit workgroups per row (k_verify_stats) and combined
// at the start of the next kernel (k_verify_chain): kernel boundaries order
// the shares, so no device-scope fence is needed.  The accept chain needs p
// and q only at the draft ids; the one replacement or bonus draw per request
// is spread over kDrawSplit workgroups (slice sums in k_verify_draw, then
// k_verify_finish walks the slice that holds the crossing).  Dropping the renormalisation by total ~ 1 (sampling.py:103-106)
// perturbs each probability by at most a few hundred ulps, so accept tests
// within 2^-40 relative of the uniform are reported with DSR_FLAG_MARGIN.
#pragma once

#include <type_traits>

#include "dsr_general.h"

namespace dsr {

constexpr int kStatThreads = 256;   // statistics workgroups: 4 waves, several resident per CU
constexpr int kStatWaves = kStatThreads / 64;
#ifndef DSR_STAT_PER
#define DSR_STAT_PER 32
#endif
#ifndef DSR_VERIFY_SPLIT
#define DSR_VERIFY_SPLIT 16
#endif
#ifndef DSR_STAT_AUX
#define DSR_STAT_AUX 2  // non-temporal: each logit is read once by this pass
#endif
// 32 logits per thread and 16 shares per row spread each workgroup's set-up
// and reductions over twice the logits of a 16-logit share: 32 requests x 9
// fp32 rows of 129,280 verify in 62.6 us against 66.3 (64 logits and 8
// shares: 62.2; 24 and 24: 67.2; 48 and 11: 64.6).
constexpr int kStatPer = DSR_STAT_PER;        // logits per thread of one share
constexpr int kVerifySplit = DSR_VERIFY_SPLIT;  // shares per distribution row
constexpr int kStatAux = DSR_STAT_AUX;        // cache policy bits of the statistics loads
constexpr int kDrawSplit = 32;   // workgroups per request (replacement / bonus draw)
constexpr int kDrawPer = 16;                         // tokens per lane of a draw workgroup
constexpr int kDrawBlocks = kStatWaves * kDrawPer;   // 64-token blocks per draw workgroup
constexpr int kDrawParts = kDrawSplit * kDrawBlocks;  // block partial sums per request
static_assert((int64_t)kDrawParts * 64 >= DSR_MAX_VOCAB, "the draw blocks cover a row");
constexpr size_t kDecisionBytes = 64;

struct VerifyStat {  // one distribution row, fast path
  double M;          // maximum logit
  double s1;         // sum of exp((v - M) / T)
  int32_t status;
  int32_t amax;      // first index of the maximum
  int32_t pad[2];
};

struct VerifyPart {  // one workgroup's share of a row
  double m, s;
  int32_t amax;
  int32_t flags;     // 1: NaN / +inf seen, 2: a finite value seen
  int32_t pad[2];
};

struct DrawPart {    // one workgroup's share of a draw
  double sum;
  long long npos;
  long long first;
  long long pad;
};

struct VerifyLayout {
  int64_t slots;     // 2K+1 distributions per request: targets 0..K, drafts K+1..2K
  int64_t stride;    // doubles per workspace row
  double* W;         // [rows * slots * stride]
  int32_t* info;     // [rows * slots * 4]: status, onehot, flags, unused
  VerifyStat* stat;  // [rows * slots]
  VerifyPart* part;  // [rows * slots * kVerifySplit]
  DrawPart* dpart;   // [rows * kDrawSplit]
  double* bsum;      // [rows * kDrawParts]: weight sum of each 64-token block of a pending draw
  struct Decision* dec;  // [rows] chain outcome handed to the draw kernels
  int64_t rows;
  int fast_inputs;   // no history, bias or allow mask
  int dists_built;   // k_verify_dists ran before k_verify_chain
};

__host__ __device__ inline size_t verify_ws_bytes(int64_t rows, int32_t K, int64_t V) {
  const size_t slots = (size_t)(2 * K + 1);
  size_t b = (size_t)rows * slots * (size_t)ws_stride(V) * sizeof(double);
  b += (size_t)rows * slots * 4 * sizeof(int32_t);
  b += (size_t)rows * slots * sizeof(VerifyStat);
  b += (size_t)rows * slots * kVerifySplit * sizeof(VerifyPart);
  b += (size_t)rows * kDrawSplit * sizeof(DrawPart);
  b += (size_t)rows * kDrawParts * sizeof(double);
  b += (size_t)rows * kDecisionBytes;
  return b;
}

__host__ inline VerifyLayout verify_layout(void* ws, int64_t rows, int32_t K, int64_t V) {
  VerifyLayout L;
  L.slots = 2 * (int64_t)K + 1;
  L.stride = ws_stride(V);
  char* p = (char*)ws;
  L.W = (double*)p;
  p += (size_t)rows * L.slots * L.stride * sizeof(double);
  L.info = (int32_t*)p;
  p += (size_t)rows * L.slots * 4 * sizeof(int32_t);
  L.stat = (VerifyStat*)p;
  p += (size_t)rows * L.slots * sizeof(VerifyStat);
  L.part = (VerifyPart*)p;
  p += (size_t)rows * L.slots * kVerifySplit * sizeof(VerifyPart);
  L.dpart = (DrawPart*)p;
  p += (size_t)rows * kDrawSplit * sizeof(DrawPart);
  L.bsum = (double*)p;
  p += (size_t)rows * kDrawParts * sizeof(double);
  L.dec = (struct Decision*)p;
  L.rows = rows;
  L.fast_inputs = 0;
  L.dists_built = 1;
  return L;
}

__device__ __forceinline__ size_t dtype_size(int dtype) { return dtype == DSR_BF16 ? 2 : (dtype == DSR_F32 ? 4 : 8); }

// Logits of distribution `slot` of request `row`.
__device__ __forceinline__ const char* verify_logits(const dsr_verify_args_t& a, int64_t row, int slot) {
  const int K = a.K;
  const size_t esz = dtype_size(a.dtype);
  return slot <= K ? (const char*)a.target + ((size_t)row * (K + 1) + slot) * (size_t)a.ld * esz
                   : (const char*)a.draft + ((size_t)row * K + (slot - K - 1)) * (size_t)a.ld * esz;
}

// The policy of request `row` read through the constant address space: the
// index is uniform, so the loads are scalar and waiting for them never waits
// for vector loads in flight.  The policy array is not written by any kernel.
__device__ __forceinline__ dsr_policy_t policy_of(const dsr_verify_args_t& a, int64_t row) {
  typedef const __attribute__((address_space(4))) dsr_policy_t* CP;
  const CP p = (CP)(uintptr_t)a.policy + row;
  dsr_policy_t r;
  r.temperature = p->temperature;
  r.top_p = p->top_p;
  r.min_p = p->min_p;
  r.repetition_penalty = p->repetition_penalty;
  r.presence_penalty = p->presence_penalty;
  r.frequency_penalty = p->frequency_penalty;
  r.top_k = p->top_k;
  r.reserved = p->reserved;
  return r;
}

// Whether request `row` takes the fast path (uniform over its workgroups).
__device__ __forceinline__ bool verify_fast_row(const dsr_verify_args_t& a, const VerifyLayout& L, int64_t row) {
  if (!L.fast_inputs) return false;
  const dsr_policy_t p = policy_of(a, row);
  return policy_ok(p) && (p.top_k == 0 || p.top_k >= a.vocab) && p.top_p >= 1.0 && p.min_p == 0.0;
}

// One request's scalar inputs: draft ids, accept uniforms, EOS ids and the
// output limit, read either from the arguments or from LDS copies.
struct Request {
  const int32_t* ids;   // [K]
  const double* ua;     // [K]
  const int32_t* eos;   // [n_eos]
  int n_eos;
  int limit;
  __device__ __forceinline__ bool is_eos(int32_t t) const {
    for (int e = 0; e < n_eos; ++e)
      if (eos[e] == t) return true;
    return false;
  }
};

template <class A>
__device__ __forceinline__ Request request_of(const A& a, int64_t row) {
  Request q;
  q.ids = a.draft_ids + row * a.K;
  q.ua = a.u_accept + row * a.K;
  q.eos = a.eos_off ? a.eos_ids + a.eos_off[row] : nullptr;
  q.n_eos = a.eos_off ? (int)(a.eos_off[row + 1] - a.eos_off[row]) : 0;
  q.limit = a.output_limit[row];
  return q;
}

// ---------------------------------------------------------------------------
// General path.

// Distribution `slot` of general-path request `row`, built in full into its
// workspace row, its status / one-hot / flags into L.info.
__device__ __forceinline__ void verify_build_dist(const dsr_verify_args_t& a, const VerifyLayout& L, int64_t row, int slot,
                                  GenShared& sh) {
  const int K = a.K;
  const bool is_target = slot <= K;
  const int j = is_target ? slot : slot - (K + 1);
  RowSpec r;
  r.V = a.vocab;
  r.dtype = a.dtype;
  r.logits = verify_logits(a, row, slot);
  r.pol = a.policy[row];
  r.pen_n = 0;
  r.pen_ids = r.pen_count = r.pen_gen = nullptr;
  if (a.pen_off) {
    int64_t o = a.pen_off[row];
    r.pen_n = a.pen_off[row + 1] - o;
    r.pen_ids = a.pen_ids + o;
    r.pen_count = a.pen_count + o;
    r.pen_gen = a.pen_gen + o;
  }
  r.prefix = a.draft_ids + row * K;
  r.prefix_n = j;
  r.bias_n = 0;
  r.bias_ids = nullptr;
  r.bias_val = nullptr;
  if (a.bias_off) {
    int64_t o = a.bias_off[row];
    r.bias_n = a.bias_off[row + 1] - o;
    r.bias_ids = a.bias_ids + o;
    r.bias_val = a.bias_val + o;
  }
  r.allow = a.allow_bits ? a.allow_bits + (row * (K + 1) + j) * a.allow_ld : nullptr;
  r.W = L.W + (row * L.slots + slot) * L.stride;
  r.kept_bits = nullptr;
  r.kept_words = 0;
  r.probs_f32 = nullptr;
  r.probs_f64 = nullptr;
  unsigned flags = 0;
  DistOut d;
  int st = general_distribution(r, sh, flags, d);
  if (threadIdx.x == 0) {
    int32_t* info = L.info + (row * L.slots + slot) * 4;
    info[0] = st;
    info[1] = (int32_t)d.onehot;
    info[2] = (int32_t)flags;
  }
}

// One workgroup per distribution of every general-path request.
__global__ __launch_bounds__(kThreads) void k_verify_dists(dsr_verify_args_t a, VerifyLayout L) {
  __shared__ GenShared sh;
  const int64_t row = blockIdx.x / L.slots;
  const int slot = (int)(blockIdx.x % L.slots);
  if (verify_fast_row(a, L, row)) return;
  verify_build_dist(a, L, row, slot, sh);
}

// Categorical draw over max(p - q, 0) / sum (correction_distribution,
// sampling.py:131-139, then categorical :118-128); q == nullptr draws from p.
struct ProbPair {
  double p, q;
};

__device__ int draw_from(const double* P, const double* Q, int64_t V, double u, GenShared& sh, int64_t& token,
                         int& used, unsigned& flags) {
  double acc = 0.0;
  long long n = 0, f = LLONG_MAX;
  row_pass<ProbPair>(
      V, [&](int64_t i) { return ProbPair{P[i], Q ? Q[i] : 0.0}; },
      [&](int64_t i, ProbPair v) {
        const double x = Q ? fmax(v.p - v.q, 0.0) : v.p;
        acc += x;
        if (x > 0.0) {
          ++n;
          if (i < f) f = i;
        }
      });
  const double total = block_sum(acc, sh.b);
  n = block_sum_i64(n, sh.b);
  f = block_min_i64(f, sh.b);
  if (Q && (!(total > 0.0) || !isfinite(total))) return DSR_E_CORRECTION;
  used = 0;
  if (n == 1) {
    token = f;
    return DSR_OK;
  }
  if (!(u >= 0.0 && u < 1.0)) return DSR_E_UNIFORM;
  used = 1;
  // CDF of the normalised residual, computed on the fly in index order.
  if (Q)
    token = cdf_search_fn(V, [&](int64_t i) { return fmax(P[i] - Q[i], 0.0) / total; }, u, n, sh, flags);
  else
    token = cdf_search_fn(V, [&](int64_t i) { return P[i]; }, u, n, sh, flags);
  return DSR_OK;
}

// The request's decision, shared by the workgroups that produce it.
struct Decision {
  int status, accepted, count, pending, stop, ua, ut, next;
  int draw_j;         // position of the replacement / bonus draw
  unsigned flags;
  int ids[DSR_MAX_DRAFTS + 1];
};
static_assert(sizeof(Decision) == kDecisionBytes, "workspace slot of a decision");

template <class A>
__device__ void write_decision(const A& a, int64_t row, const Decision& d) {
  const int K = a.K;
  int32_t* out_ids = a.out_ids + row * (K + 1);
  const bool ok = d.status == DSR_OK;
  for (int j = 0; j <= K; ++j) out_ids[j] = ok && j < d.count ? d.ids[j] : -1;
  a.out_status[row] = d.status;
  a.out_accepted[row] = ok ? d.accepted : 0;
  a.out_count[row] = ok ? d.count : 0;
  a.out_pending[row] = ok ? d.pending : -1;
  a.out_stop[row] = ok ? d.stop : DSR_STOP_NONE;
  a.out_used_accept[row] = ok ? d.ua : 0;
  a.out_used_target[row] = ok ? d.ut : 0;
  // Device draws: each domain's state moves by exactly the draws reported
  // (an error reports none, as the reference's aborted transaction restores
  // its streams).  This is the decision's last step, so every draw above read
  // the state as it was.
  if (a.rng_accept) pcg64_advance(a.rng_accept + 4 * row, ok ? d.ua : 0);
  if (a.rng_target) pcg64_advance(a.rng_target + 4 * row, ok ? d.ut : 0);
  if (a.out_flags) a.out_flags[row] = (uint8_t)d.flags;
}

// Checks made before the chain, in the reference's order (sampling.py:255-272):
// the output limit, every proposal, the first target, then token ids.
// status_of(slot) gives a distribution's status.
template <class A, class StatusOf>
__device__ void verify_precheck(const A& a, const Request& rq, StatusOf status_of, Decision& d) {
  const int K = a.K;
  const int64_t V = a.vocab;
  d.status = DSR_OK;
  d.accepted = 0;
  d.count = 0;
  d.pending = -1;
  d.stop = DSR_STOP_NONE;
  d.ua = 0;
  d.ut = 0;
  d.next = 0;
  d.draw_j = -1;
  d.flags = 0;
  if (rq.limit < 1 || rq.limit > DSR_MAX_COUNT) d.status = DSR_E_COUNTS;
  for (int j = 0; j < K && d.status == DSR_OK; ++j) d.status = status_of(K + 1 + j);
  if (d.status == DSR_OK) d.status = status_of(0);
  if (d.status == DSR_OK) {
    for (int j = 0; j < K; ++j) {
      const int32_t t = rq.ids[j];
      if (t < 0 || t >= V) d.status = DSR_E_TOKEN;
    }
    for (int e = 0; e < rq.n_eos; ++e)
      if (rq.eos[e] < 0 || rq.eos[e] >= V) d.status = DSR_E_TOKEN;
  }
}

// The sequential accept chain (sampling.py:273-294), run by one thread.
// prob(slot, j) gives distribution `slot`'s probability at draft id j,
// onehot(slot) its greedy argmax, and reach(j) is called as target j is
// reached.  On return d.next is 0 (decided), 1 (replacement draw at
// d.draw_j) or 2 (bonus draw at d.draw_j = K).
template <class A, class StatusOf, class Prob, class Onehot, class Reach>
__device__ void verify_chain(const A& a, const Request& rq, bool greedy, double margin_rel,
                             StatusOf status_of, Prob prob, Onehot onehot, Reach reach, Decision& d) {
  const int K = a.K;
  for (int j = 0; j < K && d.status == DSR_OK; ++j) {
    if (j > 0 && status_of(j) != DSR_OK) {
      d.status = status_of(j);  // the lazily built target j fails only when reached
      break;
    }
    reach(j);
    const int32_t x = rq.ids[j];
    const double q = prob(K + 1 + j, j);
    if (!(q > 0.0)) {
      d.status = DSR_E_PROPOSAL_ZERO;
      break;
    }
    bool ok;
    if (greedy) {
      ok = x == onehot(j);
    } else {
      const double u = rq.ua[j];
      ++d.ua;
      if (!(u >= 0.0 && u < 1.0)) {
        d.status = DSR_E_UNIFORM;
        break;
      }
      double ratio = prob(j, j) / q;
      ratio = ratio < 1.0 ? ratio : 1.0;
      if (fabs(u - ratio) <= margin_rel * ratio) d.flags |= DSR_FLAG_MARGIN;
      ok = u < ratio;
    }
    if (!ok) {
      d.accepted = j;
      d.next = 1;
      d.draw_j = j;
      return;
    }
    d.ids[d.count++] = x;
    if (rq.is_eos(x) || d.count >= rq.limit) {
      d.accepted = j + 1;
      d.stop = rq.is_eos(x) ? DSR_STOP_EOS : DSR_STOP_LENGTH;
      return;  // finished inside the drafts: no bonus
    }
  }
  if (d.status != DSR_OK) return;
  if (K > 0 && status_of(K) != DSR_OK) {
    d.status = status_of(K);
    return;
  }
  reach(K);
  d.next = 2;
  d.draw_j = K;
}

// Appends the replacement / bonus token `rep` and its stop reason.
template <class A>
__device__ __forceinline__ void verify_append(const A& a, const Request& rq, Decision& d, int64_t rep,
                                              int used) {
  d.ut += used;
  if (d.next == 2) d.accepted = a.K;
  const int before = d.count;
  d.ids[d.count++] = (int)rep;
  d.pending = (int)rep;
  d.stop = rq.is_eos((int32_t)rep) ? DSR_STOP_EOS : (before + 1 >= rq.limit ? DSR_STOP_LENGTH : DSR_STOP_NONE);
}

__device__ void general_decide(const dsr_verify_args_t& a, const VerifyLayout& L, int64_t row, GenShared& sh,
                               Decision& d) {
  const int K = a.K;
  const int32_t* info = L.info + row * L.slots * 4;
  auto Prow = [&](int slot) { return L.W + (row * L.slots + slot) * L.stride; };
  auto status_of = [&](int slot) { return (int)info[slot * 4]; };
  const bool greedy = a.policy[row].temperature == 0.0;
  Request rq = request_of(a, row);
  __shared__ double gua[DSR_MAX_DRAFTS];
  if (a.rng_accept) rq.ua = gua;  // the accept domain's next K draws, consumed in order
  if (threadIdx.x == 0) {
    if (a.rng_accept) pcg64_draws(a.rng_accept + 4 * row, K, gua);
    verify_precheck(a, rq, status_of, d);
    for (int j = 0; j < K; ++j) d.flags |= (unsigned)info[(K + 1 + j) * 4 + 2] & DSR_FLAG_MARGIN;
    if (d.status == DSR_OK)
      verify_chain(
          a, rq, greedy, 0x1p-48, status_of, [&](int slot, int j) { return Prow(slot)[rq.ids[j]]; },
          [&](int j) { return (int64_t)info[j * 4 + 1]; },
          [&](int j) { d.flags |= (unsigned)info[j * 4 + 2] & DSR_FLAG_MARGIN; }, d);
  }
  __syncthreads();
  if (d.status == DSR_OK && d.next != 0) {
    const int j = d.draw_j;
    int64_t rep = -1;
    int used = 0;
    int st = DSR_OK;
    unsigned flags = 0;
    if (greedy) {
      rep = info[j * 4 + 1];
    } else {
      double ut = 0.0;
      if (a.rng_target) pcg64_draws(a.rng_target + 4 * row, 1, &ut);
      else ut = a.u_target[row];
      st = draw_from(Prow(j), d.next == 1 ? Prow(K + 1 + j) : nullptr, a.vocab, ut, sh, rep, used, flags);
    }
    if (threadIdx.x == 0) {
      d.flags |= flags;
      if (st != DSR_OK) d.status = st; else verify_append(a, rq, d, rep, used);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) write_decision(a, row, d);
}

// ---------------------------------------------------------------------------
// Fast path.  Kernel boundaries order its steps; no workgroup waits for another.

// bf16 and f32 logits are held as float (exactly), f64 ones as double.
template <int DT> struct LogitT { using T = float; };
template <> struct LogitT<DSR_F64> { using T = double; };

template <int DT>
__device__ __forceinline__ typename LogitT<DT>::T logit_as(const char* base, int64_t i) {
  if constexpr (DT == DSR_BF16) return __uint_as_float((uint32_t)((const uint16_t*)base)[i] << 16);
  else if constexpr (DT == DSR_F32) return ((const float*)base)[i];
  else return ((const double*)base)[i];
}

// Reduction over the kStatWaves waves of a statistics workgroup: DPP inside
// each wave, then every lane combines the per-wave partials in wave order.
// Every call needs its own slot array.
template <class T, class Op>
__device__ __forceinline__ T stat_reduce(T x, T* slot, T id, Op op) {
  x = wave_reduce_dpp(x, op);
  if (lane_id() == 0) slot[wave_id()] = x;
  lds_barrier();  // LDS only: loads in flight for the next share keep streaming
  T y = id;
#pragma unroll
  for (int w = 0; w < kStatWaves; ++w) y = op(y, slot[w]);
  return y;
}

// Share g of a row is [g * seg, (g + 1) * seg) with seg a multiple of 8, so
// every share starts on a 16-byte boundary of an aligned row.
__host__ __device__ inline int64_t stat_segment(int64_t V) {
  return ((V + kVerifySplit - 1) / kVerifySplit + 7) & ~(int64_t)7;
}
static_assert((int64_t)kVerifySplit * kStatThreads * kStatPer >= (((DSR_MAX_VOCAB + kVerifySplit - 1) / kVerifySplit + 7) & ~7) * kVerifySplit,
              "a rounded share must fit in registers");

// Step 1: one share of one row, held in registers: its maximum, the first
// index holding it, sum exp((v - max) / T) and the NaN/+inf / finite flags.
// VEC (rows 16-byte aligned): 16-byte loads, load q of thread t holding
// elements lo + (q * kStatThreads + t) * W .. + W - 1 (W per 16 bytes), so
// each load instruction reads 4 KB in one piece; otherwise element
// lo + t + u * kStatThreads.  Either way a thread's elements increase with
// u, so a strict comparison keeps the first maximum.  Each thread sums its
// exps against its own maximum as soon as its loads land (no workgroup step
// in between) and rescales once by exp((m_t - M) / T).
struct StatShared {
  double etab[64];
  double sf[2][kStatWaves];
  long long si[kStatWaves];
  uint32_t su[kStatWaves];
};

// Share g of distribution rs: [lo, hi) and the index of the u-th element a
// thread holds.  VEC (rows 16-byte aligned): 16-byte loads, load q of thread
// t holding elements lo + (q * kStatThreads + t) * W .. + W - 1 (W per 16
// bytes), so each load instruction reads 4 KB in one piece; otherwise element
// lo + t + u * kStatThreads.  Either way a thread's elements increase with u.
template <int DT, bool VEC>
struct StatItem {
  using X = typename LogitT<DT>::T;
  static constexpr int kElt = DT == DSR_BF16 ? 2 : (int)sizeof(X);
  static constexpr int W = 16 / kElt;
  int64_t rs, lo, hi;
  int64_t row;  // request
  int slot;     // distribution of the request
  int g;
  // 32-bit index arithmetic: the grid holds fewer than 2^32 workgroups.
  __device__ StatItem(const dsr_verify_args_t& a, const VerifyLayout& L, uint32_t item) {
    const uint32_t r = item / kVerifySplit, ns = (uint32_t)L.slots;
    const uint32_t q = r / ns;
    rs = r;
    row = q;
    slot = (int)(r - q * ns);
    g = (int)(item % kVerifySplit);
    const int64_t V = a.vocab, seg = stat_segment(V);
    lo = (int64_t)g * seg < V ? (int64_t)g * seg : V;
    hi = lo + seg < V ? lo + seg : V;
  }
  __device__ __forceinline__ int64_t index_of(int u) const {
    const int t = threadIdx.x;
    if constexpr (VEC) return lo + ((int64_t)(u / W) * kStatThreads + t) * W + (u % W);
    else return lo + t + (int64_t)u * kStatThreads;
  }
  // The raw words of this thread's elements: 16-byte vectors (VEC) or one
  // element per slot at a clamped index; decoded (and masked) by elem().
  static constexpr int kRaw = VEC ? kStatPer / W : kStatPer;
  using Raw = typename std::conditional<VEC, uint4, X>::type;
  // Issues this thread's loads; nothing here waits for them.
  __device__ __forceinline__ void load(const dsr_verify_args_t& a, const VerifyLayout& L, Raw* r) const {
    const char* base = verify_logits(a, row, slot);
    if constexpr (VEC) {
      // The row as a buffer of whole 16-byte vectors (V rounded up to W
      // elements, inside the row since ld is a multiple of W): vectors past
      // it read as 0, and every element at or past hi is masked by mask().
      const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
          (void*)base, (short)0, (int)(((a.vocab + W - 1) / W) * W * kElt), 0x00020000);
#pragma unroll
      for (int q = 0; q < kRaw; ++q) {
        const int64_t e0 = index_of(q * W);
        const auto v =
            __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)(e0 < hi ? e0 * kElt : 0x7FFFFFF0), 0, kStatAux);
        r[q] = make_uint4(v[0], v[1], v[2], v[3]);
      }
    } else {
#pragma unroll
      for (int u = 0; u < kStatPer; ++u) {
        const int64_t i = index_of(u);
        r[u] = logit_as<DT>(base, i < hi ? i : (hi > 0 ? hi - 1 : 0));
      }
    }
  }
  // VEC: elements at or past hi become -inf in the raw words, once, after
  // the loads have landed (a vector is wholly in range except at the end of
  // a share), so elem() needs no index test.
  __device__ __forceinline__ void mask(Raw* r) const {
    if constexpr (VEC) {
#pragma unroll
      for (int q = 0; q < kRaw; ++q) {
        const int64_t e0 = index_of(q * W);
        if (e0 + W <= hi) continue;
        const int n = e0 < hi ? (int)(hi - e0) : 0;  // elements of this vector still in range
        uint32_t w4[4] = {r[q].x, r[q].y, r[q].z, r[q].w};
#pragma unroll
        for (int e = 0; e < W; ++e) {
          if (e < n) continue;
          if constexpr (DT == DSR_BF16) w4[e >> 1] = (w4[e >> 1] & (0xFFFF0000u >> (16 * (e & 1)))) | (0xFF80u << (16 * (e & 1)));
          else if constexpr (DT == DSR_F32) w4[e] = 0xFF800000u;
          else {
            w4[2 * e] = 0u;
            w4[2 * e + 1] = 0xFFF00000u;
          }
        }
        r[q] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
      }
    }
  }
  // Element u in the logits' own type (float for bf16 / f32, exactly):
  // -inf outside [lo, hi) (VEC: after mask()).
  __device__ __forceinline__ X elem(const Raw* r, int u) const {
    if constexpr (VEC) {
      const uint4 v = r[u / W];
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
      const int e = u % W;
      if constexpr (DT == DSR_BF16) return __uint_as_float(((w4[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) << 16);
      else if constexpr (DT == DSR_F32) return __uint_as_float(w4[e]);
      else return __longlong_as_double((long long)(((unsigned long long)w4[2 * e + 1] << 32) | w4[2 * e]));
    } else {
      return index_of(u) < hi ? r[u] : -X(INFINITY);
    }
  }
};

// exp((v - m) * iT) for v <= m (or -inf), as 2^(y / 64) with
// y = (v - m) * iT * 64 / ln 2 clamped at -68,900 (below it the result is
// 0): k = rint(y), 2^(k / 64) = 2^(k >> 6) * 2^((k & 63) / 64) from the
// table, and 2^((y - k) / 64) = exp(r), r = (y - k) ln 2 / 64, |r| <= 0.0055,
// by its degree-4 Taylor polynomial (truncation below 4e-14 relative).  v - m
// is exact for float inputs; the result is within about 1e-13 relative of
// exp, far inside the accept tests' 2^-40 band.  k & 63 indexes the table
// for every input, NaN included.
struct ExpTerm {
  double m, c1;  // c1 = iT * 64 / ln 2
  const double* etab;
  __device__ __forceinline__ double operator()(double v) const {
    constexpr double L = 0x1.62e42fefa39efp-7;  // ln 2 / 64
    constexpr double a2 = L * L / 2, a3 = L * L * L / 6, a4 = L * L * L * L / 24;
    const double y = fmax((v - m) * c1, -68900.0);
    const double kd = rint(y);
    const double f = y - kd;  // exact, |f| <= 1/2
    double p = fma(a4, f, a3);
    p = fma(p, f, a2);
    p = fma(p, f, L);
    p = fma(p, f, 1.0);
    const int k = (int)kd;
    return ldexp(etab[k & 63] * p, k >> 6);
  }
};

// ExpTerm's c1 for temperature T (every user forms it this one way).
__device__ __forceinline__ double exp_scale(double T) { return (1.0 / T) * 92.33248261689366; }

// Order key of a float (increasing with the value; -inf -> 0x007FFFFF).
__device__ __forceinline__ uint32_t float_key(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// One share held in registers -> its maximum, the first index holding it
// (greedy rows only), sum exp((v - max) / T) and the NaN/+inf / finite flags.
// The maximum pass works in the logits' own type: for bf16 / f32 a float
// maximum plus the signed and unsigned maxima of the raw bits, which reveal
// +inf / +NaN (signed >= 0x7F800000) and -NaN (unsigned > 0xFF800000); the
// workgroup then needs one 32-bit key reduction for both.  Each thread sums
// its exps against its own maximum (ExpTerm) as soon as its loads land and
// rescales once by exp((m_t - M) / T).  A -inf element adds exactly 0; a NaN
// or +inf marks the row invalid, whose statistics are then never used.
template <int DT, bool VEC>
__device__ __forceinline__ void stat_share(const dsr_verify_args_t& a, const VerifyLayout& L,
                                           const StatItem<DT, VEC>& it, typename StatItem<DT, VEC>::Raw* x,
                                           StatShared& sm) {
  using X = typename LogitT<DT>::T;
  const double* etab = sm.etab;
  const int64_t row = it.row;
  if (!verify_fast_row(a, L, row)) return;  // uniform over the workgroup
  const double T = policy_of(a, row).temperature;
  const bool greedy = T == 0.0;
  it.mask(x);
  X m = -X(INFINITY);
  double Mg;
  uint32_t flags;
  long long amg = LLONG_MAX;
  double Sg = 0.0;
  if (!greedy && DT != DSR_F64) {
    // Sampled rows: a float maximum (which passes over NaN) and a NaN test;
    // +inf shows as the maximum.
    bool nan = false;
#pragma unroll
    for (int u = 0; u < kStatPer; ++u) {
      const float v = it.elem(x, u);
      nan |= v != v;
      m = fmaxf(m, v);
    }
    const bool bad = nan || m == INFINITY;
    // The key reduction comes before the exp pass: its barrier keeps the
    // compiler from interleaving the two passes (which costs registers).
    const uint32_t K = stat_reduce(bad ? 0xFFFFFFFFu : float_key((float)m), sm.su, 0u, OpMax());
    Mg = K == 0xFFFFFFFFu ? (double)INFINITY : (double)key_float(K);
    flags = (K == 0xFFFFFFFFu ? 1u : 0u) | (K > 0x007FFFFFu && K != 0xFFFFFFFFu ? 2u : 0u);
    const double iT = 1.0 / T;
    const double mm = (double)m > -(double)INFINITY ? (double)m : 0.0;  // no finite value: exact zeros
    const ExpTerm term{mm, exp_scale(T), etab};
    double s = 0.0;
#pragma unroll
    for (int u = 0; u < kStatPer; ++u) s += term((double)it.elem(x, u));
    const double sc = (s > 0.0 && K != 0xFFFFFFFFu) ? s * exp_nonpos(((double)m - Mg) * iT, etab) : 0.0;
    Sg = stat_reduce(sc, sm.sf[1], 0.0, OpSum());
  } else {
    if constexpr (DT == DSR_F64) {
      bool nan = false;
#pragma unroll
      for (int u = 0; u < kStatPer; ++u) {
        const double v = it.elem(x, u);
        nan |= v != v;
        m = fmax(m, v);  // a NaN operand is ignored; the flag covers it
      }
      const uint32_t fl = ((nan || m == (double)INFINITY) ? 1u : 0u) | (m > -(double)INFINITY ? 2u : 0u);
      Mg = stat_reduce(m, sm.sf[0], -(double)INFINITY, OpMax());
      flags = stat_reduce(fl, sm.su, 0u, [](uint32_t p, uint32_t q) { return p | q; });
    } else {
      // Greedy rows: the signed and unsigned maxima of the raw bits reveal
      // +inf / +NaN (signed >= 0x7F800000) and -NaN (unsigned > 0xFF800000).
      int32_t smax = INT_MIN;
      uint32_t umax = 0u;
#pragma unroll
      for (int u = 0; u < kStatPer; ++u) {
        const float v = it.elem(x, u);
        const uint32_t b = __float_as_uint(v);
        smax = max(smax, (int32_t)b);
        umax = max(umax, b);
        m = fmaxf(m, v);
      }
      const bool bad = smax >= 0x7F800000 || umax > 0xFF800000u;
      const uint32_t K = stat_reduce(bad ? 0xFFFFFFFFu : float_key(m), sm.su, 0u, OpMax());
      Mg = K == 0xFFFFFFFFu ? (double)INFINITY : (double)key_float(K);
      flags = (K == 0xFFFFFFFFu ? 1u : 0u) | (K > 0x007FFFFFu && K != 0xFFFFFFFFu ? 2u : 0u);
    }
    if (greedy) {
      // The first index holding the maximum: the thread's first slot equal to
      // its own maximum, then the smallest such index over the threads at Mg.
      int mu = -1;
#pragma unroll
      for (int u = kStatPer - 1; u >= 0; --u)
        if ((double)it.elem(x, u) == (double)m) mu = u;
      amg = stat_reduce((double)m == Mg && mu >= 0 ? it.index_of(mu) : LLONG_MAX, sm.si, LLONG_MAX, OpMin());
    } else {  // f64 logits, sampled
      const double iT = 1.0 / T;
      const double mm = (double)m > -(double)INFINITY ? (double)m : 0.0;
      const ExpTerm term{mm, exp_scale(T), etab};
      double s = 0.0;
#pragma unroll
      for (int u = 0; u < kStatPer; ++u) s += term((double)it.elem(x, u));
      const double sc = s > 0.0 ? s * exp_nonpos(((double)m - Mg) * iT, etab) : 0.0;
      Sg = stat_reduce(sc, sm.sf[1], 0.0, OpSum());
    }
  }
  if (threadIdx.x == 0) {
    VerifyPart p;
    p.m = Mg;
    p.s = Sg;
    p.amax = amg == LLONG_MAX ? -1 : (int32_t)amg;
    p.flags = (int32_t)flags;
    L.part[it.rs * kVerifySplit + it.g] = p;
  }
}

// Step 1, one workgroup per share of every distribution row.
template <int DT, bool VEC>
__global__ __launch_bounds__(kStatThreads) void k_verify_stats(dsr_verify_args_t a, VerifyLayout L) {
  __shared__ StatShared sm;
  using It = StatItem<DT, VEC>;
  const It it(a, L, blockIdx.x);
  typename It::Raw x[It::kRaw];
  it.load(a, L, x);
  exp_table_init(sm.etab);
  lds_barrier();
  stat_share<DT, VEC>(a, L, it, x, sm);
}

// Combines the kVerifySplit shares of one row, in index order; called by
// every lane of one wave (lane q reads share q), result in every lane.
__device__ VerifyStat combine_shares(const VerifyPart* parts, double T, const double* etab) {
  static_assert(kVerifySplit <= 64, "one share per lane");
  const int q = lane_id();
  VerifyPart p;
  p.m = -INFINITY;
  p.s = 0.0;
  p.amax = -1;
  p.flags = 0;
  if (q < kVerifySplit) p = parts[q];
  const uint32_t any = wave_reduce_dpp((uint32_t)p.flags, [](uint32_t u, uint32_t v) { return u | v; });
  const bool f = (p.flags & 2) != 0;
  const double M = wave_reduce_dpp(f ? p.m : -(double)INFINITY, OpMax());
  const double sq = (T != 0.0 && f) ? p.s * exp_nonpos((p.m - M) / T, etab) : 0.0;
  const long long fq = (f && p.m == M) ? (long long)q : LLONG_MAX;
  const long long fw = wave_reduce_dpp(fq, OpMin());
  VerifyStat st;
  st.M = M;
  st.s1 = wave_reduce_dpp(sq, OpSum());
  st.status = (any & 1) ? DSR_E_LOGITS : ((any & 2) ? DSR_OK : DSR_E_MASKED);
  st.amax = fw == LLONG_MAX ? -1 : __shfl(p.amax, (int)fw);
  return st;
}

constexpr int kEosCached = 256;  // EOS ids copied to LDS (longer lists are read in place)

// Step 2, one workgroup per request: general requests run their whole
// decision here; fast ones combine each distribution's shares (one wave per
// distribution), fetch every input of the chain in parallel into LDS, run it
// and hand a pending draw to steps 3-4.
__global__ __launch_bounds__(kThreads) void k_verify_chain(dsr_verify_args_t a, VerifyLayout L) {
  __shared__ GenShared sh;
  __shared__ Decision d;
  __shared__ double etab[64];
  __shared__ VerifyStat sst[2 * DSR_MAX_DRAFTS + 1];
  __shared__ double sprob[2 * DSR_MAX_DRAFTS + 1];
  __shared__ int32_t sids[DSR_MAX_DRAFTS];
  __shared__ double sua[DSR_MAX_DRAFTS];
  __shared__ int32_t seos[kEosCached];
  const int64_t row = blockIdx.x;
  if (!verify_fast_row(a, L, row)) {
    if (!L.dists_built) {  // the call promised every request is fast (DSR_HINT_VERIFY_FAST); this one is not
      if (threadIdx.x == 0) {
        d.status = DSR_E_HINT;
        d.flags = 0;
        write_decision(a, row, d);
      }
      return;
    }
    general_decide(a, L, row, sh, d);
    return;
  }
  const int K = a.K;
  const double T = a.policy[row].temperature;
  const bool greedy = T == 0.0;
  const int slots = (int)L.slots;
  const int t = threadIdx.x;
  exp_table_init(etab);
  __syncthreads();
  if (wave_id() < slots) {
    const int sl = wave_id();
    const VerifyStat v = combine_shares(L.part + (row * L.slots + sl) * kVerifySplit, T, etab);
    if (lane_id() == 0) {
      sst[sl] = v;
      L.stat[row * L.slots + sl] = v;
    }
  }
  __syncthreads();
  if (t < slots) {
    const VerifyStat v = sst[t];
    const int j = t <= K ? t : t - K - 1;
    double pr = 0.0;
    if (j < K) {
      const int32_t x = a.draft_ids[row * K + j];
      if (x >= 0 && x < a.vocab && v.status == DSR_OK) {
        if (greedy) pr = x == v.amax ? 1.0 : 0.0;
        else pr = exp((load_logit(verify_logits(a, row, t), a.dtype, x) - v.M) / T) / v.s1;  // s1: this path's sum
      }
      if (t < K) {
        sids[t] = x;
        if (!a.rng_accept) sua[t] = a.u_accept[row * K + t];
      }
    }
    sprob[t] = pr;
  }
  const int n_eos = a.eos_off ? (int)(a.eos_off[row + 1] - a.eos_off[row]) : 0;
  if (n_eos <= kEosCached && t >= 64 && t < 64 + n_eos) seos[t - 64] = a.eos_ids[a.eos_off[row] + (t - 64)];
  if (a.rng_accept && t == 0) pcg64_draws(a.rng_accept + 4 * row, K, sua);  // the next K accept draws
  __syncthreads();
  if (t == 0) {
    Request rq = request_of(a, row);
    rq.ids = sids;
    rq.ua = sua;
    if (n_eos <= kEosCached) rq.eos = seos;
    auto status_of = [&](int sl) { return (int)sst[sl].status; };
    verify_precheck(a, rq, status_of, d);
    if (d.status == DSR_OK)
      verify_chain(
          a, rq, greedy, 0x1p-40, status_of, [&](int sl, int) { return sprob[sl]; },
          [&](int j) { return (int64_t)sst[j].amax; }, [](int) {}, d);
    if (d.status == DSR_OK && d.next != 0 && greedy) {
      verify_append(a, rq, d, sst[d.draw_j].amax, 0);
      d.next = 0;
    }
    L.dec[row] = d;
    if (d.status != DSR_OK || d.next == 0) write_decision(a, row, d);
  }
}

// The draw's weights at token i: p_j (bonus) or max(p_j - q_j, 0)
// (replacement, correction_distribution, sampling.py:131-139), each
// probability exp((v - M) / T) / s1 by ExpTerm.  The share sums of the draw
// kernel and the token walk of the finish use this same function.
struct DrawWeights {
  const char* P;
  const char* Q;
  int dt;
  bool resid;
  double isp, isq;
  ExpTerm ep, eq;
  __device__ __forceinline__ double weight(double vp, double vq) const {
    const double p = ep(vp) * isp;
    if (!resid) return p;
    return fmax(p - eq(vq) * isq, 0.0);
  }
  __device__ __forceinline__ double operator()(int64_t i) const {
    return weight(load_logit(P, dt, i), resid ? load_logit(Q, dt, i) : 0.0);
  }
};

// From the statistics (M, s1) of the target row at the draw (p) and of the
// matching proposal row (q, read only for a replacement).
__device__ __forceinline__ DrawWeights draw_weights_of(const dsr_verify_args_t& a, int64_t row, const Decision& d,
                                                       double T, double Mp, double sp, double Mq, double sq,
                                                       const double* etab) {
  const int K = a.K;
  const double c1 = exp_scale(T);
  DrawWeights w;
  w.resid = d.next == 1;
  w.P = verify_logits(a, row, d.draw_j);
  w.Q = w.resid ? verify_logits(a, row, K + 1 + d.draw_j) : nullptr;
  w.dt = a.dtype;
  w.isp = 1.0 / sp;
  w.isq = w.resid ? 1.0 / sq : 0.0;
  w.ep = ExpTerm{Mp, c1, etab};
  w.eq = ExpTerm{w.resid ? Mq : 0.0, c1, etab};
  return w;
}

__device__ __forceinline__ DrawWeights draw_weights(const dsr_verify_args_t& a, const VerifyLayout& L, int64_t row,
                                                    const Decision& d, const double* etab) {
  const VerifyStat* st = L.stat + row * L.slots;
  const bool resid = d.next == 1;
  const int jq = a.K + 1 + d.draw_j;
  return draw_weights_of(a, row, d, a.policy[row].temperature, st[d.draw_j].M, st[d.draw_j].s1,
                         resid ? st[jq].M : 0.0, resid ? st[jq].s1 : 1.0, etab);
}

// The 64-token block of share `owner` that holds the crossing of thr: one
// wave scans the share's block sums (one per lane, index order, from base),
// takes the last block with mass starting at or below thr, and walks it.
// margin is set when the decision sits within tol of a boundary or when
// rounding left no crossing (the last positive token is taken).
static_assert(kDrawBlocks == 64, "one block per lane");
template <class WF>
__device__ void block_cdf_search(int64_t V, const double* bsum, int owner, WF wf, double base, double thr,
                                 double tol, int64_t& tok, int& margin) {
  const int l = lane_id();
  const double b = bsum[l];
  const double incl = wave_scan_dpp(b);
  double excl = __shfl_up(incl, 1);
  if (l == 0) excl = 0.0;
  const double start = base + excl;
  const unsigned long long cb = __ballot(b > 0.0 && start <= thr);
  const unsigned long long pb = __ballot(b > 0.0);
  int m = 0, blk;
  if (cb) {
    blk = 63 - __clzll((long long)cb);
  } else {
    blk = pb ? 63 - __clzll((long long)pb) : 0;
    m = 1;
  }
  const double bbase = __shfl(start, blk);
  const int64_t lo = ((int64_t)owner * kDrawBlocks + blk) * 64;
  const int64_t hi = lo + 64 < V ? lo + 64 : V;
  int m2 = 0;
  wave_slice_cdf(wf, lo, hi, bbase, thr, tol, tok, m2);
  margin = m | m2;
}

// The end of a pending draw, run by one wave: combine the kDrawSplit shares
// in index order, then search the share that holds the crossing of
// u * total, and write the decision.  d is the workgroup's LDS copy of the
// request's decision (lane 0 completes it).
__device__ void verify_finish_wave(const dsr_verify_args_t& a, const VerifyLayout& L, int64_t row, Decision& d,
                                   const double* etab) {
  const DrawWeights wf = draw_weights(a, L, row, d, etab);
  // Lane q holds share q; sums and the share prefix come from fixed-order
  // wave reductions and scans.
  static_assert(kDrawSplit <= 64, "one share per lane");
  const int l = lane_id();
  DrawPart pq;
  pq.sum = 0.0;
  pq.npos = 0;
  pq.first = LLONG_MAX;
  if (l < kDrawSplit) pq = L.dpart[row * kDrawSplit + l];
  const double total = wave_reduce_dpp(pq.sum, OpSum());
  const long long n = wave_reduce_dpp(pq.npos, OpSum());
  const long long f = wave_reduce_dpp(pq.npos > 0 ? pq.first : LLONG_MAX, OpMin());
  int64_t rep = -1;
  int used = 0, status = DSR_OK, margin = 0;
  if (wf.resid && (!(total > 0.0) || !isfinite(total))) {
    status = DSR_E_CORRECTION;
  } else if (n == 1) {
    rep = f;  // a single positive token: no uniform is drawn (sampling.py:120-122)
  } else {
    double u = 0.0;
    if (a.rng_target) pcg64_draws(a.rng_target + 4 * row, 1, &u);
    else u = a.u_target[row];
    if (!(u >= 0.0 && u < 1.0)) {
      status = DSR_E_UNIFORM;
    } else {
      used = 1;
      const double thr = u * total;
      // The share holding the crossing: the last one with mass starting at or
      // below thr (else, rounding having left none, the last one with mass).
      const double incl = wave_scan_dpp(pq.sum);
      const double start = incl - pq.sum;
      const unsigned long long cb = __ballot(pq.sum > 0.0 && start <= thr);
      const unsigned long long pb = __ballot(pq.sum > 0.0);
      int owner;
      if (cb) {
        owner = 63 - __clzll((long long)cb);
      } else {
        owner = pb ? 63 - __clzll((long long)pb) : 0;
        margin = 1;
      }
      const double obase = __shfl(start, owner);
      const double tol = ((double)n + 16.0) * 0x1p-51 * total;
      int m2 = 0;
      block_cdf_search(a.vocab, L.bsum + row * kDrawParts + (int64_t)owner * kDrawBlocks, owner, wf, obase, thr, tol,
                       rep, m2);
      margin |= m2;
    }
  }
  if (lane_id() == 0) {
    if (margin) d.flags |= DSR_FLAG_MARGIN;
    if (status != DSR_OK) {
      d.status = status;
    } else {
      Request rq = request_of(a, row);
      verify_append(a, rq, d, rep, used);
    }
    write_decision(a, row, d);
  }
}

// Step 3: share g of a pending draw, 4,096 tokens, 1,024 per wave.  Lane l
// of wave w holds kDrawPer tokens as kDrawPer / W groups of W consecutive
// ones (W = 16 bytes of logits): group q is tokens
// g * 4096 + w * 1024 + (64 q + l) W .. + W - 1, so each load instruction of
// the wave reads 1 KB in one piece.  The 64-token block b of the wave
// (q = b / W) is then held by the LB = 64 / W lanes l with l / LB = b % W:
// each lane sums its W weights in index order, a butterfly over those lanes
// gives the block sum (bitwise the same in each of them), and the block sums
// go to L.bsum for the search.  The share's sum, positive count and first
// positive index go to its DrawPart.  VEC (rows 16-byte aligned): buffer
// loads, past the row reading as 0 and given weight 0.
static_assert(kStatThreads * kDrawPer == kDrawBlocks * 64, "a draw workgroup covers its blocks");
template <int DT, bool VEC>
__global__ __launch_bounds__(kStatThreads) void k_verify_draw(dsr_verify_args_t a, VerifyLayout L) {
  __shared__ double etab[64];
  __shared__ double sf[kStatWaves];
  __shared__ long long si[2][kStatWaves];
  using X = typename LogitT<DT>::T;
  constexpr int kElt = DT == DSR_BF16 ? 2 : (int)sizeof(X);
  constexpr int W = 16 / kElt;       // tokens per 16-byte group
  constexpr int NQ = kDrawPer / W;   // groups per lane
  constexpr int LB = 64 / W;         // lanes per 64-token block
  static_assert(NQ * W == kDrawPer && LB * W == 64, "groups tile the lane's tokens and the blocks");
  const int64_t row = blockIdx.x / kDrawSplit;
  const int g = (int)(blockIdx.x % kDrawSplit);
  const int l = lane_id(), w = wave_id();
  // The decision and the statistics of every distribution of the request
  // (lane s: distribution s) in one round trip; the draw's rows are picked
  // from them once the decision has arrived.
  const bool fast = verify_fast_row(a, L, row);
  const Decision d0 = L.dec[row];
  VerifyStat vs;
  vs.M = 0.0;
  vs.s1 = 1.0;
  if (l < (int)L.slots) vs = L.stat[row * L.slots + l];
  exp_table_init(etab);
  if (!fast || d0.status != DSR_OK || d0.next == 0) return;  // uniform over the workgroup
  __syncthreads();
  const int jq = a.K + 1 + d0.draw_j;
  const DrawWeights wf =
      draw_weights_of(a, row, d0, policy_of(a, row).temperature, __shfl(vs.M, d0.draw_j), __shfl(vs.s1, d0.draw_j),
                      __shfl(vs.M, jq), d0.next == 1 ? __shfl(vs.s1, jq) : 1.0, etab);
  const int64_t V = a.vocab;
  const int64_t wbase = (int64_t)g * (kDrawBlocks * 64) + (int64_t)w * 1024;  // this wave's first token
  auto token = [&](int q, int e) { return wbase + (int64_t)(64 * q + l) * W + e; };
  X pv[kDrawPer], qv[kDrawPer];
  if constexpr (VEC) {
    // Whole 16-byte groups (V rounded up to W elements, inside the row since
    // ld is a multiple of W); elements past V get weight 0 below.
    const int bytes = (int)(((V + W - 1) / W) * W * kElt);
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc((void*)wf.P, (short)0, bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc((void*)(wf.resid ? wf.Q : wf.P), (short)0, bytes, 0x00020000);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int64_t e0 = token(q, 0);
      const int off = e0 < V ? (int)(e0 * kElt) : 0x7FFFFFF0;
      const auto vp = __builtin_amdgcn_raw_buffer_load_b128(rp, off, 0, 0);
      const auto vq = __builtin_amdgcn_raw_buffer_load_b128(rq, wf.resid ? off : 0x7FFFFFF0, 0, 0);
      const uint32_t wp[4] = {vp[0], vp[1], vp[2], vp[3]}, wq[4] = {vq[0], vq[1], vq[2], vq[3]};
#pragma unroll
      for (int e = 0; e < W; ++e) {
        if constexpr (DT == DSR_BF16) {
          pv[q * W + e] = __uint_as_float(((wp[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) << 16);
          qv[q * W + e] = __uint_as_float(((wq[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) << 16);
        } else if constexpr (DT == DSR_F32) {
          pv[q * W + e] = __uint_as_float(wp[e]);
          qv[q * W + e] = __uint_as_float(wq[e]);
        } else {
          pv[q * W + e] = __longlong_as_double((long long)(((unsigned long long)wp[2 * e + 1] << 32) | wp[2 * e]));
          qv[q * W + e] = __longlong_as_double((long long)(((unsigned long long)wq[2 * e + 1] << 32) | wq[2 * e]));
        }
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
#pragma unroll
      for (int e = 0; e < W; ++e) {
        const int64_t i = token(q, e);
        const int64_t ic = i < V ? i : V - 1;  // past the row: any in-range element, weight forced to 0 below
        pv[q * W + e] = logit_as<DT>(wf.P, ic);
        qv[q * W + e] = wf.resid ? logit_as<DT>(wf.Q, ic) : X(0);
      }
    }
  }
  double lane_sum = 0.0;   // this lane's block sums, counted once per block (lanes l % LB == 0)
  long long npos = 0, first = LLONG_MAX;
  double* bs = L.bsum + row * kDrawParts + (int64_t)g * kDrawBlocks + w * 16;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    double part = 0.0;
#pragma unroll
    for (int e = 0; e < W; ++e) {
      const int64_t i = token(q, e);
      const double x = i < V ? wf.weight((double)pv[q * W + e], (double)qv[q * W + e]) : 0.0;
      part += x;
      npos += x > 0.0 ? 1 : 0;
      first = (first == LLONG_MAX && x > 0.0) ? i : first;
    }
    // Block sum over the LB lanes holding the block (unconditional butterfly).
#pragma unroll
    for (int off = 1; off < LB; off <<= 1) part += __shfl_xor(part, off);
    if (l % LB == 0) {
      bs[q * W + l / LB] = part;
      lane_sum += part;
    }
  }
  const double ws = wave_reduce_dpp(lane_sum, OpSum());
  const long long wn = wave_reduce_dpp(npos, OpSum());
  const long long wfst = wave_reduce_dpp(first, OpMin());
  if (l == 0) {
    sf[w] = ws;
    si[0][w] = wn;
    si[1][w] = wfst;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    DrawPart p;
    p.sum = 0.0;
    p.npos = 0;
    p.first = LLONG_MAX;
    for (int q = 0; q < kStatWaves; ++q) {
      p.sum += sf[q];
      p.npos += si[0][q];
      if (si[1][q] < p.first) p.first = si[1][q];
    }
    p.pad = 0;
    L.dpart[row * kDrawSplit + g] = p;
  }
}

// Step 4, one wave per request with a pending draw (after k_verify_draw:
// the kernel boundary orders every share's block sums and part before it).
__global__ __launch_bounds__(64) void k_verify_finish(dsr_verify_args_t a, VerifyLayout L) {
  __shared__ double etab[64];
  __shared__ Decision sd;
  const int64_t row = blockIdx.x;
  if (!verify_fast_row(a, L, row)) return;
  const int status = L.dec[row].status, next = L.dec[row].next;
  if (status != DSR_OK || next == 0) return;
  exp_table_init(etab);
  if (threadIdx.x == 0) sd = L.dec[row];
  __syncthreads();
  verify_finish_wave(a, L, row, sd, etab);
}

}  // namespace dsr
