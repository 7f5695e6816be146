/*
 * dsr_sampling.h - C ABI of the MI355X (gfx950) token-sampling hot path.
 *
 * The reference sampler (Protonburn35/DeepSeekRPC) is a Python/NumPy API with
 * no native binding: src/deepseekrpc/sampling.py (SamplingPolicy.probabilities
 * :48-106, categorical :118-128, correction_distribution :131-139,
 * verify_drafts :247-294) driven by src/deepseekrpc/terminal_sampling.py
 * (SamplingWork.distribution :127-136, verify :170-183).  Each entry point
 * below replaces one of those functions for rows that already live in device
 * memory; the reference copies them to the host first
 * (terminal_sampling.py:16-27).
 *
 * Conventions (after the reference's native extension, native/operations.cu
 * :12-15,165 and src/deepseekrpc/cuda_ops.py:11-34):
 *   - every pointer is a device pointer owned by the caller;
 *   - kernels are launched on the caller's stream; nothing synchronises;
 *   - the library never allocates: scratch memory is the caller's workspace,
 *     sized by the matching *_workspace_bytes query;
 *   - the return value is 0 or a negative DSR_ERR_* launch/argument error;
 *   - data errors are per-row status codes (DSR_E_*), one per reference
 *     ValidationError, readable with dsr_status_message().
 * Every decision-bearing quantity is computed in float64 with IEEE division
 * and no FMA contraction.  A decision whose threshold lies inside the float64
 * rounding band (where a different exp or summation order may legitimately
 * pick the neighbouring token) is still made, and flagged DSR_FLAG_MARGIN.
 */
#ifndef DSR_SAMPLING_H
#define DSR_SAMPLING_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSR_ABI_VERSION 6
#define DSR_MAX_VOCAB 129280        /* sampling.py:50 */
#define DSR_MAX_COUNT 1048576       /* sampling.py:57 */
#define DSR_MAX_DRAFTS 5            /* sampling.py:255 */
#define DSR_MAX_APPEND 16384        /* new tokens per row in one dsr_history_append call */
#define DSR_STATS_MAX_ROWS 16       /* vectors per dsr_prob_stats_rows call */

/* Logit element types. */
#define DSR_BF16 1
#define DSR_F32 2
#define DSR_F64 3

/* Per-row status codes: 0 or the reference ValidationError it stands for. */
#define DSR_OK 0
#define DSR_E_LOGITS 1          /* sampling.py:50-52: NaN / +inf logit */
#define DSR_E_MASKED 2          /* sampling.py:80-81: every token masked */
#define DSR_E_NO_MASS 3         /* sampling.py:103-105: no positive probability */
#define DSR_E_UNIFORM 4         /* sampling.py:123-125: uniform outside [0,1) */
#define DSR_E_COUNTS 5          /* sampling.py:55-58,62-65: bad history counts */
#define DSR_E_BIAS 6            /* sampling.py:69-74: bad logit bias */
#define DSR_E_PROPOSAL_ZERO 7   /* sampling.py:276-277: q[x] == 0 */
#define DSR_E_CORRECTION 8      /* sampling.py:135-138: empty residual */
#define DSR_E_TOKEN 9           /* sampling.py:271-272: token id out of range */
#define DSR_E_DISTRIBUTION 10   /* sampling.py:109-115: not a distribution */
#define DSR_E_POLICY 11         /* sampling.py:38-43: control outside its bounds */
#define DSR_E_GENERATED 12      /* sampling.py:62-65: generated counts not within counts */
#define DSR_E_HISTORY 13        /* history.py:30-36: token id outside the vocabulary, or a
                                   malformed history table */
#define DSR_E_APPEND 14         /* more than DSR_MAX_APPEND new tokens for one row */
#define DSR_E_HINT 15           /* a verifier request breaks the call's DSR_HINT_VERIFY_FAST */

/* Launch / argument errors (return values). */
#define DSR_ERR_ARG (-1)
#define DSR_ERR_LAUNCH (-2)
#define DSR_ERR_WORKSPACE (-3)

/* Device scratch of dsr_sample_rows_noalloc, in bytes (256 MiB). */
#define DSR_NOALLOC_SCRATCH_BYTES (268435456u)

/* Per-row flags. */
#define DSR_FLAG_MARGIN 1u      /* a threshold decision sat inside the rounding band */
#define DSR_FLAG_GENERAL 2u     /* decided by the general (workspace) path; bits 4-7 give
                                   the reason a row left a faster path */
#define DSR_FLAG_SPLIT 4u       /* decided from per-slice candidates (rows split over several
                                   workgroups: top-k <= 1024, greedy, top-p / min-p whose
                                   kept set lies among the row's 512 largest values, or no
                                   filter with no history or bias) */
#define DSR_FLAG_F32_TOPK 8u    /* decided by the one-workgroup FP32 top-k path (greedy or
                                   1 <= top-k <= 1024, no history or bias) */

/* Kernel-choice hints (dsr_sample_args_t.hints, dsr_verify_args_t.hints):
 * statements about the batch's policies that let the library choose its
 * launches on the host, where the device-resident policies cannot be read.
 * 0 makes no statement.
 *
 * DSR_HINT_WHOLE_SOME: at least one row is sampled (temperature > 0) with
 *   no top-k or a top-k above 1024; in a bf16 batch with no history or bias
 *   such rows then run the full-vocabulary kernel in a second launch instead
 *   of the general path.
 * DSR_HINT_WHOLE_ALL: every row is such a row; that batch runs the
 *   full-vocabulary kernel alone.
 *   The two WHOLE hints change no result: a row that contradicts them is
 *   still decided exactly, by a slower path.
 * DSR_HINT_TOPK_ALL: every row's policy is in bounds and is greedy or has
 *   1 <= top_k <= 1024 below the vocabulary; an FP32 batch with no history
 *   or bias (rows 16-byte aligned, vocab a multiple of 4, at most 131,072)
 *   then runs the one-workgroup FP32 top-k kernel.  Like the WHOLE hints it
 *   changes no result.
 * DSR_HINT_VERIFY_FAST: a promise that every request has a policy with no
 *   filter (top_k 0 or >= vocab, top_p 1, min_p 0) and that the call passes
 *   no history, bias or allow mask, so the launch that builds general-path
 *   distributions is left out.  A request that breaks the promise is not
 *   decided: its status is DSR_E_HINT (the others are unaffected). */
#define DSR_HINT_WHOLE_SOME 1u
#define DSR_HINT_WHOLE_ALL 2u
#define DSR_HINT_VERIFY_FAST 4u
#define DSR_HINT_TOPK_ALL 8u

/* Verifier stop reasons (sampling.py:286,289,294). */
#define DSR_STOP_NONE 0
#define DSR_STOP_EOS 1
#define DSR_STOP_LENGTH 2

/* One row's sampling controls: SamplingPolicy (sampling.py:28-43).  A row
 * whose controls are outside these bounds gets status DSR_E_POLICY. */
typedef struct dsr_policy {
  double temperature;          /* [0, 100]; 0 = greedy argmax */
  double top_p;                /* [0, 1]; 1 = off */
  double min_p;                /* [0, 1]; 0 = off */
  double repetition_penalty;   /* [0.01, 100] */
  double presence_penalty;     /* [-2, 2] */
  double frequency_penalty;    /* [-2, 2] */
  int32_t top_k;               /* [0, 129280]; 0 = off */
  int32_t reserved;            /* must be 0 */
} dsr_policy_t;

/* Arguments of dsr_sample_rows.  Optional pointers may be NULL.
 *
 * History counts are a per-row sparse table in CSR form: row r owns entries
 * [pen_off[r], pen_off[r+1]) of pen_ids / pen_count / pen_gen, with strictly
 * increasing token ids, 1 <= count <= 1048576, 0 <= gen <= count and a row
 * total <= 1048576.  It is exactly the reference's dense `counts` /
 * `generated_counts` pair restricted to counts > 0 (sampling.py:54-66).
 * Logit bias is a second per-row CSR table with strictly increasing ids and
 * values in [-100, 100] (sampling.py:69-74).  allow_bits holds one bit per
 * token, bit (i & 31) of word i >> 5, 1 = allowed (sampling.py:75-79).
 *
 * Draws: a row that needs its uniform (more than one positive probability,
 * sampling.py:120-125) takes uniforms[row], or, when rng_state is set, draws
 * it on the device as Generator.random() of NumPy's PCG64 does from the
 * row's state and writes the advanced state back (rng_state[4r .. 4r+3] =
 * state lo, state hi, increment lo, increment hi: the 128-bit integers of
 * the bit generator's state dict).  A row that needs no draw leaves its state
 * as it was, as the reference's `target` domain stays untouched
 * (sampling.py:120-122; terminal_sampling.py:83-95).  out_consumed reports
 * the draw either way. */
typedef struct dsr_sample_args {
  const void* logits;          /* [rows, ld] of dtype */
  int32_t dtype;               /* DSR_BF16 | DSR_F32 | DSR_F64 */
  uint32_t hints;              /* DSR_HINT_* bits, or 0; other bits: DSR_ERR_ARG */
  int64_t rows;
  int64_t vocab;               /* 1 .. 129280 */
  int64_t ld;                  /* elements between rows, >= vocab */
  const dsr_policy_t* policy;  /* [rows] */
  const int64_t* pen_off;      /* [rows + 1] or NULL (no penalties) */
  const int32_t* pen_ids;
  const int32_t* pen_count;
  const int32_t* pen_gen;
  const int64_t* bias_off;     /* [rows + 1] or NULL (no bias) */
  const int32_t* bias_ids;
  const double* bias_val;
  const uint32_t* allow_bits;  /* [rows, allow_ld] words or NULL */
  int64_t allow_ld;
  const double* uniforms;      /* [rows] pre-drawn u in [0,1), or NULL: no draw */
  int32_t* out_token;          /* [rows] sampled id, -1 on error / no draw */
  uint8_t* out_consumed;       /* [rows] 1 if the draw used its uniform */
  int32_t* out_status;         /* [rows] DSR_OK or DSR_E_* */
  uint8_t* out_flags;          /* [rows] DSR_FLAG_* or NULL */
  float* out_probs_f32;        /* [rows, probs_ld] final probabilities or NULL */
  double* out_probs_f64;       /* [rows, probs_ld] final probabilities or NULL */
  int64_t probs_ld;
  uint32_t* out_kept_bits;     /* [rows, kept_ld] tokens still finite after top-k, or NULL */
  int64_t kept_ld;
  void* workspace;             /* >= dsr_sample_workspace_bytes(rows, vocab) */
  size_t workspace_bytes;
  uint64_t* rng_state;         /* [rows, 4] or NULL; see below */
} dsr_sample_args_t;

/* Arguments of dsr_verify_drafts: the exact sampled speculative verifier for
 * `rows` requests with K drafts each (SamplingWork.verify ->
 * verify_drafts, terminal_sampling.py:170-183, sampling.py:247-294).
 * Target row j and draft row j of a request are both conditioned on the
 * accepted prefix draft_ids[:j] (each prefix token adds one to count and
 * generated count, terminal_sampling.py:127-136) and on allow mask j.
 *
 * Draws: with rng_accept set, the accept test of position j uses the
 * (j+1)-th Generator.random() of the request's accept-domain PCG64 state
 * instead of u_accept; with rng_target set, the replacement / bonus draw
 * uses the next draw of its target-domain state instead of u_target.  Each
 * state is written back advanced by exactly out_used_accept /
 * out_used_target draws (none when the request's status is an error), in the
 * layout of dsr_sample_args_t.rng_state. */
typedef struct dsr_verify_args {
  const void* target;          /* [rows, K+1, ld] logits */
  const void* draft;           /* [rows, K, ld] logits */
  int32_t dtype;
  int32_t K;                   /* 0 .. 5 */
  int64_t rows;
  int64_t vocab;
  int64_t ld;
  const int32_t* draft_ids;    /* [rows, K] */
  const dsr_policy_t* policy;  /* [rows] */
  const int64_t* pen_off;      /* as dsr_sample_args_t, per request */
  const int32_t* pen_ids;
  const int32_t* pen_count;
  const int32_t* pen_gen;
  const int64_t* bias_off;
  const int32_t* bias_ids;
  const double* bias_val;
  const uint32_t* allow_bits;  /* [rows, K+1, allow_ld] or NULL */
  int64_t allow_ld;
  const double* u_accept;      /* [rows, K] */
  const double* u_target;      /* [rows] */
  const int64_t* eos_off;      /* [rows + 1] CSR of EOS ids, or NULL */
  const int32_t* eos_ids;
  const int32_t* output_limit; /* [rows], 1 .. 1048576 */
  int32_t* out_accepted;       /* [rows] accepted drafts */
  int32_t* out_ids;            /* [rows, K+1] output ids, -1 padded */
  int32_t* out_count;          /* [rows] number of output ids */
  int32_t* out_pending;        /* [rows] pending token or -1 */
  int32_t* out_stop;           /* [rows] DSR_STOP_* */
  int32_t* out_used_accept;    /* [rows] accept-domain draws consumed */
  int32_t* out_used_target;    /* [rows] target-domain draws consumed (0/1) */
  int32_t* out_status;         /* [rows] */
  uint8_t* out_flags;          /* [rows] or NULL */
  void* workspace;             /* >= dsr_verify_workspace_bytes(rows, K, vocab) */
  size_t workspace_bytes;
  uint64_t* rng_accept;        /* [rows, 4] PCG64 states of the accept domain, or NULL */
  uint64_t* rng_target;        /* [rows, 4] PCG64 states of the target domain, or NULL */
  uint32_t hints;              /* DSR_HINT_* bits, or 0; other bits: DSR_ERR_ARG */
  uint32_t reserved;           /* must be 0 (else DSR_ERR_ARG) */
} dsr_verify_args_t;

/* Arguments of dsr_verify_probs: verify_drafts (sampling.py:247-294) on
 * float64 probability rows the caller has already built, one request per
 * `rows`, K drafts each.  Row pointers are read on the device: `target` and
 * `draft` are device arrays of device pointers, each to `vocab` float64
 * probabilities (target row j of request r at target[r * (K + 1) + j],
 * draft row j at draft[r * K + j]).  Every row is checked as
 * _distribution checks it (finite, >= 0, NumPy-ordered sum within 1e-10 of
 * 1; sampling.py:109-115), the drafts and target 0 before the chain, target
 * j > 0 when the chain reaches it.  target_status, when set, holds the
 * status of whatever built each target row: a row whose status is not
 * DSR_OK fails with that status when the chain reaches it (its pointer is
 * then never read and may be NULL), as the reference's lazily built targets
 * fail.  Draws and the write-back of rng_accept / rng_target are those of
 * dsr_verify_args_t. */
typedef struct dsr_verify_probs_args {
  const double* const* target; /* device [rows * (K+1)] device row pointers */
  const double* const* draft;  /* device [rows * K] device row pointers (unread when K == 0) */
  const int32_t* target_status;/* [rows, K+1] or NULL (every target row DSR_OK) */
  int32_t K;                   /* 0 .. 5 */
  uint32_t reserved;           /* must be 0 (else DSR_ERR_ARG) */
  int64_t rows;
  int64_t vocab;               /* 1 .. 129280 */
  const int32_t* draft_ids;    /* [rows, K] */
  const uint8_t* greedy;       /* [rows]: nonzero = verify_drafts(greedy=True), or NULL: none */
  const double* u_accept;      /* [rows, K], or NULL with rng_accept */
  const double* u_target;      /* [rows], or NULL with rng_target */
  const int64_t* eos_off;      /* [rows + 1] CSR of EOS ids, or NULL */
  const int32_t* eos_ids;
  const int32_t* output_limit; /* [rows], 1 .. 1048576 */
  int32_t* out_accepted;       /* outputs as dsr_verify_args_t */
  int32_t* out_ids;            /* [rows, K+1] */
  int32_t* out_count;
  int32_t* out_pending;
  int32_t* out_stop;
  int32_t* out_used_accept;
  int32_t* out_used_target;
  int32_t* out_status;
  uint8_t* out_flags;          /* [rows] or NULL */
  void* workspace;             /* >= dsr_verify_probs_workspace_bytes(rows, K), 8-byte aligned */
  size_t workspace_bytes;
  uint64_t* rng_accept;        /* [rows, 4] PCG64 states of the accept domain, or NULL */
  uint64_t* rng_target;        /* [rows, 4] PCG64 states of the target domain, or NULL */
} dsr_verify_probs_args_t;

/* Vocabulary projection (the terminal stage's lm_head, stage_graph.py:356-362
 * and :396).  One record per (row, DSR_HEAD_TILE-column tile) of its FP32
 * logits, written by the projection's epilogue: what the verifier's fast
 * path and the finiteness check (stage_graph.py:361) need from the row. */
#define DSR_HEAD_TILE 128           /* columns per record */
#define DSR_HEAD_MAX_ROWS 256       /* hidden rows per dsr_vocab_head call */

typedef struct dsr_head_part {
  double sum;        /* sum of exp((v - max) / T) over the tile at the row's temperature T;
                        0 for greedy rows (T == 0), T outside (0, 100], or a non-finite max */
  float max;         /* the tile's largest logit (NaN ignored; -inf if none) */
  int32_t info;      /* bit 0: a NaN or +inf logit; bit 1: a finite logit; bit 2: a -inf
                        logit; bits 8-31: the first column of the tile holding max
                        (0xFFFFFF: none) */
} dsr_head_part_t;

typedef struct dsr_head_args {
  const void* hidden;            /* [rows, dim] bf16, row-major, 16-byte aligned */
  const void* weight;            /* [vocab, dim] bf16, row-major, 16-byte aligned */
  int64_t rows;                  /* 0 .. DSR_HEAD_MAX_ROWS */
  int64_t dim;                   /* a positive multiple of 256 */
  int64_t vocab;                 /* a positive multiple of DSR_HEAD_TILE, <= DSR_MAX_VOCAB */
  const dsr_policy_t* policy;    /* or NULL: row r's temperature is
                                    policy[r / rows_per_policy].temperature */
  int32_t rows_per_policy;       /* >= 1 when policy is set */
  int32_t reserved;              /* must be 0 */
  float* logits;                 /* [rows, vocab] out, 16-byte aligned */
  dsr_head_part_t* parts;        /* [rows, vocab / DSR_HEAD_TILE] out, 8-byte aligned,
                                    or NULL: logits only */
} dsr_head_args_t;

/* ABI gate, after the reference's abi_version() (native/bindings.cpp:25). */
int32_t dsr_abi_version(void);

/* Message of a DSR_E_* status code (the reference's ValidationError text). */
const char* dsr_status_message(int32_t code);

/* Workspace queries. */
size_t dsr_sample_workspace_bytes(int64_t rows, int64_t vocab);
size_t dsr_verify_workspace_bytes(int64_t rows, int32_t K, int64_t vocab);
size_t dsr_verify_probs_workspace_bytes(int64_t rows, int32_t K);

/* Fused penalties -> temperature -> top-k -> softmax -> min-p -> top-p ->
 * categorical draw for `rows` independent rows.
 * Replaces SamplingPolicy.probabilities + categorical (sampling.py:48-128),
 * as called by TerminalSampler.begin_seed (terminal_sampling.py:83-95). */
int32_t dsr_sample_rows(const dsr_sample_args_t* args, void* stream);

/* Allocation-free dsr_sample_rows.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).
 * Arguments as dsr_sample_rows, except that workspace and workspace_bytes
 * must be 0: the workspace is a device array of DSR_NOALLOC_SCRATCH_BYTES
 * inside the library, one per device, allocated when the library's code is
 * loaded on that device and held until the process ends.  Every process
 * that uses the library on a device holds that 256 MiB there, whether or not
 * it calls this entry point.  The call uses the current
 * device's array (the stream must belong to the current device) and calls
 * no allocating routine.  A call needing more than the array, that is
 * dsr_sample_workspace_bytes(rows, vocab) > DSR_NOALLOC_SCRATCH_BYTES (more
 * than 259 rows at vocab 129,280), returns DSR_ERR_WORKSPACE and launches
 * nothing.
 * The kernels need no cleared workspace.  Calls on one device share its
 * array: calls whose work overlaps on that device (two streams, or two host
 * threads) race and must be ordered by the caller. */
int32_t dsr_sample_rows_noalloc(const dsr_sample_args_t* args, void* stream);

/* Exact sampled verifier; replaces SamplingWork.verify (terminal_sampling.py
 * :170-183) with verify_drafts (sampling.py:247-294) and the lazy
 * conditional targets (terminal_sampling.py:234-244). */
int32_t dsr_verify_drafts(const dsr_verify_args_t* args, void* stream);

/* Vocabulary projection: logits = hidden . weight^T with FP32 accumulation,
 * and with `parts` the per-tile records above.  Replaces the terminal
 * stage's logits_processor(lm_head, norm(hidden)) and its
 * torch.isfinite(logits).all() (stage_graph.py:356-362, and :396 for the
 * draft rows); a row's logits are finite exactly when none of its records
 * has info bit 0 or 2. */
int32_t dsr_vocab_head(const dsr_head_args_t* args, void* stream);

/* dsr_sample_rows on FP32 logits written by dsr_vocab_head, with that call's
 * records (`parts`, [rows, vocab / DSR_HEAD_TILE]): rows that the one-
 * workgroup FP32 top-k path takes (DSR_HINT_TOPK_ALL, no history or bias
 * table) and that carry no allow mask start from the records' per-tile
 * maxima instead of a pass over the row, and read again only the tiles whose
 * maximum reaches the k-th largest tile maximum (at most 256 tiles; more,
 * or fewer finite tiles than k, and the row takes the full pass).  Results
 * are dsr_sample_rows'; other batches are dsr_sample_rows itself.  The
 * records must be those of these logits (the projection's own output). */
int32_t dsr_sample_rows_head(const dsr_sample_args_t* args, const dsr_head_part_t* parts, void* stream);

/* dsr_verify_drafts for FP32 logits written by dsr_vocab_head together with
 * their records: the verifier's per-row statistics come from the records
 * instead of a pass over the logits.  target_parts holds the records of the
 * args->rows * (K + 1) target rows, draft_parts those of the rows * K draft
 * rows (NULL when K == 0), each computed with rows_per_policy = K + 1 (resp.
 * K) over args->policy.  Requires dtype DSR_F32, ld == vocab and vocab a
 * multiple of DSR_HEAD_TILE.  Same results and workspace as
 * dsr_verify_drafts. */
int32_t dsr_verify_drafts_head(const dsr_verify_args_t* args, const dsr_head_part_t* target_parts,
                               const dsr_head_part_t* draft_parts, void* stream);

/* Exact sampled verifier over float64 rows already on the device; replaces
 * verify_drafts (sampling.py:247-294) as SamplingWork.verify calls it
 * (terminal_sampling.py:170-183) with target rows it has built.  Four
 * launches: every row's statistics (one workgroup per 8,192 entries), the
 * chain (one wave per request), the sums of a pending replacement or bonus
 * draw (one workgroup per 8,192 entries) and the draw itself. */
int32_t dsr_verify_probs(const dsr_verify_probs_args_t* args, void* stream);

/* Probability-vector kernels behind the drop-in categorical /
 * correction_distribution / verify_drafts on float64 distributions.
 * Each works on one vector p[n] (n <= 129280) and writes a small result.
 *
 * dsr_prob_stats (sampling.py:109-115,120-122): out_sum[0] = sum of p,
 *   out_i32[0] = 1 if every entry is finite and >= 0, out_i32[1] = number of
 *   positive entries, out_i32[2] = first positive index, out_i32[3] = first
 *   index of the maximum (np.argmax). */
int32_t dsr_prob_stats(const double* p, int64_t n, double* out_sum, int32_t* out_i32, void* stream);

/* dsr_prob_stats of `count` <= DSR_STATS_MAX_ROWS float64 vectors of length n
 * in one launch (one workgroup each), for the verifier's rows
 * (sampling.py:109-115 applied to every target and proposal row).  `rows`
 * is a host array of `count` device pointers; `out` is a device float64
 * array [count, 3]: row r's sum at out[3 r], then its four int32 results
 * (as dsr_prob_stats's out_i32) in the next 16 bytes. */
int32_t dsr_prob_stats_rows(const double* const* rows, int32_t count, int64_t n, double* out, void* stream);

/* dsr_prob_categorical (sampling.py:126-128): first i with
 * cumsum(p)[i] / sum(p) > u.  out_i32[0] = token, out_i32[1] = flags. */
int32_t dsr_prob_categorical(const double* p, int64_t n, double u, int32_t* out_i32, void* stream);

/* dsr_prob_correction (sampling.py:131-139): out = max(p - q, 0) / sum;
 * out_i32[0] = status (DSR_OK or DSR_E_CORRECTION). */
int32_t dsr_prob_correction(const double* p, const double* q, int64_t n, double* out, int32_t* out_i32,
                            void* stream);

/* dsr_prob_accept (sampling.py:276-281): out_i32[0] = 1 if q[x] > 0,
 * out_i32[1] = 1 if u < min(1, p[x] / q[x]). */
int32_t dsr_prob_accept(const double* p, const double* q, int64_t n, int32_t x, double u, int32_t* out_i32,
                        void* stream);

/* The terminal window check np.isfinite(logits).all() (terminal_sampling.py
 * :25) on the device: out[r] is set to 0 when one of the n FP32 values of
 * row r (x + r * ld) is NaN or +-inf, and left as it is otherwise, so the
 * caller sets out[0 .. rows-1] to 1 first (in the same stream order).  Each
 * row is spread over workgroups of 4,096 values; nothing is read back, so
 * a caller can read the flags with its next synchronisation. */
int32_t dsr_rows_finite(const float* x, int64_t rows, int64_t n, int64_t ld, int32_t* out, void* stream);

/* Host-side scan of a terminal count vector (no device work), in one
 * read-only pass: the checks of terminal_sampling.py:58-61 (no entry
 * negative, the int64 sum).  `width` is the entry size (4 or 8);
 * `support` (room for n) receives the indices of the positive entries,
 * ascending; out3 = {positive entries, their int64 sum (wrapping as NumPy's
 * does), the largest entry}.  The caller keeps the positive entries as its
 * frozen copy of the vector (:77-79).  Returns 0, 1 when an entry is
 * negative (the other outputs are then meaningless), or DSR_ERR_ARG. */
int32_t dsr_count_scan(const void* counts, int32_t width, int64_t n, int64_t* support, int64_t* out3);

/* Device history tables: the reference's dense per-request counts and
 * generated counts (history.py:46-47,92,136-137; terminal_sampling.py
 * :127-136) kept on the device as the sparse CSR table of
 * dsr_sample_args_t (pen_off / pen_ids / pen_count / pen_gen).
 *
 * Both calls write out_off[rows + 1] (row r owns entries [out_off[r],
 * out_off[r+1]) of out_ids / out_count / out_gen) and a status per row; a
 * row with a nonzero status gets no entries.  out_off[rows] is the total the
 * call needs: if it exceeds cap, no entries are written at all (the offsets
 * and statuses still are), and the caller may repeat the call with larger
 * outputs.  Three launches each; nothing allocates or synchronises.  With
 * rows == 0 only out_off[0] = 0 is written and the input pointers may be
 * NULL.
 *
 * dsr_history_from_dense: dense counts [rows, ld] and generated counts
 * [rows, ld] (NULL: generated = counts) -> their entries with counts > 0, in
 * id order.  Validation and statuses as SamplingPolicy.probabilities does
 * it (sampling.py:54-58 then :62-65): DSR_E_COUNTS for a count outside
 * [0, 1048576] or a row total above 1048576, else DSR_E_GENERATED for a
 * generated count outside [0, count].  Replaces the dense `counts` /
 * `generated_counts` hand-over of stage_service.py:252-263. */
int32_t dsr_history_from_dense(const int32_t* counts, const int32_t* generated, int64_t rows, int64_t vocab,
                               int64_t ld, int64_t* out_off, int32_t* out_ids, int32_t* out_count,
                               int32_t* out_gen, int64_t cap, int32_t* out_status, void* stream);

/* dsr_history_append: table (off / ids / count / gen as in
 * dsr_sample_args_t; off NULL = every row empty) plus the tokens
 * tokens[tok_off[r] .. tok_off[r+1]) of each row -> the merged table.  Each
 * token adds one to its id's count (np.add.at, history.py:136-137), and one
 * to its generated count when its position within the row's tokens is at
 * least gen_from[r] (gen_from NULL: every token is generated, as for an
 * appended output token or the tentative prefix of
 * terminal_sampling.py:129-133; gen_from[r] = the row's token count: prompt
 * tokens only, as TokenHistory.set_prompt counts them, history.py:92).
 * Statuses: DSR_E_APPEND for more than DSR_MAX_APPEND tokens in a row,
 * DSR_E_HISTORY for a token outside [0, vocab) or an input row that is not
 * a valid table row (ids strictly increasing in [0, vocab), 1 <= count <=
 * 1048576, 0 <= gen <= count). */
int32_t dsr_history_append(const int64_t* off, const int32_t* ids, const int32_t* count, const int32_t* gen,
                           const int32_t* tokens, const int64_t* tok_off, const int64_t* gen_from, int64_t rows,
                           int64_t vocab, int64_t* out_off, int32_t* out_ids, int32_t* out_count, int32_t* out_gen,
                           int64_t cap, int32_t* out_status, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSR_SAMPLING_H */
