"""ctypes binding of ``libdsr_sampling.so`` (declared in include/dsr_sampling.h).

The library is built in-tree by ``deepseekrpc_amd.build`` and is loaded from
next to this file.  There is no fallback: if the library is missing, or its
ABI version differs, every device entry point raises.  This mirrors the
reference's ABI gate (src/deepseekrpc/cuda_ops.py:11-20).
"""
from __future__ import annotations

import ctypes
import os

ABI_VERSION = 6
LIB_NAME = "libdsr_sampling.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

BF16, F32, F64 = 1, 2, 3

OK = 0
E_LOGITS = 1
E_MASKED = 2
E_NO_MASS = 3
E_UNIFORM = 4
E_COUNTS = 5
E_BIAS = 6
E_PROPOSAL_ZERO = 7
E_CORRECTION = 8
E_TOKEN = 9
E_DISTRIBUTION = 10
E_POLICY = 11
E_GENERATED = 12
E_HISTORY = 13
E_APPEND = 14
E_HINT = 15
MAX_APPEND = 16384
MAX_VOCAB = 129280

FLAG_MARGIN = 1
FLAG_GENERAL = 2
FLAG_SPLIT = 4
FLAG_F32_TOPK = 8
# Kernel-choice hints (statements about a batch's policies; results never depend on them).
HINT_WHOLE_SOME = 1
HINT_WHOLE_ALL = 2
HINT_VERIFY_FAST = 4
HINT_TOPK_ALL = 8
STOP_NONE, STOP_EOS, STOP_LENGTH = 0, 1, 2

EXPORTS = (
    "dsr_abi_version", "dsr_status_message", "dsr_sample_workspace_bytes", "dsr_verify_workspace_bytes",
    "dsr_sample_rows", "dsr_verify_drafts", "dsr_prob_stats", "dsr_prob_categorical", "dsr_prob_correction",
    "dsr_prob_accept", "dsr_history_from_dense", "dsr_history_append", "dsr_sample_rows_noalloc",
    "dsr_vocab_head", "dsr_verify_drafts_head", "dsr_prob_stats_rows", "dsr_verify_probs_workspace_bytes",
    "dsr_verify_probs", "dsr_rows_finite", "dsr_count_scan", "dsr_sample_rows_head",
)
NOALLOC_SCRATCH_BYTES = 268435456
HEAD_TILE = 128
STATS_MAX_ROWS = 16
HEAD_MAX_ROWS = 256

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f64 = ctypes.c_double


class Policy(ctypes.Structure):
    """``dsr_policy_t``: one row's SamplingPolicy (sampling.py:28-43)."""
    _fields_ = [("temperature", _f64), ("top_p", _f64), ("min_p", _f64), ("repetition_penalty", _f64),
                ("presence_penalty", _f64), ("frequency_penalty", _f64), ("top_k", _i32), ("reserved", _i32)]


POLICY_DTYPE_FIELDS = [(name, "<f8") for name, _ in Policy._fields_[:6]] + [("top_k", "<i4"), ("reserved", "<i4")]


class SampleArgs(ctypes.Structure):
    _fields_ = [
        ("logits", _p), ("dtype", _i32), ("hints", ctypes.c_uint32), ("rows", _i64), ("vocab", _i64), ("ld", _i64),
        ("policy", _p), ("pen_off", _p), ("pen_ids", _p), ("pen_count", _p), ("pen_gen", _p),
        ("bias_off", _p), ("bias_ids", _p), ("bias_val", _p), ("allow_bits", _p), ("allow_ld", _i64),
        ("uniforms", _p), ("out_token", _p), ("out_consumed", _p), ("out_status", _p), ("out_flags", _p),
        ("out_probs_f32", _p), ("out_probs_f64", _p), ("probs_ld", _i64), ("out_kept_bits", _p), ("kept_ld", _i64),
        ("workspace", _p), ("workspace_bytes", ctypes.c_size_t), ("rng_state", _p),
    ]


class VerifyArgs(ctypes.Structure):
    _fields_ = [
        ("target", _p), ("draft", _p), ("dtype", _i32), ("K", _i32), ("rows", _i64), ("vocab", _i64), ("ld", _i64),
        ("draft_ids", _p), ("policy", _p), ("pen_off", _p), ("pen_ids", _p), ("pen_count", _p), ("pen_gen", _p),
        ("bias_off", _p), ("bias_ids", _p), ("bias_val", _p), ("allow_bits", _p), ("allow_ld", _i64),
        ("u_accept", _p), ("u_target", _p), ("eos_off", _p), ("eos_ids", _p), ("output_limit", _p),
        ("out_accepted", _p), ("out_ids", _p), ("out_count", _p), ("out_pending", _p), ("out_stop", _p),
        ("out_used_accept", _p), ("out_used_target", _p), ("out_status", _p), ("out_flags", _p),
        ("workspace", _p), ("workspace_bytes", ctypes.c_size_t), ("rng_accept", _p), ("rng_target", _p),
        ("hints", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
    ]


class VerifyProbsArgs(ctypes.Structure):
    _fields_ = [
        ("target", _p), ("draft", _p), ("target_status", _p), ("K", _i32), ("reserved", ctypes.c_uint32),
        ("rows", _i64), ("vocab", _i64), ("draft_ids", _p), ("greedy", _p), ("u_accept", _p), ("u_target", _p),
        ("eos_off", _p), ("eos_ids", _p), ("output_limit", _p),
        ("out_accepted", _p), ("out_ids", _p), ("out_count", _p), ("out_pending", _p), ("out_stop", _p),
        ("out_used_accept", _p), ("out_used_target", _p), ("out_status", _p), ("out_flags", _p),
        ("workspace", _p), ("workspace_bytes", ctypes.c_size_t), ("rng_accept", _p), ("rng_target", _p),
    ]


class HeadPart(ctypes.Structure):
    """``dsr_head_part_t``: one (row, 128-column tile) record of a vocabulary projection."""
    _fields_ = [("sum", _f64), ("max", ctypes.c_float), ("info", _i32)]


class HeadArgs(ctypes.Structure):
    _fields_ = [
        ("hidden", _p), ("weight", _p), ("rows", _i64), ("dim", _i64), ("vocab", _i64), ("policy", _p),
        ("rows_per_policy", _i32), ("reserved", _i32), ("logits", _p), ("parts", _p),
    ]


class NativeUnavailable(RuntimeError):
    """The HIP library is missing or incompatible; there is no CPU fallback."""


_lib = None


def load(path: str = LIB_PATH):
    """Load and ABI-check the library (cached)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise NativeUnavailable(f"{LIB_NAME} is not built; run deepseekrpc_amd.build.build() (hipcc, gfx950)")
    lib = ctypes.CDLL(path)
    lib.dsr_abi_version.restype = _i32
    lib.dsr_abi_version.argtypes = []
    if lib.dsr_abi_version() != ABI_VERSION:
        raise NativeUnavailable("libdsr_sampling ABI version mismatch")
    lib.dsr_status_message.restype = ctypes.c_char_p
    lib.dsr_status_message.argtypes = [_i32]
    lib.dsr_sample_workspace_bytes.restype = ctypes.c_size_t
    lib.dsr_sample_workspace_bytes.argtypes = [_i64, _i64]
    lib.dsr_verify_workspace_bytes.restype = ctypes.c_size_t
    lib.dsr_verify_workspace_bytes.argtypes = [_i64, _i32, _i64]
    lib.dsr_sample_rows.restype = _i32
    lib.dsr_sample_rows.argtypes = [ctypes.POINTER(SampleArgs), _p]
    lib.dsr_sample_rows_noalloc.restype = _i32
    lib.dsr_sample_rows_noalloc.argtypes = [ctypes.POINTER(SampleArgs), _p]
    lib.dsr_verify_drafts.restype = _i32
    lib.dsr_verify_drafts.argtypes = [ctypes.POINTER(VerifyArgs), _p]
    lib.dsr_prob_stats.restype = _i32
    lib.dsr_prob_stats.argtypes = [_p, _i64, _p, _p, _p]
    lib.dsr_prob_stats_rows.restype = _i32
    lib.dsr_prob_stats_rows.argtypes = [ctypes.POINTER(_p), _i32, _i64, _p, _p]
    lib.dsr_prob_categorical.restype = _i32
    lib.dsr_prob_categorical.argtypes = [_p, _i64, _f64, _p, _p]
    lib.dsr_prob_correction.restype = _i32
    lib.dsr_prob_correction.argtypes = [_p, _p, _i64, _p, _p, _p]
    lib.dsr_prob_accept.restype = _i32
    lib.dsr_prob_accept.argtypes = [_p, _p, _i64, _i32, _f64, _p, _p]
    lib.dsr_history_from_dense.restype = _i32
    lib.dsr_history_from_dense.argtypes = [_p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _p, _p]
    lib.dsr_history_append.restype = _i32
    lib.dsr_history_append.argtypes = [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _i64, _p, _p]
    lib.dsr_vocab_head.restype = _i32
    lib.dsr_vocab_head.argtypes = [ctypes.POINTER(HeadArgs), _p]
    lib.dsr_verify_drafts_head.restype = _i32
    lib.dsr_verify_drafts_head.argtypes = [ctypes.POINTER(VerifyArgs), _p, _p, _p]
    lib.dsr_verify_probs_workspace_bytes.restype = ctypes.c_size_t
    lib.dsr_verify_probs_workspace_bytes.argtypes = [_i64, _i32]
    lib.dsr_verify_probs.restype = _i32
    lib.dsr_verify_probs.argtypes = [ctypes.POINTER(VerifyProbsArgs), _p]
    lib.dsr_rows_finite.restype = _i32
    lib.dsr_rows_finite.argtypes = [_p, _i64, _i64, _i64, _p, _p]
    lib.dsr_sample_rows_head.restype = _i32
    lib.dsr_sample_rows_head.argtypes = [ctypes.POINTER(SampleArgs), _p, _p]
    lib.dsr_count_scan.restype = _i32
    lib.dsr_count_scan.argtypes = [_p, _i32, _i64, _p, _p]
    _lib = lib
    return lib


def status_message(code: int) -> str:
    return load().dsr_status_message(int(code)).decode()


def check(rc: int, what: str) -> None:
    if rc != 0:
        kind = {-1: "invalid arguments", -2: "kernel launch failed", -3: "workspace too small"}.get(rc, str(rc))
        raise RuntimeError(f"{what}: {kind}")
