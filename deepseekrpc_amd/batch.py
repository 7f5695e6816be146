"""Batched device API of the sampling hot path (rows already in HBM).

This is the interface a serving loop uses: logits ``[rows, V]`` stay on the
GPU, one launch samples every row, and the host only sees the compact
decisions.  It replaces the reference's per-row device-to-host copy and
NumPy pipeline (terminal_sampling.py:16-27,83-95; sampling.py:48-128) and
its verifier (terminal_sampling.py:170-183; sampling.py:247-294).

Uniforms are drawn on the host (the reference's PCG64 domains stay there)
and passed in; each result reports which uniforms were consumed so the host
streams advance exactly as the reference's would.
"""
from __future__ import annotations

import collections
import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _native as N

VOCAB = 129280
POLICY_DTYPE = np.dtype(N.POLICY_DTYPE_FIELDS, align=True)
assert POLICY_DTYPE.itemsize == ctypes.sizeof(N.Policy) == 56


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_current_device = getattr(torch._C, "_cuda_getDevice", None)


def _stream_handle(device=None) -> int:
    """The current stream's handle on ``device`` (default: the current
    device).  torch's raw accessor: the public ``torch.cuda.current_stream()``
    costs several microseconds a call, a sizeable part of a one-row draw's
    host time."""
    index = device.index if device is not None and device.index is not None else None
    if _raw_stream is not None and _current_device is not None:
        return _raw_stream(_current_device() if index is None else index)
    return torch.cuda.current_stream(device).cuda_stream


def _stream():
    return ctypes.c_void_p(_stream_handle())


def _require_cuda(t, name, rows_strided=False):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a device tensor")
    ok = (t.dim() == 2 and t.stride(1) == 1 and t.stride(0) >= t.shape[1]) if rows_strided else t.is_contiguous()
    if not ok:
        raise ValueError(f"{name} must be contiguous" + (" within rows" if rows_strided else ""))


def _require(t, name, dtype, numel=None):
    _require_cuda(t, name)
    if t.dtype != dtype or (numel is not None and t.numel() != numel):
        raise ValueError(f"{name} must be {dtype} with {numel} elements")


def _nonempty(table, field):
    """Tables without entries are passed as absent (an empty tensor has no data pointer)."""
    return table is not None and getattr(table, field).numel() > 0


def policy_array(policies) -> np.ndarray:
    """Pack policies (objects with the seven SamplingPolicy fields, or dicts) into ``dsr_policy_t`` rows."""
    out = np.zeros(len(policies), POLICY_DTYPE)
    for i, p in enumerate(policies):
        get = p.get if isinstance(p, dict) else (lambda k, d=None, p=p: getattr(p, k, d))
        out[i]["temperature"] = get("temperature", 1.0)
        out[i]["top_p"] = get("top_p", 1.0)
        out[i]["min_p"] = get("min_p", 0.0)
        out[i]["repetition_penalty"] = get("repetition_penalty", 1.0)
        out[i]["presence_penalty"] = get("presence_penalty", 0.0)
        out[i]["frequency_penalty"] = get("frequency_penalty", 0.0)
        out[i]["top_k"] = get("top_k", 0)
    return out


def _policy_arg(policies, dev) -> torch.Tensor:
    """Packed policies on ``dev``: a list or array is packed here; a tensor
    must be a contiguous uint8 tensor on ``dev``, as ``policy_tensor`` makes
    (the kernels read it through a device pointer)."""
    t = policies if isinstance(policies, torch.Tensor) else policy_tensor(policies, dev)
    if not t.is_cuda or t.device != dev or t.dtype != torch.uint8 or not t.is_contiguous():
        raise ValueError("a policy tensor must be a contiguous uint8 tensor on the call's device (policy_tensor)")
    return t


def policy_tensor(policies, device) -> torch.Tensor:
    """The packed policies on ``device``; the tensor keeps its host copy as
    ``dsr_policies``, from which ``sample_rows`` and ``verify_drafts`` derive
    their kernel-choice hints (a tensor without one gets no hints)."""
    arr = policies if isinstance(policies, np.ndarray) and policies.dtype == POLICY_DTYPE else policy_array(policies)
    t = torch.from_numpy(arr.view(np.uint8).copy()).to(device)
    t.dsr_policies = arr.copy()
    return t


FAST_MAX_K = 1024   # the largest top-k the bf16 register kernel cuts to


def sample_hints(arr: np.ndarray | None, vocab: int) -> int:
    """DSR_HINT_* bits for packed policies: WHOLE_* when whole rows are sampled
    (0 < T <= 100) with no top-k or one above ``FAST_MAX_K`` (the kernels'
    ``whole_row``), TOPK_ALL when every row is in bounds and greedy or has
    1 <= top_k <= ``FAST_MAX_K`` below the vocabulary.  The bits only choose
    launches; results never depend on them."""
    if arr is None or len(arr) == 0:
        return 0
    T, k = arr["temperature"], arr["top_k"]
    whole = (T > 0) & (T <= 100) & ~((k >= 1) & (k <= FAST_MAX_K) & (k < vocab))
    topk = ((T == 0) | ((k >= 1) & (k <= FAST_MAX_K) & (k < vocab))) & policies_in_bounds(arr)
    return ((N.HINT_WHOLE_SOME if whole.any() else 0) | (N.HINT_WHOLE_ALL if whole.all() else 0)
            | (N.HINT_TOPK_ALL if topk.all() else 0))


def _policy_hints(policies, vocab: int) -> int:
    """``sample_hints`` of a policy tensor, kept on the tensor per vocabulary size."""
    cached = getattr(policies, "dsr_hints", None)
    if cached is not None and cached[0] == vocab:
        return cached[1]
    arr = getattr(policies, "dsr_policies", None)
    hints = sample_hints(arr, vocab)
    if arr is not None:
        policies.dsr_hints = (vocab, hints)
    return hints


def policies_in_bounds(arr: np.ndarray) -> np.ndarray:
    """Per packed policy: the bounds of SamplingPolicy (sampling.py:38-43) as
    the kernels test them (NaN fails every comparison)."""
    return ((arr["temperature"] >= 0.0) & (arr["temperature"] <= 100.0) & (arr["top_p"] >= 0.0) & (arr["top_p"] <= 1.0)
            & (arr["min_p"] >= 0.0) & (arr["min_p"] <= 1.0) & (arr["repetition_penalty"] >= 0.01)
            & (arr["repetition_penalty"] <= 100.0) & (arr["presence_penalty"] >= -2.0)
            & (arr["presence_penalty"] <= 2.0) & (arr["frequency_penalty"] >= -2.0)
            & (arr["frequency_penalty"] <= 2.0) & (arr["top_k"] >= 0) & (arr["top_k"] <= N.MAX_VOCAB)
            & (arr["reserved"] == 0))


def verify_hints(arr: np.ndarray | None, vocab: int, plain: bool) -> int:
    """DSR_HINT_VERIFY_FAST when every request's policy is in bounds and has
    no filter, and the call carries no history, bias or allow mask
    (``plain``).  A request whose policy is out of bounds leaves the bit
    off, so its distributions are built and it reports its policy error."""
    if arr is None or len(arr) == 0 or not plain:
        return 0
    k = arr["top_k"]
    ok = ((k == 0) | (k >= vocab)) & (arr["top_p"] >= 1.0) & (arr["min_p"] == 0.0) & policies_in_bounds(arr)
    return N.HINT_VERIFY_FAST if ok.all() else 0


@dataclass
class HistoryTable:
    """Per-row sparse token-history counts in CSR form (device tensors).

    Row ``r`` owns ``ids[off[r]:off[r+1]]`` (strictly increasing) with
    ``counts`` (all history) and ``generated`` (output part only): the
    reference's dense ``counts`` / ``generated_counts`` pair restricted to
    ``counts > 0`` (sampling.py:54-66, history.py:46-47).
    """
    offsets: torch.Tensor
    ids: torch.Tensor
    counts: torch.Tensor
    generated: torch.Tensor

    @classmethod
    def from_token_lists(cls, histories, generated_start=None, device="cuda"):
        """Histories as token-id lists; ids before ``generated_start[r]`` are prompt tokens."""
        offs, ids, cnt, gen = [0], [], [], []
        for r, h in enumerate(histories):
            h = np.asarray(h, np.int64)
            s = 0 if generated_start is None else int(generated_start[r])
            u, c = np.unique(h, return_counts=True)
            if s > 0:
                gu, gc = np.unique(h[s:], return_counts=True)
                g = np.zeros(len(u), np.int64)
                g[np.searchsorted(u, gu)] = gc
            else:
                g = c
            ids.append(u)
            cnt.append(c)
            gen.append(g)
            offs.append(offs[-1] + len(u))
        return cls._upload(offs, ids, cnt, gen, device)

    @classmethod
    def from_dense(cls, counts, generated=None, device="cuda"):
        """Dense ``[rows, V]`` count arrays (NumPy), as the reference's callers hold them."""
        counts = np.atleast_2d(np.asarray(counts))
        generated = counts if generated is None else np.atleast_2d(np.asarray(generated))
        offs, ids, cnt, gen = [0], [], [], []
        for r in range(counts.shape[0]):
            nz = np.flatnonzero(counts[r] > 0)
            ids.append(nz)
            cnt.append(counts[r][nz])
            gen.append(generated[r][nz])
            offs.append(offs[-1] + len(nz))
        return cls._upload(offs, ids, cnt, gen, device)

    @classmethod
    def from_support(cls, ids, counts, generated, device="cuda"):
        """One row from its positive entries: increasing ``ids`` with their
        counts and generated counts, already validated by the caller."""
        return cls._upload([0, len(ids)], [ids], [counts], [generated], device)

    @property
    def rows(self) -> int:
        return self.offsets.numel() - 1

    # -- built on the device (dsr_history_from_dense / dsr_history_append) --

    @classmethod
    def from_dense_device(cls, counts: torch.Tensor, generated: torch.Tensor | None = None):
        """Dense ``[rows, V]`` int32 device counts (and generated counts) -> a
        table built on the device.  Returns ``(table, status)``: ``status[r]``
        is 0, E_COUNTS or E_GENERATED (sampling.py:54-58, 62-65); a rejected
        row has no entries."""
        _require_cuda(counts, "counts", rows_strided=True)
        if counts.dtype != torch.int32:
            raise ValueError("counts must be int32")
        if generated is not None:
            _require_cuda(generated, "generated", rows_strided=True)
            if generated.dtype != torch.int32 or generated.shape != counts.shape or \
                    generated.stride(0) != counts.stride(0):
                raise ValueError("generated must be int32 with the shape and row stride of counts")
        rows, vocab = counts.shape
        dev = counts.device
        off = torch.empty(rows + 1, dtype=torch.int64, device=dev)
        status = torch.empty(rows, dtype=torch.int32, device=dev)
        lib = N.load()

        def call(cap):
            out = [torch.empty(max(cap, 1), dtype=torch.int32, device=dev) for _ in range(3)]
            rc = lib.dsr_history_from_dense(_ptr(counts), _ptr(generated), rows, vocab, counts.stride(0), _ptr(off),
                                            *(_ptr(o) for o in out), cap, _ptr(status), _stream())
            N.check(rc, "dsr_history_from_dense")
            return out

        cap = rows * vocab if rows * vocab <= (1 << 22) else 0  # large batches: count first, then exact outputs
        out = call(cap)
        total = int(off[-1].item())
        if total > cap:
            out = call(total)
        return cls(off, *(o[:total] for o in out)), status

    def append(self, tokens: torch.Tensor, tok_off: torch.Tensor, gen_from: torch.Tensor | None = None,
               vocab: int = VOCAB):
        """Adds ``tokens[tok_off[r]:tok_off[r+1]]`` to row ``r`` on the device
        (np.add.at on both counts, history.py:136-137; only positions at or
        after ``gen_from[r]`` count as generated).  At most MAX_APPEND tokens
        per row.  Returns ``(table, status)``."""
        return HistoryTable._append(self, tokens, tok_off, gen_from, vocab)

    @classmethod
    def _append(cls, table, tokens, tok_off, gen_from, vocab):
        _require(tokens, "tokens", torch.int32)
        _require(tok_off, "tok_off", torch.int64)
        rows = tok_off.numel() - 1
        if table is not None and table.rows != rows:
            raise ValueError("tok_off must have one entry per table row plus one")
        if gen_from is not None:
            _require(gen_from, "gen_from", torch.int64, rows)
        dev = tok_off.device
        # The kernels read tokens[tok_off[r] .. tok_off[r+1]): the offsets must
        # start at 0, never decrease and stay inside the token buffer.
        if rows > 0 and not bool(((tok_off[1:] >= tok_off[:-1]).all() & (tok_off[0] == 0)
                                  & (tok_off[-1] <= tokens.numel())).item()):
            raise ValueError("tok_off must be non-decreasing from 0 and within tokens")
        old = 0 if table is None else table.ids.numel()
        cap = old + tokens.numel()
        off = torch.empty(rows + 1, dtype=torch.int64, device=dev)
        status = torch.empty(rows, dtype=torch.int32, device=dev)
        out = [torch.empty(max(cap, 1), dtype=torch.int32, device=dev) for _ in range(3)]
        has = table is not None and old > 0
        rc = N.load().dsr_history_append(
            _ptr(table.offsets) if has else None, _ptr(table.ids) if has else None,
            _ptr(table.counts) if has else None, _ptr(table.generated) if has else None,
            _ptr(tokens) if tokens.numel() else ctypes.c_void_p(_ptr(tok_off).value),  # never read: no tokens
            _ptr(tok_off), _ptr(gen_from), rows, vocab, _ptr(off), *(_ptr(o) for o in out), cap, _ptr(status),
            _stream())
        N.check(rc, "dsr_history_append")
        total = int(off[-1].item())
        return cls(off, *(o[:total] for o in out)), status

    @classmethod
    def from_token_lists_device(cls, histories, generated_start=None, vocab: int = VOCAB, device="cuda"):
        """Token-id histories -> a table built on the device; ids before
        ``generated_start[r]`` are prompt tokens (history.py:92-94), the rest
        output tokens (:136-137).  Rows longer than MAX_APPEND are appended in
        rounds.  Returns ``(table, status)``."""
        lens = [len(h) for h in histories]
        rounds = max(1, -(-max(lens, default=0) // N.MAX_APPEND))
        table, status = None, None
        for k in range(rounds):
            lo = k * N.MAX_APPEND
            parts = [np.asarray(h[lo:lo + N.MAX_APPEND], np.int64) for h in histories]
            off = np.zeros(len(parts) + 1, np.int64)
            off[1:] = np.cumsum([len(p) for p in parts])
            flat = np.concatenate(parts) if off[-1] else np.zeros(0, np.int64)
            flat = np.clip(flat, -1, vocab)  # ids out of range stay out of range through the int32 cast
            gf = None
            if generated_start is not None:
                gf = torch.tensor([int(s) - lo for s in generated_start], dtype=torch.int64, device=device)
            tok = torch.from_numpy(flat.astype(np.int32)).to(device)
            table, st = cls._append(table, tok, torch.from_numpy(off).to(device), gf, vocab)
            status = st if status is None else torch.where(status != 0, status, st)
        return table, status

    @classmethod
    def _upload(cls, offs, ids, cnt, gen, device):
        # ids, counts and generated counts travel in one int32 copy and are
        # handed out as three contiguous slices of it.
        n = int(offs[-1])
        body = np.empty(3 * n, np.int32)
        for part, xs in enumerate((ids, cnt, gen)):
            if n:
                body[part * n:(part + 1) * n] = np.concatenate(xs)
        packed = torch.from_numpy(body).to(device)
        return cls(torch.from_numpy(np.asarray(offs, np.int64)).to(device),
                   packed[:n], packed[n:2 * n], packed[2 * n:])


@dataclass
class BiasTable:
    """Per-row sparse logit bias in CSR form (ids strictly increasing)."""
    offsets: torch.Tensor
    ids: torch.Tensor
    values: torch.Tensor

    @classmethod
    def from_dicts(cls, biases, device="cuda"):
        offs, ids, vals = [0], [], []
        for b in biases:
            items = sorted((b or {}).items())
            ids.extend(int(t) for t, _ in items)
            vals.extend(float(v) for _, v in items)
            offs.append(len(ids))
        return cls(torch.tensor(offs, dtype=torch.int64, device=device),
                   torch.tensor(ids, dtype=torch.int32, device=device),
                   torch.tensor(vals, dtype=torch.float64, device=device))


def allow_words(vocab: int) -> int:
    return (vocab + 31) // 32


def pack_allow(allowed: np.ndarray) -> np.ndarray:
    """bool ``[..., V]`` -> uint32 ``[..., ceil(V/32)]`` with bit ``i & 31`` of word ``i >> 5``."""
    allowed = np.asarray(allowed, bool)
    V = allowed.shape[-1]
    pad = allow_words(V) * 32 - V
    a = np.concatenate([allowed, np.zeros(allowed.shape[:-1] + (pad,), bool)], axis=-1)
    return np.packbits(a.reshape(a.shape[:-1] + (-1, 32)), axis=-1, bitorder="little").view(np.uint32)[..., 0]


def unpack_bits(words: np.ndarray, vocab: int) -> np.ndarray:
    w = np.ascontiguousarray(words, np.uint32)
    bits = np.unpackbits(w.view(np.uint8), bitorder="little").reshape(w.shape[:-1] + (-1,))
    return bits[..., :vocab].astype(bool)


_DTYPES = {torch.bfloat16: N.BF16, torch.float32: N.F32, torch.float64: N.F64}


@dataclass
class SampleResult:
    tokens: torch.Tensor      # int32 [rows]
    consumed: torch.Tensor    # uint8 [rows]
    status: torch.Tensor      # int32 [rows]
    flags: torch.Tensor       # uint8 [rows]
    probs: torch.Tensor | None = None
    kept_bits: torch.Tensor | None = None
    args: object = None       # the marshalled dsr_sample_args_t of this call
    keep: tuple = ()          # every tensor ``args`` points into, kept alive with it


class Workspace:
    """Caller-owned scratch for the library (it never allocates).

    One buffer per (device, stream): calls on different streams never share
    scratch memory.  A buffer is allocated while its stream is current, so
    torch's caching allocator orders its reuse after that stream's work when
    it is replaced by a larger one or dropped.  At most ``streams`` buffers
    are kept, the least recently used dropped first, so a caller that makes
    a stream per request does not hold scratch for every stream it used."""

    def __init__(self, streams: int = 4):
        self._bufs = collections.OrderedDict()
        self._limit = max(1, int(streams))

    def get(self, nbytes: int, device, stream=None, handle: int | None = None) -> torch.Tensor:
        device = torch.device(device)
        if device.index is None:
            device = torch.device(device.type, torch.cuda.current_device())
        if handle is None:
            if stream is None:
                stream = torch.cuda.current_stream(device)
            handle = stream.cuda_stream
        key = (device.index, handle)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            if stream is None:
                stream = torch.cuda.current_stream(device)
            with torch.cuda.stream(stream):
                buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        self._bufs.move_to_end(key)
        while len(self._bufs) > self._limit:
            self._bufs.popitem(last=False)
        return buf


_default_ws = Workspace()


def sample_rows(logits: torch.Tensor, policies, *, history: HistoryTable | None = None, bias: BiasTable | None = None,
                allow_bits: torch.Tensor | None = None, uniforms: torch.Tensor | None = None,
                rng_state: torch.Tensor | None = None, probs: str | None = None, kept: bool = False,
                workspace: Workspace | None = None, noalloc: bool = False, hints: int | None = None,
                out: dict | None = None, head_parts: torch.Tensor | None = None) -> SampleResult:
    """Sample every row of ``logits [rows, V]`` on the current stream.

    ``policies`` is a device tensor made by ``policy_tensor`` or a list of
    policy objects/dicts.  ``uniforms`` (float64 ``[rows]``) are the pre-drawn
    target-domain draws.  ``rng_state`` (int64 ``[rows, 4]``, see
    ``pcg64_states``) instead lets each row that needs a draw take it on the
    device from its PCG64 state, which is advanced in place.  With neither,
    only the distribution is computed.  ``probs`` may be ``"f32"`` or
    ``"f64"`` to return the final probabilities.  ``noalloc`` launches
    through ``dsr_sample_rows_noalloc``, whose workspace is the library's own
    device array (at most ``N.NOALLOC_SCRATCH_BYTES``; calls on one device
    share it, so overlapping calls race).  ``hints`` overrides the
    DSR_HINT_* bits derived from the policies (they choose launches only).
    ``out`` may supply any of the result tensors (``tokens``, ``consumed``,
    ``status``, ``flags``, ``probs``), contiguous and of the result's dtype
    and shape, for the kernels to write in place.  ``head_parts`` (the
    ``parts`` of a ``vocab_head`` call that wrote these logits) lets FP32 top-k
    rows without a mask start from the projection's per-tile maxima instead
    of a pass over the row (``dsr_sample_rows_head``); the results are the
    same.
    """
    lib = N.load()
    _require_cuda(logits, "logits", rows_strided=True)
    if logits.dim() != 2 or logits.dtype not in _DTYPES:
        raise ValueError("logits must be a [rows, V] bf16/f32/f64 tensor")
    rows, V = logits.shape
    dev = logits.device
    policies = _policy_arg(policies, dev)
    if policies.numel() != rows * POLICY_DTYPE.itemsize:
        raise ValueError("one policy per row is required")
    out = dict(out or {})

    def result(key, shape, dtype):
        t = out.pop(key, None)
        if t is None:
            return torch.empty(*shape, dtype=dtype, device=dev)
        _require_cuda(t, key)
        if t.dtype != dtype or tuple(t.shape) != tuple(shape) or not t.is_contiguous() or t.device != dev:
            raise ValueError(f"out['{key}'] must be a contiguous {dtype} {list(shape)} tensor on {dev}")
        return t

    res = SampleResult(result("tokens", (rows,), torch.int32), result("consumed", (rows,), torch.uint8),
                       result("status", (rows,), torch.int32), result("flags", (rows,), torch.uint8))
    if probs == "f32":
        res.probs = result("probs", (rows, V), torch.float32)
    elif probs == "f64":
        res.probs = result("probs", (rows, V), torch.float64)
    elif probs is not None:
        raise ValueError("probs must be None, 'f32' or 'f64'")
    if out:
        raise ValueError(f"unused out tensors: {sorted(out)}")
    if kept:
        res.kept_bits = torch.empty(rows, allow_words(V), dtype=torch.int32, device=dev)
    if uniforms is not None:
        _require_cuda(uniforms, "uniforms")
        if uniforms.dtype != torch.float64 or uniforms.numel() != rows:
            raise ValueError("uniforms must be float64 [rows]")
    if rng_state is not None:
        _require(rng_state, "rng_state", torch.int64, rows * 4)
    if head_parts is not None:
        if noalloc:
            raise ValueError("head_parts are not taken by the allocation-free entry point")
        _require(head_parts, "head_parts", torch.int32, rows * (V // HEAD_TILE) * 4)
    if allow_bits is not None:
        _require_cuda(allow_bits, "allow_bits")
        if allow_bits.dim() != 2 or allow_bits.shape[0] != rows or allow_bits.element_size() != 4:
            raise ValueError("allow_bits must be [rows, words] 32-bit")
    need = lib.dsr_sample_workspace_bytes(rows, V)
    if noalloc and need > N.NOALLOC_SCRATCH_BYTES:
        raise ValueError(f"{rows} rows of {V} tokens need {need} bytes of scratch; the allocation-free entry point "
                         f"holds {N.NOALLOC_SCRATCH_BYTES}")
    stream = _stream_handle(dev)
    ws = None if noalloc else (workspace or _default_ws).get(need, dev, handle=stream)
    a = N.SampleArgs()
    a.logits = logits.data_ptr()
    a.dtype = _DTYPES[logits.dtype]
    a.hints = _policy_hints(policies, V) if hints is None else hints
    a.rows, a.vocab, a.ld = rows, V, logits.stride(0)
    a.policy = policies.data_ptr()
    if _nonempty(history, "ids"):
        a.pen_off, a.pen_ids = history.offsets.data_ptr(), history.ids.data_ptr()
        a.pen_count, a.pen_gen = history.counts.data_ptr(), history.generated.data_ptr()
    if _nonempty(bias, "ids"):
        a.bias_off, a.bias_ids, a.bias_val = bias.offsets.data_ptr(), bias.ids.data_ptr(), bias.values.data_ptr()
    if allow_bits is not None:
        a.allow_bits, a.allow_ld = allow_bits.data_ptr(), allow_bits.stride(0)
    if uniforms is not None:
        a.uniforms = uniforms.data_ptr()
    if rng_state is not None and rows > 0:
        a.rng_state = rng_state.data_ptr()
    a.out_token, a.out_consumed = res.tokens.data_ptr(), res.consumed.data_ptr()
    a.out_status, a.out_flags = res.status.data_ptr(), res.flags.data_ptr()
    if res.probs is not None:
        if probs == "f32":
            a.out_probs_f32 = res.probs.data_ptr()
        else:
            a.out_probs_f64 = res.probs.data_ptr()
        a.probs_ld = V
    if res.kept_bits is not None:
        a.out_kept_bits, a.kept_ld = res.kept_bits.data_ptr(), res.kept_bits.stride(0)
    handle = ctypes.c_void_p(stream)
    if noalloc:
        N.check(lib.dsr_sample_rows_noalloc(ctypes.byref(a), handle), "dsr_sample_rows_noalloc")
    else:
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        if head_parts is not None:
            N.check(lib.dsr_sample_rows_head(ctypes.byref(a), _ptr(head_parts), handle), "dsr_sample_rows_head")
        else:
            N.check(lib.dsr_sample_rows(ctypes.byref(a), handle), "dsr_sample_rows")
    res.args = a
    res.keep = (logits, policies, history, bias, allow_bits, uniforms, rng_state, ws, head_parts)
    return res


_M64 = (1 << 64) - 1


def pcg64_states(generators, device="cuda") -> torch.Tensor:
    """The PCG64 states of NumPy Generators (or PCG64 bit generators), one
    row per generator, as the int64 ``[rows, 4]`` device tensor
    ``sample_rows(rng_state=...)`` takes: state lo, state hi, increment lo,
    increment hi (the 128-bit integers of the bit generator's state dict)."""
    out = np.zeros((len(generators), 4), np.uint64)
    for i, g in enumerate(generators):
        st = getattr(g, "bit_generator", g).state
        if st["bit_generator"] != "PCG64":
            raise ValueError("device draws reproduce NumPy's PCG64 only")
        s, inc = st["state"]["state"], st["state"]["inc"]
        out[i] = (s & _M64, s >> 64, inc & _M64, inc >> 64)
    return torch.from_numpy(out.view(np.int64)).to(device)


def pcg64_restore(generators, states: torch.Tensor) -> None:
    """Write device-advanced states back into the NumPy generators, so that
    their next host draws continue the same streams."""
    words = states.cpu().numpy().view(np.uint64)
    for g, w in zip(generators, words):
        bg = getattr(g, "bit_generator", g)
        st = bg.state
        st["state"]["state"] = int(w[0]) | (int(w[1]) << 64)
        bg.state = st


class PreparedSample:
    """A ``dsr_sample_rows`` call whose arguments are marshalled once.

    ``launch()`` re-issues the same launch on the current stream (outputs are
    overwritten in place); a serving loop or a benchmark calls it per step.
    """

    def __init__(self, logits, policies, **kw):
        self.workspace = kw.pop("workspace", None) or Workspace()
        self.inputs = (logits, policies, kw)
        self.result = sample_rows(logits, policies, workspace=self.workspace, **kw)
        self.args = self.result.args
        self._lib = N.load()

    def launch(self):
        rc = self._lib.dsr_sample_rows(ctypes.byref(self.args), _stream())
        if rc != 0:
            N.check(rc, "dsr_sample_rows")
        return self.result


class PreparedHistoryAppend:
    """A ``dsr_history_append`` call with its outputs allocated once, at the
    exact upper bound (old entries plus new tokens).  ``launch()`` re-issues
    it on the current stream; ``table()`` returns the result (reading the
    total is the only synchronisation)."""

    def __init__(self, tokens: torch.Tensor, tok_off: torch.Tensor, table: HistoryTable | None = None,
                 gen_from: torch.Tensor | None = None, vocab: int = VOCAB):
        _require(tokens, "tokens", torch.int32)
        _require(tok_off, "tok_off", torch.int64)
        rows = tok_off.numel() - 1
        dev = tok_off.device
        has = table is not None and table.ids.numel() > 0
        self.cap = (table.ids.numel() if has else 0) + tokens.numel()
        self.off = torch.empty(rows + 1, dtype=torch.int64, device=dev)
        self.status = torch.empty(rows, dtype=torch.int32, device=dev)
        self.out = [torch.empty(max(self.cap, 1), dtype=torch.int32, device=dev) for _ in range(3)]
        self.inputs = (tokens, tok_off, table, gen_from)
        self._args = ((_ptr(table.offsets), _ptr(table.ids), _ptr(table.counts), _ptr(table.generated)) if has
                      else (None,) * 4) + (
            _ptr(tokens) if tokens.numel() else ctypes.c_void_p(tok_off.data_ptr()), _ptr(tok_off), _ptr(gen_from),
            rows, vocab, _ptr(self.off), *(_ptr(o) for o in self.out), self.cap, _ptr(self.status))
        self._lib = N.load()

    def launch(self):
        rc = self._lib.dsr_history_append(*self._args, _stream())
        if rc != 0:
            N.check(rc, "dsr_history_append")
        return self

    def table(self) -> HistoryTable:
        total = int(self.off[-1].item())
        return HistoryTable(self.off, *(o[:total] for o in self.out))


def _append_one(table: HistoryTable, token: torch.Tensor, bounds: torch.Tensor,
                vocab: int) -> tuple[HistoryTable, torch.Tensor]:
    """One device token appended to a one-row table (counted and generated),
    without synchronising: the outputs keep their capacity (old capacity + 1)
    and only ``offsets`` says how many entries are real, which is all the
    sampling kernels read."""
    dev = token.device
    old = table.ids.numel()
    cap = old + 1
    off = torch.empty(2, dtype=torch.int64, device=dev)
    status = torch.empty(1, dtype=torch.int32, device=dev)
    out = [torch.empty(cap, dtype=torch.int32, device=dev) for _ in range(3)]
    rc = N.load().dsr_history_append(_ptr(table.offsets), _ptr(table.ids), _ptr(table.counts),
                                     _ptr(table.generated), _ptr(token), _ptr(bounds), None, 1, vocab, _ptr(off),
                                     *(_ptr(o) for o in out), cap, _ptr(status), _stream())
    N.check(rc, "dsr_history_append")
    return HistoryTable(off, *out), status


@dataclass
class Proposals:
    """Draft proposals drawn on the device by ``propose_rows``; rows after the
    first stop token are speculative until ``finish_proposals`` cuts them."""
    tokens: torch.Tensor      # int32 [steps]
    rows: torch.Tensor        # float64 [steps, V]: each row's distribution
    consumed: torch.Tensor    # uint8 [steps]
    status: torch.Tensor      # int32 [steps]: each row's sampling status
    appended: tuple           # int32 [1] history-append status of rows 1.. (the previous proposal)
    logits: torch.Tensor      # float32 [steps, V]: each row's logits as sampled, checked for finiteness at the end
    states: torch.Tensor      # int64 [steps + 1, 4]: PCG64 state before row 0 and after each row
    keep: tuple = ()
    # (position, exception) when row_logits failed for a row after the
    # first: the chain stops there, and the error counts only if no stop
    # token comes before that row.
    deferred: tuple | None = None


def propose_rows(row_logits, seed_token: torch.Tensor, steps: int, policy, rng_state: torch.Tensor, *,
                 history: HistoryTable | None = None, bias: BiasTable | None = None,
                 allow_bits: torch.Tensor | None = None, vocab: int = VOCAB, grow: bool = True) -> Proposals:
    """Up to ``steps`` draft tokens drawn one row at a time with no host
    synchronisation (terminal_sampling.py:138-161).

    ``row_logits(position, previous)`` returns row ``position``'s FP32 logits
    on the device, conditioned on ``previous``, the previous token as a device
    int32 tensor of one element (``seed_token`` first, always a valid id): the
    caller's Markov bias step reads the token the sampling kernel wrote.  Each row is
    one ``dsr_sample_rows`` launch that draws its uniform from the ``draft``
    domain's PCG64 state in ``rng_state`` (int64 ``[1, 4]``, advanced in
    place), writes its token and distribution straight into the chain's
    tensors, and sees the history with every earlier proposal appended, as
    ``SamplingWork.distribution`` conditions it (:127-133).  Every row is
    drawn speculatively; ``finish_proposals`` keeps them up to the first stop
    token, checks the rows' logits and statuses, and restores the state saved
    after the last kept row.  With ``grow=False`` nothing is appended and
    every row carries ``history`` as given: the caller's choice when no row's
    distribution reads the prefix counts and no append could fail."""
    if steps < 0 or steps > 5:
        raise ValueError("at most five proposals")
    _require(rng_state, "rng_state", torch.int64, 4)
    _require(seed_token, "seed_token", torch.int32, 1)
    dev = rng_state.device
    pol = _policy_arg(policy if isinstance(policy, torch.Tensor) else [policy], dev)
    if pol.numel() != POLICY_DTYPE.itemsize:
        raise ValueError("one policy is required")
    tokens = torch.empty(steps, dtype=torch.int32, device=dev)
    rows = torch.empty(steps, vocab, dtype=torch.float64, device=dev)
    consumed = torch.empty(steps, dtype=torch.uint8, device=dev)
    status = torch.empty(steps, dtype=torch.int32, device=dev)
    flags = torch.empty(steps, dtype=torch.uint8, device=dev)
    states = torch.empty(steps + 1, 4, dtype=torch.int64, device=dev)
    bounds = torch.tensor([0, 1], dtype=torch.int64, device=dev)  # one token per append
    # Each row's logits as sampled (the caller may reuse its buffer for the next row).
    seen = torch.empty(steps, vocab, dtype=torch.float32, device=dev)
    keep, appended = [pol, bounds, flags], []
    table, previous = history, seed_token
    made, deferred = steps, None
    for j in range(steps):
        try:
            logits = row_logits(j, previous)
            if not (isinstance(logits, torch.Tensor) and logits.is_cuda and logits.dtype == torch.float32
                    and logits.numel() == vocab):
                raise ValueError("row_logits must return FP32 device logits of the vocabulary")
        except Exception as exc:
            # Row 0 is always kept.  A later row may lie past a stop token,
            # where the reference never asks for it: its error waits for the
            # synchronisation that knows.
            if j == 0:
                raise
            made, deferred = j, (j, exc)
            break
        logits = logits.reshape(1, vocab).contiguous()
        seen[j].copy_(logits[0])
        if j > 0 and grow:
            if table is None:
                table = HistoryTable(torch.zeros(2, dtype=torch.int64, device=dev),
                                     *(torch.zeros(1, dtype=torch.int32, device=dev) for _ in range(3)))
            table, app = _append_one(table, previous, bounds, vocab)
            appended.append(app)
        states[j].copy_(rng_state.reshape(4))
        res = sample_rows(logits, pol, history=table, bias=bias, allow_bits=allow_bits, rng_state=rng_state,
                          probs="f64", out=dict(tokens=tokens[j:j + 1], consumed=consumed[j:j + 1],
                                                status=status[j:j + 1], flags=flags[j:j + 1],
                                                probs=rows[j:j + 1]))
        keep.append((table, res))
        # A failed row writes token -1; the chain is rejected at its end, but
        # the caller's bias step and the history only ever see a valid id.
        previous = torch.clamp(tokens[j:j + 1], min=0)
    states[made].copy_(rng_state.reshape(4))
    return Proposals(tokens[:made], rows[:made], consumed[:made], status[:made], tuple(appended), seen[:made],
                     states[:made + 1], tuple(keep), deferred)


def finish_proposals(p: Proposals, eos_ids=()):
    """The one synchronisation of a proposal chain: the kept proposals (up
    to and including the first stop token), their distributions, the number
    of ``draft`` draws they consumed, the PCG64 state after the last kept row
    (int64 ``[1, 4]`` on the device, for ``pcg64_restore``), and the first row
    whose logits, sampling or history append failed
    (``(position, status)`` with status -1 for non-finite logits, or None;
    ``(position, exception)`` when the caller's ``row_logits`` failed for a
    kept row)."""
    steps = p.tokens.numel()
    if steps == 0:
        return (), p.rows[:0], 0, p.states[0:1], p.deferred
    dev = p.tokens.device
    finite = rows_finite(p.logits)
    # Row j > 0 carries the status of the append before it; a chain without appends has none.
    app = torch.cat([torch.zeros(1 if p.appended else steps, dtype=torch.int32, device=dev), *p.appended])
    info = torch.stack([p.tokens, p.consumed.to(torch.int32), p.status, app, finite]).cpu().numpy()
    toks, used, st, ap, fin = info
    count, cut = steps, False
    for j, t in enumerate(toks):
        if int(t) in eos_ids:
            count, cut = j + 1, True
            break
    failed = None
    for j in range(count):
        if not fin[j]:
            failed = (j, -1)
        elif st[j] != 0 or ap[j] != 0:
            failed = (j, int(st[j] if st[j] != 0 else ap[j]))
        if failed:
            break
    if failed is None and not cut:
        failed = p.deferred
    return tuple(int(t) for t in toks[:count]), p.rows[:count], int(used[:count].sum()), p.states[count:count + 1], \
        failed


@dataclass
class VerifyResult:
    accepted: torch.Tensor
    ids: torch.Tensor
    count: torch.Tensor
    pending: torch.Tensor
    stop: torch.Tensor
    used_accept: torch.Tensor
    used_target: torch.Tensor
    status: torch.Tensor
    flags: torch.Tensor
    args: object = None  # the marshalled dsr_verify_args_t
    keep: tuple = ()     # every tensor ``args`` points into, kept alive with it
    head: tuple | None = None  # (target records, draft records) of dsr_verify_drafts_head


def verify_drafts(target: torch.Tensor, draft: torch.Tensor, draft_ids: torch.Tensor, policies, u_accept: torch.Tensor,
                  u_target: torch.Tensor, output_limit: torch.Tensor, *, history: HistoryTable | None = None,
                  bias: BiasTable | None = None, allow_bits: torch.Tensor | None = None,
                  eos_offsets: torch.Tensor | None = None, eos_ids: torch.Tensor | None = None,
                  rng_accept: torch.Tensor | None = None, rng_target: torch.Tensor | None = None,
                  workspace: Workspace | None = None, hints: int | None = None,
                  head: tuple | None = None) -> VerifyResult:
    """Exact sampled verification of ``rows`` requests with ``K`` drafts each.

    ``target [rows, K+1, V]`` and ``draft [rows, K, V]`` are logits; row ``j``
    of both is conditioned on the prefix ``draft_ids[:, :j]``.  ``u_accept`` /
    ``u_target`` are pre-drawn uniforms; ``rng_accept`` / ``rng_target``
    (int64 ``[rows, 4]``, see ``pcg64_states``) instead draw them on the
    device from each request's accept / target PCG64 state, which is advanced
    by exactly the draws the decision uses.  ``hints`` overrides the
    DSR_HINT_VERIFY_FAST bit derived from the policies.  ``head`` =
    ``(target, draft)`` ``HeadResult`` s of the ``vocab_head`` calls that
    wrote ``target`` and ``draft``: the per-row statistics then come from
    their records (``dsr_verify_drafts_head``).
    """
    lib = N.load()
    given_policies = policies
    _require_cuda(target, "target")
    rows, K1, V = target.shape
    K = K1 - 1
    dev = target.device
    if K > 0:
        _require_cuda(draft, "draft")
        if tuple(draft.shape) != (rows, K, V) or draft.dtype != target.dtype:
            raise ValueError("draft must be [rows, K, V] of the target dtype")
        _require(draft_ids, "draft_ids", torch.int32, rows * K)
        if rng_accept is None:
            _require(u_accept, "u_accept", torch.float64, rows * K)
    if rng_accept is not None:
        _require(rng_accept, "rng_accept", torch.int64, rows * 4)
    if rng_target is None:
        _require(u_target, "u_target", torch.float64, rows)
    else:
        _require(rng_target, "rng_target", torch.int64, rows * 4)
    _require(output_limit, "output_limit", torch.int32, rows)
    if target.dtype not in _DTYPES:
        raise ValueError("target must be bf16/f32/f64")
    policies = _policy_arg(policies, dev)
    if policies.numel() != rows * POLICY_DTYPE.itemsize:
        raise ValueError("one policy per request is required")
    i32 = lambda *s: torch.empty(*s, dtype=torch.int32, device=dev)
    res = VerifyResult(i32(rows), i32(rows, K + 1), i32(rows), i32(rows), i32(rows), i32(rows), i32(rows), i32(rows),
                       torch.empty(rows, dtype=torch.uint8, device=dev))
    ws = (workspace or _default_ws).get(lib.dsr_verify_workspace_bytes(rows, K, V), dev, handle=_stream_handle(dev))
    a = N.VerifyArgs()
    a.target = target.data_ptr()
    a.draft = draft.data_ptr() if K > 0 else None
    a.dtype = _DTYPES[target.dtype]
    a.K, a.rows, a.vocab, a.ld = K, rows, V, V
    a.draft_ids = draft_ids.data_ptr() if K > 0 else None
    a.policy = policies.data_ptr()
    if _nonempty(history, "ids"):
        a.pen_off, a.pen_ids = history.offsets.data_ptr(), history.ids.data_ptr()
        a.pen_count, a.pen_gen = history.counts.data_ptr(), history.generated.data_ptr()
    if _nonempty(bias, "ids"):
        a.bias_off, a.bias_ids, a.bias_val = bias.offsets.data_ptr(), bias.ids.data_ptr(), bias.values.data_ptr()
    if allow_bits is not None:
        _require_cuda(allow_bits, "allow_bits")
        a.allow_bits, a.allow_ld = allow_bits.data_ptr(), allow_bits.shape[-1]
    a.hints = verify_hints(getattr(policies, "dsr_policies", None), V,
                           not _nonempty(history, "ids") and not _nonempty(bias, "ids") and allow_bits is None) \
        if hints is None else hints
    a.u_accept = u_accept.data_ptr() if K > 0 and u_accept is not None else None
    a.u_target = u_target.data_ptr() if u_target is not None else None
    if rng_accept is not None and rows > 0:
        a.rng_accept = rng_accept.data_ptr()
    if rng_target is not None and rows > 0:
        a.rng_target = rng_target.data_ptr()
    if eos_offsets is not None and eos_ids is not None and eos_ids.numel() > 0:
        _require(eos_offsets, "eos_offsets", torch.int64, rows + 1)
        _require_cuda(eos_ids, "eos_ids")
        a.eos_off, a.eos_ids = eos_offsets.data_ptr(), eos_ids.data_ptr()
    a.output_limit = output_limit.data_ptr()
    a.out_accepted, a.out_ids, a.out_count = res.accepted.data_ptr(), res.ids.data_ptr(), res.count.data_ptr()
    a.out_pending, a.out_stop = res.pending.data_ptr(), res.stop.data_ptr()
    a.out_used_accept, a.out_used_target = res.used_accept.data_ptr(), res.used_target.data_ptr()
    a.out_status, a.out_flags = res.status.data_ptr(), res.flags.data_ptr()
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    res.args = a
    res.keep = (target, draft, draft_ids, policies, u_accept, u_target, output_limit, history, bias, allow_bits,
                eos_offsets, eos_ids, rng_accept, rng_target, ws)
    if head is None:
        N.check(lib.dsr_verify_drafts(ctypes.byref(a), _stream()), "dsr_verify_drafts")
        return res
    th, dh = head
    def wrote(h, t):
        return h is not None and h.parts is not None and h.logits.data_ptr() == t.data_ptr() \
            and h.logits.numel() == t.numel() and t.dtype == torch.float32

    if not wrote(th, target) or (K > 0 and not wrote(dh, draft)):
        raise ValueError("head must hold the records of the vocab_head calls that wrote target and draft")
    if th.rows_per_policy != K + 1 or (K > 0 and dh.rows_per_policy != K) or \
            not _same_policies(th.policies, given_policies) or \
            (K > 0 and not _same_policies(dh.policies, given_policies)):
        raise ValueError("head records must be computed over the verifier's policies, K + 1 (target) and K "
                         "(draft) rows per request")
    res.head = (th.parts, dh.parts if K > 0 else None)
    res.keep = res.keep + res.head
    N.check(lib.dsr_verify_drafts_head(ctypes.byref(a), _ptr(res.head[0]), _ptr(res.head[1]), _stream()),
            "dsr_verify_drafts_head")
    return res


def _row_pointers(rows, count, V, dev, what, optional=False):
    """Device pointers of ``count`` float64 rows of ``V``: a ``[..., V]`` tensor
    split into its rows, or a sequence of ``[V]`` tensors (``None`` allowed
    where ``optional``)."""
    if isinstance(rows, torch.Tensor):
        rows = list(rows.reshape(-1, rows.shape[-1])) if rows.numel() else []
    rows = list(rows)
    if len(rows) != count:
        raise ValueError(f"{what}: {count} rows are required")
    out = []
    for r in rows:
        if r is None and optional:
            out.append(0)
            continue
        _require_cuda(r, what)
        if r.dtype != torch.float64 or r.numel() != V or r.device != dev or not r.is_contiguous():
            raise ValueError(f"{what} rows must be contiguous float64 [{V}] on {dev}")
        out.append(r.data_ptr())
    return out, rows


def verify_probs(target_rows, draft_rows, draft_ids: torch.Tensor, output_limit: torch.Tensor, *, vocab: int,
                 requests: int = 1, greedy: torch.Tensor | None = None, u_accept: torch.Tensor | None = None,
                 u_target: torch.Tensor | None = None, rng_accept: torch.Tensor | None = None,
                 rng_target: torch.Tensor | None = None, target_status: torch.Tensor | None = None,
                 eos_offsets: torch.Tensor | None = None, eos_ids: torch.Tensor | None = None,
                 workspace: Workspace | None = None) -> VerifyResult:
    """``verify_drafts`` (sampling.py:247-294) over float64 rows already on the
    device (``dsr_verify_probs``), for ``requests`` requests of ``K`` drafts.

    ``target_rows`` holds ``requests * (K + 1)`` rows and ``draft_rows``
    ``requests * K`` (a ``[..., V]`` tensor or a sequence of ``[V]``
    tensors), request-major.  ``target_status`` (int32, one per target row)
    is the status of whatever built each target row: a failed row is
    reported when the chain reaches it, and may be ``None`` in
    ``target_rows``.  ``greedy`` is a uint8 flag per request.  Draws come
    from ``u_accept`` / ``u_target`` or, on the device, from the PCG64 states
    ``rng_accept`` / ``rng_target`` (int64 ``[requests, 4]``), advanced by
    exactly the draws the decision uses.  The row pointers go to the device
    in one pinned upload; nothing here synchronises.
    """
    lib = N.load()
    R, V = int(requests), int(vocab)
    K = draft_ids.numel() // R if R else 0
    dev = draft_ids.device if K else output_limit.device
    tp, trows = _row_pointers(target_rows, R * (K + 1), V, dev, "target", optional=target_status is not None)
    dp, drows = _row_pointers(draft_rows if K else [], R * K, V, dev, "draft")
    if K:
        _require(draft_ids, "draft_ids", torch.int32, R * K)
        if rng_accept is None:
            _require(u_accept, "u_accept", torch.float64, R * K)
    if rng_accept is not None:
        _require(rng_accept, "rng_accept", torch.int64, R * 4)
    if rng_target is None:
        _require(u_target, "u_target", torch.float64, R)
    else:
        _require(rng_target, "rng_target", torch.int64, R * 4)
    _require(output_limit, "output_limit", torch.int32, R)
    if greedy is not None:
        _require(greedy, "greedy", torch.uint8, R)
    if target_status is not None:
        _require(target_status, "target_status", torch.int32, R * (K + 1))
    host = torch.tensor(tp + dp, dtype=torch.int64).pin_memory()
    ptrs = host.to(dev, non_blocking=True)
    i32 = lambda *sh: torch.empty(*sh, dtype=torch.int32, device=dev)
    res = VerifyResult(i32(R), i32(R, K + 1), i32(R), i32(R), i32(R), i32(R), i32(R), i32(R),
                       torch.empty(R, dtype=torch.uint8, device=dev))
    ws = (workspace or _default_ws).get(max(lib.dsr_verify_probs_workspace_bytes(R, K), 8), dev, handle=_stream_handle(dev))
    a = N.VerifyProbsArgs()
    a.target = ptrs.data_ptr()
    a.draft = ptrs.data_ptr() + 8 * R * (K + 1) if K else None
    a.target_status = target_status.data_ptr() if target_status is not None else None
    a.K, a.rows, a.vocab = K, R, V
    a.draft_ids = draft_ids.data_ptr() if K else None
    a.greedy = greedy.data_ptr() if greedy is not None else None
    a.u_accept = u_accept.data_ptr() if K and u_accept is not None else None
    a.u_target = u_target.data_ptr() if u_target is not None else None
    if rng_accept is not None and R:
        a.rng_accept = rng_accept.data_ptr()
    if rng_target is not None and R:
        a.rng_target = rng_target.data_ptr()
    if eos_offsets is not None and eos_ids is not None and eos_ids.numel() > 0:
        _require(eos_offsets, "eos_offsets", torch.int64, R + 1)
        _require_cuda(eos_ids, "eos_ids")
        a.eos_off, a.eos_ids = eos_offsets.data_ptr(), eos_ids.data_ptr()
    a.output_limit = output_limit.data_ptr()
    a.out_accepted, a.out_ids, a.out_count = res.accepted.data_ptr(), res.ids.data_ptr(), res.count.data_ptr()
    a.out_pending, a.out_stop = res.pending.data_ptr(), res.stop.data_ptr()
    a.out_used_accept, a.out_used_target = res.used_accept.data_ptr(), res.used_target.data_ptr()
    a.out_status, a.out_flags = res.status.data_ptr(), res.flags.data_ptr()
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    res.args = a
    res.keep = (trows, drows, ptrs, host, draft_ids, output_limit, greedy, u_accept, u_target, rng_accept, rng_target,
                target_status, eos_offsets, eos_ids, ws)
    N.check(lib.dsr_verify_probs(ctypes.byref(a), _stream()), "dsr_verify_probs")
    return res


class PreparedVerify:
    """A ``dsr_verify_drafts`` call whose arguments are marshalled once;
    ``launch()`` re-issues it on the current stream, overwriting the outputs."""

    def __init__(self, *args, **kw):
        self.workspace = kw.pop("workspace", None) or Workspace()
        self.inputs = (args, kw)
        self.result = verify_drafts(*args, workspace=self.workspace, **kw)
        self.args = self.result.args
        self._lib = N.load()

    def launch(self):
        head = self.result.head
        if head is None:
            rc = self._lib.dsr_verify_drafts(ctypes.byref(self.args), _stream())
        else:
            rc = self._lib.dsr_verify_drafts_head(ctypes.byref(self.args), _ptr(head[0]), _ptr(head[1]), _stream())
        if rc != 0:
            N.check(rc, "dsr_verify_drafts")
        return self.result


# ---------------------------------------------------------------------------
# Vocabulary projection (the terminal stage's lm_head) with the verifier's
# per-row statistics in its epilogue.

HEAD_TILE = N.HEAD_TILE


def _same_policies(x, y) -> bool:
    """The same policies: one object, one device tensor, or equal lists."""
    if x is y:
        return True
    if isinstance(x, torch.Tensor) or isinstance(y, torch.Tensor):
        return isinstance(x, torch.Tensor) and isinstance(y, torch.Tensor) and x.data_ptr() == y.data_ptr() \
            and x.numel() == y.numel()
    return x is not None and y is not None and np.array_equal(policy_array(x), policy_array(y))


@dataclass
class HeadResult:
    """FP32 logits ``[rows, vocab]`` and, with records, ``parts`` ``[rows,
    vocab / 128, 4]`` int32: one ``dsr_head_part_t`` per (row, 128-column
    tile), viewed by ``part_sum`` / ``part_max`` / ``part_info``."""
    logits: torch.Tensor
    parts: torch.Tensor | None
    policies: object = None
    rows_per_policy: int = 1
    args: object = None
    keep: tuple = ()

    @property
    def part_sum(self):
        return self.parts[..., 0:2].contiguous().view(torch.float64)[..., 0]

    @property
    def part_max(self):
        return self.parts[..., 2:3].contiguous().view(torch.float32)[..., 0]

    @property
    def part_info(self):
        return self.parts[..., 3]

    def finite_rows(self) -> torch.Tensor:
        """Device bool per row: every logit is finite (the terminal stage's
        torch.isfinite(logits).all() per row, stage_graph.py:361), read from
        the records' flags instead of the logits."""
        return ((self.part_info & 5) == 0).all(dim=1)


def vocab_head(hidden: torch.Tensor, weight: torch.Tensor, *, policies=None, rows_per_policy: int = 1,
               records: bool = True, out: HeadResult | None = None) -> HeadResult:
    """``logits = hidden . weight^T`` (bf16 in, FP32 accumulation and out) for
    ``hidden [rows, dim]`` and ``weight [vocab, dim]``, and with ``records``
    one ``dsr_head_part_t`` per (row, 128-column tile).  Row r samples at the
    temperature of ``policies[r // rows_per_policy]`` (a policy list or a
    ``policy_tensor``); without policies the records carry no exp sums.
    ``out`` reuses the tensors of an earlier result of the same shape."""
    lib = N.load()
    for t, name in ((hidden, "hidden"), (weight, "weight")):
        _require_cuda(t, name)
        if t.dtype != torch.bfloat16 or t.dim() != 2:
            raise ValueError(f"{name} must be a 2-D bfloat16 tensor")
    rows, dim = hidden.shape
    vocab = weight.shape[0]
    if weight.shape[1] != dim or weight.device != hidden.device:
        raise ValueError("hidden and weight must share dim and device")
    if not (0 <= rows <= N.HEAD_MAX_ROWS and dim >= 256 and dim % 256 == 0 and vocab % HEAD_TILE == 0
            and HEAD_TILE <= vocab <= VOCAB):
        raise ValueError("vocab_head needs rows <= 256, dim a multiple of 256 and vocab a multiple of 128")
    dev = hidden.device
    pol = None
    if policies is not None:
        if rows_per_policy < 1:
            raise ValueError("rows_per_policy must be >= 1")
        pol = _policy_arg(policies, dev)
        if pol.numel() * pol.element_size() < -(-rows // rows_per_policy) * ctypes.sizeof(N.Policy):
            raise ValueError("policies must cover every row")
    if out is None:
        logits = torch.empty(rows, vocab, dtype=torch.float32, device=dev)
        parts = torch.empty(rows, vocab // HEAD_TILE, 4, dtype=torch.int32, device=dev) if records else None
    else:
        logits, parts = out.logits, out.parts
        if tuple(logits.shape) != (rows, vocab) or (records and parts is None):
            raise ValueError("out does not match this call")
        parts = parts if records else None
    a = N.HeadArgs()
    a.hidden, a.weight, a.logits = hidden.data_ptr(), weight.data_ptr(), logits.data_ptr()
    a.rows, a.dim, a.vocab = rows, dim, vocab
    a.policy = pol.data_ptr() if pol is not None else None
    a.rows_per_policy = rows_per_policy if pol is not None else 0
    a.parts = parts.data_ptr() if parts is not None else None
    res = HeadResult(logits, parts, policies, rows_per_policy, a, (hidden, weight, pol))
    N.check(lib.dsr_vocab_head(ctypes.byref(a), _stream()), "dsr_vocab_head")
    return res


def vocab_head_launch(res: HeadResult) -> HeadResult:
    """Re-issue a marshalled ``vocab_head`` call on the current stream."""
    N.check(N.load().dsr_vocab_head(ctypes.byref(res.args), _stream()), "dsr_vocab_head")
    return res


# ---------------------------------------------------------------------------
# Probability-vector kernels used by the drop-in API.


def rows_finite(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """int32 ``[rows]``: 1 where every value of the FP32 row of ``x [rows, n]``
    is finite (``dsr_rows_finite``); nothing synchronises.  ``out`` may be an
    int32 device tensor of ``rows`` elements that already holds 1s (the
    kernel only clears the flags of rows with a non-finite value)."""
    lib = N.load()
    _require_cuda(x, "x", rows_strided=True)
    if x.dim() != 2 or x.dtype != torch.float32:
        raise ValueError("x must be a [rows, n] float32 tensor")
    rows, n = x.shape
    if out is None:
        out = torch.ones(rows, dtype=torch.int32, device=x.device)
    _require(out, "out", torch.int32, rows)
    N.check(lib.dsr_rows_finite(_ptr(x), rows, n, x.stride(0), _ptr(out), _stream()), "dsr_rows_finite")
    return out


def count_scan(counts: np.ndarray):
    """``dsr_count_scan`` of a host int32 / int64 count vector: ``(support,
    total, largest)`` (the increasing ids of the positive entries, their
    int64 sum, wrapping as NumPy's does, and the largest entry), or None when
    an entry is negative.  One read-only pass in native code."""
    lib = N.load()
    c = np.ascontiguousarray(counts)
    if c.ndim != 1 or c.dtype not in (np.int32, np.int64):
        raise ValueError("counts must be a 1-D int32 or int64 array")
    support = np.empty(max(c.size, 1), np.int64)
    out = np.zeros(3, np.int64)
    rc = lib.dsr_count_scan(c.ctypes.data, c.itemsize, c.size, support.ctypes.data, out.ctypes.data)
    if rc < 0:
        N.check(rc, "dsr_count_scan")
    if rc == 1:
        return None
    return support[:int(out[0])].copy(), int(out[1]), int(out[2])


def prob_stats_launch(p: torch.Tensor, slot: torch.Tensor):
    """``dsr_prob_stats`` of a float64 device vector into ``slot``, a float64
    ``[3]`` device view: the sum, then the four int32 results.  Nothing is
    synchronised; ``prob_stats_read`` decodes the slot once it is on the host."""
    lib = N.load()
    N.check(lib.dsr_prob_stats(_ptr(p), p.numel(), _ptr(slot[0:1]), _ptr(slot[1:3]), _stream()), "dsr_prob_stats")


def prob_stats_rows_launch(rows, out: torch.Tensor):
    """``dsr_prob_stats`` of every row (contiguous float64 device vectors of
    one length) into ``out``, a contiguous float64 ``[len(rows), 3]`` device
    tensor of slots, one launch per 16 rows.  Nothing is synchronised."""
    lib = N.load()
    n = rows[0].numel()
    if out.shape != (len(rows), 3) or out.dtype != torch.float64 or not out.is_contiguous():
        raise ValueError("out must be a contiguous float64 [rows, 3] tensor")
    for r in rows:
        _require(r, "row", torch.float64, n)
    for start in range(0, len(rows), N.STATS_MAX_ROWS):
        chunk = rows[start:start + N.STATS_MAX_ROWS]
        ptrs = (ctypes.c_void_p * len(chunk))(*[t.data_ptr() for t in chunk])
        N.check(lib.dsr_prob_stats_rows(ptrs, len(chunk), n, _ptr(out[start]), _stream()), "dsr_prob_stats_rows")


def prob_stats_read(slot: torch.Tensor):
    """(sum, valid, n_positive, first_positive, argmax) from a host copy of a slot."""
    o = slot[1:3].view(torch.int32).tolist()
    return float(slot[0]), bool(o[0]), int(o[1]), int(o[2]), int(o[3])


def prob_stats(p: torch.Tensor):
    """(sum, valid, n_positive, first_positive, argmax) of a float64 device vector."""
    slot = torch.empty(3, dtype=torch.float64, device=p.device)
    prob_stats_launch(p, slot)
    return prob_stats_read(slot.cpu())


def prob_categorical(p: torch.Tensor, u: float):
    lib = N.load()
    out = torch.empty(2, dtype=torch.int32, device=p.device)
    N.check(lib.dsr_prob_categorical(_ptr(p), p.numel(), float(u), _ptr(out), _stream()), "dsr_prob_categorical")
    tok, flags = out.cpu().tolist()
    return int(tok), int(flags)


def prob_correction_launch(p: torch.Tensor, q: torch.Tensor, status: torch.Tensor) -> torch.Tensor:
    """The normalised residual of ``p`` and ``q`` as a new device vector, its
    status into the int32 device view ``status``; nothing is synchronised."""
    lib = N.load()
    out = torch.empty_like(p)
    N.check(lib.dsr_prob_correction(_ptr(p), _ptr(q), p.numel(), _ptr(out), _ptr(status), _stream()),
            "dsr_prob_correction")
    return out


def prob_correction(p: torch.Tensor, q: torch.Tensor):
    st = torch.empty(1, dtype=torch.int32, device=p.device)
    out = prob_correction_launch(p, q, st)
    return out, int(st.item())


def prob_accept(p: torch.Tensor, q: torch.Tensor, x: int, u: float):
    lib = N.load()
    out = torch.empty(2, dtype=torch.int32, device=p.device)
    N.check(lib.dsr_prob_accept(_ptr(p), _ptr(q), p.numel(), int(x), float(u), _ptr(out), _stream()),
            "dsr_prob_accept")
    q_pos, ok = out.cpu().tolist()
    return bool(q_pos), bool(ok)
