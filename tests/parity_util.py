"""Shared helpers of the GPU parity tests: run a workload through the HIP
library and through the oracle on the same inputs, and compare."""
from dataclasses import dataclass, field

import numpy as np
import torch

from deepseekrpc_amd import batch, workloads
from oracle import sampling_oracle as O

# A threshold decision closer than this to its boundary may legitimately
# differ between two float64 implementations (exp ulps, summation order).
MARGIN = 1e-11


def run_gpu(w, probs="f32", kept=True, hints=None):
    d = workloads.to_device(w)
    res = batch.sample_rows(d.logits, d.policies, history=d.history, allow_bits=d.allow_bits, uniforms=d.uniforms,
                            probs=probs, kept=kept, hints=hints)
    torch.cuda.synchronize()
    out = dict(tokens=res.tokens.cpu().numpy(), consumed=res.consumed.cpu().numpy(),
               status=res.status.cpu().numpy(), flags=res.flags.cpu().numpy())
    if res.probs is not None:
        out["probs"] = res.probs.cpu().numpy()
    if res.kept_bits is not None:
        out["kept"] = batch.unpack_bits(res.kept_bits.cpu().numpy().view(np.uint32), w.logits.shape[1])
    return out


def oracle_row(w, r):
    V = w.logits.shape[1]
    counts = gen = None
    if w.histories is not None:
        counts = np.bincount(np.asarray(w.histories[r]), minlength=V).astype(np.int32)
        gen = counts
    allowed = None if w.allowed is None else w.allowed[r]
    return O.sample_row(w.logits[r], O.Policy(**w.policies[r]), float(w.uniforms[r]), counts, gen, None, allowed)


@dataclass
class Report:
    rows: int = 0
    exact: int = 0
    margin_rows: list = field(default_factory=list)   # differing rows inside the oracle's rounding band
    flagged: int = 0                                  # agreeing rows the kernel flagged as near a boundary
    mismatches: list = field(default_factory=list)    # real disagreements
    max_rel: float = 0.0


def compare(w, gpu, rows=None, prob_rtol=1e-5):
    rows = range(w.rows) if rows is None else rows
    rep = Report()
    for r in rows:
        ref = oracle_row(w, r)
        rep.rows += 1
        flagged = bool(gpu["flags"][r] & 1)  # the kernel's own rounding-band flag
        near = ref.margin < MARGIN
        if gpu["status"][r] != ref.status:
            rep.mismatches.append((r, "status", int(gpu["status"][r]), ref.status))
            continue
        if ref.status != O.OK:
            rep.exact += 1
            continue
        same = gpu["tokens"][r] == ref.token and bool(gpu["consumed"][r]) == ref.consumed
        if "kept" in gpu and not np.array_equal(gpu["kept"][r], ref.topk_kept):
            rep.mismatches.append((r, "top-k set", int(np.sum(gpu["kept"][r] != ref.topk_kept)), 0))
        if "probs" in gpu:
            g, o = gpu["probs"][r].astype(np.float64), ref.probs
            pos = o > 0
            if np.any(g[~pos] > 1e-300) and not near:
                rep.mismatches.append((r, "support", int(np.sum(g[~pos] > 0)), 0))
            if pos.any():
                rel = float(np.max(np.abs(g[pos] - o[pos]) / o[pos]))
                if not near:
                    rep.max_rel = max(rep.max_rel, rel)
                if rel > prob_rtol and not near:
                    rep.mismatches.append((r, "probs", rel, prob_rtol))
        if same:
            rep.exact += 1
            if flagged:
                rep.flagged += 1
        elif near:
            # The oracle's own decision sat within MARGIN of its threshold: a
            # different float64 exp / summation order may pick the neighbour.
            rep.margin_rows.append(r)
        else:
            rep.mismatches.append((r, "token", int(gpu["tokens"][r]), ref.token))
    return rep
