"""Write the golden vectors that only the reference itself can pin.

Run only where the reference sources are present (the GPU tests read the
committed vectors, never the reference):

    PYTHONPATH=/root/reference/src python tests/golden/make_golden.py

It imports the reference's sampling modules (src/deepseekrpc/sampling.py,
src/deepseekrpc/terminal_sampling.py) and records inputs and outputs for:

* ``SamplingPolicy.probabilities`` float64 vectors on moderate vocabularies
  (NumPy pairwise sums, double normalisation, stable tie rules) including
  near-tie rows where the sequential cumsum decides a top-p cut;
* ``categorical`` ids for fixed uniforms;
* ``verify_drafts`` decisions with fixed uniforms;
* absolute ``RandomStreams`` draws and snapshots (PCG64 via NumPy);
* ``SamplingWork.prepared()["digest"]`` bytes for fixed scenarios.

Only data is written (``sampling_golden.npz`` and ``sampling_golden.json``).
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_round(x):
    """Round-to-nearest-even float32 -> bfloat16, returned as float32."""
    a = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    a = (a + 0x7FFF + ((a >> 16) & 1)) & 0xFFFF0000
    return a.astype(np.uint32).view(np.float32)


def cases(rng):
    """Yield ``(name, logits, policy_kwargs, counts, generated, bias, allowed)``."""
    V = 4096
    yield ("c1_like", rng.normal(0, 2, V).astype(np.float32),
           dict(temperature=0.7, top_k=50, top_p=0.9), None, None, None, None)
    hist = rng.integers(0, V, 512)
    counts = np.bincount(hist, minlength=V).astype(np.int32)
    yield ("c2_like", bf16_round(rng.normal(0, 3, V)),
           dict(temperature=1.0, top_p=0.95, repetition_penalty=1.1, presence_penalty=0.5, frequency_penalty=0.3),
           counts, counts.copy(), None, None)
    x = rng.normal(0, 1, V)
    spikes = rng.choice(V, 32, replace=False)
    x[spikes] += rng.uniform(8, 15, 32)
    allowed = rng.random(V) < 0.9
    yield ("c3_like", bf16_round(x), dict(temperature=0.5, top_k=300, top_p=0.8), None, None, None, allowed)
    for i in range(3):
        y = rng.uniform(-1e-3, 1e-3, V)
        y[rng.choice(V, 8, replace=False)] = y.max()
        hist = rng.integers(0, V, 1024)
        c = np.bincount(hist, minlength=V).astype(np.int32)
        yield (f"c5_neartie_{i}", bf16_round(y),
               dict(temperature=1.0, top_p=0.9, repetition_penalty=1.1, presence_penalty=0.5, frequency_penalty=0.3),
               c, c.copy(), None, None)
    prompt = np.bincount(rng.integers(0, V, 300), minlength=V).astype(np.int32)
    gen_part = np.bincount(rng.integers(0, V, 200), minlength=V).astype(np.int32)
    bias = {int(t): float(b) for t, b in zip(rng.choice(V, 16, replace=False), rng.uniform(-5, 5, 16))}
    yield ("minp_bias_split", rng.normal(0, 1.5, V).astype(np.float32),
           dict(temperature=1.3, min_p=0.05, repetition_penalty=1.3, presence_penalty=-0.4, frequency_penalty=0.2),
           prompt + gen_part, gen_part, bias, None)
    g = bf16_round(rng.normal(0, 1, V))
    g[[17, 900, 3000]] = g.max() + 1
    yield ("greedy_ties", g, dict(temperature=0.0), None, None, None, None)
    yield ("tiny_temperature", g, dict(temperature=1e-320), None, None, None, None)
    yield ("top1", rng.normal(0, 1, V).astype(np.float32), dict(top_p=0.0, top_k=1), None, None, None, None)
    z = rng.normal(0, 4, V)
    z[rng.choice(V, 200, replace=False)] = -np.inf
    yield ("f64_neginf", z, dict(temperature=2.5, top_k=1000, top_p=0.99, min_p=0.001), None, None, None, None)
    yield ("full_vocab_default", bf16_round(rng.normal(0, 2, 129280)), dict(), None, None, None, None)
    w = rng.normal(0, 1, 129280)
    w[rng.choice(129280, 32, replace=False)] += rng.uniform(8, 15, 32)
    yield ("full_vocab_c3", bf16_round(w), dict(temperature=0.9, top_k=700, top_p=0.93), None, None, None,
           rng.random(129280) < 0.9)


class Uniforms:
    def __init__(self, accept, target):
        self.accept, self.target = list(accept), target
        self.calls = []

    def random(self, domain):
        self.calls.append(domain)
        return self.accept.pop(0) if domain == "accept" else self.target


def main():
    from deepseekrpc import sampling, terminal_sampling

    rng = np.random.default_rng(20261201)
    arrays, meta = {}, {"probabilities": [], "verify": [], "rng": [], "digests": []}
    for name, logits, kw, counts, gen, bias, allowed in cases(rng):
        policy = sampling.SamplingPolicy(**kw)
        p = policy.probabilities(logits, counts=counts, generated_counts=gen, logit_bias=bias, allowed=allowed)
        us = [float(u) for u in rng.random(3)]
        ids = [sampling.categorical(p, lambda u=u: u) for u in us]
        if len(logits) > 8192:
            # Full-vocabulary rows: bf16 logits as their 16-bit patterns, and
            # the float64 output pinned by its SHA-256 plus a few entries.
            arrays[f"{name}/logits_bf16"] = (np.asarray(logits, np.float32).view(np.uint32) >> 16).astype(np.uint16)
            top = np.argsort(-p, kind="stable")[:64]
            arrays[f"{name}/probs_top_idx"] = top
            arrays[f"{name}/probs_top_val"] = p[top]
            meta.setdefault("hashes", {})[name] = hashlib.sha256(p.tobytes()).hexdigest()
        else:
            arrays[f"{name}/logits"] = logits
            arrays[f"{name}/probs"] = p
        if counts is not None:
            arrays[f"{name}/counts"] = counts
            arrays[f"{name}/generated"] = gen
        if allowed is not None:
            arrays[f"{name}/allowed"] = np.packbits(allowed)
        meta["probabilities"].append({"name": name, "policy": policy.as_dict(), "uniforms": us, "ids": ids,
                                      "bias": None if bias is None else [[t, b] for t, b in bias.items()]})

    V, K = 512, 4
    for i, kw in enumerate([dict(), dict(temperature=0.8, top_k=40, top_p=0.9), dict(temperature=0.0)] * 2):
        policy = sampling.SamplingPolicy(**kw)
        tgt = rng.normal(0, 2, (K + 1, V)).astype(np.float32)
        drf = (tgt[:K] + rng.normal(0, 0.5, (K, V))).astype(np.float32)
        qs = [policy.probabilities(drf[j]) for j in range(K)]
        ids = [int(sampling.categorical(q, lambda: float(rng.random()))) for q in qs]
        ps = [policy.probabilities(tgt[j]) for j in range(K + 1)]
        ua = [float(u) for u in rng.random(K)]
        ut = float(rng.random())
        draws = Uniforms(ua, ut)
        limit = [10, 10, 10, 3, 2, 10][i]
        eos = [[], [], [], [], [], [ids[1]]][i]
        d = sampling.verify_drafts(ps, qs, ids, draws, greedy=policy.temperature == 0, output_limit=limit,
                                   eos_ids=frozenset(eos))
        arrays[f"verify{i}/target"] = tgt
        arrays[f"verify{i}/draft"] = drf
        meta["verify"].append({"name": f"verify{i}", "policy": policy.as_dict(), "ids": ids, "u_accept": ua,
                               "u_target": ut, "limit": limit, "eos": eos, "accepted": d.accepted_drafts,
                               "output_ids": list(d.output_ids), "pending": d.pending_token,
                               "stop": d.stop_reason, "calls": draws.calls})

    for seed in (0, 1017, (1 << 64) - 1):
        streams = sampling.RandomStreams(seed)
        snap = streams.snapshot()
        txn = streams.begin()
        draws = {d: [txn.random(d) for _ in range(8)] for d in sampling.DOMAINS}
        after = txn.commit()
        meta["rng"].append({"seed": seed, "snapshot": snap, "draws": draws, "after": after})

    # Digest scenarios (terminal_sampling.py:185-198).
    sampler = terminal_sampling.TerminalSampler(1017, vocabulary=8)
    counts = np.array([1, 0, 2, 0, 0, 1, 0, 0], np.int32)
    seed_logits = np.array([[0.5, 1.0, -0.25, 2.0, 0.0, 1.5, -1.0, 0.75]], np.float32)
    work = sampler.begin_seed(seed_logits, policy=sampling.SamplingPolicy(temperature=0.9, top_k=5),
                              counts=counts, remaining=6, eos_ids={7})
    meta["digests"].append({"name": "seed", "decision": list(work.decision.output_ids),
                            "digest": work.prepared()["digest"]})
    work.commit(work.prepared()["digest"])
    counts[work.decision.token] += 1

    class Graph:
        def draft_conditional_logits(self, result, row, previous):
            base = np.array([[0.1, 0.4, -0.3, 0.9, 0.2, 0.0, -0.6, 0.3]], np.float32)
            base[0, previous] += 0.5
            return base, None

    work = sampler.begin_verification(seed_token=work.decision.token, policy=sampling.SamplingPolicy(top_p=0.95),
                                      counts=counts, remaining=6, eos_ids={7},
                                      logit_bias={2: 1.25, 5: -0.5})
    proposals = work.propose(Graph(), None)
    target = np.linspace(-1, 1, 8 * (len(proposals) + 1), dtype=np.float32).reshape(len(proposals) + 1, 8)
    decision = work.verify(target)
    meta["digests"].append({"name": "verify", "proposals": list(proposals), "target": target.tolist(),
                            "decision": [decision.accepted_drafts, list(decision.output_ids),
                                         decision.pending_token, decision.stop_reason],
                            "digest": work.prepared()["digest"], "counts": counts.tolist()})
    work.commit(work.prepared()["digest"])
    meta["digests"].append({"name": "final_rng", "snapshot": sampler.random.snapshot()})

    np.savez_compressed(os.path.join(HERE, "sampling_golden.npz"), **arrays)
    with open(os.path.join(HERE, "sampling_golden.json"), "w") as fh:
        json.dump(meta, fh, indent=1, sort_keys=True)
    print("wrote", len(arrays), "arrays;", {k: len(v) for k, v in meta.items()})


if __name__ == "__main__":
    sys.exit(main())
