"""The calling sequence of the reference's unchanged Python decision layer
(python/cujev/systemone.py), restated as test infrastructure so the
conformance tests can drive this build's Engine exactly the way that layer
does, without shipping or running the reference's Python.

What the layer needs from the engine (python/cujev/systemone.py):
  - ``Engine(dir, device=, max_state_tokens=, max_branch_tokens=,
    max_branches=, max_candidates=256, verbose=)`` (:82-85), and the
    attributes ``name`` (:88), ``version`` (:90), ``max_state_tokens``
    (:141), ``max_branch_tokens`` (:154), ``max_branches`` (:167);
  - ``prefill(ids)`` once per distinct prefix token list (:157-160);
  - ``eval(list[Branch])`` -> per-branch float32 candidate logits in
    candidate order (:170), called on packs of branches that fit both
    budgets (:163-172); ``last_timing()`` with ``prefill_ms`` / ``eval_ms``
    (:161, :171); ``Branch(tokens, candidates)`` and the five-field
    ``Timing(prefill_ms, eval_ms, prefill_tokens, eval_tokens,
    eval_branches)`` (:192).
Answers (:174-190): softmax of the candidate logits in float64; "noul"
reports p[0]; "choice" the argmax option, the probabilities and the
confidence 1 - H(p)/ln K (:59-65; 1 for K = 1, clamped to [0, 1]); "score"
the expectation sum_i i p_i over the levels.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


def pack_plan(lengths, max_branches, max_branch_tokens):
    """Greedy in-order packing of branch lengths into eval calls: each call
    takes branches while both budgets hold (python/cujev/systemone.py:164-172).
    Returns [(start, stop)] ranges. A branch longer than the token budget is
    rejected before packing by the layer (:153-155); here it raises."""
    if lengths and max(lengths) > max_branch_tokens:
        raise ValueError("a branch exceeds max_branch_tokens")
    plan, i = [], 0
    while i < len(lengths):
        j, ntok = i, 0
        while (j < len(lengths) and j - i < max_branches
               and ntok + lengths[j] <= max_branch_tokens):
            ntok += lengths[j]
            j += 1
        plan.append((i, j))
        i = j
    return plan


def softmax64(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max())
    return e / e.sum()


def confidence(p):
    """1 - H(p)/ln K, clamped to [0, 1]; 1 when K <= 1."""
    k = len(p)
    if k <= 1:
        return 1.0
    h = -float(np.sum(p * np.log(np.clip(p, 1e-12, None))))
    return max(0.0, min(1.0, 1.0 - h / math.log(k)))


def answer(kind, logits, labels=None):
    p = softmax64(logits)
    if kind == "noul":
        return {"type": "noul", "noul": float(p[0])}
    if kind == "choice":
        return {"type": "choice", "choice": labels[int(p.argmax())],
                "probabilities": dict(zip(labels, map(float, p))), "confidence": confidence(p)}
    return {"type": "score", "score": float(np.sum(p * np.arange(len(p)))),
            "probabilities": {str(i): float(v) for i, v in enumerate(p)},
            "confidence": confidence(p)}


@dataclass
class Question:
    kind: str            # "noul" | "choice" | "score"
    tokens: list         # branch token ids (the prompt suffix)
    candidates: list     # candidate token ids, one per label
    labels: list | None = None


class Caller:
    """One engine behind the layer's lock-free core: prefix cache keyed by
    the token list, packed evals, answers."""

    def __init__(self, engine, branch_cls):
        self.engine, self.Branch = engine, branch_cls
        self.cached = None
        self.calls = []   # (branches, tokens) of every eval call made

    def evaluate(self, prefix, questions):
        if len(prefix) > self.engine.max_state_tokens:
            raise ValueError("state too long")
        hit = self.cached == list(prefix)
        if not hit:
            self.engine.prefill(prefix)
            self.cached = list(prefix)
        branches = [self.Branch(q.tokens, q.candidates) for q in questions]
        logits, eval_ms = [], 0.0
        for a, b in pack_plan([len(q.tokens) for q in questions], self.engine.max_branches,
                              self.engine.max_branch_tokens):
            logits.extend(self.engine.eval(branches[a:b]))
            t = self.engine.last_timing()
            eval_ms += t.eval_ms
            self.calls.append((b - a, sum(len(q.tokens) for q in questions[a:b]), t))
        answers = [answer(q.kind, lg, q.labels) for q, lg in zip(questions, logits)]
        return answers, logits, hit, eval_ms
