"""Drop-in conformance on the CPU: the binding exposes the surface the
reference's unchanged decision layer calls (python/cujev/systemone.py:82-192),
and the caller restatement the GPU conformance tests drive is pinned by
brute force and closed forms."""
import inspect
import math

import numpy as np
import pytest

import cujev
from cujev import _lib
from systemone_caller import answer, confidence, pack_plan, softmax64


def test_engine_constructor_takes_the_layers_keywords():
    # python/cujev/systemone.py:82-85
    params = inspect.signature(cujev.Engine.__init__).parameters
    for kw in ("device", "max_state_tokens", "max_branch_tokens", "max_branches",
               "max_candidates", "verbose"):
        assert kw in params and params[kw].kind is inspect.Parameter.KEYWORD_ONLY
    for name in ("prefill", "eval", "eval_full_logits", "last_timing", "close"):
        assert callable(getattr(cujev.Engine, name))
    assert isinstance(cujev.Engine.version, property)


def test_value_types_construct_positionally():
    # Branch(toks, cands) at :150; Timing(t_prefill, eval_ms, n, n, n) at :192
    b = cujev.Branch([1, 2, 3], [7])
    assert list(b.tokens) == [1, 2, 3] and list(b.candidates) == [7]
    t = cujev.Timing(1.5, 2.5, 10, 20, 3)
    assert (t.prefill_ms, t.eval_ms, t.prefill_tokens, t.eval_tokens, t.eval_branches) == \
        (1.5, 2.5, 10, 20, 3)
    assert issubclass(cujev.EngineError, Exception)
    assert cujev.Timing is _lib.Timing and cujev.Branch is _lib.Branch


def _brute_plan(lengths, mb, mt):
    """Greedy packing by definition: each call is the longest prefix of the
    remaining branches that fits both budgets."""
    out, i = [], 0
    while i < len(lengths):
        best = i
        for j in range(i + 1, len(lengths) + 1):
            if j - i <= mb and sum(lengths[i:j]) <= mt:
                best = j
            else:
                break
        out.append((i, best))
        i = best
    return out


@pytest.mark.parametrize("seed", range(20))
def test_pack_plan_is_greedy_within_budgets(seed):
    rng = np.random.default_rng(seed)
    mb, mt = int(rng.integers(1, 6)), int(rng.integers(8, 64))
    lengths = [int(x) for x in rng.integers(1, mt + 1, size=int(rng.integers(0, 30)))]
    plan = pack_plan(lengths, mb, mt)
    assert plan == _brute_plan(lengths, mb, mt)
    assert [i for a, b in plan for i in range(a, b)] == list(range(len(lengths)))
    for a, b in plan:
        assert 0 < b - a <= mb and sum(lengths[a:b]) <= mt


def test_pack_plan_rejects_an_oversized_branch():
    with pytest.raises(ValueError):
        pack_plan([3, 70, 2], 4, 64)


def test_confidence_closed_forms():
    assert confidence(np.array([1.0])) == 1.0
    assert confidence(np.full(7, 1 / 7)) == pytest.approx(0.0, abs=1e-12)
    assert confidence(np.array([1.0, 0, 0, 0])) == pytest.approx(1.0, abs=1e-9)
    # two labels at p, 1-p: 1 - H2(p)/ln 2
    for p in (0.1, 0.3, 0.5, 0.9):
        h = -(p * math.log(p) + (1 - p) * math.log(1 - p))
        assert confidence(np.array([p, 1 - p])) == pytest.approx(1 - h / math.log(2))


def test_answers_from_logits():
    lg = np.log(np.array([0.1, 0.6, 0.3]))
    a = answer("choice", lg, ["x", "y", "z"])
    assert a["choice"] == "y"
    assert a["probabilities"]["z"] == pytest.approx(0.3)
    s = answer("score", lg)
    assert s["score"] == pytest.approx(0.6 + 2 * 0.3)
    n = answer("noul", np.array([0.0, 0.0]))
    assert n["noul"] == pytest.approx(0.5)
    # softmax is shift-invariant and sums to one in float64
    rng = np.random.default_rng(3)
    for _ in range(3):
        x = rng.normal(size=9) * 30
        p = softmax64(x)
        assert p.sum() == pytest.approx(1.0) and np.allclose(p, softmax64(x + 1e4))
