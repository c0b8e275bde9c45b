"""Drop-in conformance on the GPU: this build's Engine driven by the
reference decision layer's calling sequence (tests/systemone_caller.py,
restating python/cujev/systemone.py:131-194), on a seeded tiny checkpoint.

  - the attributes the layer reads equal the options it passed;
  - packing under tight budgets (3 branches / 48 tokens per eval call) gives
    the answers one unpacked call gives: candidate probabilities within the
    engine tests' bar (3e-3; batch composition changes the attention key
    split and the GEMM row count, so the bf16 rounding of the two runs is
    not the same), identical choices where the top-2 margin exceeds 2e-2;
  - the prefix cache: an unchanged prefix is not prefilled again and the
    same packed calls reproduce their logits bit for bit;
  - last_timing() describes the last packed call.
"""
import numpy as np
import pytest

pytest.importorskip("torch")

from cujev import Branch, Engine, EngineError, synthetic  # noqa: E402
from systemone_caller import Caller, Question, pack_plan, softmax64  # noqa: E402

pytestmark = pytest.mark.gpu
PROB_TOL = 3e-3


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("tiny_dropin")
    cfg = synthetic.make_config(**synthetic.PRESETS["tiny"])
    synthetic.write_checkpoint(d, cfg, seed=3, norm_std=0.1)
    return str(d)


def questions(rng):
    lens = [5, 17, 30, 12, 1, 25, 9, 40, 3]
    kinds = ["noul", "choice", "score", "choice", "noul", "score", "choice", "choice", "score"]
    out = []
    for n, kind in zip(lens, kinds):
        k = {"noul": 2, "choice": int(rng.integers(2, 7)), "score": int(rng.integers(2, 11))}[kind]
        cands = [int(x) for x in rng.choice(np.arange(16, 1000), size=k, replace=False)]
        labels = [f"o{i}" for i in range(k)] if kind == "choice" else None
        out.append(Question(kind, [int(x) for x in rng.integers(16, 4096, size=n)], cands,
                            labels))
    return out


def test_packed_answers_match_one_call(ckpt):
    rng = np.random.default_rng(11)
    prefix = [int(x) for x in rng.integers(16, 4096, size=150)]
    qs = questions(rng)
    with Engine(ckpt, max_state_tokens=256, max_branch_tokens=48, max_branches=3) as tight, \
            Engine(ckpt, max_state_tokens=256, max_branch_tokens=512, max_branches=64) as wide:
        for e, (mst, mbt, mb) in ((tight, (256, 48, 3)), (wide, (256, 512, 64))):
            assert (e.max_state_tokens, e.max_branch_tokens, e.max_branches) == (mst, mbt, mb)
            assert e.max_candidates == 256 and e.name and e.version
        ct, cw = Caller(tight, Branch), Caller(wide, Branch)
        at, lt, hit_t, _ = ct.evaluate(prefix, qs)
        aw, lw, hit_w, _ = cw.evaluate(prefix, qs)
        assert not hit_t and not hit_w
        plan = pack_plan([len(q.tokens) for q in qs], 3, 48)
        assert len(ct.calls) == len(plan) >= 4 and len(cw.calls) == 1
        worst = 0.0
        for q, a, b, x, y in zip(qs, at, aw, lt, lw):
            assert x.dtype == np.float32 and x.shape == (len(q.candidates),)
            dp = np.abs(softmax64(x) - softmax64(y)).max()
            worst = max(worst, dp)
            srt = np.sort(np.asarray(y, np.float64))
            if q.kind == "choice" and srt[-1] - srt[-2] > 2e-2:
                assert a["choice"] == b["choice"]
            assert 0.0 <= a.get("confidence", 1.0) <= 1.0
        print(f"packed vs one call: max|dp| {worst:.2e} over {len(qs)} questions, "
              f"{len(plan)} packed calls")
        assert worst <= PROB_TOL


def test_prefix_cache_and_timing(ckpt):
    rng = np.random.default_rng(12)
    prefix = [int(x) for x in rng.integers(16, 4096, size=90)]
    qs = questions(rng)
    with Engine(ckpt, max_state_tokens=128, max_branch_tokens=48, max_branches=3) as e:
        c = Caller(e, Branch)
        _, l1, hit1, _ = c.evaluate(prefix, qs)
        t_first = e.last_timing()
        _, l2, hit2, _ = c.evaluate(prefix, qs)
        assert not hit1 and hit2
        for x, y in zip(l1, l2):
            assert np.array_equal(x, y)
        # the last packed call's timing record
        n_br, n_tok, t = c.calls[-1]
        assert (t.eval_branches, t.eval_tokens) == (n_br, n_tok)
        assert t.prefill_tokens == len(prefix) and t.eval_ms > 0 and t_first.prefill_ms > 0
        # a new prefix is prefilled and changes the answers
        _, l3, hit3, _ = c.evaluate(prefix[:-1] + [17], qs)
        assert not hit3 and any(not np.array_equal(x, y) for x, y in zip(l1, l3))
        # what the layer's own checks keep out, the engine refuses too
        with pytest.raises(EngineError):
            e.eval([Branch(list(range(16, 16 + 49)), [20])])
        with pytest.raises(EngineError):
            e.eval([Branch([20], [21])] * 4)
        with pytest.raises(EngineError):
            e.prefill(list(range(16, 16 + 129)))


def test_deferred_prefill_under_the_layer(ckpt, monkeypatch):
    """The same calling sequence with CUJEV_DEFER_PREFILL=1: the first packed
    eval after a prefill runs the fused pass (prefill + branches), later ones
    read the state it left. Answers as the default engine's (the bar above);
    the repeat hits the prefix cache and reproduces every packed call but the
    first (which ran fused the first time) bit for bit; the prefill reports
    no time of its own."""
    rng = np.random.default_rng(13)
    prefix = [int(x) for x in rng.integers(16, 4096, size=120)]
    qs = questions(rng)
    opts = dict(max_state_tokens=256, max_branch_tokens=48, max_branches=3)
    with Engine(ckpt, **opts) as eager:
        _, le, _, _ = Caller(eager, Branch).evaluate(prefix, qs)
    monkeypatch.setenv("CUJEV_DEFER_PREFILL", "1")
    with Engine(ckpt, **opts) as e:
        c = Caller(e, Branch)
        _, l1, hit1, _ = c.evaluate(prefix, qs)
        assert not hit1 and e.last_timing().prefill_ms == 0
        _, l2, hit2, _ = c.evaluate(prefix, qs)
        assert hit2
    worst = max(np.abs(softmax64(x) - softmax64(y)).max() for x, y in zip(l1, le))
    first = c.calls[0][0]  # branches of the first packed call
    for x, y in list(zip(l1, l2))[first:]:
        assert np.array_equal(x, y)
    print(f"deferred vs default engine: max|dp| {worst:.2e}; first packed call "
          f"{first} branches")
    assert worst <= PROB_TOL
