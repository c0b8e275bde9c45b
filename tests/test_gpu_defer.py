"""Deferred prefill (CUJEV_DEFER_PREFILL) through the public C ABI, on the
seeded tiny checkpoint of the engine tests.

With =1 a prefill only stages its tokens; the state's next eval runs one
pass over [state ++ branch tokens]: embedding, projections and norms once
over all of them, attention and GDN per group (the state's group writes the
K/V cache, S and conv tail that the branch group then reads). With =2 the
eval runs the staged prefill on its own first, i.e. the same kernels as an
eager prefill followed by an eval.

Checked: fused evals against the eager engine and the float64 oracle, at
state and branch lengths that straddle the 16/32-token query tiles, 64-key
tiles and 64-token GDN chunks, with the GEMMs on the few-token, hand-tiled
and hipBLASLt paths (the call's token count picks them) and with packed GDN
chunks; the state left behind by a fused eval against an eager prefill's;
full-vocabulary logits; the =2 path bit for bit against eager; timing and
argument checks. Bars as in test_gpu_engine.py: candidate probabilities
within 3e-3 of the oracle (the engine's bf16 rounding points, and float64),
and of the eager engine, whose GEMMs sum the state tokens' projections over
another token count (another tile and split choice: an equally valid fp32
order, so not bit for bit).
"""
import os
from contextlib import contextmanager

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from cujev import Branch, Engine, EngineError, synthetic  # noqa: E402
from oracle import qwen35 as orc  # noqa: E402

pytestmark = pytest.mark.gpu
PROB_TOL = 3e-3
OPTS = dict(max_state_tokens=1024, max_branch_tokens=512, max_branches=64, max_candidates=256)


@contextmanager
def env(**kv):
    old = {k: os.environ.get(k) for k in kv}
    os.environ.update({k: str(v) for k, v in kv.items()})
    try:
        yield
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def open_engine(ckpt, mode):
    with env(CUJEV_DEFER_PREFILL=mode):
        return Engine(ckpt, **OPTS)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("tiny_defer")
    cfg = synthetic.make_config(**synthetic.PRESETS["tiny"])
    synthetic.write_checkpoint(d, cfg, seed=0, norm_std=0.1)
    return str(d)


@pytest.fixture(scope="module")
def oracle(ckpt):
    return orc.load_checkpoint(ckpt)


@pytest.fixture(scope="module")
def engines(ckpt):
    es = {m: open_engine(ckpt, m) for m in ("0", "1", "2")}
    yield es
    for e in es.values():
        e.close()


def rand_ids(rng, n, vocab=4096):
    return [int(x) for x in rng.integers(16, vocab, size=n)]


def softmax(x):
    x = np.asarray(x, np.float64)
    p = np.exp(x - x.max())
    return p / p.sum()


def max_dp(a, b):
    return float(np.abs(softmax(a) - softmax(b)).max())


def run(e, prefix, branches):
    e.prefill(prefix)
    return e.eval(branches)


SHAPES = [  # (state length, branch lengths)
    (1, [1]),
    (17, [4, 20, 20, 20]),
    (64, [33]),
    (65, [70, 5, 1]),   # a branch over two GDN chunks
    (200, [20] * 4),
    (530, [20] * 4),    # the config-4 request shape
    (300, [12] * 30),   # many short branches
]


@pytest.mark.parametrize("plen,blens", SHAPES)
def test_fused_matches_eager_and_oracle(engines, oracle, plen, blens):
    cfg, W = oracle
    rng = np.random.default_rng(plen * 7 + len(blens))
    prefix = rand_ids(rng, plen)
    branches = [Branch(rand_ids(rng, n), [int(x) for x in rng.integers(16, 4096, size=6)])
                for n in blens]
    print(f"case P={plen} branches={blens}", flush=True)
    eager = run(engines["0"], prefix, branches)
    fused = run(engines["1"], prefix, branches)
    worst = max(max_dp(f, e) for f, e in zip(fused, eager))
    for b, lg in list(zip(branches, fused))[:: max(1, len(branches) // 3)]:
        ids = prefix + list(b.tokens)
        ref = orc.model_last_logits(cfg, W, ids, engine_numerics=True)[list(b.candidates)]
        ref64 = orc.model_last_logits(cfg, W, ids)[list(b.candidates)]
        d, d64 = max_dp(lg, ref), max_dp(lg, ref64)
        print(f"  branch len {len(b.tokens)}: vs oracle max|dp| {d:.2e}, vs fp64 {d64:.2e}")
        assert d <= PROB_TOL and d64 <= PROB_TOL
    print(f"  fused vs eager engine: max|dp| {worst:.2e}")
    assert worst <= PROB_TOL


@pytest.mark.parametrize("pack_min", ["0", "-1"])
def test_fused_with_packed_chunks(engines, oracle, monkeypatch, pack_min):
    """The branch group's GDN chunks packed several branches to a chunk
    (threshold 0) and one per chunk (packing off), behind a 90-token state."""
    monkeypatch.setenv("CUJEV_GDN_PACK_MIN_UNITS", pack_min)
    rng = np.random.default_rng(21)
    prefix = rand_ids(rng, 90)
    branches = [Branch(rand_ids(rng, int(n)), [int(x) for x in rng.integers(16, 4096, size=5)])
                for n in rng.integers(1, 12, size=24)]
    eager = run(engines["0"], prefix, branches)
    fused = run(engines["1"], prefix, branches)
    worst = max(max_dp(f, e) for f, e in zip(fused, eager))
    print(f"packing threshold {pack_min}: fused vs eager max|dp| {worst:.2e}")
    assert worst <= PROB_TOL


def test_state_after_fused_eval(engines):
    """After a fused eval the state is current: later evals (eager, then
    replayed from a captured graph) agree with an eager prefill's."""
    rng = np.random.default_rng(4)
    prefix = rand_ids(rng, 150)
    first = [Branch(rand_ids(rng, 9), [1, 2, 3])]
    later = [Branch(rand_ids(rng, 20), [int(x) for x in rng.integers(16, 4096, size=8)])
             for _ in range(3)]
    e0, e1 = engines["0"], engines["1"]
    e0.prefill(prefix)
    ref = e0.eval(later)
    e1.prefill(prefix)
    e1.eval(first)
    got = [e1.eval(later) for _ in range(3)]  # eager, captured, replayed
    for g in got:
        assert max(max_dp(a, b) for a, b in zip(g, ref)) <= PROB_TOL
    np.testing.assert_array_equal(np.asarray(got[1]), np.asarray(got[2]))


def test_full_logits_with_pending_prefill(engines):
    rng = np.random.default_rng(8)
    prefix, suffix = rand_ids(rng, 70), rand_ids(rng, 6)
    engines["0"].prefill(prefix)
    ref = engines["0"].eval_full_logits([Branch(suffix, [])])[0]
    engines["1"].prefill(prefix)
    got = engines["1"].eval_full_logits([Branch(suffix, [])])[0]
    d = max_dp(got, ref)
    print(f"full logits, fused vs eager: max|dp| {d:.2e}")
    assert d <= PROB_TOL and np.all(np.isfinite(got))


def test_staged_prefill_is_the_eager_path(engines):
    """=2 runs the staged prefill by itself at the eval: the same kernels on
    the same inputs as an eager prefill, so the same bits."""
    rng = np.random.default_rng(6)
    prefix = rand_ids(rng, 97)
    branches = [Branch(rand_ids(rng, n), [7, 8, 9, 10]) for n in (5, 40, 17)]
    a = run(engines["0"], prefix, branches)
    b = run(engines["2"], prefix, branches)
    np.testing.assert_array_equal(np.asarray(a), np.asarray(b))


def test_restaged_prefill_and_timing(engines):
    """A second prefill replaces a staged one; the staged prefill reports
    0 ms, the eval that runs it reports the whole pass."""
    e0, e1 = engines["0"], engines["1"]
    rng = np.random.default_rng(9)
    p1, p2 = rand_ids(rng, 40), rand_ids(rng, 55)
    br = [Branch(rand_ids(rng, 7), [3, 4, 5])]
    e1.prefill(p1)
    e1.prefill(p2)
    t = e1.last_timing()
    assert t.prefill_ms == 0 and t.prefill_tokens == 55
    got = e1.eval(br)[0]
    t = e1.last_timing()
    assert t.eval_ms > 0 and t.eval_tokens == 7 and t.eval_branches == 1
    assert max_dp(got, run(e0, p2, br)[0]) <= PROB_TOL


def test_deferred_prefill_checks_arguments(engines):
    e = engines["1"]
    with pytest.raises(EngineError):
        e.prefill([1] * 1025)
    with pytest.raises(EngineError):
        e.prefill([e.vocab_size])
    e.prefill([1, 2, 3])
    with pytest.raises(EngineError):
        e.eval([Branch([4] * 513, [1])])
    lg = e.eval([Branch([4, 5], [1, 2])])[0]
    assert np.all(np.isfinite(lg))
