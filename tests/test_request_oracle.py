"""The streaming request oracle (oracle/request.py) against the whole-model
oracle (oracle.qwen35.model_last_logits, itself pinned by transformers'
golden logits in tests/test_golden.py) on a seeded tiny checkpoint.

A request's shared-prefix decomposition -- the state prefilled once, each
branch attending to the state's K/V plus its own prefix and continuing the
state's GDN recurrence and conv tail -- must give every branch the logits of
plain causal processing of [state ++ branch] (REF src/engine/forward.c:50-149):
  * "f64" track == model_last_logits in float64, to summation-order roundoff;
  * "engine" track == model_last_logits(engine_numerics=True): the same bf16
    rounding points (bit-equal on this request; the bar, 1e-6 absolute,
    leaves room only for float64 reordering that crosses no bf16 boundary);
  * candidate logits are the full logits at the candidate ids;
  * a planted mistake (the state one token short) is caught.
"""
import numpy as np
import pytest

from cujev import synthetic
from oracle import qwen35 as q35
from oracle import request as rq


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    d = tmp_path_factory.mktemp("tiny_req")
    cfg = synthetic.make_config(**synthetic.PRESETS["tiny"])
    synthetic.write_checkpoint(d, cfg, seed=5, norm_std=0.1)
    return str(d), q35.load_checkpoint(str(d))


def request(seed=0):
    rng = np.random.default_rng(seed)
    state = [int(x) for x in rng.integers(16, 4096, size=70)]
    branches = []
    for n in (20, 1, 65):
        toks = [int(x) for x in rng.integers(16, 4096, size=n)]
        cands = [int(x) for x in rng.choice(np.arange(16, 4096), size=5, replace=False)]
        branches.append((toks, cands))
    return state, branches


def test_request_oracle_equals_whole_model(tiny):
    path, (cfg, W) = tiny
    state, branches = request()
    out = rq.request_logits(path, state, branches, modes=("f64", "engine"), full=True)
    for i, (toks, cands) in enumerate(branches):
        ids = state + toks
        ref64 = q35.model_last_logits(cfg, W, ids)
        refe = q35.model_last_logits(cfg, W, ids, engine_numerics=True)
        got64, gote = out["f64"]["full"][i], out["engine"]["full"][i]
        e64 = np.abs(got64 - ref64).max() / np.abs(ref64).max()
        ee = np.abs(gote - refe).max()
        print(f"branch {i} (len {len(toks)}): f64 rel {e64:.2e}, engine max |dlogit| {ee:.2e}")
        assert e64 <= 1e-9
        assert ee <= 1e-6
        for m in ("f64", "engine"):
            assert np.array_equal(out[m]["cand"][i], out[m]["full"][i][cands])


def test_request_oracle_catches_a_short_state(tiny):
    path, (cfg, W) = tiny
    state, branches = request(1)
    out = rq.request_logits(path, state[:-1], branches[:1], modes=("f64",), full=True)
    ref = q35.model_last_logits(cfg, W, state + branches[0][0])
    assert np.abs(out["f64"]["full"][0] - ref).max() / np.abs(ref).max() > 1e-3


def _scan_inputs(seed=3, T=150, H=2, d=32):
    rng = np.random.default_rng(seed)
    rb = lambda x: q35.bf16_round(np.asarray(x, np.float32)).astype(np.float64)
    # q and k as the kernel stages them (about 16 significant bits: the
    # split pair), so that their single bf16 operands Q and KT are roundings
    # of their own
    q = rng.normal(size=(T, H, d)) / np.sqrt(d)
    k = rng.normal(size=(T, H, d))
    k = k / np.linalg.norm(k, axis=-1, keepdims=True)
    v = rb(rng.normal(size=(T, H, d)))
    g = -np.log1p(np.exp(rng.normal(size=(T, H))))
    beta = 1.0 / (1.0 + np.exp(-rng.normal(size=(T, H))))
    S0 = rng.normal(size=(H, d, d)) * 0.1
    return q, k, v, g, beta, S0


OPS = ("S", "Vp", "T", "W", "U", "Q", "QK", "KT", "O")


def test_emulated_kernel_scan_is_pinned_to_the_chunked_form():
    """oracle.request.gdn_chunk_emulated (the kernel's rounding points, used
    for attribution statistics): with every operand carried as a split pair
    it is the float64 chunked scan to split-bf16 precision; leaving any one
    operand as plain bf16 moves it by about a bf16 rounding."""
    q, k, v, g, beta, S0 = _scan_inputs()
    o_ref, S_ref = q35.gdn_chunked(q, k, v, g, beta, S0)
    rel = lambda a, b: float(np.abs(a - b).max() / np.abs(b).max())
    o_all, S_all = rq.gdn_chunk_emulated(q, k, v, g, beta, S0, split=OPS)
    assert rel(o_all, o_ref) <= 1e-4 and rel(S_all, S_ref) <= 1e-4
    for op in OPS:
        o1, S1 = rq.gdn_chunk_emulated(q, k, v, g, beta, S0, split=tuple(x for x in OPS if x != op))
        e = max(rel(o1, o_ref), rel(S1, S_ref))
        print(f"{op} as plain bf16: {e:.2e}")
        assert 2e-5 < e <= 3e-2, op
