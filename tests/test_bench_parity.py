"""bench.py's parity field against the config-4 golden fixture, on the CPU:
the comparison logic is fed vectors whose answers the fixture already holds.

* The fixture's own "engine" label logits as the engine's output: zero
  deviation from the "engine" oracle, identical argmax everywhere, and the
  "f64" deviation equals the reference numerics' own distance from float64.
* A jitter seed's label logits as the engine's output: bench.py's max |dp|
  equals the statistic make_request_4b.py stored for that seed (computed
  there from the full logits, independently of bench.py).
* A request that is not the fixture's is refused (no comparison made).
"""
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests" / "golden"))

import bench  # noqa: E402
import make_request_4b as fx  # noqa: E402


@pytest.fixture(scope="module")
def g():
    return np.load(fx.OUT, allow_pickle=False)


def _labels(g, mode):
    modes = [str(m) for m in g["label_modes"]]
    v = g["label_logits"][modes.index(mode)]
    offs = np.concatenate([[0], np.cumsum(g["cand_len"])])
    return [v[offs[i]:offs[i + 1]] for i in range(len(offs) - 1)]


def test_fixture_request_is_the_bench_request(g):
    rng = np.random.default_rng(0)
    state, brs = bench.make_request(rng, 248320)
    s2, b2 = fx.request()
    assert state == s2 and brs == b2


def test_parity_field_on_known_vectors(g):
    pin = {"checkpoint_sha256": str(g["checkpoint_sha256"]),
           "fixture_sha256": str(g["checkpoint_sha256"]), "matches": True}
    req = fx.request()
    outs = {"deferred": _labels(g, "engine"), "eager": _labels(g, "engine~1")}
    full = np.zeros((4, 248320))
    full[:, g["sample_ids"]] = g["sample_engine"]
    r = bench.fixture_parity(pin, req, outs, full)
    assert r["request_matches_fixture"]
    d = r["engine"]["deferred"]
    assert d["max_abs_dprob_vs_engine_oracle"] == 0.0
    assert d["argmax_identical_engine_oracle"]
    assert d["rms_dlogit_vs_engine_oracle"] < 1e-6  # float32 storage of the sample
    assert d["max_abs_dprob_vs_f64_oracle"] == r["reference_engine_vs_f64"]["max_abs_dprob"]
    stats = dict(zip([str(m) for m in g["stat_modes"]], g["stat_values"]))
    e = r["engine"]["eager"]
    assert e["max_abs_dprob_vs_engine_oracle"] == pytest.approx(stats["engine~1"][2], abs=1e-5)
    assert r["noise_floor"]["max_abs_dprob"] == pytest.approx(
        max(v[2] for m, v in stats.items() if m.startswith("engine~")), abs=1e-5)
    for b in d["branches"]:
        assert b["argmax_agrees"] and b["margin_engine"] == b["margin_engine_oracle"]


def test_parity_field_refuses_another_request(g):
    pin = {"checkpoint_sha256": "x", "fixture_sha256": str(g["checkpoint_sha256"]),
           "matches": False}
    r = bench.fixture_parity(pin, fx.request(), {"deferred": _labels(g, "engine")}, None)
    assert not r["request_matches_fixture"] and "error" in r
