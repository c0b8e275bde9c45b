"""Config 1 on the CPU: the oracle's shared-prefix gated attention layer
(oracle.qwen35.gated_attention_layer: projection, q/k norm, partial RoPE,
state + own-prefix attention, sigmoid gate, o_proj) against transformers'
Qwen3_5Attention run over every [state ++ branch] sequence
(tests/golden/attention_layer_cfg1.npz, written by
tests/golden/make_attention_layer.py), at config 1's shapes and seed.

Bar: max |oracle - transformers| / max |transformers| <= 1e-5 (float64
against float32). Planted mistakes in the oracle (RoPE base, gate, GQA head
map, state keys dropped) must each break it.
"""
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle import qwen35 as orc

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_attention_layer as cfg1  # noqa: E402

GOLDEN = Path(__file__).resolve().parent / "golden" / "attention_layer_cfg1.npz"


def oracle_branch_out(theta=cfg1.THETA, **plant):
    xs, xb, w = cfg1.config1_inputs()
    f = lambda a: np.asarray(a, np.float64)
    Wqkv = np.concatenate([f(w["q_proj"]), f(w["k_proj"]), f(w["v_proj"])], 0)
    own_base = np.repeat(np.arange(cfg1.B) * cfg1.L, cfg1.L)
    if plant.get("no_state"):
        xs = xs[:0]
    if plant.get("kv_swap"):  # q-head h reads the other kv-head
        nq = cfg1.HQ * 2 * cfg1.D
        k = Wqkv[nq: nq + 2 * cfg1.D].copy()
        Wqkv[nq: nq + cfg1.D], Wqkv[nq + cfg1.D: nq + 2 * cfg1.D] = k[cfg1.D:], k[:cfg1.D]
    _, out = orc.gated_attention_layer(
        xs, xb, own_base, Wqkv, f(w["o_proj"]), 1.0 + f(w["q_norm"]), 1.0 + f(w["k_norm"]),
        cfg1.HQ, cfg1.HKV, cfg1.ROT, theta, cfg1.EPS, cfg1.D)
    return out


def rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / np.abs(b).max())


def test_oracle_layer_matches_transformers_golden():
    ref = np.load(GOLDEN, allow_pickle=False)["branch_out"].astype(np.float64)
    e = rel(oracle_branch_out(), ref)
    print(f"config 1 oracle vs transformers fp32: {e:.2e}")
    assert e <= 1e-5


@pytest.mark.parametrize("plant", [{"theta": 1e4}, {"no_state": True}, {"kv_swap": True}])
def test_planted_mistakes_break_the_match(plant):
    ref = np.load(GOLDEN, allow_pickle=False)["branch_out"].astype(np.float64)
    assert rel(oracle_branch_out(**plant), ref) > 1e-2


def test_gate_is_applied(monkeypatch):
    """The sigmoid gate multiplies the attention output: with it removed the
    oracle no longer matches."""
    ref = np.load(GOLDEN, allow_pickle=False)["branch_out"].astype(np.float64)
    monkeypatch.setattr(orc, "sigmoid", lambda x: np.ones_like(np.asarray(x, np.float64)))
    assert rel(oracle_branch_out(), ref) > 1e-2
