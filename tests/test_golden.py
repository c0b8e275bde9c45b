"""The CPU oracle's whole-model forward against golden vectors from
transformers' Qwen3_5ForCausalLM (float32, CPU; tests/golden/make_golden.py):
last-token logits of a seeded micro Qwen3.5 checkpoint (3 Gated DeltaNet
layers + 1 gated attention layer) for sequences of 1..130 tokens.

This pins what only the composed model fixes: weight names and the fused row
order, tied embeddings, the zero-centred (1 + w) norms, norm placement, the
gated-attention and GDN layer wiring, and the 1-D RoPE that text-only
positions reduce to. Bar: max |oracle - golden| <= 1e-5 * max(1, max|golden|)
(the two differ by float32 vs float64 rounding, ~1e-6 here).
"""
import sys
import tempfile
from pathlib import Path

import numpy as np
import pytest

pytest.importorskip("torch")
pytest.importorskip("safetensors")

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))

import make_golden  # noqa: E402
from oracle import qwen35 as orc  # noqa: E402

FIXTURE = HERE / "golden" / "qwen35_micro.npz"


@pytest.fixture(scope="module")
def golden():
    return np.load(FIXTURE, allow_pickle=False)


@pytest.fixture(scope="module")
def model(golden):
    d = tempfile.mkdtemp()
    cfg, digest = make_golden.build_checkpoint(d)
    assert digest == str(golden["checkpoint_sha256"]), \
        "rebuilt checkpoint differs from the one the golden logits were made on"
    return orc.load_checkpoint(d)


def split(golden):
    off = 0
    for n, ref in zip(golden["lengths"], golden["logits"]):
        yield golden["ids"][off:off + n], ref.astype(np.float64)
        off += n


@pytest.mark.parametrize("chunked", [True, False])
def test_oracle_matches_transformers(golden, model, chunked):
    cfg, W = model
    for ids, ref in split(golden):
        got = orc.model_last_logits(cfg, W, ids, chunked=chunked)
        err = np.abs(got - ref).max()
        assert err <= 1e-5 * max(1.0, np.abs(ref).max()), (len(ids), err)


def test_golden_is_sensitive(golden, model):
    """Plausible mistakes -- the conv taps in reverse order, a norm weight left
    out -- move the logits far beyond the bar, so the comparison can fail."""
    cfg, W = model
    ids, ref = list(split(golden))[-1]
    bar = 1e-5 * max(1.0, np.abs(ref).max())
    conv = next(k for k in W if k.endswith("conv1d.weight"))
    norm = next(k for k in W if k.endswith("input_layernorm.weight"))
    for name, value in ((conv, W[conv][..., ::-1].copy()), (norm, np.zeros_like(W[norm]))):
        W2 = dict(W)
        W2[name] = value
        got = orc.model_last_logits(cfg, W2, ids)
        assert np.abs(got - ref).max() > 100 * bar, name
