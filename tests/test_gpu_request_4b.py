"""Config 4 decision parity on the GPU: the engine through the public C ABI
on the seeded 4B-shaped checkpoint and the first bench request (530-token
state + 4 branches x 20 tokens, 3/2/2/4 labels), against the float64 oracle
vectors of tests/golden/request_4b.npz (tests/golden/make_request_4b.py):
"engine" = the reference engine's bf16 rounding points, "f64" =
transformers' math.

What the bars are, and why. On this random-init 32-layer model the bf16
rounding noise is large: the reference engine's own numerics sit at max
|dp| 2.2e-2 and RMS dlogit 0.045 from float64, and the same numerics with
another valid fp32 summation order (2^-24 jitter before every bf16 rounding,
three seeds, stored in the fixture) drift from "engine" by max |dp| up to
1.05e-2 and RMS dlogit 0.022 -- an order of magnitude above a 1e-3
probability bar, which no bf16 engine that is not bit-identical to the
oracle's arithmetic can meet. The test therefore asserts, against "engine":
  * identical argmax on every branch (every top-2 label margin in the fixture
    is >= 0.58 logits; the jitter seeds move single label logits by at most
    0.04);
  * RMS dlogit over 4096+ vocabulary ids <= 1.5 x the largest jitter-seed
    RMS (the engine is as close to the reference numerics as another valid
    summation order is);
  * max |dp| over the labels <= 1.5 x the largest jitter-seed max |dp|;
and prints max |dp| against both oracles next to the 1e-3 figure.
"""
import os
import sys
import tempfile
from pathlib import Path

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from cujev import Branch, Engine  # noqa: E402

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_request_4b as fx  # noqa: E402

pytestmark = pytest.mark.gpu
FLOOR_FACTOR = 1.5


def softmax(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max())
    return e / e.sum()


def test_config4_request_against_oracle():
    g = np.load(fx.OUT, allow_pickle=False)
    base = "/dev/shm" if os.path.isdir("/dev/shm") else None
    with tempfile.TemporaryDirectory(dir=base) as d:
        print("building the seeded 4B checkpoint", flush=True)
        digest = fx.build_checkpoint(d)
        assert digest == str(g["checkpoint_sha256"]), "checkpoint differs from the fixture's"
        state, brs = fx.request()
        e = Engine(d, max_state_tokens=1024, max_branch_tokens=256, max_branches=16,
                   max_candidates=256)
        try:
            e.prefill(state)
            cand = e.eval([Branch(t, c) for t, c in brs])
            full = e.eval_full_logits([Branch(t, []) for t, _ in brs])
        finally:
            e.close()
    ids = g["sample_ids"]
    offs = np.concatenate([[0], np.cumsum(g["cand_len"])])
    ref = {m: [g[f"cand_{m}"][offs[i]:offs[i + 1]] for i in range(len(brs))]
           for m in ("engine", "f64")}
    dp = {m: max(np.abs(softmax(cand[i]) - softmax(ref[m][i])).max() for i in range(len(brs)))
          for m in ref}
    rms = {m: float(np.sqrt(np.mean((full[:, ids] - g[f"sample_{m}"]) ** 2))) for m in ref}
    stats = dict(zip([str(s) for s in g["stat_modes"]], g["stat_values"]))
    floor_rms = max(v[1] for m, v in stats.items() if m.startswith("engine~"))
    floor_dp = max(v[2] for m, v in stats.items() if m.startswith("engine~"))
    print(f"engine vs reference-engine oracle: max|dp| {dp['engine']:.3e}, "
          f"RMS dlogit {rms['engine']:.4f}", flush=True)
    print(f"engine vs float64 oracle:          max|dp| {dp['f64']:.3e}, "
          f"RMS dlogit {rms['f64']:.4f}", flush=True)
    print(f"noise floor (jitter seeds vs oracle): max|dp| {floor_dp:.3e}, RMS dlogit "
          f"{floor_rms:.4f}; 1e-3 bar met: {dp['engine'] <= 1e-3}", flush=True)
    for m, v in stats.items():
        print(f"  fixture {m}: RMS {v[1]:.4f}, max|dp| {v[2]:.3e}", flush=True)
    for i in range(len(brs)):
        r = ref["engine"][i]
        margin = np.sort(r)[-1] - np.sort(r)[-2]
        assert np.argmax(cand[i]) == np.argmax(r), (i, margin)
        np.testing.assert_allclose(cand[i], full[i, brs[i][1]], rtol=1e-3, atol=1e-3)
    assert rms["engine"] <= FLOOR_FACTOR * floor_rms
    assert dp["engine"] <= FLOOR_FACTOR * floor_dp
