"""Config 5's numerics on the GPU: the engine through the public C ABI on a
seeded 9B-dims checkpoint cut to 4 layers (three Gated DeltaNet layers and
one full-attention layer; hidden 4096, intermediate 12288, head_dim 256,
untied LM head), one request shaped like config 5's at reduced size (a
320-token state, 4 branches x 16 tokens, 8 labels), against the float64
oracle vectors of tests/golden/request_9b.npz (tests/golden/
make_request_9b.py): "engine" = the reference engine's bf16 rounding
points, "f64" = transformers' math.

Bars. The reference engine's numerics re-run with a 2^-24 relative jitter
before every bf16 rounding (three seeds: other valid fp32 summation orders)
drift from "engine" by RMS dlogit 0.008-0.009 and max |dp| 2.1e-3 -
3.2e-3 on this 4-layer model; "engine" itself sits at max |dp| 1.58e-2
and RMS 0.021 from float64. Asserted:
  * identical argmax where the fixture's top-2 label margin exceeds 8x the
    floor's RMS (three of the four branches);
  * RMS dlogit against "engine" over 4096+ vocabulary ids within 1.5x the
    largest jitter seed's;
  * against float64, max |dp| and RMS within 1.5x of "engine"'s own: the
    engine is no further from the exact math than the reference engine is;
  * max |dp| against "engine" within 1.5x the jitter floor.
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
import make_request_9b as fx  # noqa: E402

pytestmark = pytest.mark.gpu
FLOOR_FACTOR = 1.5


def softmax(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max())
    return e / e.sum()


def test_config5_numerics_against_oracle():
    g = np.load(fx.OUT, allow_pickle=False)
    base = "/dev/shm" if os.path.isdir("/dev/shm") else None
    with tempfile.TemporaryDirectory(dir=base) as d:
        print("building the seeded 4-layer 9B-dims checkpoint", flush=True)
        digest = fx.build_checkpoint(d)
        assert digest == str(g["checkpoint_sha256"]), "checkpoint differs from the fixture's"
        state, brs = fx.request()
        assert np.array_equal(g["state"], state)
        e = Engine(d, max_state_tokens=512, max_branch_tokens=128, max_branches=8,
                   max_candidates=256)
        try:
            e.prefill(state)
            cand = e.eval([Branch(t, c) for t, c in brs])
            full = e.eval_full_logits([Branch(t, []) for t, _ in brs])
        finally:
            e.close()
    ids = g["sample_ids"]
    stats = dict(zip([str(s) for s in g["stat_modes"]], g["stat_values"]))
    floor_rms = max(v[1] for m, v in stats.items() if m.startswith("engine~"))
    floor_dp = max(v[2] for m, v in stats.items() if m.startswith("engine~"))
    dp = {m: max(np.abs(softmax(cand[i]) - softmax(g[f"cand_{m}"][i])).max()
                 for i in range(len(brs))) for m in ("engine", "f64")}
    rms = {m: float(np.sqrt(np.mean((full[:, ids] - g[f"sample_{m}"]) ** 2)))
           for m in ("engine", "f64")}
    print(f"engine vs reference-engine oracle: max|dp| {dp['engine']:.3e}, "
          f"RMS dlogit {rms['engine']:.4f}", flush=True)
    print(f"engine vs float64 oracle:          max|dp| {dp['f64']:.3e}, "
          f"RMS dlogit {rms['f64']:.4f}", flush=True)
    print(f"noise floor (jitter seeds vs oracle): max|dp| {floor_dp:.3e}, RMS dlogit "
          f"{floor_rms:.4f}; 1e-3 bar met: {dp['engine'] <= 1e-3}", flush=True)
    for i, (_, c) in enumerate(brs):
        r = g["cand_engine"][i]
        srt = np.sort(r)
        np.testing.assert_allclose(cand[i], full[i, c], rtol=1e-3, atol=1e-3)
        if srt[-1] - srt[-2] > 8 * floor_rms:
            assert np.argmax(cand[i]) == np.argmax(r), (i, srt[-1] - srt[-2])
    ref_dp = max(np.abs(softmax(g["cand_engine"][i]) - softmax(g["cand_f64"][i])).max()
                 for i in range(len(brs)))
    ref_rms = float(np.sqrt(np.mean((g["sample_engine"].astype(np.float64) -
                                     g["sample_f64"]) ** 2)))
    print(f"reference numerics vs float64:     max|dp| {ref_dp:.3e}, RMS dlogit {ref_rms:.4f}",
          flush=True)
    assert rms["engine"] <= FLOOR_FACTOR * floor_rms
    assert dp["f64"] <= FLOOR_FACTOR * ref_dp and rms["f64"] <= FLOOR_FACTOR * ref_rms
    assert dp["engine"] <= FLOOR_FACTOR * floor_dp
