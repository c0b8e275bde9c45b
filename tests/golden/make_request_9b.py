"""Golden vectors for config 5's numerics: a 9B-dims checkpoint cut to 4
layers (three Gated DeltaNet layers, then full attention; hidden 4096,
intermediate 12288, untied LM head) and one request shaped like config 5's
at reduced size (a 320-token state, 4 branches x 16 tokens, 8 labels each),
through the streaming request oracle (oracle/request.py) in float64
("f64"), with the reference engine's bf16 rounding points ("engine"), and
with three jitter seeds of the engine numerics ("engine~1..3": other valid
fp32 summation orders, the noise floor the GPU test's bar is stated
against).

The checkpoint is rebuilt bit for bit from its seed with cujev.synthetic's
"blocks" generator and pinned by its SHA-256. Stored: the request, every
branch's label logits per mode, the logits at a fixed sample of 4096
vocabulary ids (plus each branch's 16 largest f64 logits) for "f64" and
"engine", and the floor statistics. About 5 minutes on 8 cores:

    python tests/golden/make_request_9b.py /path/to/checkpoint_dir
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
OUT = HERE / "request_9b.npz"
SEED = 5
LAYERS = 4
STATE, BRANCH, NB, LABELS = 320, 16, 4, 8
MODES = ("f64", "engine", "engine~1", "engine~2", "engine~3")


def _paths():
    for p in (str(ROOT), str(ROOT / "cu-jev_amd")):
        if p not in sys.path:
            sys.path.insert(0, p)


def config():
    _paths()
    from cujev import synthetic
    return synthetic.make_config(**dict(synthetic.PRESETS["9b"], num_layers=LAYERS))


def request():
    """ids in [1000, 60000), distinct labels in [16, 1000) (bench.py's
    config-5 draw, smaller)."""
    rng = np.random.default_rng(SEED)
    state = [int(x) for x in rng.integers(1000, 60000, size=STATE)]
    branches = []
    for _ in range(NB):
        toks = [int(x) for x in rng.integers(1000, 60000, size=BRANCH)]
        cands = [int(x) for x in rng.choice(np.arange(16, 1000), size=LABELS, replace=False)]
        branches.append((toks, cands))
    return state, branches


def vocab_sample(vocab):
    return np.sort(np.random.default_rng(2).choice(vocab, size=4096, replace=False))


def build_checkpoint(path):
    """Writes the seeded 4-layer 9B-dims checkpoint under `path`; returns its
    SHA-256."""
    _paths()
    from cujev import synthetic
    synthetic.write_checkpoint(path, config(), seed=SEED, generator="blocks")
    return sha256(Path(path) / "model.safetensors")


def sha256(file):
    h = hashlib.sha256()
    with open(file, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    return h.hexdigest()


def softmax(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max())
    return e / e.sum()


def main(ckpt):
    _paths()
    from oracle import request as rq
    ckpt = Path(ckpt)
    if not (ckpt / "model.safetensors").exists():
        digest = build_checkpoint(ckpt)
    else:
        digest = sha256(ckpt / "model.safetensors")
    state, brs = request()
    out = rq.request_logits(str(ckpt), state, brs, modes=MODES, full=True,
                            progress=lambda l: print(f"layer {l}", flush=True))
    full = {m: out[m]["full"] for m in MODES}
    V = full["f64"].shape[1]
    top = np.argsort(-full["f64"], axis=1)[:, :16]
    ids = np.unique(np.concatenate([vocab_sample(V), top.ravel()]))
    stats = {}
    for m in MODES[2:]:
        d = full[m] - full["engine"]
        dp = max(np.abs(softmax(full[m][i, c]) - softmax(full["engine"][i, c])).max()
                 for i, (_, c) in enumerate(brs))
        stats[m] = (float(np.sqrt(np.mean(d ** 2))), float(np.sqrt(np.mean(d[:, ids] ** 2))),
                    float(dp))
    np.savez_compressed(
        OUT, checkpoint_sha256=digest, state=np.asarray(state, np.int32),
        branch_tokens=np.asarray([t for t, _ in brs], np.int32),
        cand=np.asarray([c for _, c in brs], np.int32),
        cand_f64=np.stack([full["f64"][i, c] for i, (_, c) in enumerate(brs)]),
        cand_engine=np.stack([full["engine"][i, c] for i, (_, c) in enumerate(brs)]),
        sample_ids=ids.astype(np.int32),
        sample_f64=full["f64"][:, ids].astype(np.float32),
        sample_engine=full["engine"][:, ids].astype(np.float32),
        # per jitter seed vs "engine": RMS dlogit over the whole vocabulary,
        # over the sample, and max |dp| over the labels
        stat_modes=np.asarray(MODES[2:]),
        stat_values=np.asarray([stats[m] for m in MODES[2:]]),
        # every mode's label logits (rows in MODES order, labels flattened in
        # branch order): the jitter seeds' label deviations set the noise
        # floor of a decision's top-2 margin
        label_modes=np.asarray(MODES),
        label_logits=np.stack([np.concatenate([full[m][i, c] for i, (_, c) in enumerate(brs)])
                               for m in MODES]))
    for m, v in stats.items():
        print(f"{m} vs engine: rms dlogit {v[0]:.4f} (sample {v[1]:.4f}), max|dp| {v[2]:.2e}")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main(sys.argv[1])
