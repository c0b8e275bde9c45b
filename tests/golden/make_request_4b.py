"""Golden vectors for config 4: the first bench request (530-token state +
4 branches x 20 tokens, 3/2/2/4 labels) on the seeded 4B-shaped checkpoint,
through the streaming request oracle (oracle/request.py), in float64
("f64": transformers' math) and with the reference engine's bf16 rounding
points ("engine").

The noise floor is kept too: the "engine" numerics re-run with a 2^-24
relative jitter before every bf16 rounding (three seeds: three other,
equally valid fp32 summation orders) drift from "engine" by the amount any
two correct bf16 engines drift apart on this model; the GPU test's bar is
stated against it. "mfma" (this build's former Gated DeltaNet rounding
points, emulated) is kept as a statistic only.

The checkpoint is rebuilt bit for bit from its seed with
cujev.synthetic's "blocks" generator (numpy PCG64 per tensor block) and
pinned by its SHA-256. Stored: the request, every branch's candidate
logits per mode, the logits at a fixed sample of 4096 vocabulary ids (plus
each branch's 16 largest f64 logits) for "f64" and "engine", and the floor
statistics. Runs in about 15 minutes on 8 cores:

    python tests/golden/make_request_4b.py /path/to/checkpoint_dir
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
OUT = HERE / "request_4b.npz"
SEED = 0
STATE, BRANCH, LABELS = 530, 20, (3, 2, 2, 4)
MODES = ("f64", "engine", "engine~1", "engine~2", "engine~3", "mfma")


def request():
    """The first request of bench.py's config-4 stream (same generator and
    draw order): ids in [1000, 60000), distinct labels in [16, 1000)."""
    rng = np.random.default_rng(SEED)
    state = [int(x) for x in rng.integers(1000, 60000, size=STATE)]
    branches = []
    for n in LABELS:
        toks = [int(x) for x in rng.integers(1000, 60000, size=BRANCH)]
        cands = [int(x) for x in rng.choice(np.arange(16, 1000), size=n, replace=False)]
        branches.append((toks, cands))
    return state, branches


def vocab_sample(vocab):
    return np.sort(np.random.default_rng(1).choice(vocab, size=4096, replace=False))


def build_checkpoint(path):
    """Writes the seeded 4B checkpoint under `path`; returns its SHA-256."""
    for p in (str(ROOT), str(ROOT / "cu-jev_amd")):
        if p not in sys.path:
            sys.path.insert(0, p)
    from cujev import synthetic
    cfg = synthetic.make_config(**synthetic.PRESETS["4b"])
    synthetic.write_checkpoint(path, cfg, seed=SEED, generator="blocks")
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
    for p in (str(ROOT), str(ROOT / "cu-jev_amd")):
        if p not in sys.path:
            sys.path.insert(0, p)
    from oracle import request as rq
    ckpt = Path(ckpt)
    if not (ckpt / "model.safetensors").exists():
        digest = build_checkpoint(ckpt)
    else:
        digest = sha256(ckpt / "model.safetensors")
    state, brs = request()
    out = rq.request_logits(str(ckpt), state, brs, modes=MODES, full=True,
                            progress=lambda l: print(f"layer {l}", flush=True))
    write_fixture({m: out[m]["full"] for m in MODES}, digest)


def write_fixture(full, digest):
    """full: {mode: [4, vocab] float64 last-token logits} of request()."""
    state, brs = request()
    V = full["f64"].shape[1]
    sample = vocab_sample(V)
    top = np.argsort(-full["f64"], axis=1)[:, :16]
    ids = np.unique(np.concatenate([sample, top.ravel()]))
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
        cand_flat=np.concatenate([c for _, c in brs]).astype(np.int32),
        cand_len=np.asarray([len(c) for _, c in brs], np.int32),
        cand_f64=np.concatenate([full["f64"][i, c] for i, (_, c) in enumerate(brs)]),
        cand_engine=np.concatenate([full["engine"][i, c] for i, (_, c) in enumerate(brs)]),
        sample_ids=ids.astype(np.int32),
        sample_f64=full["f64"][:, ids].astype(np.float32),
        sample_engine=full["engine"][:, ids].astype(np.float32),
        # per mode vs "engine": RMS dlogit over the whole vocabulary, over the
        # sample, and max |dp| over the labels
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
