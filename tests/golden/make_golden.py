"""Writes tests/golden/qwen35_micro.npz: last-token logits of transformers'
Qwen3_5ForCausalLM (float32, CPU) on a seeded random-init checkpoint of a
micro Qwen3.5 shape, for token sequences that straddle the 64-token GDN
chunks and the attention query/key tiles.

The checkpoint is not stored: it is rebuilt from the seed by
cujev.synthetic with numpy's PCG64 generator (the same stream on every host),
and the fixture keeps the SHA-256 of its model.safetensors so a test can tell
when the rebuild differs.

    python tests/golden/make_golden.py          # needs transformers (CPU)
"""
import hashlib
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "cu-jev_amd"))

from cujev import synthetic  # noqa: E402

# 3 Gated DeltaNet layers + 1 gated full-attention layer (layer 3)
MICRO = dict(hidden_size=256, num_layers=4, vocab_size=512, intermediate_size=512,
             num_heads=4, num_kv_heads=1, lin_k_heads=2, lin_v_heads=4, tie=True)
SEED, NORM_STD = 5, 0.1
LENGTHS = (1, 2, 17, 64, 65, 130)
OUT = Path(__file__).with_name("qwen35_micro.npz")


def build_checkpoint(path):
    cfg = synthetic.make_config(**MICRO)
    synthetic.write_checkpoint(path, cfg, seed=SEED, norm_std=NORM_STD, generator="numpy")
    digest = hashlib.sha256((Path(path) / "model.safetensors").read_bytes()).hexdigest()
    return cfg, digest


def sequences():
    rng = np.random.default_rng(11)
    return [rng.integers(16, MICRO["vocab_size"], n).astype(np.int32) for n in LENGTHS]


def main():
    import torch
    import transformers
    from transformers import AutoModelForCausalLM

    d = tempfile.mkdtemp()
    _, digest = build_checkpoint(d)
    model = AutoModelForCausalLM.from_pretrained(d, dtype=torch.float32).eval()
    seqs = sequences()
    logits = []
    with torch.no_grad():
        for ids in seqs:
            out = model(torch.tensor(ids[None].astype(np.int64))).logits[0, -1]
            logits.append(out.double().numpy())
    ids_flat = np.concatenate(seqs)
    np.savez_compressed(
        OUT, ids=ids_flat, lengths=np.array(LENGTHS, np.int32),
        logits=np.stack(logits).astype(np.float32),
        checkpoint_sha256=np.array(digest), transformers_version=np.array(transformers.__version__),
        torch_version=np.array(torch.__version__))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes), checkpoint sha256 {digest[:16]}..")


if __name__ == "__main__":
    main()
