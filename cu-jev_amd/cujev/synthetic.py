"""Seeded random-init Qwen3.5-shaped checkpoints written to a local directory
(config.json + model.safetensors) in the Hugging Face layout, so that the
engine and transformers load the very same file. Nothing is downloaded.

Matrices (every tensor with >= 2 dims, conv1d included) are bf16 ~ N(0, std).
1-D parameters follow the transformers init of Qwen3.5 (modeling_qwen3_5.py
_init_weights): zero-centred RMSNorm weights 0, gated-norm weight 1,
dt_bias 1, A_log = log U(0, 16) -- unless ``norm_std`` > 0, which adds
N(0, norm_std) to the norm weights (used by parity tests to exercise the
zero-centred 1 + w path).
"""
from __future__ import annotations

import json
import os
from pathlib import Path


def make_config(hidden_size, num_layers, vocab_size, intermediate_size, *, num_heads=16,
                num_kv_heads=4, lin_k_heads=16, lin_v_heads=32, tie=True, rope_theta=1e7,
                eps=1e-6, full_every=4):
    layer_types = ["full_attention" if (i + 1) % full_every == 0 else "linear_attention"
                   for i in range(num_layers)]
    return {
        "architectures": ["Qwen3_5ForCausalLM"],
        "model_type": "qwen3_5_text",
        "hidden_size": hidden_size,
        "intermediate_size": intermediate_size,
        "num_hidden_layers": num_layers,
        "num_attention_heads": num_heads,
        "num_key_value_heads": num_kv_heads,
        "head_dim": 256,
        "hidden_act": "silu",
        "vocab_size": vocab_size,
        "rms_norm_eps": eps,
        "tie_word_embeddings": tie,
        "attention_bias": False,
        "linear_conv_kernel_dim": 4,
        "linear_key_head_dim": 128,
        "linear_value_head_dim": 128,
        "linear_num_key_heads": lin_k_heads,
        "linear_num_value_heads": lin_v_heads,
        "layer_types": layer_types,
        "max_position_embeddings": 32768,
        "rope_parameters": {"rope_type": "default", "rope_theta": rope_theta,
                            "partial_rotary_factor": 0.25, "mrope_section": [11, 11, 10],
                            "mrope_interleaved": True},
        "torch_dtype": "bfloat16",
    }


# Shapes used by the benchmarks and tests. The 4B dims beyond hidden/layers/
# vocab (which the workload fixes) are the Qwen3.5 defaults: 16/4 attention
# heads of 256, 16/32 GDN heads of 128, intermediate 9216.
PRESETS = {
    "4b": dict(hidden_size=2560, num_layers=32, vocab_size=248320, intermediate_size=9216,
               tie=True),
    "9b": dict(hidden_size=4096, num_layers=32, vocab_size=248320, intermediate_size=12288,
               tie=False),
    "tiny": dict(hidden_size=512, num_layers=4, vocab_size=4096, intermediate_size=1024,
                 num_heads=4, num_kv_heads=1, lin_k_heads=2, lin_v_heads=4, tie=True),
}


def tensor_shapes(cfg):
    """(name, shape) of every tensor of the text model, HF names."""
    H, I, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    Hq, Hkv, D = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    Hk, Hv = cfg["linear_num_key_heads"], cfg["linear_num_value_heads"]
    dk, dv = cfg["linear_key_head_dim"], cfg["linear_value_head_dim"]
    C = 2 * Hk * dk + Hv * dv
    out = [("model.embed_tokens.weight", (V, H))]
    for i, lt in enumerate(cfg["layer_types"]):
        p = f"model.layers.{i}."
        out += [(p + "input_layernorm.weight", (H,)), (p + "post_attention_layernorm.weight", (H,))]
        if lt == "full_attention":
            a = p + "self_attn."
            out += [(a + "q_proj.weight", (Hq * 2 * D, H)), (a + "k_proj.weight", (Hkv * D, H)),
                    (a + "v_proj.weight", (Hkv * D, H)), (a + "o_proj.weight", (H, Hq * D)),
                    (a + "q_norm.weight", (D,)), (a + "k_norm.weight", (D,))]
        else:
            g = p + "linear_attn."
            out += [(g + "in_proj_qkv.weight", (C, H)), (g + "in_proj_z.weight", (Hv * dv, H)),
                    (g + "in_proj_b.weight", (Hv, H)), (g + "in_proj_a.weight", (Hv, H)),
                    (g + "conv1d.weight", (C, 1, 4)), (g + "dt_bias", (Hv,)),
                    (g + "A_log", (Hv,)), (g + "norm.weight", (dv,)),
                    (g + "out_proj.weight", (H, Hv * dv))]
        m = p + "mlp."
        out += [(m + "gate_proj.weight", (I, H)), (m + "up_proj.weight", (I, H)),
                (m + "down_proj.weight", (H, I))]
    out.append(("model.norm.weight", (H,)))
    if not cfg["tie_word_embeddings"]:
        out.append(("lm_head.weight", (V, H)))
    return out


def write_checkpoint(path, cfg, *, seed=0, std=0.02, norm_std=0.0, device="cpu",
                     generator="torch"):
    """Write config.json + model.safetensors under `path`; returns the path.

    generator="torch" draws with torch's generator on `device` (fast for the
    multi-GiB shapes); generator="numpy" draws with numpy's PCG64, whose
    streams are the same on every host, so the file is bit-identical wherever
    it is rebuilt (used for committed golden vectors)."""
    import numpy as np
    import torch
    from safetensors.torch import save_file

    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    if generator == "blocks":
        return _write_blocks(path, cfg, seed=seed, std=std, norm_std=norm_std)
    if generator == "numpy":
        rng = np.random.default_rng(seed)

        def randn(shape):
            return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32))

        def rand(shape):
            return torch.from_numpy(rng.random(shape, dtype=np.float32))
        dev = "cpu"
    else:
        gen = torch.Generator(device=device).manual_seed(seed)

        def randn(shape):
            return torch.randn(shape, generator=gen, device=device, dtype=torch.float32)

        def rand(shape):
            return torch.rand(shape, generator=gen, device=device, dtype=torch.float32)
        dev = device
    tensors = {}
    for name, shape in tensor_shapes(cfg):
        leaf = name.rsplit(".", 1)[0] if name.endswith(".weight") else name
        if len(shape) >= 2:
            t = (randn(shape) * std).to(torch.bfloat16)
        elif name.endswith("A_log"):
            u = (rand(shape) * 16.0).clamp_min(1e-3)
            if generator == "numpy":  # scalar libm log: no vector-path ulp differences
                import math
                t = torch.tensor([math.log(float(x)) for x in u.reshape(-1)],
                                 dtype=torch.float32).reshape(shape)
            else:
                t = torch.log(u)
        elif name.endswith("dt_bias"):
            t = torch.ones(shape, dtype=torch.float32, device=dev)
        elif leaf.endswith("linear_attn.norm"):
            t = torch.ones(shape, dtype=torch.float32, device=dev)
            if norm_std > 0:
                t = t + randn(shape) * norm_std
            t = t.to(torch.bfloat16)
        else:  # zero-centred RMSNorm weights
            t = torch.zeros(shape, dtype=torch.float32, device=dev)
            if norm_std > 0:
                t = t + randn(shape) * norm_std
            t = t.to(torch.bfloat16)
        tensors[name] = t.cpu().contiguous()
    save_file(tensors, str(path / "model.safetensors"), metadata={"format": "pt"})
    with open(path / "config.json", "w") as f:
        json.dump(cfg, f, indent=1)
    return str(path)


BLOCK_ROWS_ELEMS = 1 << 22  # elements per independently seeded block


def _write_blocks(path, cfg, *, seed, std, norm_std):
    """generator="blocks": the numpy draws of generator="numpy" made parallel.
    Tensor i (in tensor_shapes order) is cut into row blocks of about 4M
    elements; block j is drawn from PCG64 seeded with the entropy list
    [seed, i, j], so the bits do not depend on the thread count or the host,
    and the blocks are drawn on a thread pool (numpy releases the GIL while
    filling). Matrices ~ N(0, std) in float32, then rounded to bf16; 1-D
    parameters as in write_checkpoint (A_log = log U(0, 16) through scalar
    libm, dt_bias 1, norms 0 / 1 (+ N(0, norm_std)))."""
    import math
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    import torch
    from safetensors.torch import save_file

    shapes = tensor_shapes(cfg)
    jobs = []
    out = {}
    for i, (name, shape) in enumerate(shapes):
        if len(shape) >= 2:
            rows = shape[0]
            per_row = int(np.prod(shape[1:]))
            step = max(1, BLOCK_ROWS_ELEMS // per_row)
            t = torch.empty(shape, dtype=torch.bfloat16)
            out[name] = t
            for j, r0 in enumerate(range(0, rows, step)):
                jobs.append((t, i, j, r0, min(rows, r0 + step)))
            continue
        rng = np.random.default_rng([seed, i, 0])
        leaf = name.rsplit(".", 1)[0] if name.endswith(".weight") else name
        if name.endswith("A_log"):
            u = np.maximum(rng.random(shape, dtype=np.float32) * np.float32(16.0), np.float32(1e-3))
            t = torch.tensor([math.log(float(x)) for x in u.reshape(-1)], dtype=torch.float32)
        elif name.endswith("dt_bias"):
            t = torch.ones(shape, dtype=torch.float32)
        else:
            base = 1.0 if leaf.endswith("linear_attn.norm") else 0.0
            v = np.full(shape, base, np.float32)
            if norm_std > 0:
                v = v + rng.standard_normal(shape, dtype=np.float32) * np.float32(norm_std)
            t = torch.from_numpy(v).to(torch.bfloat16)
        out[name] = t.reshape(shape)

    def fill(job):
        t, i, j, r0, r1 = job
        rng = np.random.default_rng([seed, i, j])
        blk = rng.standard_normal((r1 - r0,) + tuple(t.shape[1:]), dtype=np.float32)
        blk *= np.float32(std)
        t[r0:r1] = torch.from_numpy(blk).to(torch.bfloat16)

    threads = max(1, min(32, len(os.sched_getaffinity(0))))
    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(fill, jobs))
    save_file(out, str(path / "model.safetensors"), metadata={"format": "pt"})
    with open(path / "config.json", "w") as f:
        json.dump(cfg, f, indent=1)
    return str(path)


def ensure_checkpoint(path, preset="4b", *, seed=0, device="cpu", generator="torch",
                      sha256=None, **overrides):
    """Write the preset checkpoint once (reused when config.json already
    matches and, when `sha256` is given, the weights file hashes to it)."""
    kw = dict(PRESETS[preset])
    kw.update(overrides)
    cfg = make_config(**kw)
    path = Path(path)
    cfg_file = path / "config.json"
    if cfg_file.exists() and (path / "model.safetensors").exists():
        try:
            if json.loads(cfg_file.read_text()) == cfg and (
                    sha256 is None or file_sha256(path / "model.safetensors") == sha256):
                return str(path)
        except ValueError:
            pass
    return write_checkpoint(path, cfg, seed=seed, device=device, generator=generator)


def file_sha256(file):
    """SHA-256 hex digest of a file, read in 16 MiB pieces."""
    import hashlib
    h = hashlib.sha256()
    with open(file, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    return h.hexdigest()


if __name__ == "__main__":  # python -m cujev.synthetic <dir> [preset]
    import sys
    out = sys.argv[1]
    preset = sys.argv[2] if len(sys.argv) > 2 else "4b"
    print(ensure_checkpoint(out, preset, device=os.environ.get("CUJEV_SYNTH_DEVICE", "cpu")))
