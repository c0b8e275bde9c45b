"""Golden vectors for config 1: one gated GQA attention layer of transformers'
Qwen3.5 (Qwen3_5Attention, float32, CPU), at config 1's shapes and seed.

Config 1: hidden 1024, 8 q-heads / 2 kv-heads of 256, RoPE theta 1e7 on the
first 64 dims (partial_rotary_factor 0.25), sigmoid output gate; weights
~N(0, 0.02) (the zero-centred q/k norm weights too, so their effective scale
is 1 + N(0, 0.02)); hidden states ~N(0, 1); a state of 512 tokens, then 4
branches of 32 tokens. transformers runs every [state ++ branch] sequence as
one causal sequence (positions 0..543, eager attention); the fixture keeps
the outputs at the branch positions. Everything is drawn from numpy's PCG64
(seed 0) in the order of `config1_inputs`, so the tests rebuild the inputs
bit for bit on any host.

    python tests/golden/make_attention_layer.py   # writes attention_layer_cfg1.npz
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
OUT = HERE / "attention_layer_cfg1.npz"
H, HQ, HKV, D, ROT, THETA, EPS = 1024, 8, 2, 256, 64, 1e7, 1e-6
P, B, L = 512, 4, 32


def config1_inputs(seed=0):
    """(x_state [P, H], x_branch [B*L, H], weights dict) as float32."""
    rng = np.random.default_rng(seed)
    f = lambda *shape, std=1.0: (rng.standard_normal(shape, dtype=np.float32) * np.float32(std))
    w = {"q_proj": f(HQ * 2 * D, H, std=0.02), "k_proj": f(HKV * D, H, std=0.02),
         "v_proj": f(HKV * D, H, std=0.02), "o_proj": f(H, HQ * D, std=0.02),
         "q_norm": f(D, std=0.02), "k_norm": f(D, std=0.02)}
    x_state = f(P, H)
    x_branch = f(B * L, H)
    return x_state, x_branch, w


def transformers_branch_outputs(x_state, x_branch, w):
    """[B*L, H] outputs of Qwen3_5Attention at the branch positions, each
    branch run as the causal sequence [state ++ branch] (float32)."""
    import torch
    from transformers.models.qwen3_5 import modeling_qwen3_5 as tf
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig

    cfg = Qwen3_5TextConfig(hidden_size=H, num_attention_heads=HQ, num_key_value_heads=HKV,
                            head_dim=D, rms_norm_eps=EPS, num_hidden_layers=4,
                            intermediate_size=2048, vocab_size=1024,
                            rope_parameters={"rope_type": "default", "rope_theta": THETA,
                                             "partial_rotary_factor": ROT / D,
                                             "mrope_section": [11, 11, 10],
                                             "mrope_interleaved": True})
    cfg._attn_implementation = "eager"
    attn = tf.Qwen3_5Attention(cfg, layer_idx=3).eval()
    rope = tf.Qwen3_5TextRotaryEmbedding(cfg)
    with torch.no_grad():
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            getattr(attn, name).weight.copy_(torch.from_numpy(w[name]))
        attn.q_norm.weight.copy_(torch.from_numpy(w["q_norm"]))
        attn.k_norm.weight.copy_(torch.from_numpy(w["k_norm"]))
        T = P + L
        mask = torch.full((T, T), float("-inf")).triu(1)[None, None]
        pos = torch.arange(T)[None]
        outs = []
        for b in range(B):
            x = torch.from_numpy(np.concatenate([x_state, x_branch[b * L:(b + 1) * L]]))[None]
            cos_sin = rope(x, pos)
            y, _ = attn(x, cos_sin, mask)
            outs.append(y[0, P:].numpy())
    return np.concatenate(outs).astype(np.float32)


if __name__ == "__main__":
    xs, xb, w = config1_inputs()
    out = transformers_branch_outputs(xs, xb, w)
    import transformers
    np.savez_compressed(OUT, branch_out=out, transformers_version=transformers.__version__)
    print(f"wrote {OUT} ({out.shape}, |out| max {np.abs(out).max():.3f})")
