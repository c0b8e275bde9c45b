"""CPU baseline of the hot path: transformers' own PyTorch implementation of
Qwen3.5 in float32 on the host cores (the reference's oracle path; REF
tests/python/oracle_fp32.py, benchmarks/benefit.py:77-92). Used by bench.py
only. It is a reported baseline, never the thing measured as `value`.

  request_baseline   the whole request, HF-batched: every [state ++ branch]
                     row in one batch, logits_to_keep=1, candidate logits
                     gathered; one full-size warm-up, then `reps` timed
                     requests, p50.
  layer_baselines    configs 1-3 one layer at a time: the gated attention
                     layer (Qwen3_5Attention), the Gated DeltaNet mixer from
                     its projection output (conv + torch_chunk_gated_delta_rule
                     + gated norm, prefill and 64 branches x 16), and the
                     shared-prefix attention at capacity (eager-style softmax
                     attention over [state ++ branch] per branch).

Every timing uses torch.set_num_threads(len(os.sched_getaffinity(0))): all
cores this process may run on; the count and the CPU model are reported.
"""
from __future__ import annotations

import os
import statistics
import time


def cpu_info() -> dict:
    threads = len(os.sched_getaffinity(0))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"threads": threads, "cpu_model": model}


def _setup():
    import torch
    n = cpu_info()["threads"]
    torch.set_num_threads(n)
    return torch, n


def request_baseline(ckpt, state, branches, reps=5, log=print):
    """transformers fp32 (timed, `reps` requests after a full-size warm-up)
    and bf16 (one run) on one request; returns timings and the last-token
    logits [B, vocab] of both."""
    torch, n = _setup()
    from transformers import AutoModelForCausalLM
    ids = torch.tensor([list(state) + list(t) for t, _ in branches])
    model = AutoModelForCausalLM.from_pretrained(ckpt, dtype=torch.float32).eval()
    times = []
    with torch.no_grad():
        model(ids, logits_to_keep=1)  # warm-up on the full request
        for _ in range(reps):
            t0 = time.perf_counter()
            lg32 = model(ids, logits_to_keep=1).logits[:, -1, :]
            times.append(time.perf_counter() - t0)
    lg32 = lg32.double().numpy()
    log(f"transformers fp32 on {n} threads: p50 {statistics.median(times) * 1e3:.0f} ms/request")
    del model
    model = AutoModelForCausalLM.from_pretrained(ckpt, dtype=torch.bfloat16).eval()
    with torch.no_grad():
        lg16 = model(ids, logits_to_keep=1).logits[:, -1, :].double().numpy()
    del model
    return {"threads": n, "times_s": times, "fp32_logits": lg32, "bf16_logits": lg16}


def _timed(fn, reps):
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts) * 1e3


def layer_baselines(reps=3, log=print):
    """Median ms of configs 1-3 on the CPU (transformers' torch code, fp32)."""
    torch, n = _setup()
    import torch.nn.functional as F
    from transformers.models.qwen3_5 import modeling_qwen3_5 as tf
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    g = torch.Generator().manual_seed(0)
    randn = lambda *s, std=1.0: torch.randn(*s, generator=g) * std
    out = {}
    with torch.no_grad():
        # config 1: one gated attention layer, 512-token state + 4 x 32 branches
        cfg = Qwen3_5TextConfig(hidden_size=1024, num_attention_heads=8, num_key_value_heads=2,
                                head_dim=256, num_hidden_layers=4, intermediate_size=2048,
                                vocab_size=1024,
                                rope_parameters={"rope_type": "default", "rope_theta": 1e7,
                                                 "partial_rotary_factor": 0.25,
                                                 "mrope_section": [11, 11, 10],
                                                 "mrope_interleaved": True})
        cfg._attn_implementation = "eager"
        attn = tf.Qwen3_5Attention(cfg, layer_idx=3).eval()
        for p in attn.parameters():
            p.copy_(randn(*p.shape, std=0.02))
        rope = tf.Qwen3_5TextRotaryEmbedding(cfg)
        x = randn(4, 544, 1024)
        pos = torch.arange(544)[None].expand(4, -1)
        cs = rope(x, pos)
        mask = torch.full((544, 544), float("-inf")).triu(1)[None, None]
        out["config1_attention_layer_ms"] = round(_timed(lambda: attn(x, cs, mask), reps), 2)
        log(f"cpu config 1 layer: {out['config1_attention_layer_ms']} ms")

        # config 2: GDN mixer from its projection output, Hk 16 / Hv 32
        Hk, Hv, T, dk = 16, 32, 2048, 128
        C = (2 * Hk + Hv) * dk
        w = randn(C, 1, 4, std=0.5)
        norm = tf.Qwen3_5RMSNormGated(dk, eps=1e-6)

        def gdn(xqkv, z, a, b, S0, conv_pre):
            L = xqkv.shape[1]
            xc = torch.cat([conv_pre, xqkv], 1).transpose(1, 2)  # [B, C, 3 + L]
            xc = F.silu(F.conv1d(xc, w, groups=C)).transpose(1, 2)
            q, k, v = torch.split(xc, [Hk * dk, Hk * dk, Hv * dk], -1)
            q = q.reshape(*q.shape[:2], Hk, dk).repeat_interleave(2, 2)
            k = k.reshape(*k.shape[:2], Hk, dk).repeat_interleave(2, 2)
            v = v.reshape(*v.shape[:2], Hv, dk)
            gg = -F.softplus(a)
            o, S = tf.torch_chunk_gated_delta_rule(q, k, v, g=gg, beta=b.sigmoid(),
                                                   initial_state=S0, output_final_state=True,
                                                   use_qk_l2norm_in_kernel=True)
            return norm(o.reshape(-1, dk), z.reshape(-1, dk)), S

        xq, z, a, b = randn(1, T, C), randn(1, T, Hv * dk), randn(1, T, Hv), randn(1, T, Hv)
        out["config2_gdn_prefill_ms"] = round(
            _timed(lambda: gdn(xq, z, a, b, None, torch.zeros(1, 3, C)), reps), 2)
        _, S = gdn(xq, z, a, b, None, torch.zeros(1, 3, C))
        Bn, Lb = 64, 16
        xq2, z2 = randn(Bn, Lb, C), randn(Bn, Lb, Hv * dk)
        a2, b2 = randn(Bn, Lb, Hv), randn(Bn, Lb, Hv)
        S0, tail = S.expand(Bn, -1, -1, -1).contiguous(), xq[:, -3:].expand(Bn, -1, -1)
        out["config2_gdn_branches_ms"] = round(
            _timed(lambda: gdn(xq2, z2, a2, b2, S0, tail), reps), 2)
        log(f"cpu config 2: prefill {out['config2_gdn_prefill_ms']} ms, "
            f"branches {out['config2_gdn_branches_ms']} ms")

        # config 3: shared-prefix attention at capacity, Hq 16 / Hkv 4, D 256
        P, Bn, Lb, Hq, Hkv, D = 8192, 256, 16, 16, 4, 256
        ks, vs = randn(Hkv, P, D), randn(Hkv, P, D)
        q, gate = randn(Bn, Lb, Hq, D), randn(Bn, Lb, Hq, D)
        ko, vo = randn(Bn, Lb, Hkv, D), randn(Bn, Lb, Hkv, D)
        own_mask = torch.full((Lb, Lb), float("-inf")).triu(1)

        def att3(step=16):
            res = []
            for b0 in range(0, Bn, step):
                qb = q[b0:b0 + step].permute(0, 2, 1, 3).reshape(step, Hkv, 4 * Lb, D)
                kb = torch.cat([ks.expand(step, -1, -1, -1),
                                ko[b0:b0 + step].permute(0, 2, 1, 3)], 2)
                vb = torch.cat([vs.expand(step, -1, -1, -1),
                                vo[b0:b0 + step].permute(0, 2, 1, 3)], 2)
                s = qb @ kb.transpose(-1, -2) / 16.0
                s[..., P:] += own_mask.repeat(4, 1)
                o = torch.softmax(s, -1) @ vb
                o = o.reshape(step, Hq, Lb, D).permute(0, 2, 1, 3)
                res.append(o * torch.sigmoid(gate[b0:b0 + step]))
            return torch.cat(res)

        out["config3_attention_ms"] = round(_timed(att3, max(1, reps - 1)), 2)
        log(f"cpu config 3 attention: {out['config3_attention_ms']} ms")
    out["threads"] = n
    return out
