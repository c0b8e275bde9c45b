#!/usr/bin/env python3
"""Benchmark of the branch-forward hot path on one MI355X.

Workload (BASELINE.json metric, config 4): a random-init Qwen3.5-4B-shaped
hybrid model (32 layers, every 4th full gated attention, hidden 2560, vocab
248320, bf16 weights ~ N(0, 0.02)); one request = a fresh 530-token
random-id state prefill + 4 question branches of 20 tokens, read out over
3/2/2/4 single-token labels. A step is one request. `value` is requests/s
(one request = one decision, the Starfighter sense); branch-decisions/s
(4 per request, the cujev-bench sense) and p50 ms/request are reported next
to it.

Also measured, each in its own timed loop with HIP events on the stream the
kernel is launched on:
  roofline       the shared-prefix attention kernel at config 3 (Hq 16/Hkv 4,
                 state 8192, 256 branches x 16 tokens) against the bf16 dense
                 MFMA peak;
  gdn_roofline   the Gated DeltaNet layer at config 2 (T=2048 prefill) against
                 the HBM peak, from its compulsory bytes.
cpu_baseline: transformers' Qwen3_5ForCausalLM in fp32 on the host cores, on
the same checkpoint file and the same first request (the HF-batched method
of the reference's benchmarks/benefit.py:77-92); it is also the parity check
of the request's decision probabilities.

The request loop runs in a child process that imports only numpy and the
ctypes binding, as the reference's Python layer does (python/cujev/_lib.py,
systemone.py): a process that imported torch first would run the engine on
torch's bundled HIP runtime and hipBLASLt instead of the system ROCm's.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "cu-jev_amd"))
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
STATE_TOKENS = 530
BRANCH_TOKENS = 20
LABELS = [3, 2, 2, 4]      # labels per question (Starfighter-style)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_request(rng, vocab):
    state = [int(x) for x in rng.integers(1000, 60000, size=STATE_TOKENS)]
    branches = []
    for n in LABELS:
        toks = [int(x) for x in rng.integers(1000, 60000, size=BRANCH_TOKENS)]
        cands = [int(x) for x in rng.choice(np.arange(16, 1000), size=n, replace=False)]
        branches.append((toks, cands))
    return state, branches


# --------------------------------------------------------------------------
# end to end
# --------------------------------------------------------------------------
def run_e2e(ckpt, steps, warmup, seed=0):
    from cujev import Branch, Engine
    eng = Engine(ckpt, max_state_tokens=1024, max_branch_tokens=256, max_branches=16,
                 max_candidates=256)
    rng = np.random.default_rng(seed)
    reqs = [make_request(rng, eng.vocab_size) for _ in range(warmup + steps)]
    first_out = None
    wall, gpu = [], []
    for i, (state, brs) in enumerate(reqs):
        t0 = time.perf_counter()
        eng.prefill(state)
        pre_ms = eng.last_timing().prefill_ms
        out = eng.eval([Branch(t, c) for t, c in brs])
        t1 = time.perf_counter()
        ev_ms = eng.last_timing().eval_ms
        if i == 0:
            first_out = out
        if i >= warmup:
            wall.append((t1 - t0) * 1e3)
            gpu.append(pre_ms + ev_ms)
    # eval only, state cached (benchmarks/benefit.py:62-66)
    state, brs = reqs[-1]
    eng.prefill(state)
    ev_only = []
    for _ in range(max(steps, 5)):
        t0 = time.perf_counter()
        eng.eval([Branch(t, c) for t, c in brs])
        ev_only.append((time.perf_counter() - t0) * 1e3)
    # full-vocabulary logits of the first request, for the parity check
    state, brs = reqs[0]
    eng.prefill(state)
    first_full = eng.eval_full_logits([Branch(t, []) for t, _ in brs])
    info = dict(name=eng.name, weight_gib=eng.weight_bytes / 2 ** 30)
    eng.close()
    return dict(wall_ms=wall, gpu_ms=gpu, eval_only_ms=ev_only, first_req=reqs[0],
                first_out=first_out, first_full=first_full, info=info)


def e2e_child(a):
    """--e2e-child: the request loop without torch in the process; prints one
    JSON line, the full-vocabulary logits go to a .npy file."""
    assert "torch" not in sys.modules
    r = run_e2e(a.ckpt, a.steps, a.warmup)
    np.save(a.full_out, np.asarray(r["first_full"], np.float32), allow_pickle=False)
    r["first_full"] = None
    r["first_out"] = [np.asarray(o, np.float64).tolist() for o in r["first_out"]]
    r["torch_loaded"] = "torch" in sys.modules
    print(json.dumps(r), flush=True)


def run_e2e_in_child(ckpt, steps, warmup):
    import subprocess
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        full = os.path.join(d, "full.npy")
        cmd = [sys.executable, str(Path(__file__).resolve()), "--e2e-child", "--ckpt", ckpt,
               "--steps", str(steps), "--warmup", str(warmup), "--full-out", full]
        p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=sys.stderr, text=True)
        if p.returncode != 0:
            raise SystemExit(f"e2e child failed with status {p.returncode}")
        r = json.loads(p.stdout.strip().splitlines()[-1])
        r["first_full"] = np.load(full, allow_pickle=False)
    r["first_out"] = [np.asarray(o) for o in r["first_out"]]
    return r


# --------------------------------------------------------------------------
# kernel rooflines (operator C ABI, HIP events on the launch stream)
# --------------------------------------------------------------------------
# The first ~25 launches of a kernel in a fresh process run while the GPU's
# clocks ramp up (the first attention launch takes over 1 ms, later ones
# 484-490 us): the kernel cases warm up for ROOF_WARMUP launches and then time
# ROOF_ITERS, the steady state.
ROOF_WARMUP, ROOF_ITERS = 40, 50


def attention_roofline(iters=ROOF_ITERS, warmup=ROOF_WARMUP):
    from cujev import kernel_bench
    launch, info = kernel_bench.attention_case()
    us = kernel_bench.time_launches(launch, iters, warmup)
    return dict(us=us, flop=info["flop"], tflops=info["flop"] / (us * 1e-6) / 1e12)


def gdn_roofline(iters=ROOF_ITERS, case="gdn", warmup=ROOF_WARMUP):
    from cujev import kernel_bench
    launch, info = kernel_bench.CASES[case]()
    us = kernel_bench.time_launches(launch, iters, warmup)
    return dict(us=us, bytes=info["bytes"], gbs=info["bytes"] / (us * 1e-6) / 1e9)


# --------------------------------------------------------------------------
# CPU baseline: transformers fp32 on the host cores (and the parity check)
# --------------------------------------------------------------------------
def _softmax(x):
    x = np.asarray(x, np.float64)
    p = np.exp(x - x.max())
    return p / p.sum()


def cpu_baseline(ckpt, req, eng_out, eng_full):
    """transformers fp32 on the host cores: the timed baseline and the parity
    reference. transformers' own bf16 run on the same request is reported next
    to the engine's deviation: on a random-init 32-layer model the bf16 rounding
    of GEMM inputs alone moves logits by a few tenths, for any bf16 engine."""
    try:
        import torch
        from transformers import AutoModelForCausalLM
    except Exception as e:  # pragma: no cover
        return None, {"error": f"CPU baseline unavailable: {e}"}
    threads = min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "16")))
    torch.set_num_threads(threads)
    state, brs = req
    ids = torch.tensor([state + t for t, _ in brs])
    t0 = time.perf_counter()
    model = AutoModelForCausalLM.from_pretrained(ckpt, dtype=torch.float32).eval()
    log(f"transformers fp32 loaded on CPU in {time.perf_counter() - t0:.1f}s ({threads} threads)")
    with torch.no_grad():
        model(ids[:, :8], logits_to_keep=1)  # warm-up
        t0 = time.perf_counter()
        lg32 = model(ids, logits_to_keep=1).logits[:, -1, :].double().numpy()
        dt = time.perf_counter() - t0
    del model
    model = AutoModelForCausalLM.from_pretrained(ckpt, dtype=torch.bfloat16).eval()
    with torch.no_grad():
        lg16 = model(ids, logits_to_keep=1).logits[:, -1, :].double().numpy()
    del model

    def dev(logits_labels, logits_full):
        dp = max(float(np.abs(_softmax(logits_labels[i]) - _softmax(lg32[i, c])).max())
                 for i, (_, c) in enumerate(brs))
        agree = all(int(np.argmax(logits_labels[i])) == int(np.argmax(lg32[i, c]))
                    for i, (_, c) in enumerate(brs))
        dl = float(np.abs(np.asarray(logits_full) - lg32).max())
        return {"max_abs_dprob_labels": round(dp, 5), "argmax_identical": agree,
                "max_abs_dlogit_full_vocab": round(dl, 4)}

    eng = dev([np.asarray(o, np.float64) for o in eng_out], eng_full)
    hf16 = dev([lg16[i, c] for i, (_, c) in enumerate(brs)], lg16)
    margins = [round(float(np.sort(lg32[i, c])[-1] - np.sort(lg32[i, c])[-2]), 4)
               for i, (_, c) in enumerate(brs)]
    base = {"value": round(1.0 / dt, 5), "unit": "requests/s", "cores": threads,
            "kind": "reference",
            "sample": (f"1 request (4 branches x [{STATE_TOKENS}+{BRANCH_TOKENS}] tokens, one "
                       f"batch, logits_to_keep=1) through transformers Qwen3_5ForCausalLM fp32 "
                       f"on {threads} host threads: {dt:.1f} s"),
            "ms_per_request": round(dt * 1e3, 1)}
    parity = {"reference": "transformers Qwen3_5ForCausalLM fp32 (CPU), same checkpoint and request",
              "engine": eng, "transformers_bf16": hf16, "label_top2_logit_margins": margins}
    return base, parity


def kernel_rooflines():
    """The kernel roofline entries of the JSON line (attention, GDN prefill,
    GDN branches), each timed in its steady state."""
    res = {}
    from cujev import kernel_bench
    att = attention_roofline()
    log(f"attention config 3: {att['us']:.1f} us, {att['tflops']:.1f} TFLOP/s")
    res["roofline"] = {"kernel": "attention_kernel (ops library), config 3",
                       "bound": "mfma", "achieved": round(att["tflops"], 2),
                       "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                       "frac": round(att["tflops"] / PEAK_BF16_TFLOPS, 4),
                       "traffic": kernel_bench.measured_traffic("attention"),
                       "traffic_source": "rocprofv3 --pmc FETCH_SIZE x2 + WRITE_SIZE x1 "
                                         "(copy-calibrated), bytes per launch",
                       "us_per_launch": round(att["us"], 2),
                       "flop_per_launch": att["flop"]}
    gdn = gdn_roofline()
    log(f"gdn config 2 prefill: {gdn['us']:.1f} us, {gdn['gbs']:.1f} GB/s")
    res["gdn_roofline"] = {"kernel": "gdn layer call: conv_tail + chunk_a (conv and gates "
                                     "inside) + chunk_b + norm_gate, config 2 T=2048 "
                                     "prefill", "bound": "hbm",
                           "achieved": round(gdn["gbs"], 1), "peak": PEAK_HBM_GBS,
                           "unit": "GB/s", "frac": round(gdn["gbs"] / PEAK_HBM_GBS, 4),
                           "us_per_layer": round(gdn["us"], 2),
                           "compulsory_bytes": gdn["bytes"],
                           "traffic": kernel_bench.measured_traffic("gdn")}
    gbr = gdn_roofline(case="gdn_branch")
    log(f"gdn config 2 branches: {gbr['us']:.1f} us, {gbr['gbs']:.1f} GB/s")
    res["gdn_branch_roofline"] = {"kernel": "gdn layer call: chunk_a (conv and gates inside, "
                                            "packed chunks) + short_b (norm inside), config "
                                            "2, 64 branches x 16 tokens", "bound": "hbm",
                                  "achieved": round(gbr["gbs"], 1), "peak": PEAK_HBM_GBS,
                                  "unit": "GB/s", "frac": round(gbr["gbs"] / PEAK_HBM_GBS, 4),
                                  "us_per_layer": round(gbr["us"], 2),
                                  "compulsory_bytes": gbr["bytes"],
                                  "traffic": kernel_bench.measured_traffic("gdn_branch")}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--ckpt", default=os.environ.get("CUJEV_BENCH_CKPT", "/tmp/cujev_synth_4b"))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernels", action="store_true")
    ap.add_argument("--kernels-only", action="store_true",
                    help="only the kernel roofline entries (no request loop, no CPU baseline)")
    ap.add_argument("--e2e-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--full-out", help=argparse.SUPPRESS)
    a = ap.parse_args()
    if a.e2e_child:
        return e2e_child(a)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: the engine is single-device (one process, one "
              "stream per model) and this build runs no multi-GPU path; use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if a.kernels_only:
        print(json.dumps(kernel_rooflines()), flush=True)
        return
    from cujev import synthetic
    t0 = time.perf_counter()
    ckpt = synthetic.ensure_checkpoint(a.ckpt, "4b", seed=0, device="cuda")
    torch.cuda.empty_cache()
    log(f"checkpoint ready at {ckpt} ({time.perf_counter() - t0:.1f}s)")

    e2e = run_e2e_in_child(ckpt, a.steps, a.warmup)
    wall = e2e["wall_ms"]
    ms = statistics.mean(wall)
    p50 = statistics.median(wall)
    log(f"e2e: {ms:.2f} ms/request mean, p50 {p50:.2f} ms, GPU p50 "
        f"{statistics.median(e2e['gpu_ms']):.2f} ms")
    res = {
        "metric": "decisions/sec + p50 ms/request (4B shape, 530-tok state); attn MFMA util %",
        "value": round(1e3 / ms, 3),
        "unit": "decisions/s (requests/s; 1 request = 4 questions)",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 3),
        "p50_ms_per_request": round(p50, 3),
        "branch_decisions_per_s": round(4 * 1e3 / ms, 2),
        "gpu_ms_per_request_p50": round(statistics.median(e2e["gpu_ms"]), 3),
        "eval_only_ms_p50": round(statistics.median(e2e["eval_only_ms"]), 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random token ids, random-init bf16 weights ~N(0,0.02))",
        "config": {"workload": "Qwen3.5-4B-shaped hybrid, fresh 530-token state prefill + 4 "
                               "branches x 20 tokens, 3/2/2/4 labels per request",
                   "model": e2e["info"]["name"], "layers": 32, "hidden": 2560,
                   "vocab": 248320, "weights_gib": round(e2e["info"]["weight_gib"], 2)},
    }
    if not a.no_kernels:
        res.update(kernel_rooflines())
    if not a.no_cpu_baseline:
        torch.cuda.empty_cache()
        base, parity = cpu_baseline(ckpt, e2e["first_req"], e2e["first_out"], e2e["first_full"])
        res["cpu_baseline"] = base
        res["parity"] = parity
        if base:
            log(f"cpu baseline: {base['ms_per_request']:.0f} ms/request; parity {parity}")
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
