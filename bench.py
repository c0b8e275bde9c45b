#!/usr/bin/env python3
"""Benchmark of the branch-forward hot path on one MI355X.

Workload (BASELINE.json metric, config 4): a random-init Qwen3.5-4B-shaped
hybrid model (32 layers, every 4th full gated attention, hidden 2560, vocab
248320, bf16 weights ~ N(0, 0.02)); one request = a fresh 530-token
random-id state prefill + 4 question branches of 20 tokens, read out over
3/2/2/4 single-token labels. A step is one request. `value` is requests/s
(one request = one decision, the Starfighter sense); branch-decisions/s
(4 per request, the cujev-bench sense) and p50 ms/request are reported next
to it. The request makes the reference's API calls (prefill, then eval) on
an engine opened with CUJEV_DEFER_PREFILL=1: the prefill's tokens are staged
and run inside the eval, one pass over state and branch tokens, so each
layer's weights are streamed once per request. The default engine (each
prefill runs when called) is timed first and reported as `eager_prefill`.

Also measured:
  config5        config 5 end to end: a random-init Qwen3.5-9B-shaped model
                 (hidden 4096, intermediate 12288, untied LM head) at the
                 engine's default capacity: 8192-token state, 256 branches x
                 16 tokens, 8 labels each (no CPU leg at this size);
  roofline       the shared-prefix attention kernel at config 3 (Hq 16/Hkv 4,
                 state 8192, 256 branches x 16 tokens) against the bf16 dense
                 MFMA peak, HIP events on its launch stream;
  gdn_roofline   the Gated DeltaNet layer at config 2 (T=2048 prefill; and
                 the 64 x 16 branches) against the HBM peak, from its
                 compulsory bytes.
cpu_baseline: transformers' Qwen3_5ForCausalLM in fp32 on every host core
this process may use, on the same checkpoint file and the first request (the
HF-batched method of the reference's benchmarks/benefit.py:77-92): one
full-size warm-up, then 5 timed requests, p50; configs 1-3 one layer at a
time beside it. The same fp32 run is the parity reference of the request's
decision probabilities.

The request loops run in a child process that imports only numpy and the
ctypes binding, as the reference's Python layer does (python/cujev/_lib.py,
systemone.py): a process that imported torch first would run the engine on
torch's bundled HIP runtime and hipBLASLt instead of the system ROCm's.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-config5]
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
# the request of each end-to-end workload and the engine capacities it runs at
WORKLOADS = {
    "config4": dict(preset="4b", ckpt="/tmp/cujev_synth_4b", state=530, branch=20,
                    labels=[3, 2, 2, 4],
                    opts=dict(max_state_tokens=1024, max_branch_tokens=256, max_branches=16,
                              max_candidates=256)),
    "config5": dict(preset="9b", ckpt="/tmp/cujev_synth_9b", state=8192, branch=16,
                    labels=[8] * 256,
                    opts=dict(max_state_tokens=8192, max_branch_tokens=4096, max_branches=256,
                              max_candidates=8)),
}
STATE_TOKENS, BRANCH_TOKENS = 530, 20


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_request(rng, vocab, wl="config4"):
    """(state ids, [(branch ids, candidate ids)]) of one request: ids in
    [1000, 60000) as in the reference's tests/python/test_engine.py:56-58,
    distinct single-token labels in [16, 1000)."""
    w = WORKLOADS[wl]
    state = [int(x) for x in rng.integers(1000, 60000, size=w["state"])]
    branches = []
    for n in w["labels"]:
        toks = [int(x) for x in rng.integers(1000, 60000, size=w["branch"])]
        cands = [int(x) for x in rng.choice(np.arange(16, 1000), size=n, replace=False)]
        branches.append((toks, cands))
    return state, branches


# --------------------------------------------------------------------------
# end to end
# --------------------------------------------------------------------------
def run_e2e(ckpt, steps, warmup, wl="config4", seed=0, full_logits=True):
    from cujev import Branch, Engine
    eng = Engine(ckpt, **WORKLOADS[wl]["opts"])
    rng = np.random.default_rng(seed)
    reqs = [make_request(rng, eng.vocab_size, wl) for _ in range(warmup + steps)]
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
    # full-vocabulary logits of the first request: the parity check (config
    # 4) or the readout property (candidate logits == full logits)
    state, brs = reqs[0]
    eng.prefill(state)
    first_full = eng.eval_full_logits([Branch(t, []) for t, _ in brs]) if full_logits else None
    checks = {"finite": bool(all(np.all(np.isfinite(o)) for o in first_out))}
    if first_full is not None:
        checks["candidates_equal_full_logits_max_abs"] = float(max(
            np.abs(np.asarray(o) - first_full[i, c]).max() for i, (o, (_, c)) in
            enumerate(zip(first_out, brs))))
    info = dict(name=eng.name, weight_gib=eng.weight_bytes / 2 ** 30,
                workspace_gib=eng.workspace_bytes / 2 ** 30)
    eng.close()
    return dict(wall_ms=wall, gpu_ms=gpu, eval_only_ms=ev_only, first_req=reqs[0],
                first_out=first_out, first_full=first_full, info=info, checks=checks)


# The reference's own benchmark shapes (tools/bench.c:41-74; its published
# RTX 5090 rows, README.md:233-235, 4B and 9B): prefill P tokens, then one
# eval of B branches x L tokens with C candidates each, timed by the
# library's own GPU timing (cujev_last_timing), decisions/s = B / eval time.
REF_BENCH_SHAPES = [
    {"model": "4b", "P": 1024, "B": 16, "L": 40, "C": 8,
     "rtx5090": {"prefill_ms": 60.0, "eval_ms": 37.0, "decisions_per_s": 430}},
    {"model": "4b", "P": 8192, "B": 64, "L": 40, "C": 8,
     "rtx5090": {"prefill_ms": 550.0, "eval_ms": 185.0, "decisions_per_s": 350}},
    {"model": "9b", "P": 1024, "B": 16, "L": 40, "C": 8,
     "rtx5090": {"prefill_ms": 106.0, "eval_ms": 61.0, "decisions_per_s": 262}},
]


def run_ref_shapes(ckpt, model="4b", iters=5):
    """tools/bench.c's method on this engine: deterministic token ids
    1000 + (7919 i mod 50000), candidates 32..32+C-1, one warm-up, then the
    mean of `iters` prefill and eval timings."""
    from cujev import Branch, Engine
    out = []
    eng = Engine(ckpt, max_state_tokens=8192, max_branch_tokens=4096, max_branches=256,
                 max_candidates=256)
    try:
        for sh in [x for x in REF_BENCH_SHAPES if x["model"] == model]:
            P, B, L, C = sh["P"], sh["B"], sh["L"], sh["C"]
            tok = [1000 + (i * 7919) % 50000 for i in range(P + B * L)]
            cands = list(range(32, 32 + C))
            brs = [Branch(tok[P + b * L: P + (b + 1) * L], cands) for b in range(B)]
            eng.prefill(tok[:P])
            eng.eval(brs)
            pre = ev = 0.0
            for _ in range(iters):
                eng.prefill(tok[:P])
                pre += eng.last_timing().prefill_ms
                eng.eval(brs)
                ev += eng.last_timing().eval_ms
            pre, ev = pre / iters, ev / iters
            out.append({"model": model, "state_tokens": P, "branches": B, "branch_tokens": L,
                        "candidates": C,
                        "prefill_ms": round(pre, 3), "prefill_tok_per_s": round(P / pre * 1e3),
                        "eval_ms": round(ev, 3), "decisions_per_s": round(B / ev * 1e3, 1),
                        "iters": iters, "reference_rtx5090": sh["rtx5090"]})
    finally:
        eng.close()
    return out


def e2e_child(a):
    """--e2e-child: the request loop without torch in the process; prints one
    JSON line, the full-vocabulary logits go to a .npy file."""
    assert "torch" not in sys.modules
    if a.workload.startswith("ref_shapes"):
        model = a.workload.split(":")[1] if ":" in a.workload else "4b"
        print(json.dumps({"ref_shapes": run_ref_shapes(a.ckpt, model)}), flush=True)
        return
    r = run_e2e(a.ckpt, a.steps, a.warmup, wl=a.workload)
    if r["first_full"] is not None and a.workload == "config4":
        np.save(a.full_out, np.asarray(r["first_full"], np.float32), allow_pickle=False)
    r["first_full"] = None
    r["first_out"] = [np.asarray(o, np.float64).tolist() for o in r["first_out"]]
    r["torch_loaded"] = "torch" in sys.modules
    print(json.dumps(r), flush=True)


def run_e2e_in_child(ckpt, steps, warmup, wl="config4", defer=False):
    """defer: the engine opened with CUJEV_DEFER_PREFILL=1, so each request's
    prefill runs inside its eval as one pass over state and branch tokens
    (same API calls, same outputs; each layer's weights streamed once)."""
    import subprocess
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        full = os.path.join(d, "full.npy")
        cmd = [sys.executable, str(Path(__file__).resolve()), "--e2e-child", "--ckpt", ckpt,
               "--workload", wl, "--steps", str(steps), "--warmup", str(warmup),
               "--full-out", full]
        env = dict(os.environ, CUJEV_DEFER_PREFILL="1" if defer else "0")
        p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=sys.stderr, text=True, env=env)
        if p.returncode != 0:
            raise SystemExit(f"e2e child ({wl}) failed with status {p.returncode}")
        r = json.loads(p.stdout.strip().splitlines()[-1])
        r["first_full"] = np.load(full, allow_pickle=False) if os.path.exists(full) else None
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


def cpu_baseline(ckpt, req, eng_out, eng_full, reps=5):
    """transformers fp32 on every host core this process may use: the timed
    baseline (p50 of `reps` requests after a full-size warm-up) and the
    parity reference; configs 1-3 timed one layer at a time beside it.
    transformers' own bf16 run on the same request is reported next to the
    engine's deviation: on a random-init 32-layer model the bf16 rounding of
    GEMM inputs alone moves logits by a few tenths, for any bf16 engine."""
    try:
        from cujev import cpu_baseline as cb
        import transformers  # noqa: F401
    except Exception as e:  # pragma: no cover
        return None, {"error": f"CPU baseline unavailable: {e}"}
    info = cb.cpu_info()
    state, brs = req
    t0 = time.perf_counter()
    r = cb.request_baseline(ckpt, state, brs, reps=reps, log=log)
    lg32, lg16 = r["fp32_logits"], r["bf16_logits"]
    layers = cb.layer_baselines(log=log)
    log(f"cpu baseline legs took {time.perf_counter() - t0:.0f} s")

    def dev(logits_labels, logits_full):
        dp = max(float(np.abs(_softmax(logits_labels[i]) - _softmax(lg32[i, c])).max())
                 for i, (_, c) in enumerate(brs))
        agree = all(int(np.argmax(logits_labels[i])) == int(np.argmax(lg32[i, c]))
                    for i, (_, c) in enumerate(brs))
        full = np.asarray(logits_full, np.float64)
        dl = float(np.abs(full - lg32).max())
        l1 = max(float(np.abs(_softmax(full[i]) - _softmax(lg32[i])).sum())
                 for i in range(len(brs)))
        return {"max_abs_dprob_labels": round(dp, 5), "argmax_identical": agree,
                "max_abs_dlogit_full_vocab": round(dl, 4),
                "max_L1_full_vocab_distribution": round(l1, 4)}

    eng = dev([np.asarray(o, np.float64) for o in eng_out], eng_full)
    hf16 = dev([lg16[i, c] for i, (_, c) in enumerate(brs)], lg16)
    margins = [round(float(np.sort(lg32[i, c])[-1] - np.sort(lg32[i, c])[-2]), 4)
               for i, (_, c) in enumerate(brs)]
    p50 = statistics.median(r["times_s"])
    w = WORKLOADS["config4"]
    base = {"value": round(1.0 / p50, 5), "unit": "requests/s", "cores": r["threads"],
            "kind": "reference",
            "sample": (f"{reps} requests after one full-size warm-up, p50: each request = "
                       f"{len(brs)} rows of [{w['state']}+{w['branch']}] tokens in one batch, "
                       f"logits_to_keep=1, through transformers Qwen3_5ForCausalLM fp32 on "
                       f"{r['threads']} host threads ({info['cpu_model']})"),
            "ms_per_request_p50": round(p50 * 1e3, 1),
            "ms_per_request_all": [round(t * 1e3, 1) for t in r["times_s"]],
            "cpu_model": info["cpu_model"],
            "layers": layers}
    parity = {"reference": "transformers Qwen3_5ForCausalLM fp32 (CPU), same checkpoint and request",
              "engine": eng, "transformers_bf16": hf16, "label_top2_logit_margins": margins,
              "reference_repo_bar": "full-vocabulary L1 to fp32 < 0.05 "
                                    "(tests/python/oracle_fp32.py:52)"}
    return base, parity


FIXTURE_4B = ROOT / "tests" / "golden" / "request_4b.npz"


def config4_checkpoint(path):
    """Config 4's checkpoint is the golden fixture's: cujev.synthetic's
    "blocks" generator (numpy PCG64 per tensor block, the same bits on every
    host) with seed 0, so the bench's first request is the fixture's request
    on the very same weights. Returns (dir, pin) where pin records the
    file's SHA-256 against the one the fixture stores."""
    from cujev import synthetic
    want = str(np.load(FIXTURE_4B, allow_pickle=False)["checkpoint_sha256"])
    ckpt = synthetic.ensure_checkpoint(path, "4b", seed=0, generator="blocks", sha256=want)
    got = synthetic.file_sha256(Path(ckpt) / "model.safetensors")
    return ckpt, {"checkpoint_sha256": got, "fixture_sha256": want, "matches": got == want}


def fixture_parity(pin, req, outs, full):
    """The first request's decisions against the config-4 golden fixture
    (tests/golden/request_4b.npz: the same checkpoint and request through the
    float64 oracle, "f64" = transformers' math, and with the reference
    engine's bf16 rounding points, "engine"; three jitter seeds of "engine"
    give the noise floor between two correct bf16 engines).

    outs: {engine mode: candidate logits per branch}; full: [B, vocab] full
    logits of the first mode. Per branch: the label top-2 margin in the
    "engine" vectors and in "f64", and whether the argmax agrees; a margin
    is resolvable when it exceeds twice the largest label-logit deviation
    of any jitter seed (each of the two labels may move by that much)."""
    g = np.load(FIXTURE_4B, allow_pickle=False)
    state, brs = req
    same = (pin["matches"] and [int(x) for x in g["state"]] == list(state)
            and all([int(x) for x in g["branch_tokens"][i]] == list(t) for i, (t, _) in
                    enumerate(brs))
            and [int(x) for x in g["cand_flat"]] == [int(x) for _, c in brs for x in c])
    res = {"fixture": "tests/golden/request_4b.npz (tests/golden/make_request_4b.py)",
           "checkpoint": pin, "request_matches_fixture": bool(same)}
    if not same:
        res["error"] = "the bench checkpoint or request differs from the fixture's"
        return res
    offs = np.concatenate([[0], np.cumsum(g["cand_len"])]).astype(int)
    split = lambda v: [np.asarray(v[offs[i]:offs[i + 1]], np.float64) for i in range(len(brs))]
    lab = {str(m): split(v) for m, v in zip(g["label_modes"], g["label_logits"])}
    jit = [m for m in lab if m.startswith("engine~")]
    stats = dict(zip([str(m) for m in g["stat_modes"]], g["stat_values"]))
    floor_dp = max(float(stats[m][2]) for m in jit)
    floor_rms = max(float(stats[m][1]) for m in jit)
    floor_lab = max(float(np.abs(lab[m][i] - lab["engine"][i]).max()) for m in jit
                    for i in range(len(brs)))
    ids = g["sample_ids"]

    def margin(v):
        s = np.sort(v)
        return float(s[-1] - s[-2])

    def versus(o, ref):
        return max(float(np.abs(_softmax(o[i]) - _softmax(ref[i])).max())
                   for i in range(len(brs)))

    engines = {}
    for mode, out in outs.items():
        o = [np.asarray(x, np.float64) for x in out]
        e = {"max_abs_dprob_vs_engine_oracle": round(versus(o, lab["engine"]), 5),
             "max_abs_dprob_vs_f64_oracle": round(versus(o, lab["f64"]), 5),
             "argmax_identical_engine_oracle": all(
                 int(np.argmax(o[i])) == int(np.argmax(lab["engine"][i])) for i in range(len(brs))),
             "argmax_identical_f64_oracle": all(
                 int(np.argmax(o[i])) == int(np.argmax(lab["f64"][i])) for i in range(len(brs)))}
        if full is not None and mode == next(iter(outs)):
            f = np.asarray(full, np.float64)[:, ids]
            e["rms_dlogit_vs_engine_oracle"] = round(
                float(np.sqrt(np.mean((f - g["sample_engine"]) ** 2))), 4)
            e["rms_dlogit_vs_f64_oracle"] = round(
                float(np.sqrt(np.mean((f - g["sample_f64"]) ** 2))), 4)
        e["branches"] = [{"labels": len(brs[i][1]),
                          "margin_engine_oracle": round(margin(lab["engine"][i]), 4),
                          "margin_f64_oracle": round(margin(lab["f64"][i]), 4),
                          "margin_engine": round(margin(o[i]), 4),
                          "resolvable": margin(lab["engine"][i]) > 2 * floor_lab,
                          "argmax_agrees": int(np.argmax(o[i])) == int(np.argmax(lab["engine"][i]))}
                         for i in range(len(brs))]
        e["argmax_identical_where_resolvable"] = all(
            b["argmax_agrees"] for b in e["branches"] if b["resolvable"])
        engines[mode] = e
    res["engine"] = engines
    res["noise_floor"] = {"what": "the reference-engine numerics under three other valid fp32 "
                                  "summation orders (2^-24 jitter before every bf16 rounding)",
                          "max_abs_dprob": round(floor_dp, 5), "rms_dlogit": round(floor_rms, 4),
                          "max_abs_label_dlogit": round(floor_lab, 4)}
    res["reference_engine_vs_f64"] = {"max_abs_dprob": round(versus(lab["engine"], lab["f64"]), 5)}
    first = engines[next(iter(outs))]
    res["bars"] = {"north_star_max_abs_dprob_1e-3": first["max_abs_dprob_vs_engine_oracle"] <= 1e-3,
                   "floor_relative_1.5x": bool(
                       first["max_abs_dprob_vs_engine_oracle"] <= 1.5 * floor_dp
                       and first.get("rms_dlogit_vs_engine_oracle", 0.0) <= 1.5 * floor_rms),
                   "note": "the 1e-3 bar lies below the noise floor: two correct bf16 engines "
                           "(the jitter seeds) already differ by max |dp| "
                           f"{floor_dp:.1e} on this checkpoint and request"}
    res["summary"] = {m: {k: v for k, v in e.items() if k != "branches"}
                      for m, e in engines.items()}
    return res


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
                                         "(copy-calibrated), bytes per launch, measured at "
                                         + kernel_bench.MEASURED_AT["attention"],
                       "us_per_launch": round(att["us"], 2),
                       "flop_per_launch": att["flop"]}
    gdn = gdn_roofline()
    log(f"gdn config 2 prefill: {gdn['us']:.1f} us, {gdn['gbs']:.1f} GB/s")
    res["gdn_roofline"] = {"kernel": "gdn layer call: chunk_a (conv and gates inside) + "
                                     "chunk_b (conv tail copied by extra workgroups) + "
                                     "norm_gate, config 2 T=2048 prefill", "bound": "hbm",
                           "achieved": round(gdn["gbs"], 1), "peak": PEAK_HBM_GBS,
                           "unit": "GB/s", "frac": round(gdn["gbs"] / PEAK_HBM_GBS, 4),
                           "us_per_layer": round(gdn["us"], 2),
                           "compulsory_bytes": gdn["bytes"],
                           "traffic": kernel_bench.measured_traffic("gdn"),
                           "traffic_measured_at": kernel_bench.MEASURED_AT["gdn"]}
    gbr = gdn_roofline(case="gdn_branch")
    log(f"gdn config 2 branches: {gbr['us']:.1f} us, {gbr['gbs']:.1f} GB/s")
    res["gdn_branch_roofline"] = {"kernel": "gdn layer call: chunk_a (conv and gates inside, "
                                            "packed chunks) + short_b (norm inside), config "
                                            "2, 64 branches x 16 tokens", "bound": "hbm",
                                  "achieved": round(gbr["gbs"], 1), "peak": PEAK_HBM_GBS,
                                  "unit": "GB/s", "frac": round(gbr["gbs"] / PEAK_HBM_GBS, 4),
                                  "us_per_layer": round(gbr["us"], 2),
                                  "compulsory_bytes": gbr["bytes"],
                                  "traffic": kernel_bench.measured_traffic("gdn_branch"),
                                  "traffic_measured_at": kernel_bench.MEASURED_AT["gdn_branch"]}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--ckpt", default=os.environ.get("CUJEV_BENCH_CKPT",
                                                     WORKLOADS["config4"]["ckpt"]))
    ap.add_argument("--ckpt9b", default=os.environ.get("CUJEV_BENCH_CKPT9B",
                                                       WORKLOADS["config5"]["ckpt"]))
    ap.add_argument("--no-config5", action="store_true", help="skip the 9B capacity line")
    ap.add_argument("--config5-steps", type=int, default=5)
    ap.add_argument("--workload", default="config4", help=argparse.SUPPRESS)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ref-shapes", action="store_true",
                    help="skip the reference's published cujev-bench shapes")
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
    t0 = time.perf_counter()
    ckpt, ckpt_pin = config4_checkpoint(a.ckpt)
    log(f"checkpoint ready at {ckpt} ({time.perf_counter() - t0:.1f}s): {ckpt_pin}")

    # the default engine (each prefill runs when called, the reference's
    # timing split), then prefills deferred into the eval: `value`
    eager = run_e2e_in_child(ckpt, a.steps, a.warmup)
    ems, ep50 = statistics.mean(eager["wall_ms"]), statistics.median(eager["wall_ms"])
    log(f"e2e, eager prefill: {ems:.2f} ms/request mean, p50 {ep50:.2f} ms, GPU p50 "
        f"{statistics.median(eager['gpu_ms']):.2f} ms")
    e2e = run_e2e_in_child(ckpt, a.steps, a.warmup, defer=True)
    wall = e2e["wall_ms"]
    ms = statistics.mean(wall)
    p50 = statistics.median(wall)
    log(f"e2e, deferred prefill: {ms:.2f} ms/request mean, p50 {p50:.2f} ms, GPU p50 "
        f"{statistics.median(e2e['gpu_ms']):.2f} ms")
    same = max(float(np.abs(np.asarray(x) - np.asarray(y)).max())
               for x, y in zip(e2e["first_out"], eager["first_out"]))
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
                   "vocab": 248320, "weights_gib": round(e2e["info"]["weight_gib"], 2),
                   "prefill": "deferred (CUJEV_DEFER_PREFILL=1): the request's prefill and "
                              "eval calls run as one pass over state + branch tokens"},
        "eager_prefill": {"value": round(1e3 / ems, 3), "ms_per_step": round(ems, 3),
                          "p50_ms_per_request": round(ep50, 3),
                          "gpu_ms_per_request_p50": round(statistics.median(eager["gpu_ms"]), 3),
                          "first_request_max_abs_dlogit_vs_deferred": same,
                          "note": "the default engine: each prefill runs when called"},
    }
    res["e2e_checks"] = e2e["checks"]
    try:
        fxp = fixture_parity(ckpt_pin, e2e["first_req"],
                             {"deferred": e2e["first_out"], "eager": eager["first_out"]},
                             e2e["first_full"])
    except (KeyError, ValueError, OSError) as ex:  # a fixture without these fields
        fxp = {"fixture": str(FIXTURE_4B), "error": f"{type(ex).__name__}: {ex}"}
    log(f"parity vs the config-4 fixture: {json.dumps(fxp.get('summary', fxp))}")
    if not a.no_config5:
        res["config5"] = config5_line(a)
    if not a.no_ref_shapes:
        res["reference_bench_shapes"] = ref_shapes_line(
            ckpt, a.ckpt9b if os.path.isdir(a.ckpt9b) else None)
    if not a.no_kernels:
        res.update(kernel_rooflines())
    if not a.no_cpu_baseline:
        torch.cuda.empty_cache()
        base, parity = cpu_baseline(ckpt, e2e["first_req"], e2e["first_out"], e2e["first_full"])
        res["cpu_baseline"] = base
        fxp["transformers_fp32"] = parity
        if base:
            log(f"cpu baseline: {base['ms_per_request_p50']:.0f} ms/request p50; parity {parity}")
    res["parity"] = fxp
    print(json.dumps(res), flush=True)


def config5_line(a):
    """Config 5: the 9B-shaped model (untied LM head) at capacity, a fresh
    8192-token state + 256 branches x 16 tokens with 8 labels each per
    request, in the torch-free child. The checkpoint is written once on the
    device (torch's generator) and reused; there is no CPU leg at this size."""
    import torch
    from cujev import synthetic
    t0 = time.perf_counter()
    ckpt = synthetic.ensure_checkpoint(a.ckpt9b, "9b", seed=0, device="cuda")
    torch.cuda.empty_cache()
    log(f"9B checkpoint ready at {ckpt} ({time.perf_counter() - t0:.1f}s)")
    re = run_e2e_in_child(ckpt, a.config5_steps, 1, wl="config5")
    ems = statistics.mean(re["wall_ms"])
    log(f"config 5, eager prefill: {ems:.1f} ms/request mean, p50 "
        f"{statistics.median(re['wall_ms']):.1f} ms")
    r = run_e2e_in_child(ckpt, a.config5_steps, 1, wl="config5", defer=True)
    wall = r["wall_ms"]
    ms, p50 = statistics.mean(wall), statistics.median(wall)
    nb = len(WORKLOADS["config5"]["labels"])
    log(f"config 5, deferred prefill: {ms:.1f} ms/request mean, p50 {p50:.1f} ms, checks "
        f"{r['checks']}")
    return {"workload": "Qwen3.5-9B-shaped hybrid (hidden 4096, intermediate 12288, 32 layers, "
                        "8 full attention, untied LM head), fresh 8192-token state prefill + 256 "
                        "branches x 16 tokens, 8 labels per branch",
            "requests_per_s": round(1e3 / ms, 3), "branch_decisions_per_s": round(nb * 1e3 / ms, 1),
            "ms_per_request_mean": round(ms, 2), "p50_ms_per_request": round(p50, 2),
            "gpu_ms_per_request_p50": round(statistics.median(r["gpu_ms"]), 2),
            "eval_only_ms_p50": round(statistics.median(r["eval_only_ms"]), 2),
            "steps": a.config5_steps, "warmup": 1, "checks": r["checks"],
            "weights_gib": round(r["info"]["weight_gib"], 2),
            "workspace_gib": round(r["info"]["workspace_gib"], 2),
            "prefill": "deferred (CUJEV_DEFER_PREFILL=1)",
            "eager_prefill": {"ms_per_request_mean": round(ems, 2),
                              "p50_ms_per_request": round(statistics.median(re["wall_ms"]), 2),
                              "workspace_gib": round(re["info"]["workspace_gib"], 2)},
            "cpu_baseline": None}


def ref_shapes_line(ckpt, ckpt9b=None):
    """The reference benchmark's shapes on the same synthetic checkpoints (the
    9B row when its checkpoint is there), each model in a torch-free child;
    the RTX 5090 figures are the reference's published numbers on other
    hardware, for context only."""
    import subprocess
    rows = []
    for model, path in (("4b", ckpt), ("9b", ckpt9b)):
        if not path:
            continue
        cmd = [sys.executable, str(Path(__file__).resolve()), "--e2e-child", "--ckpt", path,
               "--workload", f"ref_shapes:{model}"]
        p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=sys.stderr, text=True)
        if p.returncode != 0:
            raise SystemExit(f"reference-shape child ({model}) failed with status {p.returncode}")
        rows += json.loads(p.stdout.strip().splitlines()[-1])["ref_shapes"]
    for r in rows:
        log(f"cujev-bench shape {r['model']} P={r['state_tokens']} {r['branches']}x"
            f"{r['branch_tokens']}: prefill {r['prefill_ms']:.2f} ms, eval {r['eval_ms']:.2f} ms, "
            f"{r['decisions_per_s']:.0f} decisions/s")
    return {"method": "tools/bench.c:41-74 (prefill then one eval, cujev_last_timing GPU ms, "
                      "decisions/s = branches / eval ms), the 4B and 9B shapes of "
                      "README.md:233-235",
            "rows": rows}


if __name__ == "__main__":
    main()
