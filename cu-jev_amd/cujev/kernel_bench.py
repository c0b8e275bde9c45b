"""Kernel-level workloads of the hot path through the operator C ABI, used by
bench.py (timed with HIP events on the launch stream) and runnable on their
own for profilers:

    python -m cujev.kernel_bench attention|gdn|gdn_branch|gemm_*|blas_*|wide_*|copy [iters [warmup]]

attention  config 3: Hq 16 / Hkv 4, D 256, state 8192 keys, 256 branches x 16
gdn        config 2: Hk 16 / Hv 32, T = 2048 prefill through the one-call GDN
           layer (conv+gates inside the scan, norm); config 2's gates:
           A_neg_exp = -1, dt_bias = 0, so g = -softplus(a), a ~ N(0, 1)
gdn_branch config 2 branches: 64 branches x 16 tokens continuing one state
           (S and the conv tail read, nothing written back), packed chunks
gdn_split, gdn_branch_split: the same through conv_prep + scan (two calls)
gemm_<p>    the few-token kernel on projection p (qkv, in, gate_up, down, o) at
           N = 80 with cold weights; blas_<p> the same on hipBLASLt; wide_<p>
           the prefill kernel at the deferred pass's 610 tokens on the
           engine's plan (tile, splits), cold weights
wide_sweep the prefill GEMM: for each 4B projection and token count (argv[2],
           comma-separated, default 610), hipBLASLt and every tile and split
           of the hand-tiled kernel, cold weights; one line per launch kind
copy       a plain device-to-device copy of 256 MiB (scale factor for the
           FETCH_SIZE / WRITE_SIZE counters)
"""
from __future__ import annotations

import sys

# HBM traffic per launch, measured with rocprofv3 --pmc on MI355X (one
# counter per run): FETCH_SIZE and WRITE_SIZE in KiB per dispatch, summed
# over the kernels of the case. A plain 256 MiB device copy reads 131085 KiB
# of FETCH_SIZE and writes 262144 KiB of WRITE_SIZE, so FETCH_SIZE is scaled
# by 2 and WRITE_SIZE by 1. MEASURED_AT names the commit each case's counters
# were taken at; re-measure after changing one of its kernels.
COPY_SCALE = {"FETCH_SIZE": 2.0, "WRITE_SIZE": 1.0}
MEASURED_AT = {"attention": "06180c0", "gdn": "06180c0", "gdn_branch": "06180c0"}
MEASURED_KIB = {
    "attention": {"FETCH_SIZE": 115108.0, "WRITE_SIZE": 32807.7},
    # chunk_a<1>, chunk_b (with the conv-tail workgroups), norm_gate
    "gdn": {"FETCH_SIZE": 18172.3 + 57601.8 + 24595.2,
            "WRITE_SIZE": 90400.3 + 34912.0 + 16384.0},
    # chunk_a<2>, short_b
    "gdn_branch": {"FETCH_SIZE": 9839.4 + 30838.9, "WRITE_SIZE": 45189.4 + 8192.0},
}


def measured_traffic(case):
    """HBM bytes per launch of a case from the counter figures above (None
    while not measured for the kernels of this tree)."""
    kib = MEASURED_KIB.get(case)
    if kib is None:
        return None
    return int(sum(kib[c] * COPY_SCALE[c] for c in kib) * 1024)


def attention_case():
    import torch
    from . import ops
    ops.load()
    D, Hq, Hkv, P, B, L = 256, 16, 4, 8192, 256, 16
    N = B * L
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(1)
    ps, os_ = ops.kv_stride(P), ops.kv_stride(N)
    t = dict(
        pk=torch.randn(Hkv, ps, D, device=dev, generator=g).to(torch.bfloat16),
        pvt=torch.randn(Hkv, D, ps, device=dev, generator=g).to(torch.bfloat16),
        ok=torch.randn(Hkv, os_, D, device=dev, generator=g).to(torch.bfloat16),
        ovt=torch.randn(Hkv, D, os_, device=dev, generator=g).to(torch.bfloat16),
        q=(torch.randn(N, Hq, D, device=dev, generator=g) * (1.4426950408889634 / 16)).to(
            torch.bfloat16),
        gate=torch.randn(N, Hq, D, device=dev, generator=g).to(torch.bfloat16),
        own_base=torch.arange(N, device=dev, dtype=torch.int32) // L * L,
        out=torch.empty(N, Hq * D, dtype=torch.bfloat16, device=dev))

    def launch():
        ops.attention(t["q"], t["gate"], Hq * D, D, t["pk"], t["pvt"], P, ps, t["ok"], t["ovt"],
                      os_, t["own_base"], Hq, Hkv, t["out"])

    flop = 4.0 * D * Hq * (N * P + B * L * (L + 1) / 2)  # QK^T + PV, exact causal count
    return launch, {"flop": flop}


def gdn_case(fused=True):
    import torch
    from . import ops
    ops.load()
    Hk, Hv, T = 16, 32, 2048
    C = (2 * Hk + Hv) * 128
    Wd = C + Hv * 128 + 2 * Hv
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(2)
    proj = torch.randn(T, Wd, device=dev, generator=g).to(torch.bfloat16)
    conv_w = torch.randn(C, 4, device=dev, generator=g) * 0.5
    A_neg = -torch.ones(Hv, device=dev)  # config 2: g = -softplus(a)
    dt_bias = torch.zeros(Hv, device=dev)
    norm_w = torch.ones(128, device=dev)
    own_base = torch.zeros(T, dtype=torch.int32, device=dev)
    q = torch.empty(T, Hk, 128, dtype=torch.float32, device=dev)
    k = torch.empty_like(q)
    v = torch.empty(T, Hv, 128, dtype=torch.float32, device=dev)
    gg = torch.empty(T, Hv, device=dev)
    beta = torch.empty_like(gg)
    conv_out = torch.empty(C, 3, device=dev)
    S_out = torch.empty(Hv, 128, 128, device=dev)
    y = torch.empty(T, Hv * 128, dtype=torch.bfloat16, device=dev)
    tok0, clen, seg0, segn = (torch.as_tensor(a).to(dev) for a in ops.chunk_table([T]))
    scratch = torch.empty(ops.gdn_scratch_bytes(len(tok0), Hv, T), dtype=torch.uint8, device=dev)

    def launch():
        if fused:
            ops.gdn_layer(proj, conv_w, None, conv_out, T, own_base, A_neg, dt_bias, tok0, clen,
                          seg0, segn, None, S_out, norm_w, 1e-6, Hk, Hv, y, scratch)
            return
        ops.gdn_conv_prep(proj, conv_w, None, conv_out, T, own_base, A_neg, dt_bias, Hk, Hv, q, k,
                          v, gg, beta)
        ops.gdn_scan(q, k, v, gg, beta, tok0, clen, seg0, segn, None, S_out, proj[:, C:],
                     proj.stride(0), norm_w, 1e-6, Hk, Hv, y, scratch)

    # compulsory bytes: pre-conv qkv, a/b, conv w, z, bf16 out, S_out, conv tail
    nbytes = T * C * 2 + T * 2 * Hv * 2 + C * 4 * 4 + T * Hv * 128 * 2 + T * Hv * 128 * 2 \
        + Hv * 128 * 128 * 4 + C * 3 * 4
    return launch, {"bytes": nbytes}


def gdn_branch_case(B=64, L=16, fused=True):
    import torch
    from . import ops
    ops.load()
    Hk, Hv = 16, 32
    N = B * L
    C = (2 * Hk + Hv) * 128
    Wd = C + Hv * 128 + 2 * Hv
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(3)
    proj = torch.randn(N, Wd, device=dev, generator=g).to(torch.bfloat16)
    conv_w = torch.randn(C, 4, device=dev, generator=g) * 0.5
    conv_in = torch.randn(C, 3, device=dev, generator=g)
    A_neg = -torch.ones(Hv, device=dev)  # config 2: g = -softplus(a)
    dt_bias = torch.zeros(Hv, device=dev)
    norm_w = torch.ones(128, device=dev)
    S_in = torch.randn(Hv, 128, 128, device=dev, generator=g) * 0.1
    own_base = (torch.arange(N, device=dev, dtype=torch.int32) // L) * L
    q = torch.empty(N, Hk, 128, dtype=torch.float32, device=dev)
    k = torch.empty_like(q)
    v = torch.empty(N, Hv, 128, dtype=torch.float32, device=dev)
    gg = torch.empty(N, Hv, device=dev)
    beta = torch.empty_like(gg)
    y = torch.empty(N, Hv * 128, dtype=torch.bfloat16, device=dev)
    # the engine's eval table: whole branches packed into 64-token chunks
    tok0, clen, starts = (torch.as_tensor(a).to(dev) for a in ops.packed_chunk_table([L] * B))
    scratch = torch.empty(ops.gdn_scratch_bytes(len(tok0), Hv, N), dtype=torch.uint8, device=dev)

    def launch():
        if fused:
            ops.gdn_layer(proj, conv_w, conv_in, None, N, own_base, A_neg, dt_bias, tok0, clen,
                          None, None, S_in, None, norm_w, 1e-6, Hk, Hv, y, scratch,
                          max_seg_chunks=1, chunk_starts=starts)
            return
        ops.gdn_conv_prep(proj, conv_w, conv_in, None, N, own_base, A_neg, dt_bias, Hk, Hv, q, k,
                          v, gg, beta)
        ops.gdn_scan(q, k, v, gg, beta, tok0, clen, None, None, S_in, None, proj[:, C:],
                     proj.stride(0), norm_w, 1e-6, Hk, Hv, y, scratch, max_seg_chunks=1,
                     chunk_starts=starts)

    # compulsory bytes: pre-conv qkv, a/b, conv w, conv tail, S (once), z, bf16 out
    nbytes = N * C * 2 + N * 2 * Hv * 2 + C * 4 * 4 + C * 3 * 4 + Hv * 128 * 128 * 4 \
        + N * Hv * 128 * 2 + N * Hv * 128 * 2
    return launch, {"bytes": nbytes}


# The eval's projections at 4B shape: (rows M, inner K, gated gate|up pair)
GEMM_SHAPES = {"qkv": (10240, 2560, False), "in": (12352, 2560, False),
               "gate_up": (18432, 2560, True), "down": (2560, 9216, False),
               "o": (2560, 4096, False)}


def gemm_case(name, small=True, N=80):
    """One projection of an 80-token eval with cold weights: every launch uses
    the next of enough weight copies (> 1.2 GB in all) that none is still in
    the 256 MB MALL, as in a request, where the other 31 layers evict a
    layer's weights. small=True runs the few-token kernel on pre-tiled
    weights (split-K partials where the engine uses them, the fused
    silu(gate)*up for gate_up); small=False the hipBLASLt GEMM."""
    import torch
    from . import ops
    ops.load()
    M, K, gated = GEMM_SHAPES[name]
    dev = "cuda"
    ncopy = max(2, int(1.2e9 // (M * K * 2)))
    g = torch.Generator(device=dev).manual_seed(5)
    X = torch.randn(N, K, device=dev, generator=g).to(torch.bfloat16)
    Ws = [(torch.randn(M, K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
          for _ in range(ncopy)]
    Y = torch.empty(N, M, dtype=torch.bfloat16, device=dev)
    if small:
        Ws = [ops.gemm_small_tile(W) for W in Ws]
        sp = ops.gemm_small_splits(M, K)
        P = torch.empty(max(sp, 1), N, M, dtype=torch.float32, device=dev)
        A = torch.empty(N, M // 2, dtype=torch.bfloat16, device=dev)
        if gated:
            run = lambda W: ops.gemm_small(X, W, Y=A, gated=True)
        elif M <= 4096 and sp > 1:  # residual projections: partials to the add
            run = lambda W: ops.gemm_small(X, W, P=P, splits=sp)
        else:
            run = lambda W: ops.gemm_small(X, W, Y=Y)
    else:
        run = lambda W: ops.gemm(X, W, Y)
    state = {"i": 0}

    def launch():
        run(Ws[state["i"] % ncopy])
        state["i"] += 1

    return launch, {"bytes": M * K * 2, "copies": ncopy}


def wide_case(name, N=610):
    """One projection of the deferred config-4 pass (610 tokens) on the
    prefill kernel with the engine's plan (tile and, for the residual
    projections, split count), cold weights (> 800 MB of copies, launched
    in turn)."""
    import torch
    from . import ops
    ops.load()
    M, K, gated = GEMM_SHAPES[name]
    residual = M <= 4096
    rg, ng, sp = ops.gemm_wide_plan(N, M, K, gated, 8 if residual else 1)
    dev = "cuda"
    ncopy = max(2, int(800e6 // (M * K * 2)) + 1)
    g = torch.Generator(device=dev).manual_seed(7)
    X = torch.randn(N, K, device=dev, generator=g).to(torch.bfloat16)
    Wt = [ops.gemm_small_tile((torch.randn(M, K, device=dev, generator=g) * 0.02)
                              .to(torch.bfloat16)) for _ in range(ncopy)]
    Y = torch.empty(N, M // 2 if gated else M, dtype=torch.bfloat16, device=dev)
    P = torch.empty(sp, N, M, dtype=torch.float32, device=dev)
    if sp > 1:
        run = lambda W: ops.gemm_wide(X, W, P=P, splits=sp, rg=rg, ng=ng)
    else:
        run = lambda W: ops.gemm_wide(X, W, Y=Y, gated=gated, rg=rg, ng=ng)
    state = {"i": 0}

    def launch():
        run(Wt[state["i"] % ncopy])
        state["i"] += 1

    return launch, {"N": N, "plan": (rg, ng, sp), "copies": ncopy}


def copy_case(nbytes=256 << 20):
    import torch
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)

    def launch():
        b.copy_(a)

    return launch, {"bytes": nbytes}


def time_launches(launch, iters=20, warmup=3):
    """Average microseconds per launch, HIP events on torch's current stream
    (the stream the operator ABI launches on)."""
    import torch
    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(iters):
        launch()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters * 1e3


WIDE_TILES = [(2, 8), (2, 12), (3, 8), (3, 12), (4, 6), (4, 8), (4, 10), (4, 12), (6, 4),
              (6, 6), (6, 8), (8, 4), (8, 6)]


def wide_sweep(token_counts, reps=15):
    """Prefill GEMM timings behind the engine's routing and the plan model's
    fit: `ROW <projection> <N> blas 0 0 0 <us>` for hipBLASLt on the plain
    rows and `ROW <projection> <N> wide <RG> <NG> <splits> <us>` for each
    tile and split of the hand-tiled kernel (fp32 partials where splits >
    1, the fused silu(gate) * up for gate_up), cold weights (> 800 MB of
    copies, launched in turn)."""
    import torch
    from . import ops
    ops.load()
    shapes = [("qkv", 10240, 2560, False, 1), ("in", 12352, 2560, False, 1),
              ("gate_up", 18432, 2560, True, 1), ("o", 2560, 4096, False, 8),
              ("down", 2560, 9216, False, 8)]
    for N in token_counts:
        for name, M, K, gated, max_splits in shapes:
            g = torch.Generator(device="cuda").manual_seed(7)
            X = torch.randn(N, K, device="cuda", generator=g).to(torch.bfloat16)
            ncopy = max(2, int(800e6 // (M * K * 2)) + 1)
            W = [(torch.randn(M, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
                 for _ in range(ncopy)]
            Wt = [ops.gemm_small_tile(w) for w in W]
            Y = torch.empty(N, M, dtype=torch.bfloat16, device="cuda")
            act = torch.empty(N, M // 2, dtype=torch.bfloat16, device="cuda")
            P = torch.empty(min(max_splits, max(1, int(2e9 // (N * M * 4)))), N, M,
                            dtype=torch.float32, device="cuda")
            it = [0]

            def timed(fn):
                def launch():
                    fn(it[0] % ncopy)
                    it[0] += 1
                return time_launches(launch, reps, 3)

            print(f"ROW {name} {N} blas 0 0 0 {timed(lambda i: ops.gemm(X, W[i], Y)):.2f}",
                  flush=True)
            for rg, ng in WIDE_TILES:
                if gated and rg % 2:
                    continue
                for sp in range(1, max_splits + 1):
                    if (K // 128) % sp or sp > P.shape[0]:
                        continue
                    if sp == 1:
                        fn = (lambda i, rg=rg, ng=ng: ops.gemm_wide(
                            X, Wt[i], Y=act if gated else Y, gated=gated, rg=rg, ng=ng))
                    else:
                        fn = (lambda i, rg=rg, ng=ng, sp=sp: ops.gemm_wide(
                            X, Wt[i], P=P, splits=sp, rg=rg, ng=ng))
                    print(f"ROW {name} {N} wide {rg} {ng} {sp} {timed(fn):.2f}", flush=True)
            del W, Wt, P
            torch.cuda.empty_cache()


CASES = {"attention": attention_case, "gdn": gdn_case, "gdn_branch": gdn_branch_case,
         "gdn_split": lambda: gdn_case(fused=False),
         "gdn_branch_split": lambda: gdn_branch_case(fused=False), "copy": copy_case}
for _g in GEMM_SHAPES:
    CASES["gemm_" + _g] = lambda _g=_g: gemm_case(_g, small=True)
    CASES["blas_" + _g] = lambda _g=_g: gemm_case(_g, small=False)
    CASES["wide_" + _g] = lambda _g=_g: wide_case(_g)

if __name__ == "__main__":
    name = sys.argv[1]
    if name == "wide_sweep":
        wide_sweep([int(n) for n in (sys.argv[2] if len(sys.argv) > 2 else "610").split(",")])
        sys.exit(0)
    iters = int(sys.argv[2]) if len(sys.argv) > 2 else 20
    warmup = int(sys.argv[3]) if len(sys.argv) > 3 else 3
    launch, info = CASES[name]()
    us = time_launches(launch, iters, warmup)
    tbs = f", {info['bytes'] / us / 1e6:.2f} TB/s" if "bytes" in info else ""
    print(f"{name}: {us:.1f} us per launch{tbs} {info}", flush=True)
