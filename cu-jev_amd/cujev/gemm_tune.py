"""Builds the tuned hipBLASLt algorithm table the engine reads at model open
(gemm_table_gfx950_hipblaslt<version>.txt next to libcujev.so, or the file
CUJEV_GEMM_TABLE names): for every projection GEMM shape of a model and every
token count, the fastest hipBLASLt solution found by timing all supported
ones.

    python -m cujev.gemm_tune --preset 4b --out-dir cu-jev_amd/cujev

This process imports torch, so it tunes the hipBLASLt torch ships with (the
one the engine uses inside torch processes, e.g. the tests). The torch-free
tuner cu-jev_amd/cujev/cujev_gemm_tune does the same for the system
hipBLASLt (the one the reference's ctypes layer or a C caller loads).
Solution indices are only valid for the version in the file name and header.
"""
from __future__ import annotations

import argparse
import os
import sys
import time

from . import ops, synthetic


def projection_shapes(cfg):
    """Unique (M, K) of Y[N,M] = X[N,K] W[M,K]^T over the layer types."""
    H, I = cfg["hidden_size"], cfg["intermediate_size"]
    Hq, Hkv, D = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    Hk, Hv = cfg["linear_num_key_heads"], cfg["linear_num_value_heads"]
    dk, dv = cfg["linear_key_head_dim"], cfg["linear_value_head_dim"]
    C = 2 * Hk * dk + Hv * dv
    shapes = [(Hq * 2 * D + 2 * Hkv * D, H),   # fused q|gate, k, v
              (H, Hq * D),                     # o_proj
              (C + Hv * dv + 2 * Hv, H),       # fused GDN in-projection
              (H, Hv * dv),                    # GDN out_proj
              (2 * I, H),                      # fused gate|up
              (H, I)]                          # down
    return list(dict.fromkeys(shapes))


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--preset", default="4b", choices=sorted(synthetic.PRESETS))
    ap.add_argument("--tokens", default="16,32,64,80,128,256,512,530,1024")
    ap.add_argument("--out-dir", required=True)
    a = ap.parse_args(argv)
    import torch
    cfg = synthetic.make_config(**synthetic.PRESETS[a.preset])
    tokens = [int(t) for t in a.tokens.split(",")]
    ver = ops.blaslt_version()
    lines = [f"# hipblaslt {ver}",
             f"# {a.preset} projection GEMMs, tokens {a.tokens}; columns: N M K f32out index"]
    g = torch.Generator(device="cuda").manual_seed(0)
    for M, K in projection_shapes(cfg):
        W = (torch.randn(M, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        for N in tokens:
            X = torch.randn(N, K, device="cuda", generator=g).to(torch.bfloat16)
            Y = torch.empty(N, M, device="cuda", dtype=torch.bfloat16)
            t0 = time.time()
            idx, best, heur = ops.gemm_tune(X, W, Y)
            lines.append(f"{N} {M} {K} 0 {idx}")
            print(f"N={N:5d} M={M:6d} K={K:5d}: heuristic {heur:7.1f} us -> {best:7.1f} us "
                  f"(x{heur / best:.2f}, solution {idx}, {time.time() - t0:.1f} s)", flush=True)
    out = os.path.join(a.out_dir, f"gemm_table_gfx950_hipblaslt{ver}.txt")
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(f"wrote {out}")


if __name__ == "__main__":
    sys.exit(main())
