"""GPU parity of the few-token weight-streaming GEMM (cujev_op_gemm_small) and
of the residual add + RMSNorm that consumes its split-K partials, through the
operator C ABI, against float32 references of the same bf16 inputs.

The GEMM replaces the reference's cuBLAS call (src/kernels/elementwise.cu:56-75)
at eval shapes; the gated form replaces GEMM + silu_mul (:42-54). Tolerance:
the only rounding besides fp32 accumulation order is the bf16 output, so
max |gpu - ref| / max |ref| <= 1e-2.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
TOL = 1e-2


def ops():
    from cujev import ops as o
    o.load()
    return o


def rel(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def rand_bf16(*shape, seed, scale=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(*shape, device="cuda", generator=g) * scale).to(torch.bfloat16)


# (N, M, K): eval shapes of the 4B model (qkv, in_proj) and edge token counts
@pytest.mark.parametrize("N,M,K", [(80, 10240, 2560), (80, 12352, 2560), (1, 2560, 2560),
                                   (17, 640, 384), (96, 256, 1024), (33, 4160, 2560)])
def test_gemm_small_matches_fp32(N, M, K):
    o = ops()
    print(f"gemm_small N={N} M={M} K={K}", flush=True)
    X = rand_bf16(N, K, seed=1)
    W = rand_bf16(M, K, seed=2, scale=0.02)
    Y = torch.empty(N, M, dtype=torch.bfloat16, device="cuda")
    o.gemm_small(X, o.gemm_small_tile(W), Y=Y)
    torch.cuda.synchronize()
    ref = X.float() @ W.float().t()
    e = rel(Y.float(), ref)
    print(f"rel err {e:.3e}")
    assert e <= TOL


# 9216 and 12288 (the 4B and 9B widths) take the 48 + 48-row workgroups;
# 8224 would need 257 workgroups of 32 + 32 rows but does not divide by 48
@pytest.mark.parametrize("N,I,H", [(80, 9216, 2560), (5, 128, 256), (96, 512, 640),
                                   (80, 12288, 4096), (7, 8224, 256)])
def test_gemm_small_gated_is_silu_mul(N, I, H):
    o = ops()
    print(f"gated N={N} I={I} H={H}", flush=True)
    X = rand_bf16(N, H, seed=3)
    W = rand_bf16(2 * I, H, seed=4, scale=0.05)
    act = torch.empty(N, I, dtype=torch.bfloat16, device="cuda")
    o.gemm_small(X, o.gemm_small_tile(W), Y=act, gated=True)
    torch.cuda.synchronize()
    gu = (X.float() @ W.float().t()).to(torch.bfloat16).float()  # the GEMM's bf16 output
    ref = torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]
    e = rel(act.float(), ref)
    print(f"rel err {e:.3e}")
    assert e <= TOL


@pytest.mark.parametrize("N,H,K", [(80, 2560, 9216), (80, 2560, 4096), (7, 2560, 2560),
                                   (96, 1024, 1024)])
def test_split_partials_feed_add_rmsnorm(N, H, K):
    """splits > 1: fp32 partials summed in split order by add_rmsnorm equal the
    bf16-output path (GEMM into y, then the add) up to the bf16 rounding of y."""
    o = ops()
    sp = o.gemm_small_splits(H, K)
    print(f"split N={N} H={H} K={K} splits={sp}", flush=True)
    assert sp >= 1
    X = rand_bf16(N, K, seed=5)
    W = rand_bf16(H, K, seed=6, scale=0.02)
    w = (1.0 + 0.1 * torch.randn(H, device="cuda")).float()
    g = torch.Generator(device="cuda").manual_seed(7)
    x0 = torch.randn(N, H, device="cuda", generator=g)
    P = torch.empty(max(sp, 1), N, H, dtype=torch.float32, device="cuda")
    out = torch.empty(N, H, dtype=torch.bfloat16, device="cuda")
    x = x0.clone()
    Wt = o.gemm_small_tile(W)
    if sp > 1:
        o.gemm_small(X, Wt, P=P, splits=sp)
        o.add_rmsnorm(x, w, out, 1e-6, yp=P, splits=sp)
    else:
        y = torch.empty(N, H, dtype=torch.bfloat16, device="cuda")
        o.gemm_small(X, Wt, Y=y)
        o.add_rmsnorm(x, w, out, 1e-6, y=y)
    torch.cuda.synchronize()
    y_ref = (X.float() @ W.float().t()).to(torch.bfloat16).float()
    v = x0 + y_ref
    ref = v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + 1e-6) * w
    assert rel(x, v) <= TOL          # residual written back
    e = rel(out.float(), ref)
    print(f"rel err {e:.3e}")
    assert e <= TOL
    if sp > 1:  # deterministic: a second run is bit-identical
        x2, out2 = x0.clone(), torch.empty_like(out)
        o.gemm_small(X, Wt, P=P, splits=sp)
        o.add_rmsnorm(x2, w, out2, 1e-6, yp=P, splits=sp)
        torch.cuda.synchronize()
        assert torch.equal(out, out2) and torch.equal(x, x2)


@pytest.mark.parametrize("N,M,K,splits", [(80, 2560, 4096, 6), (33, 640, 1024, 3),
                                          (80, 2560, 2560, 7)])
def test_split_ranges(N, M, K, splits):
    """Split s holds the product over the 128-wide K chunks [s C / S,
    (s+1) C / S) of the C = K / 128, so ranges may differ by one chunk."""
    o = ops()
    print(f"split ranges N={N} M={M} K={K} splits={splits}", flush=True)
    X = rand_bf16(N, K, seed=12)
    W = rand_bf16(M, K, seed=13, scale=0.02)
    P = torch.full((splits, N, M), float("nan"), dtype=torch.float32, device="cuda")
    o.gemm_small(X, o.gemm_small_tile(W), P=P, splits=splits)
    torch.cuda.synchronize()
    C = K // 128
    worst = 0.0
    for s in range(splits):
        k0, k1 = 128 * (s * C // splits), 128 * ((s + 1) * C // splits)
        ref = X[:, k0:k1].float() @ W[:, k0:k1].float().t()
        worst = max(worst, rel(P[s], ref))
    print(f"worst split rel err {worst:.3e}")
    assert worst <= 1e-4


def tile_reference(W):
    """The tiled layout restated with tensor indexing: blocks of 16 rows x 128
    k in chunk-major order (block c * M/16 + g), element 512 i + 8 l + e =
    W[16 g + l%16][128 c + 64 (i//2) + 16 (l//16) + 8 (i%2) + e]."""
    M, K = W.shape
    t = W.reshape(M // 16, 16, K // 128, 2, 4, 2, 8)   # g, r, c, j, q, hf, e
    t = t.permute(2, 0, 3, 5, 4, 1, 6)                  # c, g, j, hf, q, r, e
    return t.reshape(M, K)


@pytest.mark.parametrize("M,K", [(64, 128), (48, 384), (12352, 2560)])
def test_gemm_small_tile_layout(M, K):
    """The tiling kernel is an exact permutation (bit-exact against the
    indexing restatement) and round-trips every element."""
    o = ops()
    W = rand_bf16(M, K, seed=10)
    Wt = o.gemm_small_tile(W)
    torch.cuda.synchronize()
    assert torch.equal(Wt, tile_reference(W))
    assert torch.equal(torch.sort(Wt.view(-1).view(torch.int16))[0],
                       torch.sort(W.view(-1).view(torch.int16))[0])


def test_gemm_small_rejects_unsupported_shapes():
    o = ops()
    X = rand_bf16(8, 100, seed=8)
    W = rand_bf16(64, 100, seed=9)
    Y = torch.empty(8, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(o.OpsError):
        o.gemm_small(X, W, Y=Y)           # K not a multiple of 128
    X = rand_bf16(97, 128, seed=8)
    W = rand_bf16(64, 128, seed=9)
    Y = torch.empty(97, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(o.OpsError):
        o.gemm_small(X, W, Y=Y)           # more than 96 tokens
    assert o.gemm_small_splits(100, 256) == 0
