"""GPU parity of the prefill GEMM (cujev_op_gemm_wide) through the operator
C ABI: against float32 references of the same bf16 inputs (bar as for the
few-token kernel: the only rounding besides fp32 accumulation order is the
bf16 output, max |gpu - ref| / max |ref| <= 1e-2), and bit for bit against the
few-token kernel where both run (N <= 96): both walk K in the same order with
the same k assignment per MFMA, so their sums are the same.

Replaces the reference's cuBLAS projection GEMM (src/kernels/elementwise.cu:56-75)
and, gated, GEMM + silu_mul (:42-54) at prefill token counts.
"""
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
TOL = 1e-2
TILES = [(2, 8), (2, 12), (3, 8), (3, 12), (4, 6), (4, 8), (4, 10), (4, 12), (6, 4), (6, 6),
         (6, 8), (8, 4), (8, 6)]


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


# prefill shapes of the 4B model at the config-4 state (530 tokens), and
# ragged token / row counts: a last token block of 1..31 rows, M not a
# multiple of the tile, one token, and a strided X
@pytest.mark.parametrize("N,M,K", [(530, 10240, 2560), (530, 12352, 2560), (1, 256, 128),
                                   (17, 640, 384), (200, 2608, 1024), (1100, 1024, 1152)])
def test_gemm_wide_matches_fp32(N, M, K):
    o = ops()
    X = rand_bf16(N, K, seed=1)
    W = rand_bf16(M, K, seed=2, scale=0.02)
    Wt = o.gemm_small_tile(W)
    ref = X.float() @ W.float().t()
    for rg, ng in TILES:
        print(f"gemm_wide N={N} M={M} K={K} rg={rg} ng={ng}", flush=True)
        Y = torch.full((N, M), float("nan"), dtype=torch.bfloat16, device="cuda")
        o.gemm_wide(X, Wt, Y=Y, rg=rg, ng=ng)
        torch.cuda.synchronize()
        e = rel(Y.float(), ref)
        print(f"  rel err {e:.3e}")
        assert torch.isfinite(Y.float()).all() and e <= TOL


def test_gemm_wide_strided_x_and_output():
    o = ops()
    N, M, K = 130, 512, 640
    Xb = rand_bf16(N, K + 256, seed=3)
    X = Xb[:, 128:128 + K]
    W = rand_bf16(M, K, seed=4, scale=0.02)
    Yb = torch.zeros(N, M + 64, dtype=torch.bfloat16, device="cuda")
    Y = Yb[:, :M]
    o.gemm_wide(X, o.gemm_small_tile(W), Y=Y, rg=3, ng=12)
    torch.cuda.synchronize()
    assert rel(Y.float(), X.float() @ W.float().t()) <= TOL
    assert (Yb[:, M:] == 0).all()  # nothing written past the row's M outputs


@pytest.mark.parametrize("N,M,K", [(80, 10240, 2560), (33, 4160, 2560), (96, 256, 1024)])
def test_gemm_wide_equals_few_token_kernel(N, M, K):
    o = ops()
    X = rand_bf16(N, K, seed=5)
    W = rand_bf16(M, K, seed=6, scale=0.02)
    Wt = o.gemm_small_tile(W)
    ys = torch.empty(N, M, dtype=torch.bfloat16, device="cuda")
    o.gemm_small(X, Wt, Y=ys)
    for rg, ng in TILES:
        yw = torch.empty_like(ys)
        o.gemm_wide(X, Wt, Y=yw, rg=rg, ng=ng)
        torch.cuda.synchronize()
        assert torch.equal(yw, ys), (rg, ng)


@pytest.mark.parametrize("N,I,H", [(530, 9216, 2560), (80, 9216, 2560), (45, 160, 256)])
def test_gemm_wide_gated_is_silu_mul(N, I, H):
    o = ops()
    X = rand_bf16(N, H, seed=7)
    W = rand_bf16(2 * I, H, seed=8, scale=0.05)
    Wt = o.gemm_small_tile(W)
    gu = (X.float() @ W.float().t()).to(torch.bfloat16).float()  # the GEMM's bf16 output
    ref = torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]
    small = None
    if N <= 96 and I % 32 == 0:
        small = torch.empty(N, I, dtype=torch.bfloat16, device="cuda")
        o.gemm_small(X, Wt, Y=small, gated=True)
    for rg, ng in [(2, 8), (2, 12), (4, 6), (4, 8), (4, 10), (4, 12), (6, 4), (6, 6), (6, 8),
                   (8, 4), (8, 6)]:
        print(f"gated N={N} I={I} H={H} rg={rg} ng={ng}", flush=True)
        act = torch.full((N, I), float("nan"), dtype=torch.bfloat16, device="cuda")
        o.gemm_wide(X, Wt, Y=act, gated=True, rg=rg, ng=ng)
        torch.cuda.synchronize()
        e = rel(act.float(), ref)
        print(f"  rel err {e:.3e}")
        assert torch.isfinite(act.float()).all() and e <= TOL
        if small is not None:
            assert torch.equal(act, small)


@pytest.mark.parametrize("N,H,K,splits", [(530, 2560, 9216, 4), (530, 2560, 4096, 8),
                                          (77, 1024, 1024, 2), (300, 512, 768, 3)])
def test_gemm_wide_split_partials_feed_add_rmsnorm(N, H, K, splits):
    o = ops()
    X = rand_bf16(N, K, seed=9)
    W = rand_bf16(H, K, seed=10, scale=0.02)
    w = (1.0 + 0.1 * torch.randn(H, device="cuda")).float()
    g = torch.Generator(device="cuda").manual_seed(11)
    x0 = torch.randn(N, H, device="cuda", generator=g)
    Wt = o.gemm_small_tile(W)
    y_ref = (X.float() @ W.float().t()).to(torch.bfloat16).float()
    v = x0 + y_ref
    ref = v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + 1e-6) * w
    outs = []
    for rg, ng in [(2, 8), (4, 12), (8, 6)]:
        print(f"split N={N} H={H} K={K} splits={splits} rg={rg} ng={ng}", flush=True)
        P = torch.full((splits, N, H), float("nan"), dtype=torch.float32, device="cuda")
        out = torch.empty(N, H, dtype=torch.bfloat16, device="cuda")
        x = x0.clone()
        o.gemm_wide(X, Wt, P=P, splits=splits, rg=rg, ng=ng)
        o.add_rmsnorm(x, w, out, 1e-6, yp=P, splits=splits)
        torch.cuda.synchronize()
        assert rel(x, v) <= TOL
        e = rel(out.float(), ref)
        print(f"  rel err {e:.3e}")
        assert e <= TOL
        outs.append(out)
    # the partials of one split do not depend on the tile: same sums
    assert torch.equal(outs[0], outs[1])

