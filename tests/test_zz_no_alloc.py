"""cujev_op_attention_noalloc (the operator ABI's entry point that allocates
nothing: key-split partials in the library's static per-GPU scratch) against
cujev_op_attention_ws with a caller-allocated workspace. Both run the same
kernels with the same split count, so the outputs must be bit-identical;
two calls in a row, the second with a smaller input (the scratch keeps the
first call's contents), and a one-pass shape (no partials at all).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
D = 256


def case(seed, N, P, Hq, Hkv, lens):
    from cujev import ops
    g = torch.Generator(device="cuda").manual_seed(seed)
    ps, os_ = ops.kv_stride(P), ops.kv_stride(N)
    rnd = lambda *s: torch.randn(*s, device="cuda", generator=g).to(torch.bfloat16)
    t = dict(q=(torch.randn(N, Hq, D, device="cuda", generator=g) * 0.09).to(torch.bfloat16),
             gate=rnd(N, Hq, D), pk=rnd(Hkv, ps, D), pvt=rnd(Hkv, D, ps), ok=rnd(Hkv, os_, D),
             ovt=rnd(Hkv, D, os_))
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    t["own"] = torch.as_tensor(np.repeat(starts, lens).astype(np.int32)).cuda()
    return t, ps, os_


def run(t, ps, os_, N, P, Hq, Hkv, noalloc):
    from cujev import ops
    out = torch.empty(N, Hq * D, dtype=torch.bfloat16, device="cuda")
    args = (t["q"], t["gate"], Hq * D, D, t["pk"], t["pvt"], P, ps, t["ok"], t["ovt"], os_,
            t["own"], Hq, Hkv, out)
    if noalloc:
        ops.attention_noalloc(*args)
    else:
        wsb = ops.attention_ws_bytes(N, Hq, Hkv, P)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda") if wsb else None
        ops.attention(*args, ws=ws)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("shapes", [
    # (N, P, Hq, Hkv, branch lengths): the engine's 4B eval, then a smaller one
    [(80, 530, 16, 4, [20] * 4), (20, 100, 16, 4, [5, 15])],
    # the largest partials the kernel can ask for (16 splits x 128 tokens x 16
    # heads), then a shape that runs in one pass (no partials)
    [(128, 4096, 16, 4, [32] * 4), (512, 64, 8, 2, [256, 256])],
])
def test_noalloc_matches_workspace_entry(shapes):
    from cujev import ops
    ops.load()
    for i, (N, P, Hq, Hkv, lens) in enumerate(shapes):
        print(f"noalloc call {i}: N={N} P={P} Hq={Hq} Hkv={Hkv} "
              f"partials {ops.attention_ws_bytes(N, Hq, Hkv, P)} B", flush=True)
        assert ops.attention_ws_bytes(N, Hq, Hkv, P) <= 33816576
        t, ps, os_ = case(100 + i, N, P, Hq, Hkv, lens)
        a = run(t, ps, os_, N, P, Hq, Hkv, noalloc=True)
        b = run(t, ps, os_, N, P, Hq, Hkv, noalloc=False)
        assert torch.isfinite(a.float()).all()
        assert torch.equal(a, b), f"call {i}: noalloc differs from the workspace entry point"
