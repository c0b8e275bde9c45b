"""Config 1 on the GPU: the whole gated GQA attention layer through the
operator C ABI, the way the engine runs it -- hipBLASLt q|k|v projection,
attn_prep (q/k norm, RoPE 1e7 on 64 dims, K / V^T cache write), shared-prefix
attention, hipBLASLt o_proj -- for a 512-token state (prefill: P = 0, the
state's own cache) and then 4 branches of 32 tokens over that state.

Config 1's inputs and weights (tests/golden/make_attention_layer.py, seed 0)
are rounded to bf16 for the device. Compared with the oracle layer
(oracle.qwen35.gated_attention_layer) on the same bf16 inputs, once with the
reference engine's bf16 rounding points and once in float64, and with
transformers' float32 outputs of tests/golden/attention_layer_cfg1.npz.
Bar: max relative error <= 2e-2 on the bf16 layer outputs.
"""
import sys
from pathlib import Path

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import qwen35 as orc  # noqa: E402

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_attention_layer as cfg1  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = 2e-2


def rel(a, b):
    b = np.asarray(b, np.float64)
    return float(np.abs(np.asarray(a, np.float64) - b).max() / np.abs(b).max())


def bfr(a):
    return orc.bf16_round(np.asarray(a, np.float32)).astype(np.float64)


def test_config1_attention_layer():
    from cujev import ops
    ops.load()
    H, Hq, Hkv, D, rot = cfg1.H, cfg1.HQ, cfg1.HKV, cfg1.D, cfg1.ROT
    P, B, L = cfg1.P, cfg1.B, cfg1.L
    N = B * L
    xs, xb, w = cfg1.config1_inputs()
    Wqkv = np.concatenate([w["q_proj"], w["k_proj"], w["v_proj"]], 0)
    Wqkv_b, Wo_b, xs_b, xb_b = bfr(Wqkv), bfr(w["o_proj"]), bfr(xs), bfr(xb)
    qn, kn = 1.0 + w["q_norm"].astype(np.float64), 1.0 + w["k_norm"].astype(np.float64)
    own_base = np.repeat(np.arange(B) * L, L).astype(np.int32)

    dev = "cuda"
    tb = lambda a: torch.as_tensor(np.asarray(a, np.float32)).to(dev).to(torch.bfloat16)
    tf = lambda a: torch.as_tensor(np.asarray(a, np.float32)).to(dev)
    ti = lambda a: torch.as_tensor(np.asarray(a, np.int32)).to(dev)
    Wd, Wod = tb(Wqkv_b), tb(Wo_b)
    wq = Wqkv.shape[0]
    ps, bs = ops.kv_stride(P), ops.kv_stride(N)
    rope = ops.rope_table(cfg1.THETA, rot, P + N)
    q_scale = D ** -0.5 * orc.LOG2E
    pk = torch.zeros(Hkv, ps, D, dtype=torch.bfloat16, device=dev)
    pvt = torch.zeros(Hkv, D, ps, dtype=torch.bfloat16, device=dev)
    bk = torch.zeros(Hkv, bs, D, dtype=torch.bfloat16, device=dev)
    bvt = torch.zeros(Hkv, D, bs, dtype=torch.bfloat16, device=dev)

    def layer(x, pos, base, Pkeys, kc, vc, stride):
        n = x.shape[0]
        proj = torch.empty(n, wq, dtype=torch.bfloat16, device=dev)
        ops.gemm(tb(x), Wd, proj)
        q = torch.empty(n, Hq, D, dtype=torch.bfloat16, device=dev)
        ops.attn_prep(proj, tf(qn), tf(kn), ti(pos), Hq, Hkv, rot, rope, cfg1.EPS, q_scale,
                      q, kc, vc, stride)
        att = torch.empty(n, Hq * D, dtype=torch.bfloat16, device=dev)
        wsb = ops.attention_ws_bytes(n, Hq, Hkv, Pkeys)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev) if wsb else None
        ops.attention(q, proj[:, D:], wq, 2 * D, pk, pvt, Pkeys, ps, kc, vc, stride, ti(base),
                      Hq, Hkv, att, ws=ws)
        out = torch.empty(n, H, dtype=torch.bfloat16, device=dev)
        ops.gemm(att, Wod, out)
        return out

    print("config 1: state prefill (P = 0, 512 tokens)", flush=True)
    out_s = layer(xs_b, np.arange(P), np.zeros(P), 0, pk, pvt, ps)
    print("config 1: 4 branches x 32 over the 512-token state", flush=True)
    out_b = layer(xb_b, P + np.arange(N) - own_base, own_base, P, bk, bvt, bs)
    torch.cuda.synchronize()
    got_s, got_b = out_s.float().cpu().numpy(), out_b.float().cpu().numpy()

    eng_s, eng_b = orc.gated_attention_layer(xs_b, xb_b, own_base, Wqkv_b, Wo_b, qn, kn, Hq, Hkv,
                                             rot, cfg1.THETA, cfg1.EPS, D, rnd=bfr)
    f64_s, f64_b = orc.gated_attention_layer(xs_b, xb_b, own_base, Wqkv_b, Wo_b, qn, kn, Hq, Hkv,
                                             rot, cfg1.THETA, cfg1.EPS, D)
    golden = np.load(cfg1.OUT, allow_pickle=False)["branch_out"]
    errs = {"state vs engine-numerics oracle": rel(got_s, eng_s),
            "state vs float64 oracle": rel(got_s, f64_s),
            "branches vs engine-numerics oracle": rel(got_b, eng_b),
            "branches vs float64 oracle": rel(got_b, f64_b),
            "branches vs transformers fp32 (fp32 weights)": rel(got_b, golden)}
    for k, v in errs.items():
        print(f"  {k}: {v:.3e}", flush=True)
    assert all(v <= TOL for v in errs.values()), errs
