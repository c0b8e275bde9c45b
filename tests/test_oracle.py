"""Pins of the CPU oracle (oracle/qwen35.py) on the CPU: closed forms,
brute-force special cases and invariants chosen so that a dropped term, a
wrong sign or index or a transposed operand fails at least one of them.
The golden vectors written by transformers are checked in test_golden.py."""
import numpy as np
import pytest

from oracle import qwen35 as orc


def test_bf16_round_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-8, 8, 10000),
                        np.array([1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -0.0, 65504.0, 3.0e38],
                                 dtype=np.float32)])
    ref = torch.tensor(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(orc.bf16_round(x), ref)
    # ties go to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7
    assert orc.bf16_round(np.float32(1 + 2 ** -8)) == 1.0
    assert orc.bf16_round(np.float32(1 + 3 * 2 ** -8)) == np.float32(1 + 2 ** -6)


def test_rmsnorm_closed_form():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 256)) * 3
    y = orc.rmsnorm(x, np.ones(256), 0.0)
    np.testing.assert_allclose(np.sqrt((y * y).mean(-1)), 1.0, rtol=1e-12)
    w = rng.standard_normal(256)
    np.testing.assert_allclose(orc.rmsnorm(x, w, 0.0), y * w, rtol=1e-12)


def test_rope_identity_norm_and_complex_form():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 2, 256))
    inv = orc.rope_inv_freq(1e7, 64)
    np.testing.assert_allclose(orc.apply_rope(x, np.zeros(3), inv, 64), x)
    pos = np.array([1.0, 17.0, 8191.0])
    y = orc.apply_rope(x, pos, inv, 64)
    np.testing.assert_allclose(y[..., 64:], x[..., 64:])  # pass-through dims
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1))
    # rotate_half pairs dim i with i + 32: (x_i + i x_{i+32}) * e^{i pos f_i}
    z = (x[..., :32] + 1j * x[..., 32:64]) * np.exp(1j * pos[:, None, None] * inv[None, None, :])
    np.testing.assert_allclose(y[..., :32], z.real, atol=1e-12)
    np.testing.assert_allclose(y[..., 32:64], z.imag, atol=1e-12)
    # inv_freq[1] = theta^(-2/64)
    assert abs(inv[1] - 1e7 ** (-2 / 64)) < 1e-15


def _attn_inputs(seed, N, P, Hq=8, Hkv=2, D=256):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((N, Hq, D)), rng.standard_normal((N, Hq, D)),
            rng.standard_normal((P, Hkv, D)), rng.standard_normal((P, Hkv, D)),
            rng.standard_normal((N, Hkv, D)), rng.standard_normal((N, Hkv, D)))


def test_shared_prefix_equals_causal_over_concatenation():
    q, g, ks, vs, ko, vo = _attn_inputs(3, 12, 20)
    segs = [5, 7]
    own_base = np.array([0] * 5 + [5] * 7)
    out = orc.shared_prefix_attention(q, g, ks, vs, ko, vo, own_base)
    start = 0
    for L in segs:
        sl = slice(start, start + L)
        # full causal sequence [state ++ branch]; the state rows' queries are dummies
        rng = np.random.default_rng(9)
        qf = np.concatenate([rng.standard_normal((20, 8, 256)), q[sl]])
        gf = np.concatenate([rng.standard_normal((20, 8, 256)), g[sl]])
        kf = np.concatenate([ks, ko[sl]])
        vf = np.concatenate([vs, vo[sl]])
        ref = orc.causal_gqa_attention(qf, gf, kf, vf)[20:]
        np.testing.assert_allclose(out[sl], ref, rtol=1e-10, atol=1e-12)
        start += L


def test_shared_prefix_equals_causal_with_engine_rounding():
    """The engine track's tiles follow the concatenated key index [state ++
    own], so the shared-prefix form equals causal attention over the
    concatenation with the rounding points included (state of 70 keys: the
    branch rows' tiles straddle the state/own boundary)."""
    rng = np.random.default_rng(11)
    P, L = 70, 9
    q, g = rng.standard_normal((L, 8, 256)), rng.standard_normal((L, 8, 256))
    ks, vs = rng.standard_normal((P, 2, 256)), rng.standard_normal((P, 2, 256))
    ko, vo = rng.standard_normal((L, 2, 256)), rng.standard_normal((L, 2, 256))
    kw = dict(scale=0.05, bf16_p=True)
    out = orc.shared_prefix_attention(q, g, ks, vs, ko, vo, np.zeros(L, int), **kw)
    qf = np.concatenate([rng.standard_normal((P, 8, 256)), q])
    gf = np.concatenate([rng.standard_normal((P, 8, 256)), g])
    ref = orc.causal_gqa_attention(qf, gf, np.concatenate([ks, ko]), np.concatenate([vs, vo]),
                                   **kw)[P:]
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-14)


def _final_max_pv(s, v):
    """bf16(p) against the row's final max (the rounding the tiled form must
    reduce to when no later tile raises the max)."""
    p = np.exp(s - s.max())
    pb = orc.bf16_round(p.astype(np.float32)).astype(np.float64)
    return pb @ v / p.sum()


def test_tiled_bf16_softmax_rounding_points():
    """Pins oracle.qwen35._tiled_pv, the reference kernel's online softmax
    with P rounded to bf16 per 64-key tile against the running max."""
    rng = np.random.default_rng(12)
    L, D = 200, 16
    v = rng.standard_normal((L, D))
    ln2 = np.log(2.0)
    # all scores equal: p = 1 exactly in every tile, o = mean(v)
    np.testing.assert_allclose(orc._tiled_pv(np.zeros(L), v), v.mean(0), rtol=1e-13)
    # one tile: the final max is the running max
    s = rng.standard_normal(50) * 2
    np.testing.assert_allclose(orc._tiled_pv(s, v[:50]), _final_max_pv(s, v[:50]), rtol=1e-13)
    # the max in the first tile, at its last key (63): later tiles never move
    # it, so every p is rounded against the final max
    s = rng.uniform(-4, 0, L) * ln2
    s[63] = 3.0 * ln2
    np.testing.assert_allclose(orc._tiled_pv(s, v), _final_max_pv(s, v), rtol=1e-13)
    # the max at key 64 (the second tile's first): tile 0 was rounded against
    # a lower running max, which is not a whole number of octaves below, so
    # the bf16 roundings differ
    s2 = s.copy()
    s2[63], s2[64] = s[64], 3.37 * ln2
    a, b = orc._tiled_pv(s2, v), _final_max_pv(s2, v)
    assert np.abs(a - b).max() > 1e-6 * np.abs(b).max()
    np.testing.assert_allclose(a, b, rtol=2e-2, atol=2e-2)
    # running maxima a whole number of octaves apart (0, then 3 in tile 1):
    # 2^(s-0) and 2^(s-3) differ by 2^3, which bf16 rounding commutes with
    s3 = rng.uniform(-6, -1, L) * ln2
    s3[5], s3[100] = 0.0, 3.0 * ln2
    np.testing.assert_allclose(orc._tiled_pv(s3, v), _final_max_pv(s3, v), rtol=1e-12)
    # masked keys (-inf) contribute nothing, wherever they sit in a tile
    s4 = s.copy()
    s4[[0, 70, 150]] = -np.inf
    keep = np.isfinite(s4)
    np.testing.assert_allclose(orc._tiled_pv(s4, v), orc._tiled_pv(s4, np.where(keep[:, None], v, 7.0)),
                               rtol=0, atol=0)


def test_attention_single_key_and_gqa_mapping():
    q, g, _, _, ko, vo = _attn_inputs(4, 1, 0)
    out = orc.shared_prefix_attention(q, g, np.zeros((0, 2, 256)), np.zeros((0, 2, 256)), ko, vo,
                                      np.zeros(1, int))
    # one visible key: softmax = 1, q-head h reads kv-head h // 4
    for h in range(8):
        np.testing.assert_allclose(out[0, h], orc.sigmoid(g[0, h]) * vo[0, h // 4])


def test_attention_siblings_do_not_leak():
    q, g, ks, vs, ko, vo = _attn_inputs(5, 10, 8)
    own_base = np.array([0] * 4 + [4] * 6)
    a = orc.shared_prefix_attention(q, g, ks, vs, ko, vo, own_base)
    ko2, vo2 = ko.copy(), vo.copy()
    ko2[4:] *= -3.0
    vo2[4:] += 5.0
    b = orc.shared_prefix_attention(q, g, ks, vs, ko2, vo2, own_base)
    np.testing.assert_array_equal(a[:4], b[:4])


def test_conv_with_tail_equals_concatenation():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((20, 16))
    w = rng.standard_normal((16, 4))
    full = orc.gdn_conv(x, w)
    tail = orc.gdn_conv_tail(x[:9])
    np.testing.assert_allclose(orc.gdn_conv(x[9:], w, tail), full[9:], rtol=1e-12)
    np.testing.assert_array_equal(tail, x[6:9].T)
    # the first output only sees w[:, 3] * x[0]
    np.testing.assert_allclose(full[0], orc.silu(w[:, 3] * x[0]))
    # short segment: tail of a 2-token segment after a tail keeps the older input
    t2 = orc.gdn_conv_tail(x[9:11], tail)
    np.testing.assert_array_equal(t2, np.stack([x[8], x[9], x[10]], 1))


def test_prep_norms_and_gates():
    rng = np.random.default_rng(7)
    Hk, Hv = 2, 4
    xc = rng.standard_normal((3, (2 * Hk + Hv) * 128))
    b, a = rng.standard_normal((3, Hv)), rng.standard_normal((3, Hv))
    A_log, dt = rng.standard_normal(Hv), rng.standard_normal(Hv)
    q, k, v, g, beta = orc.gdn_prep(xc, b, a, A_log, dt, Hk, Hv)
    np.testing.assert_allclose(np.linalg.norm(k, axis=-1), 1.0, rtol=1e-5)
    np.testing.assert_allclose(np.linalg.norm(q, axis=-1), 128 ** -0.5, rtol=1e-5)
    # repeat_interleave: v-heads 0,1 read k-head 0, v-heads 2,3 read k-head 1
    np.testing.assert_array_equal(k[:, 0], k[:, 1])
    np.testing.assert_array_equal(k[:, 2], k[:, 3])
    assert not np.allclose(k[:, 1], k[:, 2])
    np.testing.assert_allclose(g, -np.exp(A_log) * np.log1p(np.exp(a + dt)))
    np.testing.assert_allclose(beta, 1 / (1 + np.exp(-b)))


def _scan_inputs(seed, T, H=3, dk=16, dv=8):
    rng = np.random.default_rng(seed)
    q = orc.l2norm(rng.standard_normal((T, H, dk))) / np.sqrt(dk)
    k = orc.l2norm(rng.standard_normal((T, H, dk)))
    v = rng.standard_normal((T, H, dv))
    g = -orc.softplus(rng.standard_normal((T, H)))
    beta = orc.sigmoid(rng.standard_normal((T, H)))
    S0 = rng.standard_normal((H, dk, dv))
    return q, k, v, g, beta, S0


def test_scan_special_cases():
    q, k, v, g, beta, S0 = _scan_inputs(8, 1)
    # one token from S = 0: o = beta (q.k) v
    o, S = orc.gdn_recurrent(q, k, v, g, beta)
    ref = beta[0][:, None] * np.einsum("hk,hk->h", q[0], k[0])[:, None] * v[0]
    np.testing.assert_allclose(o[0], ref, rtol=1e-12)
    # beta = 0: pure decay, o = (e^g S0)^T q
    o, S = orc.gdn_recurrent(q, k, v, g, np.zeros_like(beta), S0)
    Sd = S0 * np.exp(g[0])[:, None, None]
    np.testing.assert_allclose(S, Sd)
    np.testing.assert_allclose(o[0], np.einsum("hkv,hk->hv", Sd, q[0]))
    # g = 0, beta = 1, orthonormal keys: exact overwrite S^T k_t = v_t
    T = 4
    rng = np.random.default_rng(10)
    basis = np.linalg.qr(rng.standard_normal((16, 16)))[0][:, :T].T  # T orthonormal rows
    kk = np.repeat(basis[:, None, :], 3, axis=1)
    vv = rng.standard_normal((T, 3, 8))
    _, S = orc.gdn_recurrent(q[:1].repeat(T, 0), kk, vv, np.zeros((T, 3)), np.ones((T, 3)), S0)
    for t in range(T):
        np.testing.assert_allclose(np.einsum("hkv,hk->hv", S, kk[t]), vv[t], atol=1e-12)


@pytest.mark.parametrize("T", [1, 5, 64, 65, 150])
def test_chunked_equals_recurrent(T):
    q, k, v, g, beta, S0 = _scan_inputs(T, T)
    o1, S1 = orc.gdn_recurrent(q, k, v, g, beta, S0)
    o2, S2 = orc.gdn_chunked(q, k, v, g, beta, S0, chunk=64)
    np.testing.assert_allclose(o2, o1, rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(S2, S1, rtol=1e-9, atol=1e-10)
    o3, _ = orc.gdn_chunked(q, k, v, g, beta, S0, chunk=16)
    np.testing.assert_allclose(o3, o1, rtol=1e-9, atol=1e-10)


def test_scan_continuation_equals_concatenation():
    q, k, v, g, beta, _ = _scan_inputs(11, 40)
    o_full, S_full = orc.gdn_recurrent(q, k, v, g, beta)
    o_a, S_a = orc.gdn_recurrent(q[:25], k[:25], v[:25], g[:25], beta[:25])
    o_b, S_b = orc.gdn_recurrent(q[25:], k[25:], v[25:], g[25:], beta[25:], S_a)
    np.testing.assert_allclose(np.concatenate([o_a, o_b]), o_full, rtol=1e-12)
    np.testing.assert_allclose(S_b, S_full, rtol=1e-12)


def test_gated_rmsnorm_closed_form():
    rng = np.random.default_rng(12)
    o = rng.standard_normal((4, 2, 128))
    z = rng.standard_normal((4, 2, 128))
    w = rng.standard_normal(128)
    y = orc.gated_rmsnorm(o, z, w, 1e-6, bf16_roundtrip=False)
    hn = y / (w * orc.silu(z))
    np.testing.assert_allclose(np.sqrt((hn ** 2).mean(-1)), 1.0, rtol=1e-5)
    yb = orc.gated_rmsnorm(o, z, w, 1e-6, bf16_roundtrip=True)
    assert np.abs(yb - y).max() > 0  # the round trip is really applied
    np.testing.assert_allclose(yb, y, rtol=1e-2)
