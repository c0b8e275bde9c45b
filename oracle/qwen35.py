"""CPU oracle for the branch-forward hot path (TEST INFRASTRUCTURE ONLY).

This module is a numpy restatement of the math the reference engine computes
on its hot path and of the transformers implementation it is tested against.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may use it, and only as the checker. Nothing in the product path imports
it.

Citations:
  REF  = the reference repository (dtunai/cu-Jev), path:line.
  TF   = transformers 5.15.0 ``models/qwen3_5/modeling_qwen3_5.py`` (the
         oracle the reference tests against; pinned at transformers 5.17.0
         in the reference's uv.lock:1933-1934).

Every function is pinned by tests/test_oracle.py against golden vectors
written by transformers (tests/golden/), closed forms or brute-force
invariants; the pin of each function is listed in its docstring.

Numerics: everything is float64 unless a function says it emulates a bf16
rounding point of the engine (``bf16_round``).
"""
from __future__ import annotations

import numpy as np

LOG2E = 1.4426950408889634


# --------------------------------------------------------------------------
# bf16 helpers
# --------------------------------------------------------------------------
def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round to the nearest bfloat16 (ties to even), returned as float32.

    Same rounding as REF src/engine/model.c:36-41 (f32_to_bf16) and the device
    conversion. Pinned by tests/test_oracle.py::test_bf16_round (exact values).
    """
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32)
    # NaN stays NaN
    return np.where(np.isnan(f), f, out)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float -> uint16 bfloat16 bit patterns (round to nearest even)."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------
# norms, activations
# --------------------------------------------------------------------------
def rmsnorm(x, w_eff, eps):
    """x * rsqrt(mean(x^2) + eps) * w_eff over the last axis.

    Zero-centred norms pass w_eff = 1 + w (TF:720-734 Qwen3_5RMSNorm; the
    engine adds the 1 at load, REF src/engine/model.c:196-205). Pinned by a
    closed form (unit RMS output) in tests/test_oracle.py.
    """
    x = np.asarray(x, dtype=np.float64)
    var = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(var + eps) * np.asarray(w_eff, dtype=np.float64)


def sigmoid(x):
    x = np.asarray(x, dtype=np.float64)
    return 1.0 / (1.0 + np.exp(-x))


def silu(x):
    x = np.asarray(x, dtype=np.float64)
    return x * sigmoid(x)


def softplus(x):
    """log(1 + e^x), linear above 20 (torch.nn.functional.softplus default;
    REF src/kernels/common.cuh:11-13)."""
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


# --------------------------------------------------------------------------
# RoPE
# --------------------------------------------------------------------------
def rope_inv_freq(theta: float, rot: int) -> np.ndarray:
    """inv_freq[i] = 1 / theta^(2i/rot), i < rot/2 (TF:117-125; REF
    src/kernels/attention.cu:91-93 computes it in double). Pinned by the
    closed form pos=0 -> identity and by the golden attention vectors."""
    i = np.arange(0, rot, 2, dtype=np.float64)
    return 1.0 / theta ** (i / rot)


def apply_rope(x, pos, inv_freq, rot):
    """rotate_half RoPE on x[..., :rot] (TF:546-589); x: [T, H, D], pos: [T].

    Text-only positions make the interleaved MRoPE of TF:149-164 reduce to
    1-D RoPE (all three position streams are equal).
    """
    x = np.asarray(x, dtype=np.float64)
    ang = np.asarray(pos, dtype=np.float64)[:, None] * inv_freq[None, :]  # [T, rot/2]
    cos = np.cos(np.concatenate([ang, ang], -1))[:, None, :]
    sin = np.sin(np.concatenate([ang, ang], -1))[:, None, :]
    xr, xp = x[..., :rot], x[..., rot:]
    half = rot // 2
    rot_half = np.concatenate([-xr[..., half:], xr[..., :half]], -1)
    return np.concatenate([xr * cos + rot_half * sin, xp], -1)


# --------------------------------------------------------------------------
# full (gated GQA) attention
# --------------------------------------------------------------------------
def attn_split_proj(proj, Hq, Hkv, D=256):
    """Split the fused projection row [Hq x (q|gate)] [Hkv x K] [Hkv x V]
    (REF src/engine/model.c:207-210, attention.cu:48-53; TF:667-671)."""
    T = proj.shape[0]
    qg = proj[:, : Hq * 2 * D].reshape(T, Hq, 2 * D)
    q, gate = qg[..., :D], qg[..., D:]
    k = proj[:, Hq * 2 * D: Hq * 2 * D + Hkv * D].reshape(T, Hkv, D)
    v = proj[:, Hq * 2 * D + Hkv * D: Hq * 2 * D + 2 * Hkv * D].reshape(T, Hkv, D)
    return q, gate, k, v


def attn_prep(proj, q_norm_eff, k_norm_eff, pos, Hq, Hkv, rot, theta, eps, D=256):
    """Per-head zero-centred RMSNorm then partial RoPE on q and k; v raw.

    REF src/kernels/attention.cu:11-81; TF:672-677 (norm before RoPE).
    Returns float64 q [T,Hq,D], gate [T,Hq,D], k [T,Hkv,D], v [T,Hkv,D].
    Pinned by the golden attention-layer vectors and pos=0 identity.
    """
    q, gate, k, v = attn_split_proj(np.asarray(proj, np.float64), Hq, Hkv, D)
    inv = rope_inv_freq(theta, rot)
    q = apply_rope(rmsnorm(q, q_norm_eff, eps), pos, inv, rot)
    k = apply_rope(rmsnorm(k, k_norm_eff, eps), pos, inv, rot)
    return q, gate, k, v.astype(np.float64)


KEY_TILE = 64  # keys per online-softmax step of the reference kernel (REF attention.cu:188, ATT_BC)


def _tiled_pv(s, v, tile=KEY_TILE):
    """Online softmax over key tiles with the probabilities rounded to bf16
    for the PV product, as the reference kernel runs it
    (REF src/kernels/attention.cu:188-297):

      for each tile of `tile` consecutive keys (boundaries at multiples of
      `tile` of the key index):
        m_new = max(m, max over the tile);  sc = e^(m - m_new)
        l = l sc + sum p;  o = o sc + bf16(p) V   with p = e^(s - m_new)

    so each tile's p is rounded against the running max after that tile, not
    against the row's final max. l sums the unrounded p. Masked keys carry
    s = -inf (p = 0). Returns o / l.

    s: [..., L] scores in the exponent's own units (the engine's log2-domain
    scores times ln 2, so e^s = 2^(s / ln 2)); v: [..., L, D], or [H, L, D]
    shared by every row when s is [H, T, L] (causal attention).
    Pinned by tests/test_oracle.py::test_tiled_bf16_softmax_rounding_points
    (one tile, or a first-tile max, gives the final-max rounding bit for bit;
    running maxima an integer number of octaves apart give it exactly too;
    a maximum in a later tile changes it; without rounding it is the plain
    softmax to 1e-15).
    """
    L = s.shape[-1]
    sub = "htl,hld->htd" if v.ndim == s.ndim else "...l,...ld->...d"
    m = np.full(s.shape[:-1], -np.inf)
    l = np.zeros(s.shape[:-1])
    o = np.zeros(s.shape[:-1] + (v.shape[-1],))
    for k0 in range(0, L, tile):
        st = s[..., k0:k0 + tile]
        mn = np.maximum(m, st.max(-1))
        ms = np.where(np.isfinite(mn), mn, 0.0)
        with np.errstate(invalid="ignore"):
            sc = np.where(np.isfinite(m), np.exp(m - ms), 0.0)
        p = np.exp(st - ms[..., None])
        l = l * sc + p.sum(-1)
        pb = bf16_round(p.astype(np.float32)).astype(np.float64)
        o = o * sc[..., None] + np.einsum(sub, pb, v[..., k0:k0 + tile, :])
        m = mn
    return o / l[..., None]


def shared_prefix_attention(q, gate, k_state, v_state, k_own, v_own, own_base,
                            scale=1.0 / 16.0, bf16_p=False):
    """Gated GQA attention of the engine (REF src/kernels/attention.cu:138-332).

    q, gate: [N, Hq, D]; k_state/v_state: [P, Hkv, D]; k_own/v_own: [N, Hkv, D]
    indexed by packed token; own_base: [N] segment start of each token.
    Token n sees state keys [0, P) and own keys [own_base[n], n].
    out[n, h] = sigmoid(gate[n, h]) * sum_j softmax_j(q.k_j * scale) v_j with
    q-head h reading kv-head h // (Hq // Hkv) (TF:592-601).

    bf16_p=True emulates the engine's rounding of the probabilities to bf16
    before the PV product, per 64-key tile of the concatenated key index
    [state ++ own] against the running max (`_tiled_pv`), while the row sum
    stays in full precision (REF attention.cu:188-297).

    Pinned by: equality with causal attention over [state ++ branch]
    (tests/test_oracle.py), the single-visible-key closed form sigma(g)*v,
    and the transformers golden layer vectors.
    """
    N, Hq, D = q.shape
    P = k_state.shape[0]
    Hkv = k_state.shape[1] if P > 0 else k_own.shape[1]
    grp = Hq // Hkv
    out = np.zeros((N, Hq, D), dtype=np.float64)
    for n in range(N):
        b = int(own_base[n])
        ks = np.concatenate([k_state, k_own[b: n + 1]], 0).astype(np.float64)  # [L, Hkv, D]
        vs = np.concatenate([v_state, v_own[b: n + 1]], 0).astype(np.float64)
        kr = np.repeat(ks.transpose(1, 0, 2), grp, axis=0)  # [Hq, L, D]
        vr = np.repeat(vs.transpose(1, 0, 2), grp, axis=0)
        s = np.einsum("hld,hd->hl", kr, q[n].astype(np.float64)) * scale
        if bf16_p:
            out[n] = _tiled_pv(s, vr)
        else:
            p = np.exp(s - s.max(-1, keepdims=True))
            out[n] = np.einsum("hl,hld->hd", p, vr) / p.sum(-1)[:, None]
    return out * sigmoid(gate)


def causal_gqa_attention(q, gate, k, v, scale=1.0 / 16.0, bf16_p=False):
    """transformers-style causal attention over one sequence
    (TF:604-626 eager_attention_forward + repeat_kv TF:592-601, gate TF:697-700).
    q, gate: [T, Hq, D]; k, v: [T, Hkv, D]. bf16_p: the probabilities are
    rounded to bf16 before the PV product per 64-key tile against the
    running max, the row sum is not (engine semantics, `_tiled_pv`,
    REF attention.cu:188-297)."""
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    grp = Hq // Hkv
    kr = np.repeat(k, grp, axis=1)
    vr = np.repeat(v, grp, axis=1)
    s = np.einsum("thd,shd->hts", q, kr) * scale
    mask = np.triu(np.ones((T, T), dtype=bool), 1)
    s = np.where(mask[None], -np.inf, s)
    if bf16_p:
        o = _tiled_pv(s, np.ascontiguousarray(vr.transpose(1, 0, 2), dtype=np.float64))
        return o.transpose(1, 0, 2) * sigmoid(gate)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    l = p.sum(-1, keepdims=True)
    o = np.einsum("hts,shd->thd", p / l, vr)
    return o * sigmoid(gate)


def gated_attention_layer(h_state, h_branch, own_base, Wqkv, Wo, q_norm_eff, k_norm_eff, Hq,
                          Hkv, rot, theta, eps, D=256, rnd=None):
    """One gated GQA attention layer (projection to o_proj) over a shared
    state and packed branches, as the engine runs it (REF
    src/engine/forward.c:99-118, src/kernels/attention.cu:41-100, :138-332):
    the state's tokens (positions 0..P-1) attend causally among themselves,
    branch token n (position P + its index in its branch) attends to the
    whole state plus [own_base[n], n].

    h_state [P, H], h_branch [N, H]: the layer inputs (after the input norm);
    Wqkv [Hq*2D + 2*Hkv*D, H] row-fused q|gate (per head), k, v; Wo [H, Hq*D].
    rnd: None for float64 throughout, or a bf16 rounding function applied at
    the reference engine's rounding points (projection output, q after its
    scale, K cache, probabilities, attention output, o_proj output).
    Returns (out_state [P, H], out_branch [N, H]).
    Pinned by tests/test_attention_layer.py against transformers'
    Qwen3_5Attention over every [state ++ branch] at config 1's shapes."""
    e = rnd is not None
    r = rnd if e else (lambda x: x)
    P, N = len(h_state), len(h_branch)
    own_base = np.asarray(own_base)
    pos_b = P + np.arange(N) - own_base
    qs, gs, ks, vs = attn_prep(r(np.asarray(h_state, np.float64) @ Wqkv.T), q_norm_eff,
                               k_norm_eff, np.arange(P), Hq, Hkv, rot, theta, eps, D)
    qb, gb, kb, vb = attn_prep(r(np.asarray(h_branch, np.float64) @ Wqkv.T), q_norm_eff,
                               k_norm_eff, pos_b, Hq, Hkv, rot, theta, eps, D)
    if e:
        sc = D ** -0.5 * LOG2E
        qs, qb, ks, kb = r(qs * sc), r(qb * sc), r(ks), r(kb)
        kw = dict(scale=np.log(2.0), bf16_p=True)
    else:
        kw = dict(scale=D ** -0.5)
    o_s = causal_gqa_attention(qs, gs, ks, vs, **kw) if P else np.zeros((0, Hq, D))
    o_b = shared_prefix_attention(qb, gb, ks, vs, kb, vb, own_base, **kw)
    return r(r(o_s.reshape(P, Hq * D)) @ Wo.T), r(r(o_b.reshape(N, Hq * D)) @ Wo.T)


# --------------------------------------------------------------------------
# Gated DeltaNet
# --------------------------------------------------------------------------
def gdn_split_proj(proj, Hk, Hv, dk=128, dv=128):
    """Fused GDN projection row [q Hk*dk | k Hk*dk | v Hv*dv | z Hv*dv | b Hv | a Hv]
    (REF src/engine/model.c:218-222, src/engine/forward.c:125; TF:426-429)."""
    K, V = Hk * dk, Hv * dv
    C = 2 * K + V
    x = proj[:, :C]
    z = proj[:, C: C + V]
    b = proj[:, C + V: C + V + Hv]
    a = proj[:, C + V + Hv: C + V + 2 * Hv]
    return x, z, b, a


def gdn_conv(x, w, tail=None):
    """Depthwise causal conv (width 4, no bias) + SiLU over channels.

    x: [T, C] pre-conv inputs; w: [C, 4]; tail: [C, 3] last three pre-conv
    inputs of the prefix (None = zeros). out[t,c] = silu(sum_j w[c,j] x[t-3+j,c])
    with x[t<0] taken from the tail. REF src/kernels/gdn.cu:4-24; TF:219-239.
    Pinned by: conv with tail == conv over the concatenated sequence, and the
    golden GDN layer vectors.
    """
    x = np.asarray(x, np.float64)
    T, C = x.shape
    pre = np.zeros((3, C)) if tail is None else np.asarray(tail, np.float64).T  # [3, C]
    xx = np.concatenate([pre, x], 0)
    acc = np.zeros((T, C))
    for j in range(4):
        acc += xx[j: j + T] * np.asarray(w, np.float64)[None, :, j]
    return silu(acc)


def gdn_conv_tail(x, tail=None):
    """Last three pre-conv inputs after a segment, as [C, 3] (oldest first)
    (REF src/kernels/gdn.cu:26-43; TF:199-216 conv state)."""
    x = np.asarray(x, np.float64)
    C = x.shape[1]
    pre = np.zeros((3, C)) if tail is None else np.asarray(tail, np.float64).T
    xx = np.concatenate([pre, x], 0)
    return xx[-3:].T.copy()


def l2norm(x, eps=1e-6):
    """x * rsqrt(sum x^2 + eps) (TF:242-245)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + eps)


def gdn_prep(xc, b, a, A_log, dt_bias, Hk, Hv, dk=128, dv=128):
    """Post-conv qkv -> q, k (l2-normalised, q * dk^-1/2, k-heads repeated to
    Hv), v, g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b).

    REF src/kernels/gdn.cu:57-96; TF:483-502 and :262-279 (l2norm in kernel).
    Pinned by the l2-norm closed form and the golden GDN layer vectors.
    """
    T = xc.shape[0]
    K = Hk * dk
    q = xc[:, :K].reshape(T, Hk, dk)
    k = xc[:, K: 2 * K].reshape(T, Hk, dk)
    v = xc[:, 2 * K:].reshape(T, Hv, dv)
    rep = Hv // Hk
    q = np.repeat(l2norm(q), rep, axis=1) / np.sqrt(dk)
    k = np.repeat(l2norm(k), rep, axis=1)
    g = -np.exp(np.asarray(A_log, np.float64))[None, :] * softplus(
        np.asarray(a, np.float64) + np.asarray(dt_bias, np.float64)[None, :])
    beta = sigmoid(b)
    return q, k, np.asarray(v, np.float64), g, beta


def gdn_recurrent(q, k, v, g, beta, S0=None):
    """Gated delta rule, recurrent form, per head.

    q,k: [T,H,dk] (q already scaled), v: [T,H,dv], g,beta: [T,H]; S: [H,dk,dv].
      S <- e^{g_t} S;  kv = S^T k_t;  delta = beta_t (v_t - kv);
      S <- S + k_t delta^T;  o_t = S^T q_t
    REF src/kernels/gdn.cu:140-176; TF:331-380. Pinned by brute-force special
    cases (beta=0 pure decay, one token from S=0 gives beta (q.k) v, exact
    overwrite with orthonormal keys) in tests/test_oracle.py.
    """
    T, H, dk = k.shape
    dv = v.shape[-1]
    S = np.zeros((H, dk, dv)) if S0 is None else np.array(S0, dtype=np.float64)
    o = np.zeros((T, H, dv))
    for t in range(T):
        S = S * np.exp(g[t])[:, None, None]
        kv = np.einsum("hkv,hk->hv", S, k[t])
        delta = beta[t][:, None] * (v[t] - kv)
        S = S + k[t][:, :, None] * delta[:, None, :]
        o[t] = np.einsum("hkv,hk->hv", S, q[t])
    return o, S


def gdn_chunked(q, k, v, g, beta, S0=None, chunk=64):
    """Chunked WY/UT form of the same recurrence (TF:249-327, FLA's
    chunk_gated_delta_rule). Per chunk with cumulative log-decay G:
      A = tril(diag(beta) K K^T * e^{G_i - G_j}, -1); T = (I + A)^-1
      W = T diag(beta e^G) K;  U = T diag(beta) V
      V' = U - W S;  O = (Q e^G) S + tril(Q K^T e^{G_i-G_j}) V'
      S <- e^{G_last} S + (K e^{G_last - G})^T V'
    Pinned by equality with gdn_recurrent (tests/test_oracle.py)."""
    T, H, dk = k.shape
    dv = v.shape[-1]
    S = np.zeros((H, dk, dv)) if S0 is None else np.array(S0, dtype=np.float64)
    o = np.zeros((T, H, dv))
    for c0 in range(0, T, chunk):
        c1 = min(T, c0 + chunk)
        L = c1 - c0
        for h in range(H):
            Q, K, Vv = q[c0:c1, h], k[c0:c1, h], v[c0:c1, h]
            bt = beta[c0:c1, h]
            G = np.cumsum(g[c0:c1, h])
            with np.errstate(over="ignore"):  # only the masked upper part overflows
                Gam = np.exp(G[:, None] - G[None, :])
            A = np.tril((bt[:, None] * (K @ K.T)) * Gam, -1)
            Tm = np.linalg.inv(np.eye(L) + A)
            W = Tm @ (K * (bt * np.exp(G))[:, None])
            U = Tm @ (Vv * bt[:, None])
            Vn = U - W @ S[h]
            QK = np.tril((Q @ K.T) * Gam)
            o[c0:c1, h] = (Q * np.exp(G)[:, None]) @ S[h] + QK @ Vn
            S[h] = np.exp(G[-1]) * S[h] + (K * np.exp(G[-1] - G)[:, None]).T @ Vn
    return o, S


def gated_rmsnorm(o, z, w, eps, bf16_roundtrip=True):
    """y = (w * bf16(o * rsqrt(mean o^2 + eps))) * silu(z) per head (last axis).

    TF:168-184 Qwen3_5RMSNormGated (w is NOT zero-centred); the bf16 round trip
    of TF:181 happens for bf16 activations and is kept by the engine
    (REF src/kernels/gdn.cu:213). Pinned by the closed form and the golden
    GDN layer vectors."""
    o = np.asarray(o, np.float64)
    var = np.mean(o * o, axis=-1, keepdims=True)
    hn = o / np.sqrt(var + eps)
    if bf16_roundtrip:
        hn = bf16_round(hn.astype(np.float32)).astype(np.float64)
    return hn * np.asarray(w, np.float64) * silu(z)


# --------------------------------------------------------------------------
# whole model (transformers Qwen3_5ForCausalLM semantics, float64)
# --------------------------------------------------------------------------
def load_checkpoint(path):
    """config.json + *.safetensors of a local directory -> (cfg, {name: f64}).
    Reads with safetensors' torch loader (no pickle); text model only."""
    import json
    from pathlib import Path

    from safetensors.torch import load_file

    path = Path(path)
    cfg = json.loads((path / "config.json").read_text())
    cfg = cfg.get("text_config", cfg)
    W = {}
    for f in sorted(path.glob("*.safetensors")):
        for k, v in load_file(str(f)).items():
            W[k.replace("model.language_model.", "model.")] = v.float().numpy().astype(np.float64)
    return cfg, W


def _b(x, on):
    """bf16 rounding point of the engine, applied when `on`."""
    return bf16_round(np.asarray(x, np.float32)).astype(np.float64) if on else x


def model_last_logits(cfg, W, ids, chunked=True, engine_numerics=False):
    """Next-token logits at the last position of one causal sequence `ids`.

    Decoder layer TF:740-793 (pre-norm, residual), full attention TF:656-701,
    GDN TF:432-543 in its fp32 form (no bf16 round trip inside the gated norm),
    MLP TF:704-717, final norm and LM head (tied: the embedding) TF:1571-1650.
    Pinned by the transformers golden logits (tests/test_golden.py) and by the
    engine invariants it is used for (branch = [state ++ branch]).

    engine_numerics=True rounds to bf16 where the reference engine stores
    bf16 (REF docs/ARCHITECTURE.md:67-75, src/kernels/*.cu): every GEMM input
    and output, q (after its scale * log2 e), the K/V cache, the attention
    probabilities, the attention and GDN outputs, silu*up, the final-norm row,
    and the gated-norm round trip (REF gdn.cu:213); the residual stays full
    precision. This is the reference engine's own path on the same weights."""
    ids = np.asarray(ids)
    T = len(ids)
    e = engine_numerics
    eps = cfg["rms_norm_eps"]
    Hq, Hkv, D = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    Hk, Hv = cfg["linear_num_key_heads"], cfg["linear_num_value_heads"]
    rp = cfg.get("rope_parameters") or {}
    theta = rp.get("rope_theta", cfg.get("rope_theta", 10000.0))
    rot = int(D * rp.get("partial_rotary_factor", cfg.get("partial_rotary_factor", 0.25)))
    pos = np.arange(T)
    x = W["model.embed_tokens.weight"][ids]
    for i, lt in enumerate(cfg["layer_types"]):
        p = f"model.layers.{i}."
        h = _b(rmsnorm(x, 1.0 + W[p + "input_layernorm.weight"], eps), e)
        if lt == "full_attention":
            a = p + "self_attn."
            proj = _b(np.concatenate([h @ W[a + "q_proj.weight"].T, h @ W[a + "k_proj.weight"].T,
                                      h @ W[a + "v_proj.weight"].T], -1), e)
            q, gate, k, v = attn_prep(proj, 1.0 + W[a + "q_norm.weight"],
                                      1.0 + W[a + "k_norm.weight"], pos, Hq, Hkv, rot, theta, eps, D)
            if e:
                qs = _b(q * (D ** -0.5 * LOG2E), True)
                o = causal_gqa_attention(qs, gate, _b(k, True), v, scale=np.log(2.0), bf16_p=True)
            else:
                o = causal_gqa_attention(q, gate, k, v, scale=D ** -0.5)
            o = _b(o.reshape(T, Hq * D), e)
            x = x + _b(o @ W[a + "o_proj.weight"].T, e)
        else:
            g_ = p + "linear_attn."
            xq = _b(h @ W[g_ + "in_proj_qkv.weight"].T, e)
            z = _b(h @ W[g_ + "in_proj_z.weight"].T, e)
            b = _b(h @ W[g_ + "in_proj_b.weight"].T, e)
            aa = _b(h @ W[g_ + "in_proj_a.weight"].T, e)
            xc = gdn_conv(xq, W[g_ + "conv1d.weight"].reshape(-1, 4))
            q, k, v, g, beta = gdn_prep(xc, b, aa, W[g_ + "A_log"], W[g_ + "dt_bias"], Hk, Hv)
            if chunked:
                o, _ = gdn_chunked(q, k, v, g, beta)
            else:
                o, _ = gdn_recurrent(q, k, v, g, beta)
            y = gated_rmsnorm(o, z.reshape(T, Hv, -1), W[g_ + "norm.weight"], eps,
                              bf16_roundtrip=e)
            y = _b(y.reshape(T, -1), e)
            x = x + _b(y @ W[g_ + "out_proj.weight"].T, e)
        m = p + "mlp."
        h = _b(rmsnorm(x, 1.0 + W[p + "post_attention_layernorm.weight"], eps), e)
        gu_g = _b(h @ W[m + "gate_proj.weight"].T, e)
        gu_u = _b(h @ W[m + "up_proj.weight"].T, e)
        act = _b(silu(gu_g) * gu_u, e)
        x = x + _b(act @ W[m + "down_proj.weight"].T, e)
    hl = _b(rmsnorm(x[-1], 1.0 + W["model.norm.weight"], eps), e)
    head = W["lm_head.weight"] if "lm_head.weight" in W else W["model.embed_tokens.weight"]
    return head @ hl
