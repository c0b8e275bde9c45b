"""Streaming request oracle (TEST INFRASTRUCTURE ONLY).

One shared-prefix request -- a state of P tokens, then B branches that each
continue it -- through a whole Qwen3.5 checkpoint, one layer at a time, so a
4B/9B-shaped model never has to sit in host memory in float64 (a 4B model is
~32 GB in float64; one layer is ~1 GB). Only ``tests/``, ``bench.py``'s
cpu_baseline leg and the fixture scripts under ``tests/golden/`` may use it,
and only as the checker.

The request is computed the way the reference engine computes it
(REF src/engine/forward.c:50-149): the state is prefilled once, each branch
attends to the state's K/V plus its own causal prefix and starts its Gated
DeltaNet recurrence from the state's final S and conv tail. This
decomposition equals plain causal processing of every ``[state ++ branch]``
sequence (``qwen35.model_last_logits``); tests/test_oracle.py pins each step
(shared-prefix attention == causal attention over the concatenation,
continuing from S_final == scanning the concatenation, conv with the tail ==
conv over the concatenation) and tests/test_request_oracle.py pins the whole
function against ``model_last_logits`` on small checkpoints.

Several numerics "tracks" share one pass over the weights:
  "f64"     transformers' math in float64 (the fp32 oracle, without fp32's
            own roundoff);
  "engine"  the reference engine's bf16 rounding points on float64 math
            (``model_last_logits(engine_numerics=True)``, REF
            docs/ARCHITECTURE.md:67-75): its GDN recurrence is fp32;
  "mfma"    "engine" with the Gated DeltaNet replaced by an emulation of this
            build's chunked gfx950 kernel rounding points
            (``gdn_chunk_emulated``), for attributing deviations;
  "engine~<n>" "engine" with a 2^-24 relative jitter (seed n) before every
            bf16 rounding: another valid fp32 summation order, the noise
            floor between two correct bf16 engines;
  "mfma:<ops>" the same with the listed operands carried as split bf16
            pairs (hi + lo), e.g. "mfma:S" or "mfma:S,Vp,T".
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from . import qwen35 as q35

_b = q35._b


# --------------------------------------------------------------------------
# weights, one tensor at a time
# --------------------------------------------------------------------------
class StreamedWeights:
    """float64 views of single tensors of a local safetensors checkpoint,
    read on demand (no pickle: safetensors' own reader)."""

    def __init__(self, path):
        from safetensors import safe_open

        self.path = Path(path)
        cfg = json.loads((self.path / "config.json").read_text())
        self.cfg = cfg.get("text_config", cfg)
        self._files = [safe_open(str(f), framework="pt") for f in
                       sorted(self.path.glob("*.safetensors"))]
        self._where = {}
        for f in self._files:
            for k in f.keys():
                self._where[k.replace("model.language_model.", "model.")] = (f, k)

    def has(self, name):
        return name in self._where

    def get(self, name, dtype=np.float64):
        f, k = self._where[name]
        return f.get_tensor(k).float().numpy().astype(dtype, copy=False)

    def rows(self, name, idx):
        """Selected rows of a 2-D tensor (embedding lookups)."""
        f, k = self._where[name]
        t = f.get_slice(k)
        idx = np.asarray(idx)
        uniq, inv = np.unique(idx, return_inverse=True)
        out = np.stack([t[int(i): int(i) + 1].float().numpy()[0] for i in uniq])
        return out[inv].astype(np.float64)

    def head_matvec(self, h, block=16384):
        """[B, H] float64 -> [B, vocab] logits through the LM head (tied: the
        embedding), streamed in row blocks."""
        name = "lm_head.weight" if self.has("lm_head.weight") else "model.embed_tokens.weight"
        f, k = self._where[name]
        sl = f.get_slice(k)
        V = sl.get_shape()[0]
        out = np.empty((h.shape[0], V))
        for r0 in range(0, V, block):
            r1 = min(V, r0 + block)
            w = sl[r0:r1].float().numpy().astype(np.float64)
            out[:, r0:r1] = h @ w.T
        return out


# --------------------------------------------------------------------------
# this build's Gated DeltaNet kernel numerics (for attribution)
# --------------------------------------------------------------------------
def _rb(x, split=False):
    """bf16 operand, or a split pair hi + lo (about 16 significant bits)."""
    hi = q35.bf16_round(np.asarray(x, np.float32)).astype(np.float64)
    if not split:
        return hi
    lo = q35.bf16_round(np.asarray(x - hi, np.float32)).astype(np.float64)
    return hi + lo


def gdn_chunk_emulated(q, k, v, g, beta, S0=None, chunk=64, split=()):
    """The chunked delta rule with the rounding points of this build's gfx950
    kernels (cu-jev_amd/csrc/kernels/gdn.hip: gdn_chunk_a_kernel,
    gdn_chunk_b_kernel / gdn_short_b_kernel), float64 elsewhere.

    q, k, v are the bf16 values the kernel stages (conv, l2-norm and scale
    already applied and rounded). Per chunk and head:
      A = tril(beta_i k_i.k_j e^{G_i-G_j}, -1);  T = (I + A)^-1   (fp32)
      W = bf16(bf16(T) bf16(beta e^G K)),  U = bf16(bf16(T) bf16(beta V))
      Q = bf16(q), QKm = bf16(tril(q.k e^{G_i-G_j})), KT = bf16(K) (per k-head)
      V' = bf16(U - W bf16(S)),  D = bf16(e^{Gl-G} (U - W bf16(S)))
      O = e^G (Q bf16(S)) + QKm V'
      S = e^{Gl} S + KT^T D       (S itself stays fp32)
    O is returned rounded to bf16, as the kernel stores it. `split` names
    operands carried as hi + lo bf16 pairs instead: any of "S", "Vp" (V' and
    D), "T", "W", "U", "Q", "QK", "KT", "O" (and, in request_logits, "qkv"
    for the staged q, k, v).
    Pinned by tests/test_request_oracle.py: with every operand split it
    matches gdn_chunked to ~1e-4, and each unsplit rounding point moves the
    result by the size a bf16 rounding implies.
    """
    sp = set(split)
    T_, H, dk = k.shape
    dv = v.shape[-1]
    S = np.zeros((H, dk, dv)) if S0 is None else np.array(S0, dtype=np.float64)
    o = np.zeros((T_, H, dv))
    for c0 in range(0, T_, chunk):
        c1 = min(T_, c0 + chunk)
        L = c1 - c0
        for h in range(H):
            Q, K, Vv = q[c0:c1, h], k[c0:c1, h], v[c0:c1, h]
            bt = beta[c0:c1, h]
            G = np.cumsum(g[c0:c1, h])
            dG = np.minimum(G[:, None] - G[None, :], 0.0)
            dec = np.exp(dG)
            A = np.tril(bt[:, None] * (K @ K.T) * dec, -1)
            Tm = np.linalg.inv(np.eye(L) + A)
            Tb = _rb(Tm, "T" in sp)
            W = _rb(Tb @ _rb(K * (bt * np.exp(G))[:, None], "W" in sp), "W" in sp)
            U = _rb(Tb @ _rb(Vv * bt[:, None], "U" in sp), "U" in sp)
            Qb = _rb(Q, "Q" in sp)
            QK = _rb(np.tril((Q @ K.T) * dec), "QK" in sp)
            Kb = _rb(K, "KT" in sp)
            Sb = _rb(S[h], "S" in sp)
            Vx = U - W @ Sb
            Vn = _rb(Vx, "Vp" in sp)
            Vd = _rb(Vx * np.exp(G[-1] - G)[:, None], "Vp" in sp)
            oc = np.exp(G)[:, None] * (Qb @ Sb) + QK @ Vn
            o[c0:c1, h] = _rb(oc, "O" in sp)
            S[h] = np.exp(G[-1]) * S[h] + Kb.T @ Vd
    return o, S


def _gdn_prep_kernel_rounding(xc, b, a, A_log, dt_bias, Hk, Hv, split=False):
    """gdn_prep with the kernel's bf16 staging of q, k, v (the gates stay
    fp32): what gdn_chunk_a_kernel holds in LDS (split: hi + lo pairs)."""
    qh, kh, vh, g, beta = q35.gdn_prep(xc, b, a, A_log, dt_bias, Hk, Hv)
    return _rb(qh, split), _rb(kh, split), _rb(vh, split), g, beta


# --------------------------------------------------------------------------
# one request
# --------------------------------------------------------------------------
class _Track:
    def __init__(self, mode):
        self.mode = mode
        base, _, jseed = mode.partition("~")
        self.e = base != "f64"
        # "engine~<n>": fp32-sized relative jitter (2^-24, seed n) on every
        # value before its bf16 rounding, i.e. another equally valid fp32
        # summation order; the control for how far two correct bf16 engines
        # drift apart
        self.jitter = 2.0 ** -24 if "~" in mode else 0.0
        self._rng = np.random.default_rng(int(jseed) if jseed else 12345)
        self.gdn = "mfma" if mode.startswith("mfma") else "ref"
        self.split = tuple(s for s in mode.split(":", 1)[1].split(",") if s) if ":" in mode else ()
        self.xs = None  # state residual [P, H]
        self.xb = None  # branch residual [N, H]
        self.taps = []  # per layer: the branch rows' residual when recording

    def rnd(self, x):
        """This track's bf16 rounding point (identity for "f64")."""
        if not self.e:
            return x
        if self.jitter:
            x = x * (1.0 + self.jitter * self._rng.standard_normal(np.shape(x)))
        return _b(x, True)


def request_logits(ckpt, state, branches, modes=("f64", "engine"), full=False, record=False,
                   progress=None):
    """Last-token logits of every branch of one request, for each numerics
    mode in `modes` (see the module docstring).

    state: token ids of the shared prefix; branches: list of (tokens,
    candidates). Returns {mode: {"cand": [np.ndarray per branch],
    "full": [B, vocab] or None, "hidden": [B, H] final-norm rows,
    "taps": per-layer residuals when `record`}}.
    """
    Wt = StreamedWeights(ckpt)
    cfg = Wt.cfg
    eps = cfg["rms_norm_eps"]
    Hq, Hkv, D = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    Hk, Hv = cfg["linear_num_key_heads"], cfg["linear_num_value_heads"]
    rp = cfg.get("rope_parameters") or {}
    theta = rp.get("rope_theta", cfg.get("rope_theta", 10000.0))
    rot = int(D * rp.get("partial_rotary_factor", cfg.get("partial_rotary_factor", 0.25)))
    P = len(state)
    lens = [len(t) for t, _ in branches]
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(int)
    N = int(sum(lens))
    br_ids = np.concatenate([np.asarray(t) for t, _ in branches])
    pos_s = np.arange(P)
    pos_b = np.concatenate([P + np.arange(n) for n in lens])
    own_base = np.repeat(starts, lens)

    tracks = [_Track(m) for m in modes]
    emb_s = Wt.rows("model.embed_tokens.weight", state)
    emb_b = Wt.rows("model.embed_tokens.weight", br_ids)
    for tr in tracks:
        tr.xs, tr.xb = emb_s.copy(), emb_b.copy()

    for li, lt in enumerate(cfg["layer_types"]):
        p = f"model.layers.{li}."
        w_in = 1.0 + Wt.get(p + "input_layernorm.weight")
        w_post = 1.0 + Wt.get(p + "post_attention_layernorm.weight")
        if lt == "full_attention":
            a = p + "self_attn."
            Wqkv = np.concatenate([Wt.get(a + "q_proj.weight"), Wt.get(a + "k_proj.weight"),
                                   Wt.get(a + "v_proj.weight")], 0)
            Wo = Wt.get(a + "o_proj.weight")
            qn, kn = 1.0 + Wt.get(a + "q_norm.weight"), 1.0 + Wt.get(a + "k_norm.weight")
            for tr in tracks:
                e = tr.e
                hs = tr.rnd(q35.rmsnorm(tr.xs, w_in, eps))
                hb = tr.rnd(q35.rmsnorm(tr.xb, w_in, eps))
                ys, yb = q35.gated_attention_layer(hs, hb, own_base, Wqkv, Wo, qn, kn, Hq, Hkv,
                                                   rot, theta, eps, D, tr.rnd if e else None)
                tr.xs, tr.xb = tr.xs + ys, tr.xb + yb
        else:
            g_ = p + "linear_attn."
            Wq = Wt.get(g_ + "in_proj_qkv.weight")
            Wz = Wt.get(g_ + "in_proj_z.weight")
            Wb = Wt.get(g_ + "in_proj_b.weight")
            Wa = Wt.get(g_ + "in_proj_a.weight")
            Wout = Wt.get(g_ + "out_proj.weight")
            cw = Wt.get(g_ + "conv1d.weight").reshape(-1, 4)
            A_log, dtb = Wt.get(g_ + "A_log"), Wt.get(g_ + "dt_bias")
            nw = Wt.get(g_ + "norm.weight")
            for tr in tracks:
                e = tr.e
                emu = tr.gdn == "mfma"
                if emu:
                    def prep(*args, _sp="qkv" in tr.split):
                        return _gdn_prep_kernel_rounding(*args, split=_sp)
                else:
                    prep = q35.gdn_prep

                def scan(qq, kk, vv, gg, bb, S0):
                    if emu:
                        return gdn_chunk_emulated(qq, kk, vv, gg, bb, S0, split=tr.split)
                    return q35.gdn_chunked(qq, kk, vv, gg, bb, S0)

                def mixer(h, tail, S0):
                    xq = tr.rnd(h @ Wq.T)
                    z, bb, aa = tr.rnd(h @ Wz.T), tr.rnd(h @ Wb.T), tr.rnd(h @ Wa.T)
                    xc = q35.gdn_conv(xq, cw, tail)
                    qq, kk, vv, gg, be = prep(xc, bb, aa, A_log, dtb, Hk, Hv)
                    o, S = scan(qq, kk, vv, gg, be, S0)
                    y = q35.gated_rmsnorm(o, z.reshape(len(h), Hv, -1), nw, eps, bf16_roundtrip=e)
                    return tr.rnd(y.reshape(len(h), -1)), S, q35.gdn_conv_tail(xq, tail)

                hs = tr.rnd(q35.rmsnorm(tr.xs, w_in, eps))
                ys, S_fin, tail = mixer(hs, None, None)
                hb = tr.rnd(q35.rmsnorm(tr.xb, w_in, eps))
                yb = np.zeros((N, Hv * 128))
                for b0, n in zip(starts, lens):
                    yb[b0: b0 + n] = mixer(hb[b0: b0 + n], tail, S_fin)[0]
                tr.xs = tr.xs + tr.rnd(ys @ Wout.T)
                tr.xb = tr.xb + tr.rnd(yb @ Wout.T)
        m = p + "mlp."
        Wg, Wu, Wd = Wt.get(m + "gate_proj.weight"), Wt.get(m + "up_proj.weight"), \
            Wt.get(m + "down_proj.weight")
        for tr in tracks:
            e = tr.e
            for side in ("xs", "xb"):
                x = getattr(tr, side)
                h = tr.rnd(q35.rmsnorm(x, w_post, eps))
                act = tr.rnd(q35.silu(tr.rnd(h @ Wg.T)) * tr.rnd(h @ Wu.T))
                setattr(tr, side, x + tr.rnd(act @ Wd.T))
            if record:
                rows = starts + np.asarray(lens) - 1
                tr.taps.append(tr.xb[rows].copy())
        if progress:
            progress(li)

    wf = 1.0 + Wt.get("model.norm.weight")
    rows = starts + np.asarray(lens) - 1
    out = {}
    for tr in tracks:
        hl = tr.rnd(q35.rmsnorm(tr.xb[rows], wf, eps))
        res = {"hidden": hl, "taps": tr.taps if record else None}
        if full:
            res["full"] = Wt.head_matvec(hl)
            res["cand"] = [res["full"][i, np.asarray(c, int)] for i, (_, c) in
                           enumerate(branches)]
        else:
            name = "lm_head.weight" if Wt.has("lm_head.weight") else "model.embed_tokens.weight"
            res["full"] = None
            res["cand"] = [Wt.rows(name, np.asarray(c, int)) @ hl[i] if len(c) else np.zeros(0)
                           for i, (_, c) in enumerate(branches)]
        out[tr.mode] = res
    return out
