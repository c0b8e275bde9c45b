"""ctypes binding of libcujev_ops.so (include/cujev_ops.h): the hot-path
kernels one by one, on device buffers.

torch is used only as device-memory plumbing: callers pass torch CUDA tensors
and this module hands their raw pointers and the current HIP stream to the C
ABI. There is no fallback: if the library is missing or a call fails, an
``OpsError`` is raised.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent


class OpsError(RuntimeError):
    pass


_lib = None

_P = C.c_void_p
_I = C.c_int
_F = C.c_float
_D = C.c_double

# name -> argtypes (all return int status)
_SIGS = {
    "cujev_op_gemm": [_P, _P, _P, _I, _I, _I, _I, _P, C.c_size_t, _P],
    "cujev_op_rope_table": [_D, _I, _I, _P],
    "cujev_op_attn_prep": [_P, _I, _P, _P, _P, _I, _I, _I, _I, _P, _F, _F, _P, _P, _P, _I, _P],
    "cujev_op_attn_prep_pair": [_P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _P, _F, _F, _P, _P, _P,
                                _I, _P, _P, _I, _P],
    "cujev_op_attention": [_P, _P, _I, _I, _P, _P, _I, _I, _P, _P, _I, _P, _I, _I, _I, _P, _P],
    "cujev_op_attention_ws": [_P, _P, _I, _I, _P, _P, _I, _I, _P, _P, _I, _P, _I, _I, _I, _P, _P,
                              C.c_size_t, _P],
    "cujev_op_attention_noalloc": [_P, _P, _I, _I, _P, _P, _I, _I, _P, _P, _I, _P, _I, _I, _I,
                                   _P, _P],
    # q, gate, gts, ghs, pk, pvt, p_stride, own_base, out, Hq, Hkv,
    # Na, Pa, oka, ovta, oa_stride, Nb, Pb, okb, ovtb, ob_stride, stream
    "cujev_op_attention_pair": [_P, _P, _I, _I, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P, _P, _I,
                                _I, _I, _P, _P, _I, _P],
    "cujev_op_gdn_conv_prep": [_P, _I, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _P, _P, _P, _P,
                               _P, _P],
    "cujev_op_gemm_small": [_P, _I, _P, _I, _I, _I, _I, _I, _P, _I, _P, _P],
    "cujev_op_gemm_small_tile": [_P, _I, _I, _P, _P],
    "cujev_op_gemm_wide": [_P, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P, _I, _P, _P],
    "cujev_op_add_rmsnorm": [_P, _P, _P, _I, _P, _P, _I, _I, _F, _P, _I, _P],
    "cujev_op_gdn_recur": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _F, _I, _I, _I, _P,
                           _P, _P],
    "cujev_op_gdn_layer": [_P, _I, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _P, _P,
                           _P, _P, _F, _I, _I, _I, _P, _P, _P],
    "cujev_op_gdn_scan": [_P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _P, _P, _P, _P, _I, _P,
                          _F, _I, _I, _I, _P, _P, _P],
}


def library_path() -> str:
    return os.environ.get("CUJEV_OPS_LIBRARY", str(_HERE / "libcujev_ops.so"))


def load():
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not os.path.exists(path):
        raise OpsError(f"{path} not found: build it with `make -C cu-jev_amd` "
                       "(or __graft_entry__.build())")
    lib = C.CDLL(path)
    lib.cujev_ops_kv_stride.argtypes = [_I]
    lib.cujev_ops_kv_stride.restype = _I
    lib.cujev_ops_last_error.restype = C.c_char_p
    lib.cujev_ops_gdn_scratch_bytes.argtypes = [_I, _I, _I]
    lib.cujev_ops_gdn_scratch_bytes.restype = C.c_size_t
    lib.cujev_ops_gemm_small_splits.argtypes = [_I, _I]
    lib.cujev_ops_gemm_small_splits.restype = _I
    lib.cujev_ops_gemm_wide_plan.argtypes = [_I, _I, _I, _I, _I, C.POINTER(_I), C.POINTER(_I),
                                             C.POINTER(_I)]
    lib.cujev_ops_gemm_wide_plan.restype = _I
    lib.cujev_ops_attention_ws_bytes.argtypes = [_I, _I, _I, _I]
    lib.cujev_ops_attention_ws_bytes.restype = C.c_size_t
    lib.cujev_ops_blaslt_version.argtypes = []
    lib.cujev_ops_blaslt_version.restype = _I
    lib.cujev_op_gemm_tune.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, _I, _I, _I, _I,
                                       C.c_void_p, C.c_size_t, C.c_void_p,
                                       C.POINTER(_I), C.POINTER(C.c_float), C.POINTER(C.c_float)]
    lib.cujev_op_gemm_tune.restype = _I
    for name, args in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _I
    _lib = lib
    return lib


def exported_symbols():
    return ["cujev_ops_kv_stride", "cujev_ops_last_error", "cujev_ops_gdn_scratch_bytes",
            "cujev_ops_gemm_small_splits", "cujev_ops_gemm_wide_plan", "cujev_ops_attention_ws_bytes",
            "cujev_ops_blaslt_version", "cujev_op_gemm_tune", *_SIGS]


def _ptr(t):
    if t is None:
        return None
    return C.c_void_p(t.data_ptr())


def _stream():
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _call(name, *args):
    lib = load()
    st = getattr(lib, name)(*args)
    if st != 0:
        raise OpsError(f"{name}: status {st}: {lib.cujev_ops_last_error().decode()}")


def kv_stride(max_tokens: int) -> int:
    return load().cujev_ops_kv_stride(int(max_tokens))


def rope_table(theta, rot, npos):
    """Device RoPE table for attn_prep (torch float32 [npos, rot/2, 2])."""
    import torch
    t = torch.empty(npos, rot // 2, 2, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    _call("cujev_op_rope_table", float(theta), int(rot), int(npos), _ptr(t))
    return t


def attn_prep(proj, q_norm_w, k_norm_w, pos, Hq, Hkv, rot, rope, eps, q_scale,
              q_out, k_cache, vt_cache, cache_stride):
    N = proj.shape[0]
    _call("cujev_op_attn_prep", _ptr(proj), proj.stride(0), _ptr(q_norm_w), _ptr(k_norm_w),
          _ptr(pos), N, Hq, Hkv, rot, _ptr(rope), float(eps), float(q_scale), _ptr(q_out),
          _ptr(k_cache), _ptr(vt_cache), cache_stride, _stream())


def attn_prep_pair(proj, q_norm_w, k_norm_w, pos, Na, Hq, Hkv, rot, rope, eps, q_scale, q_out,
                   k_cache, vt_cache, cache_stride, k_cache2, vt_cache2, cache_stride2):
    """attn_prep of rows [0, Na) into (k_cache, vt_cache) and of the rest into
    (k_cache2, vt_cache2), one launch."""
    Nb = proj.shape[0] - Na
    _call("cujev_op_attn_prep_pair", _ptr(proj), proj.stride(0), _ptr(q_norm_w), _ptr(k_norm_w),
          _ptr(pos), int(Na), int(Nb), Hq, Hkv, rot, _ptr(rope), float(eps), float(q_scale),
          _ptr(q_out), _ptr(k_cache), _ptr(vt_cache), cache_stride, _ptr(k_cache2),
          _ptr(vt_cache2), cache_stride2, _stream())


def attention_ws_bytes(N, Hq, Hkv, P) -> int:
    return int(load().cujev_ops_attention_ws_bytes(int(N), int(Hq), int(Hkv), int(P)))


def attention(q, gate, gate_tok_stride, gate_head_stride, pk, pvt, P, p_stride, ok, ovt,
              o_stride, own_base, Hq, Hkv, out, ws=None):
    """ws: optional uint8 device workspace (attention_ws_bytes) that lets a
    few-workgroup shape split its key tiles."""
    N = q.shape[0]
    if ws is not None:
        _call("cujev_op_attention_ws", _ptr(q), _ptr(gate), gate_tok_stride, gate_head_stride,
              _ptr(pk), _ptr(pvt), int(P), p_stride, _ptr(ok), _ptr(ovt), o_stride,
              _ptr(own_base), N, Hq, Hkv, _ptr(out), _ptr(ws), ws.numel(), _stream())
        return
    _call("cujev_op_attention", _ptr(q), _ptr(gate), gate_tok_stride, gate_head_stride,
          _ptr(pk), _ptr(pvt), int(P), p_stride, _ptr(ok), _ptr(ovt), o_stride, _ptr(own_base),
          N, Hq, Hkv, _ptr(out), _stream())


def attention_pair(q, gate, gate_tok_stride, gate_head_stride, pk, pvt, p_stride, own_base, Hq,
                   Hkv, out, Na, Pa, oka, ovta, oa_stride, Pb, okb, ovtb, ob_stride):
    """Two problems in one launch: rows [0, Na) of q / gate / own_base / out
    over the state's first Pa keys and own keys (oka, ovta), the remaining
    rows over Pb keys and (okb, ovtb)."""
    Nb = q.shape[0] - Na
    _call("cujev_op_attention_pair", _ptr(q), _ptr(gate), gate_tok_stride, gate_head_stride,
          _ptr(pk), _ptr(pvt), p_stride, _ptr(own_base), _ptr(out), Hq, Hkv, int(Na), int(Pa),
          _ptr(oka), _ptr(ovta), oa_stride, int(Nb), int(Pb), _ptr(okb), _ptr(ovtb), ob_stride,
          _stream())


def attention_noalloc(q, gate, gate_tok_stride, gate_head_stride, pk, pvt, P, p_stride, ok, ovt,
                      o_stride, own_base, Hq, Hkv, out):
    """attention_ws with the key-split partials in the library's static
    per-GPU scratch (no allocation by the call)."""
    N = q.shape[0]
    _call("cujev_op_attention_noalloc", _ptr(q), _ptr(gate), gate_tok_stride, gate_head_stride,
          _ptr(pk), _ptr(pvt), int(P), p_stride, _ptr(ok), _ptr(ovt), o_stride, _ptr(own_base),
          N, Hq, Hkv, _ptr(out), _stream())


def gdn_conv_prep(proj, conv_w, conv_in, conv_out, seg0_len, own_base, A_neg_exp, dt_bias,
                  Hk, Hv, q, k, v, g, beta):
    N = proj.shape[0]
    _call("cujev_op_gdn_conv_prep", _ptr(proj), proj.stride(0), _ptr(conv_w), _ptr(conv_in),
          _ptr(conv_out), int(seg0_len), _ptr(own_base), _ptr(A_neg_exp), _ptr(dt_bias), N, Hk,
          Hv, _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _stream())


def packed_chunk_table(seg_lens, chunk=64):
    """Host-side table of whole segments packed into chunks of at most `chunk`
    tokens (consecutive segments while they fit), with the per-chunk bit mask
    of segment starts. Every segment must fit one chunk. Returns chunk_tok0,
    chunk_len (int32) and chunk_starts (uint64 bits in an int64 array)."""
    import numpy as np
    tok0, clen, starts = [], [], []
    start = 0
    for L in seg_lens:
        if L > chunk:
            raise ValueError("packed_chunk_table: segment longer than a chunk")
        if L <= 0:
            continue
        if not tok0 or clen[-1] + L > chunk:
            tok0.append(start)
            clen.append(0)
            starts.append(0)
        starts[-1] |= 1 << clen[-1]
        clen[-1] += L
        start += L
    as_i = lambda x: np.asarray(x, dtype=np.int32)
    return as_i(tok0), as_i(clen), np.asarray(starts, dtype=np.uint64).view(np.int64)


def chunk_table(seg_lens, chunk=64):
    """Host-side chunk table: every segment cut into `chunk`-token pieces."""
    import numpy as np
    tok0, clen, seg0, segn = [], [], [], []
    start = 0
    for L in seg_lens:
        seg0.append(len(tok0))
        n = 0
        for c in range(0, L, chunk):
            tok0.append(start + c)
            clen.append(min(chunk, L - c))
            n += 1
        segn.append(n)
        start += L
    as_i = lambda x: np.asarray(x, dtype=np.int32)
    return as_i(tok0), as_i(clen), as_i(seg0), as_i(segn)


def gdn_scratch_bytes(num_chunks, Hv, N):
    return int(load().cujev_ops_gdn_scratch_bytes(int(num_chunks), int(Hv), int(N)))


def gdn_scan(q, k, v, g, beta, chunk_tok0, chunk_len, seg_chunk0, seg_nchunk, S_in, S_out, z,
             z_stride, norm_w, eps, Hk, Hv, y, scratch, max_seg_chunks=0, chunk_starts=None):
    """max_seg_chunks: the largest seg_nchunk entry when the caller knows it
    (0 = not given); 1 with S_out None takes the branch path. chunk_starts
    (int64 device tensor from packed_chunk_table, seg_chunk0 / seg_nchunk then
    None) packs whole segments into chunks."""
    nseg = seg_chunk0.shape[0] if seg_chunk0 is not None else 0
    _call("cujev_op_gdn_scan", _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(chunk_tok0),
          _ptr(chunk_len), chunk_tok0.shape[0], _ptr(seg_chunk0), _ptr(seg_nchunk),
          nseg, int(max_seg_chunks), _ptr(chunk_starts), _ptr(S_in), _ptr(S_out), _ptr(z),
          int(z_stride), _ptr(norm_w), float(eps), Hk, Hv, q.shape[0], _ptr(y), _ptr(scratch),
          _stream())


def gdn_layer(proj, conv_w, conv_in, conv_out, seg0_len, own_base, A_neg_exp, dt_bias,
              chunk_tok0, chunk_len, seg_chunk0, seg_nchunk, S_in, S_out, norm_w, eps, Hk, Hv, y,
              scratch, max_seg_chunks=0, chunk_starts=None):
    """gdn_conv_prep + gdn_scan in one call (z from proj's columns after the
    conv channels); q, k, v, g, beta stay on chip."""
    N = proj.shape[0]
    nseg = seg_chunk0.shape[0] if seg_chunk0 is not None else 0
    _call("cujev_op_gdn_layer", _ptr(proj), proj.stride(0), _ptr(conv_w), _ptr(conv_in),
          _ptr(conv_out), int(seg0_len), _ptr(own_base), _ptr(A_neg_exp), _ptr(dt_bias),
          _ptr(chunk_tok0), _ptr(chunk_len), chunk_tok0.shape[0], _ptr(seg_chunk0),
          _ptr(seg_nchunk), nseg, int(max_seg_chunks), _ptr(chunk_starts), _ptr(S_in),
          _ptr(S_out), _ptr(norm_w), float(eps), Hk, Hv, N, _ptr(y), _ptr(scratch), _stream())


def gdn_recur(proj, conv_w, conv_in, A_neg_exp, dt_bias, chunk_tok0, chunk_len, seg_chunk0,
              max_seg_len, S_in, norm_w, eps, Hk, Hv, y, scratch):
    """The token-by-token fp32 path for eval branches (each <= 32 tokens, one
    chunk per segment): conv, gates, recurrence from S_in, gated norm."""
    N = proj.shape[0]
    _call("cujev_op_gdn_recur", _ptr(proj), proj.stride(0), _ptr(conv_w), _ptr(conv_in),
          _ptr(A_neg_exp), _ptr(dt_bias), _ptr(chunk_tok0), _ptr(chunk_len), _ptr(seg_chunk0),
          seg_chunk0.shape[0], int(max_seg_len), _ptr(S_in), _ptr(norm_w), float(eps), Hk, Hv, N,
          _ptr(y), _ptr(scratch), _stream())


_gemm_ws = None


def gemm(X, W, Y, f32out=False):
    """Y[N,M] = X[N,K] . W[M,K]^T (bf16 in, fp32 accumulate)."""
    import torch
    global _gemm_ws
    if _gemm_ws is None:
        _gemm_ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    N, K = X.shape
    M = W.shape[0]
    _call("cujev_op_gemm", _ptr(X), _ptr(W), _ptr(Y), int(bool(f32out)), N, M, K, _ptr(_gemm_ws),
          _gemm_ws.numel(), _stream())


def gemm_small_splits(M, K) -> int:
    return int(load().cujev_ops_gemm_small_splits(int(M), int(K)))


def gemm_small_tile(W):
    """The tiled copy of W [M, K] that gemm_small reads (same shape and dtype;
    the content is permuted into one 4 KiB block per 16 rows x 128 k)."""
    import torch
    Wt = torch.empty_like(W)
    M, K = W.shape
    _call("cujev_op_gemm_small_tile", _ptr(W), int(M), int(K), _ptr(Wt), _stream())
    return Wt


def gemm_small(X, W, Y=None, P=None, splits=1, gated=False, N=None, K=None):
    """Few-token GEMM: Y[N,M] = X[N,K] . W[M,K]^T (splits == 1, bf16 Y; gated:
    Y = act[N, M/2]) or fp32 partials P[splits][N][M] (splits > 1). W is the
    tiled copy from gemm_small_tile."""
    N = X.shape[0] if N is None else N
    K = W.shape[1] if K is None else K
    M = W.shape[0]
    _call("cujev_op_gemm_small", _ptr(X), X.stride(0), _ptr(W), int(N), int(M), int(K),
          int(bool(gated)), int(splits), _ptr(Y), Y.stride(0) if Y is not None else 0, _ptr(P),
          _stream())


def gemm_wide_plan(N, M, K, gated=False, max_splits=1):
    """(rg, ng, splits) the engine's planner picks for a prefill GEMM shape."""
    a, b, c = _I(), _I(), _I()
    if load().cujev_ops_gemm_wide_plan(int(N), int(M), int(K), int(bool(gated)), int(max_splits),
                                       C.byref(a), C.byref(b), C.byref(c)) != 0:
        raise OpsError(f"gemm_wide_plan: unsupported shape N={N} M={M} K={K}")
    return a.value, b.value, c.value


def gemm_wide(X, W, Y=None, P=None, splits=1, gated=False, rg=None, ng=None):
    """Prefill GEMM on the tiled W: Y[N,M] = X[N,K] . W[M,K]^T (bf16 Y; gated:
    Y = act[N, M/2]) or fp32 partials P[splits][N][M]. rg/ng default to the
    planner's tile for this shape and split count."""
    N, K = X.shape[0], W.shape[1]
    M = W.shape[0]
    if rg is None or ng is None:
        rg, ng, _ = gemm_wide_plan(N, M, K, gated, 1)
        if splits > 1:
            rg, ng, s = gemm_wide_plan(N, M, K, gated, splits)
            if s != splits:
                rg, ng = 2, 8
    _call("cujev_op_gemm_wide", _ptr(X), X.stride(0), _ptr(W), int(N), int(M), int(K),
          int(bool(gated)), int(rg), int(ng), int(splits), _ptr(Y),
          Y.stride(0) if Y is not None else 0, _ptr(P), _stream())


def add_rmsnorm(x, w, out, eps, y=None, yp=None, splits=0, rows=None):
    N, H = x.shape
    R = rows.shape[0] if rows is not None else 0
    _call("cujev_op_add_rmsnorm", _ptr(x), _ptr(y), _ptr(yp), int(splits), _ptr(w), _ptr(out),
          N, H, float(eps), _ptr(rows), R, _stream())


def blaslt_version() -> int:
    return load().cujev_ops_blaslt_version()


def gemm_tune(X, W, Y, f32out=False):
    """Exhaustive hipBLASLt search for Y = X W^T: (solution index, best us,
    heuristic us)."""
    import torch
    global _gemm_ws
    if _gemm_ws is None:
        _gemm_ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    N, K = X.shape
    M = W.shape[0]
    idx, best, heur = _I(0), C.c_float(0), C.c_float(0)
    lib = load()
    st = lib.cujev_op_gemm_tune(_ptr(X), _ptr(W), _ptr(Y), int(bool(f32out)), N, M, K,
                                _ptr(_gemm_ws), _gemm_ws.numel(), _stream(), C.byref(idx),
                                C.byref(best), C.byref(heur))
    if st != 0:
        raise OpsError(f"cujev_op_gemm_tune: status {st}: {lib.cujev_ops_last_error().decode()}")
    return idx.value, best.value, heur.value
