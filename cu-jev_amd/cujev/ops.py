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
    "cujev_op_attn_prep": [_P, _I, _P, _P, _P, _I, _I, _I, _I, _D, _F, _F, _P, _P, _P, _I, _P],
    "cujev_op_attention": [_P, _P, _I, _I, _P, _P, _I, _I, _P, _P, _I, _P, _I, _I, _I, _P, _P],
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
    for name, args in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _I
    _lib = lib
    return lib


def exported_symbols():
    return ["cujev_ops_kv_stride", "cujev_ops_last_error", *_SIGS]


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


def attn_prep(proj, q_norm_w, k_norm_w, pos, Hq, Hkv, rot, theta, eps, q_scale,
              q_out, k_cache, vt_cache, cache_stride):
    N = proj.shape[0]
    _call("cujev_op_attn_prep", _ptr(proj), proj.stride(0), _ptr(q_norm_w), _ptr(k_norm_w),
          _ptr(pos), N, Hq, Hkv, rot, float(theta), float(eps), float(q_scale), _ptr(q_out),
          _ptr(k_cache), _ptr(vt_cache), cache_stride, _stream())


def attention(q, gate, gate_tok_stride, gate_head_stride, pk, pvt, P, p_stride, ok, ovt,
              o_stride, own_base, Hq, Hkv, out):
    N = q.shape[0]
    _call("cujev_op_attention", _ptr(q), _ptr(gate), gate_tok_stride, gate_head_stride,
          _ptr(pk), _ptr(pvt), int(P), p_stride, _ptr(ok), _ptr(ovt), o_stride, _ptr(own_base),
          N, Hq, Hkv, _ptr(out), _stream())
