"""ctypes binding of libcujev.so, written from include/cujev.h.

Public surface, the one callers of the reference's Python layer use
(python/cujev/_lib.py:61-238 there): ``Engine(checkpoint_dir, *, device=0,
max_state_tokens=8192, max_branch_tokens=4096, max_branches=256,
max_candidates=256, verbose=False)`` with ``prefill``, ``eval``,
``eval_full_logits``, ``last_timing``, ``close``, ``version``,
``state_tokens`` and the model-info attributes; ``Branch(tokens,
candidates)``; ``Timing``; ``EngineError``, raised for every non-zero
``cujev_status`` as ``"<call>: <status name>: <cujev_last_error()>"``.

Only the structure layouts below have to match the reference's mirrors
(python/cujev/_lib.py:17-59 there) byte for byte; they follow the C
declarations in include/cujev.h.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Sequence

import numpy as np


class EngineError(RuntimeError):
    """A libcujev call returned a non-zero cujev_status (or was misused)."""


# ---- C structures (include/cujev.h) ---------------------------------------
class _Options(C.Structure):  # cujev_options, 24 bytes
    _fields_ = [(name, C.c_int) for name in (
        "device", "max_state_tokens", "max_branch_tokens", "max_branches", "max_candidates",
        "verbose")]


class _Info(C.Structure):  # cujev_model_info, 112 bytes on LP64
    _fields_ = [("name", C.c_char * 64)] + [(name, C.c_int) for name in (
        "hidden_size", "num_layers", "num_full_attention_layers", "vocab_size",
        "max_state_tokens", "max_branch_tokens", "max_branches")] + [
        ("device_bytes_weights", C.c_size_t), ("device_bytes_workspace", C.c_size_t)]


_I32P = C.POINTER(C.c_int32)


class _Branch(C.Structure):  # cujev_branch, 32 bytes on LP64
    _fields_ = [("tokens", _I32P), ("num_tokens", C.c_int),
                ("candidates", _I32P), ("num_candidates", C.c_int)]


class _Timing(C.Structure):  # cujev_timing, 20 bytes
    _fields_ = [("prefill_ms", C.c_float), ("eval_ms", C.c_float),
                ("prefill_tokens", C.c_int), ("eval_tokens", C.c_int),
                ("eval_branches", C.c_int)]


_VP, _FP = C.c_void_p, C.POINTER(C.c_float)
_STATUS = C.c_int

# name -> (restype, argtypes), in header order
_PROTOTYPES = {
    "cujev_options_default": (None, [C.POINTER(_Options)]),
    "cujev_model_open": (_STATUS, [C.c_char_p, C.POINTER(_Options), C.POINTER(_VP)]),
    "cujev_model_close": (None, [_VP]),
    "cujev_model_info_get": (_STATUS, [_VP, C.POINTER(_Info)]),
    "cujev_state_create": (_STATUS, [_VP, C.POINTER(_VP)]),
    "cujev_state_destroy": (None, [_VP]),
    "cujev_state_prefill": (_STATUS, [_VP, _VP, _I32P, C.c_int]),
    "cujev_state_num_tokens": (C.c_int, [_VP]),
    "cujev_eval": (_STATUS, [_VP, _VP, C.POINTER(_Branch), C.c_int, _FP, C.c_int]),
    "cujev_eval_full_logits": (_STATUS, [_VP, _VP, C.POINTER(_Branch), C.c_int, _FP]),
    "cujev_last_timing": (None, [_VP, C.POINTER(_Timing)]),
    "cujev_status_string": (C.c_char_p, [C.c_int]),
    "cujev_last_error": (C.c_char_p, []),
    "cujev_version": (C.c_char_p, []),
}
PUBLIC_SYMBOLS = tuple(_PROTOTYPES)


def library_path() -> str:
    """CUJEV_LIBRARY if set, else the libcujev.so built next to this file."""
    override = os.environ.get("CUJEV_LIBRARY")
    if override:
        return override
    built = Path(__file__).resolve().with_name("libcujev.so")
    if built.is_file():
        return str(built)
    raise EngineError(f"{built} is missing: build it with `make -C cu-jev_amd` "
                      "(or point CUJEV_LIBRARY at a libcujev.so)")


class _Native:
    """The loaded library with every prototype declared, and a checked call
    that turns a non-zero status into EngineError."""

    _shared: "_Native | None" = None

    def __init__(self, path: str):
        self.dll = C.CDLL(path)
        for name, (res, args) in _PROTOTYPES.items():
            fn = getattr(self.dll, name)
            fn.restype, fn.argtypes = res, args

    @classmethod
    def get(cls) -> "_Native":
        if cls._shared is None:
            cls._shared = cls(library_path())
        return cls._shared

    def checked(self, name: str, *args, what: str | None = None) -> None:
        status = getattr(self.dll, name)(*args)
        if status:
            raise EngineError(f"{what or name}: {self.dll.cujev_status_string(status).decode()}: "
                              f"{self.dll.cujev_last_error().decode()}")


def _load():
    """The shared library handle (loaded on first use)."""
    return _Native.get().dll


# ---- Python-side values ----------------------------------------------------
@dataclass
class Branch:
    tokens: Sequence[int]
    candidates: Sequence[int]


@dataclass
class Timing:
    prefill_ms: float
    eval_ms: float
    prefill_tokens: int
    eval_tokens: int
    eval_branches: int


class _BranchBatch:
    """A list of Branch as one cujev_branch[B] whose token and candidate
    pointers index two contiguous int32 arrays this object keeps alive."""

    def __init__(self, branches: Sequence[Branch]):
        toks = [np.asarray(b.tokens, dtype=np.int32).ravel() for b in branches]
        cands = [np.asarray(b.candidates, dtype=np.int32).ravel() for b in branches]
        self.ncand = [len(c) for c in cands]
        self._tok = np.ascontiguousarray(np.concatenate(toks) if toks else np.zeros(0, np.int32))
        self._cand = np.ascontiguousarray(np.concatenate(cands) if any(self.ncand)
                                          else np.zeros(1, np.int32))
        self.array = (_Branch * len(branches))()
        t_addr, c_addr = self._tok.ctypes.data, self._cand.ctypes.data
        t_off = c_off = 0
        for slot, t, n_c in zip(self.array, toks, self.ncand):
            slot.tokens = C.cast(t_addr + 4 * t_off, _I32P)
            slot.num_tokens = len(t)
            slot.candidates = C.cast(c_addr + 4 * c_off, _I32P)
            slot.num_candidates = n_c
            t_off += len(t)
            c_off += n_c

    def __len__(self):
        return len(self.array)


def _as_f32p(a: np.ndarray):
    return a.ctypes.data_as(_FP)


class Engine:
    """One loaded model and one reusable state (the shared prefix)."""

    def __init__(self, checkpoint_dir: str | os.PathLike, *, device: int = 0,
                 max_state_tokens: int = 8192, max_branch_tokens: int = 4096,
                 max_branches: int = 256, max_candidates: int = 256, verbose: bool = False):
        self._native = _Native.get()
        self._lib = self._native.dll
        self._model, self._state = _VP(), _VP()
        opts = _Options(device=device, max_state_tokens=max_state_tokens,
                        max_branch_tokens=max_branch_tokens, max_branches=max_branches,
                        max_candidates=max_candidates, verbose=int(bool(verbose)))
        self._native.checked("cujev_model_open", os.fsencode(os.fspath(checkpoint_dir)),
                             C.byref(opts), C.byref(self._model), what="model_open")
        try:
            self._native.checked("cujev_state_create", self._model, C.byref(self._state),
                                 what="state_create")
            info = _Info()
            self._native.checked("cujev_model_info_get", self._model, C.byref(info),
                                 what="model_info")
        except EngineError:
            self.close()
            raise
        self.name = info.name.decode()
        for field in ("hidden_size", "num_layers", "num_full_attention_layers", "vocab_size",
                      "max_state_tokens", "max_branch_tokens", "max_branches"):
            setattr(self, field, getattr(info, field))
        self.max_candidates = max_candidates
        self.weight_bytes = info.device_bytes_weights
        self.workspace_bytes = info.device_bytes_workspace
        self._state_tokens: list[int] | None = None

    # -- lifetime ------------------------------------------------------------
    def close(self) -> None:
        """Frees the state and the model (idempotent)."""
        state, model = getattr(self, "_state", None), getattr(self, "_model", None)
        if state is not None and state.value:
            self._lib.cujev_state_destroy(state)
            self._state = _VP()
        if model is not None and model.value:
            self._lib.cujev_model_close(model)
            self._model = _VP()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def version(self) -> str:
        return self._lib.cujev_version().decode()

    # -- requests --------------------------------------------------------------
    def prefill(self, tokens: Sequence[int]) -> None:
        """Runs the shared prefix and keeps it as this engine's state."""
        ids = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).ravel())
        self._native.checked("cujev_state_prefill", self._model, self._state,
                             ids.ctypes.data_as(_I32P), int(ids.size), what="prefill")
        self._state_tokens = ids.tolist()

    @property
    def state_tokens(self) -> list[int] | None:
        return self._state_tokens

    def _need_state(self) -> None:
        if self._state_tokens is None:
            raise EngineError("prefill() first")

    def eval(self, branches: Sequence[Branch]) -> list[np.ndarray]:
        """Candidate logits at the last token of every branch (float32)."""
        self._need_state()
        batch = _BranchBatch(branches)
        ld = max(batch.ncand, default=0) or 1
        out = np.zeros((len(batch), ld), dtype=np.float32)
        self._native.checked("cujev_eval", self._model, self._state, batch.array, len(batch),
                             _as_f32p(out), ld, what="eval")
        return [out[i, :n].copy() for i, n in enumerate(batch.ncand)]

    def eval_full_logits(self, branches: Sequence[Branch]) -> np.ndarray:
        """[B, vocab] float32 logits at the last token of every branch (test path)."""
        self._need_state()
        batch = _BranchBatch(branches)
        out = np.zeros((len(batch), self.vocab_size), dtype=np.float32)
        self._native.checked("cujev_eval_full_logits", self._model, self._state, batch.array,
                             len(batch), _as_f32p(out), what="eval_full_logits")
        return out

    def last_timing(self) -> Timing:
        """GPU milliseconds of this model's last prefill and eval."""
        t = _Timing()
        self._lib.cujev_last_timing(self._model, C.byref(t))
        return Timing(float(t.prefill_ms), float(t.eval_ms), int(t.prefill_tokens),
                      int(t.eval_tokens), int(t.eval_branches))
