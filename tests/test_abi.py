"""The drop-in boundary on the CPU: both libraries load, export exactly what
include/cujev.h and include/cujev_ops.h declare, the ctypes mirrors have the C
sizes, and every error the reference raises before touching a device
(REF src/api/cujev.c:20-33 then src/core/config.c:42-133) comes back with the
same status code. No compute call is made here."""
import ctypes as C
import json
import re
import subprocess
from pathlib import Path

import pytest

from cujev import _lib as L
from cujev import synthetic

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "cu-jev_amd" / "cujev" / "libcujev.so"
OPS = ROOT / "cu-jev_amd" / "cujev" / "libcujev_ops.so"


def declared(header):
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(cujev_\w+)\s*\(", text)) - {"cujev_status"}


def exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True,
                         check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


def test_public_library_exports_exactly_the_abi():
    assert declared("cujev.h") == set(L.PUBLIC_SYMBOLS)
    assert exported(LIB) == set(L.PUBLIC_SYMBOLS)


def test_ops_library_exports_its_header():
    from cujev import ops
    assert exported(OPS) == declared("cujev_ops.h") == set(ops.exported_symbols())
    ops.load()  # binds every symbol with its argtypes


def test_struct_layouts_match_c():
    assert C.sizeof(L._Options) == 24
    assert C.sizeof(L._Info) == 112
    assert C.sizeof(L._Branch) == 32
    assert C.sizeof(L._Timing) == 20
    assert L._Info.device_bytes_weights.offset == 96


def test_options_default_status_strings_version():
    lib = L._load()
    o = L._Options()
    lib.cujev_options_default(C.byref(o))
    assert (o.device, o.max_state_tokens, o.max_branch_tokens, o.max_branches,
            o.max_candidates, o.verbose) == (0, 8192, 4096, 256, 256, 0)
    assert lib.cujev_status_string(0) == b"ok"
    assert lib.cujev_status_string(6) == b"capacity exceeded"
    assert lib.cujev_status_string(99) == b"unknown"
    assert lib.cujev_version() == b"0.1.0"


def open_status(path):
    lib = L._load()
    m = C.c_void_p()
    st = lib.cujev_model_open(str(path).encode() if path is not None else None, None, C.byref(m))
    assert not m.value
    return st, lib.cujev_last_error().decode()


def write_cfg(tmp_path, **changes):
    cfg = synthetic.make_config(**synthetic.PRESETS["tiny"])
    cfg.update(changes)
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    return tmp_path


def test_open_errors_before_any_device_call(tmp_path):
    assert open_status(None)[0] == 1                                  # INVALID_ARGUMENT
    assert open_status(tmp_path / "missing")[0] == 2                  # IO
    (tmp_path / "config.json").write_text("{not json")
    st, msg = open_status(tmp_path)
    assert st == 3 and "JSON" in msg                                  # FORMAT
    st, msg = open_status(write_cfg(tmp_path, model_type="llama"))
    assert st == 7 and "qwen3_5" in msg                               # UNSUPPORTED
    assert open_status(write_cfg(tmp_path, head_dim=128))[0] == 7
    assert open_status(write_cfg(tmp_path, num_attention_heads=6, num_key_value_heads=1))[0] == 7
    assert open_status(write_cfg(tmp_path, linear_conv_kernel_dim=3))[0] == 7
    assert open_status(write_cfg(tmp_path, linear_key_head_dim=64))[0] == 7
    st, msg = open_status(write_cfg(tmp_path, layer_types=["linear_attention"]))
    assert st == 3 and "layer_types" in msg
    assert open_status(write_cfg(tmp_path, layer_types=["full_attention"] * 3 + ["moe"]))[0] == 7
    cfg = synthetic.make_config(**synthetic.PRESETS["tiny"])
    del cfg["hidden_size"]
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    assert open_status(tmp_path)[0] == 3


def test_text_config_nesting_and_rope_defaults(tmp_path):
    """A multimodal config keeps the text model under text_config; a valid
    config with no weights fails on the checkpoint (IO), i.e. after parsing."""
    cfg = synthetic.make_config(**synthetic.PRESETS["tiny"])
    (tmp_path / "config.json").write_text(json.dumps({"model_type": "qwen3_5",
                                                      "text_config": cfg}))
    st, msg = open_status(tmp_path)
    assert st in (2, 4), msg  # no *.safetensors (or no device on this host)


def test_engine_error_surface():
    with pytest.raises(L.EngineError):
        L.Engine("/nonexistent/checkpoint")
