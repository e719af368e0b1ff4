"""The C-ABI library loads (no GPU needed) and exports every function
include/llamd_hip.h declares; the Python binding covers all of them."""
import re
from pathlib import Path

from llamd_rs_amd import _lib

ROOT = Path(__file__).resolve().parent.parent


def declared():
    text = (ROOT / "include" / "llamd_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(llamd_\w+)\s*\(", text)))


def test_header_declares_the_reference_names():
    names = declared()
    for ref in ["llamd_rocm_device_count", "llamd_rocm_device_info", "llamd_rocm_free_mem",
                "llamd_rocm_upload", "llamd_rocm_release", "llamd_rocm_matvec_q6k_resident",
                "llamd_rocm_matvec_grouped", "llamd_rocm_matvec_grouped_bench",
                "llamd_rocm_quantize_q8k", "llamd_rocm_matvec_bench", "llamd_fwd_matvec",
                "llamd_fwd_matvec_grouped", "llamd_fwd_matvec_grouped_pa", "llamd_fwd_quantize",
                "llamd_fwd_router", "llamd_fwd_silu_mul", "llamd_fwd_moe_combine_add",
                "llamd_fwd_argmax", "llamd_fwd_matvec_f32", "llamd_fwd_sync"]:
        assert ref in names, ref


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    missing = [n for n in declared() if not hasattr(L, n)]
    assert not missing, missing


def test_binding_covers_the_header():
    missing = [n for n in declared() if n not in _lib.SIGNATURES]
    assert not missing, missing


def test_no_device_calls_fail_cleanly():
    """Without a GPU (this container) the inventory reports zero devices."""
    import os
    if os.path.exists("/dev/kfd"):
        return
    assert _lib.lib().llamd_rocm_device_count() == 0


# ---- link compatibility with the reference's llamd-rocm crate ----------------
# tests/golden/llamd_rocm_ffi.json holds every function the reference binds in
# crates/llamd-rocm/src/{lib,forward,batch,udot}.rs (make_ffi_fixture.py).

def _ffi():
    import json
    return json.loads((ROOT / "tests" / "golden" / "llamd_rocm_ffi.json").read_text())


def _rust_kind(t: str) -> str:
    t = t.strip()
    if t.startswith("*"):
        inner = t.split()[-1].split("::")[-1]
        return "ptr:" + {"c_void": "void", "c_char": "i8", "i8": "i8", "u8": "u8", "f32": "f32",
                         "i32": "i32", "c_int": "i32", "usize": "usize", "i16": "i16"}[inner]
    return {"c_int": "i32", "i32": "i32", "usize": "usize", "f32": "f32", "()": "void"}[t]


def _c_kind(t: str) -> str:
    t = t.replace("const", "").strip()
    if "*" in t:
        base = t.replace("*", "").strip()
        return "ptr:" + {"void": "void", "char": "i8", "int8_t": "i8", "uint8_t": "u8",
                         "float": "f32", "int32_t": "i32", "int": "i32", "size_t": "usize",
                         "int16_t": "i16"}[base]
    return {"int": "i32", "size_t": "usize", "float": "f32", "void": "void"}[t]


def _header_decls():
    text = (ROOT / "include" / "llamd_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"^[ \t]*((?:const\s+)?\w+[\s\*]*?)\b(llamd_\w+)\s*\(([^;{]*?)\)\s*;", text,
                         re.S | re.M):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        ps = [] if params.strip() in ("", "void") else [p.strip() for p in params.split(",")]
        # drop the parameter name (and array brackets): keep the type
        types = [re.sub(r"\[.*?\]", "*", re.sub(r"\b\w+\s*(\[.*?\])?$", r"\1", p)).strip() for p in ps]
        decls[name] = (ret.strip(), types)
    return decls


def test_every_reference_ffi_symbol_is_exported():
    L = _lib.lib()
    missing = sorted(n for n in _ffi() if not hasattr(L, n))
    assert not missing, missing


def test_reference_ffi_signatures_match_the_header():
    decls = _header_decls()
    bad = []
    for name, ref in _ffi().items():
        assert name in decls, f"{name} ({ref['file']}) is not declared in include/llamd_hip.h"
        ret, types = decls[name]
        want = [_rust_kind(t) for t in ref["params"]]
        got = [_c_kind(t) for t in types]
        ret_c = _c_kind(ret.replace("*", "").strip()) if "*" not in ret else "ptr:void"
        ret_r = _rust_kind(ref["ret"])
        if got != want or ret_c != ret_r:
            bad.append((name, ref["file"], want, got, ret_r, ret_c))
    assert not bad, bad
