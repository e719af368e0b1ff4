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
