"""Loader for libllamd_hip.so (built in-tree by llamd_rs_amd/build.py).

The product path has no fallback: if the library is missing, every entry
point raises HipUnavailable instead of computing anything on the CPU.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libllamd_hip.so"


class HipUnavailable(RuntimeError):
    """The HIP library is not built, or no ROCm device is visible."""


class HipError(RuntimeError):
    """A C-ABI call returned -1 / NULL; the message is the library's."""


_lib = None

vp, i32, sz, f32p, i8p, i16p, i32p, u8p, u16, u32, u64, f = (
    C.c_void_p, C.c_int, C.c_size_t, C.POINTER(C.c_float), C.POINTER(C.c_int8),
    C.POINTER(C.c_int16), C.POINTER(C.c_int32), C.POINTER(C.c_uint8), C.c_uint16, C.c_uint32,
    C.c_uint64, C.c_float)
dp = C.POINTER(C.c_double)
cp = C.c_char_p

# name: (restype, argtypes) for every symbol of include/llamd_hip.h and the
# host-side synthetic-data helpers.
SIGNATURES = {
    "llamd_rocm_device_count": (i32, []),
    "llamd_rocm_device_info": (i32, [i32, cp, i32, cp, i32, C.POINTER(sz), i32p, i32p]),
    "llamd_rocm_free_mem": (sz, []),
    "llamd_hip_last_error": (cp, []),
    "llamd_hip_tune": (i32, [cp, i32]),
    "llamd_rocm_upload": (vp, [vp, sz]),
    "llamd_rocm_release": (None, [vp]),
    "llamd_fwd_get_stream": (vp, []),
    "llamd_fwd_stream_init": (i32, []),
    "llamd_fwd_begin_capture": (i32, []),
    "llamd_fwd_end_capture": (i32, []),
    "llamd_fwd_graph_launch": (i32, []),
    "llamd_fwd_has_graph": (i32, []),
    "llamd_fwd_graph_destroy": (None, []),
    "llamd_fwd_alloc": (vp, [sz]),
    "llamd_fwd_free": (None, [vp]),
    "llamd_fwd_upload": (i32, [vp, vp, sz]),
    "llamd_fwd_download": (i32, [vp, vp, sz]),
    "llamd_fwd_sync": (i32, []),
    "llamd_fwd_last_error": (i32, []),
    "llamd_hip_q6k_tiled_bytes": (sz, [i32, i32]),
    "llamd_hip_q6k_tile": (i32, [vp, i32, i32, vp]),
    "llamd_hip_q6k_untile": (i32, [vp, i32, i32, vp]),
    "llamd_hip_q8_0_planar_bytes": (sz, [i32, i32]),
    "llamd_hip_q8_0_planarize": (i32, [vp, i32, i32, vp]),
    "llamd_rocm_upload_q6k": (vp, [vp, i32, i32]),
    "llamd_rocm_upload_q6k_experts": (vp, [vp, i32, i32, i32]),
    "llamd_hip_upload_q8_0": (vp, [vp, i32, i32]),
    "llamd_rocm_matvec_q6k_resident": (i32, [vp, vp, vp, vp, i32, i32]),
    "llamd_rocm_matvec_grouped": (i32, [vp, vp, vp, vp, vp, i32, i32, i32]),
    "llamd_hip_matvec_grouped_pa": (i32, [vp, vp, vp, vp, vp, i32, i32, i32]),
    "llamd_hip_matvec_q6k_batched": (i32, [vp, vp, vp, vp, i32, i32, i32]),
    "llamd_rocm_quantize_q8k": (i32, [vp, i32, vp, vp, vp]),
    "llamd_hip_swiglu_q8k": (i32, [vp, vp, i32, vp, vp, vp, vp]),
    "llamd_hip_dequant_q6k": (i32, [vp, i32, i32, vp]),
    "llamd_hip_dequant_q8_0": (i32, [vp, i32, i32, vp]),
    "llamd_hip_matvec_q8_0": (i32, [vp, vp, vp, i32, i32]),
    "llamd_hip_route": (i32, [vp, i32, i32, vp, vp]),
    "llamd_hip_argmax": (i32, [vp, i32, i32, vp]),
    "llamd_fwd_matvec": (None, [vp, vp, vp, vp, i32, i32]),
    "llamd_fwd_matvec_grouped": (None, [vp, vp, vp, vp, vp, i32, i32, i32]),
    "llamd_fwd_matvec_grouped_pa": (None, [vp, vp, vp, vp, vp, i32, i32, i32]),
    "llamd_fwd_matvec_x3": (None, [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32]),
    "llamd_fwd_matvec_x3_splitk": (None, [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32]),
    "llamd_fwd_matvec_grouped_x2": (None, [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32]),
    "llamd_fwd_matvec_grouped_x2_splitk": (None, [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32]),
    "llamd_fwd_matvec_grouped_pa_splitk": (None, [vp, vp, vp, vp, vp, i32, i32, i32, i32]),
    "llamd_fwd_moe_combine": (None, [vp, vp, vp, i32, i32]),
    "llamd_fwd_rms_norm_mul": (None, [vp, vp, vp, i32, f]),
    "llamd_fwd_head_rms_norm_mul": (None, [vp, vp, vp, i32, i32, f]),
    "llamd_fwd_rms_norm_quant": (None, [vp, vp, vp, vp, vp, vp, i32, f]),
    "llamd_fwd_quantize": (None, [vp, vp, vp, i32]),
    "llamd_fwd_silu_mul": (None, [vp, vp, vp, i32]),
    "llamd_fwd_router": (None, [vp, i32, i32, vp, vp, vp]),
    "llamd_fwd_moe_combine_add": (None, [vp, vp, vp, vp, i32, i32]),
    "llamd_fwd_argmax": (None, [vp, i32, vp, vp, vp, i32]),
    "llamd_fwd_matvec_f32": (None, [vp, vp, vp, i32, i32]),
    "llamd_hip_fwd_matvec_q8_0": (None, [vp, vp, vp, i32, i32]),
    "llamd_hip_moe_create": (vp, [vp, vp, vp, vp, i32, i32, i32, i32]),
    "llamd_hip_moe_destroy": (None, [vp]),
    "llamd_hip_moe_forward": (i32, [vp, vp, vp, vp, i32]),
    "llamd_hip_moe_forward_host": (i32, [vp, vp, vp, vp, vp, vp, vp, i32]),
    "llamd_hip_moe_prefill": (i32, [vp, vp, vp, vp, vp, i32]),
    "llamd_hip_moe_prefill_host": (i32, [vp, vp, vp, vp, vp, i32]),
    "llamd_hip_moe_prefill_ex": (i32, [vp, vp, vp, vp, vp, i32, i32]),
    "llamd_hip_moe_prefill_host_ex": (i32, [vp, vp, vp, vp, vp, i32, i32]),
    "llamd_hip_moe_stats": (i32, [vp, i32p, i32p]),
    "llamd_hip_moe_forward_batch": (i32, [vp, vp, vp, vp, i32]),
    "llamd_hip_moe_forward_batch_host": (i32, [vp, vp, vp, vp, vp, vp, vp, i32]),
    "llamd_hip_moe_counters": (i32, [vp, i32p, vp]),
    "llamd_gguf_open": (vp, [cp]),
    "llamd_gguf_close": (None, [vp]),
    "llamd_gguf_header": (i32, [vp, vp, vp, vp, vp, vp, vp]),
    "llamd_gguf_kv": (i32, [vp, u64, vp, sz, vp, vp, vp]),
    "llamd_gguf_find_kv": (C.c_int64, [vp, cp]),
    "llamd_gguf_kv_bits": (i32, [vp, u64, u64, vp]),
    "llamd_gguf_kv_str": (i32, [vp, u64, u64, vp, sz, vp]),
    "llamd_gguf_get_u64": (i32, [vp, cp, vp]),
    "llamd_gguf_get_f32": (i32, [vp, cp, vp]),
    "llamd_gguf_tensor": (i32, [vp, u64, vp, sz, vp, vp, vp, vp]),
    "llamd_gguf_find_tensor": (C.c_int64, [vp, cp]),
    "llamd_gguf_tensor_data": (vp, [vp, u64, vp]),
    "llamd_gguf_upload_q6k": (vp, [vp, cp]),
    "llamd_gguf_moe_create": (vp, [vp, i32]),
    "llamd_hip_model_create": (vp, [vp, i32]),
    "llamd_hip_model_destroy": (None, [vp]),
    "llamd_hip_model_info": (i32, [vp, i32p, i32p, i32p, i32p]),
    "llamd_hip_model_forward": (i32, [vp, i32, i32, vp, vp]),
    "llamd_hip_lmhead_create": (vp, [vp, i32, i32, i32]),
    "llamd_hip_lmhead_destroy": (None, [vp]),
    "llamd_hip_lmhead_forward": (i32, [vp, vp, i32, vp, vp]),
    "llamd_hip_lmhead_forward_ex": (i32, [vp, vp, i32, vp, vp, i32]),
    "llamd_hip_kernel_clock": (i32, [vp, i32]),
    "llamd_hip_lmhead_forward_noalloc": (i32, [vp, i32, i32, vp, i32, vp, vp]),
    "llamd_hip_lmhead_noalloc_scratch_bytes": (sz, []),
    "llamd_hip_event_create": (vp, []),
    "llamd_hip_event_destroy": (None, [vp]),
    "llamd_hip_event_record": (i32, [vp]),
    "llamd_hip_event_elapsed_ms": (f, [vp, vp]),
    "llamd_hip_copy_calibration": (i32, [vp, vp, sz]),
    "llamd_hip_read_many": (i32, [vp, sz, i32, i32]),
    "llamd_rocm_matvec_bench": (i32, [vp, vp, vp, i32, i32, i32, f32p]),
    "llamd_rocm_matvec_grouped_bench": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, f32p]),
    "llamd_fwd_memset": (i32, [vp, i32, sz]),
    "llamd_fwd_free_mem": (sz, []),
    "llamd_fwd_matvec_splitk": (None, [vp, vp, vp, vp, i32, i32, i32]),
    "llamd_rocm_splitk_bench": (i32, [vp, vp, vp, i32, i32, i32, i32, f32p]),
    "llamd_fwd_planar_matvec": (None, [vp, vp, vp, vp, vp, i32, i32]),
    "llamd_fwd_planar_grouped": (None, [vp, vp, vp, vp, vp, vp, i32, i32, i32]),
    "llamd_fwd_planar_grouped_pa": (None, [vp, vp, vp, vp, vp, vp, i32, i32, i32]),
    "llamd_fwd_planar_x3": (None, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32]),
    "llamd_fwd_planar_grouped_x2": (None, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32]),
    "llamd_rocm_planar_matvec": (i32, [vp, vp, vp, vp, vp, i32, i32]),
    "llamd_rocm_planar_bench": (i32, [vp, vp, vp, vp, i32, i32, i32, f32p]),
    "llamd_fwd_embed": (None, [vp, i32, vp, i32]),
    "llamd_fwd_embed_meta": (None, [vp, vp, vp, i32]),
    "llamd_fwd_rope": (None, [vp, i32, i32, i32, f]),
    "llamd_fwd_norm_rope": (None, [vp, vp, i32, i32, vp, f, f]),
    "llamd_fwd_k_norm_rope_store": (None, [vp, vp, vp, vp, vp, i32, i32, i32, vp, f, f]),
    "llamd_fwd_kv_store": (None, [vp, vp, vp, vp, i32, i32]),
    "llamd_fwd_attention": (None, [vp, vp, vp, vp, vp, i32, i32, i32, i32]),
    "llamd_fwd_attention_meta": (None, [vp, vp, vp, vp, vp, i32, i32, i32, vp, i32]),
    "llamd_fwd_add": (None, [vp, vp, vp, i32]),
    "llamd_batch_max_seq": (i32, []),
    "llamd_b_embed": (None, [vp, vp, vp, i32, i32]),
    "llamd_b_rms_norm_quant": (None, [vp, vp, vp, vp, vp, vp, i32, i32, f]),
    "llamd_b_rms_norm_mul": (None, [vp, vp, vp, i32, i32, f]),
    "llamd_b_quantize": (None, [vp, vp, vp, i32]),
    "llamd_b_matvec": (None, [vp, vp, vp, vp, i32, i32, i32]),
    "llamd_b_matvec_x3": (None, [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32]),
    "llamd_b_grouped_x2": (None, [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32]),
    "llamd_b_grouped_pa": (None, [vp, vp, vp, vp, vp, i32, i32, i32, i32]),
    "llamd_b_norm_rope": (None, [vp, vp, i32, i32, vp, i32, f, f]),
    "llamd_b_k_norm_rope_store": (None, [vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, i32, f, f]),
    "llamd_b_attention": (None, [vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, i32]),
    "llamd_b_add": (None, [vp, vp, vp, i32]),
    "llamd_b_silu_mul": (None, [vp, vp, vp, i32]),
    "llamd_b_matvec_f32": (None, [vp, vp, vp, i32, i32, i32]),
    "llamd_b_router": (None, [vp, i32, i32, vp, vp, vp, i32]),
    "llamd_b_moe_combine_add": (None, [vp, vp, vp, vp, i32, i32, i32]),
    "llamd_b_argmax": (None, [vp, i32, vp, vp, vp, i32, i32]),
    "llamd_u_set_tile": (None, [i32]),
    "llamd_u_get_tile": (i32, []),
    "llamd_u_bias_sums": (None, [vp, vp, vp, i32]),
    "llamd_u_norm_quant": (None, [vp, vp, vp, vp, vp, vp, vp, i32, i32, f]),
    "llamd_u_quantize": (None, [vp, vp, vp, vp, i32]),
    "llamd_u_matvec": (None, [vp, vp, vp, vp, vp, vp, i32, i32, i32]),
    "llamd_u_x3": (None, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32]),
    "llamd_u_grouped_x2": (None, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32]),
    "llamd_u_grouped_pa": (None, [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32]),
    "llamd_u_norm_quant_host": (i32, [vp, vp, i32, i32, f, vp, vp, vp, vp]),
    "llamd_u_quantize_host": (i32, [vp, i32, vp, vp, vp]),
    "llamd_u_matvec_host": (i32, [vp, vp, vp, vp, vp, i32, i32, i32]),
    "llamd_u_matvec_bench": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, f32p]),
    "llamd_hip_matvec_many": (i32, [vp, vp, vp, vp, vp, vp, i32]),
    "llamd_hip_be_rms_norm": (i32, [vp, vp, i32, i32, f]),
    "llamd_hip_be_softmax": (i32, [vp, vp, i32, i32]),
    "llamd_hip_be_silu": (i32, [vp, vp, sz]),
    "llamd_hip_be_add": (i32, [vp, vp, vp, sz]),
    "llamd_hip_be_mul": (i32, [vp, vp, vp, sz]),
    "llamd_hip_be_scale": (i32, [vp, f, vp, sz]),
    "llamd_hip_be_matmul": (i32, [vp, vp, vp, i32, i32, i32]),
    "llamd_hip_be_rope": (i32, [vp, i32, i32, vp, i32, f, f]),
    "llamd_hip_be_get_rows": (i32, [vp, i32, i32, vp, i32, vp]),
    # host-side synthetic data (llamd_rs_amd/csrc/host/synth.cpp)
    "llamd_synth_normal": (None, [u64, f, vp, sz]),
    "llamd_synth_f32_to_f16": (u16, [f]),
    "llamd_synth_quantize_q6k": (i32, [vp, sz, sz, vp]),
    "llamd_synth_quantize_q8_0": (i32, [vp, sz, sz, vp]),
    "llamd_synth_q6k_matrix": (i32, [u64, f, sz, sz, vp]),
    "llamd_synth_q8_0_matrix": (i32, [u64, f, sz, sz, vp]),
    "llamd_synth_zipf_routing": (i32, [u64, C.c_double, sz, sz, sz, vp, vp]),
}


def lib():
    """The loaded library; raises HipUnavailable if it was never built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise HipUnavailable(
                f"{LIB_PATH} is not built; run `python -m llamd_rs_amd.build` "
                "(there is no CPU fallback)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return (lib().llamd_hip_last_error() or b"").decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise HipError(f"{what}: {last_error()}")


def check_ptr(p, what: str):
    if not p:
        raise HipError(f"{what}: {last_error()}")
    return p
