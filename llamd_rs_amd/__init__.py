"""llamd_rs_amd -- MI355X (gfx950) implementation of llamd.rs's quantized
matmul hot path: Q6_K / Q8_0 matvecs, the expert-grouped Q6_K GEMM, and the
MoE route -> experts -> SwiGLU -> combine step, behind the C ABI in
include/llamd_hip.h. `rocm` mirrors the reference's llamd-rocm wrappers.
"""
from ._lib import HipError, HipUnavailable  # noqa: F401
