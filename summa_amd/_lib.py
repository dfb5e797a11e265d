"""ctypes binding of the C ABI in ``include/summa_amd.h``.

The library is the in-tree ``summa_amd/libsumma_amd.so`` built by
``summa_amd.build``. There is no fallback: if it is missing or fails to load,
every op raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

# SUMMA_AMD_LIB selects another build of the library (the AddressSanitizer
# build of the host code, python -m summa_amd.build --asan)
LIB_PATH = Path(os.environ.get("SUMMA_AMD_LIB",
                               Path(__file__).resolve().parent / "libsumma_amd.so"))

SM_OK = 0
SM_F32, SM_BF16, SM_F16, SM_F16X2 = 0, 1, 2, 3
(SM_EPI_STORE_F32, SM_EPI_STORE_BF16, SM_EPI_ADD_F32, SM_EPI_SWIGLU_BF16, SM_EPI_SWIGLU_F16,
 SM_EPI_SWIGLU_F16X2) = 0, 1, 2, 3, 4, 5

_lib = None


class GemvJob(C.Structure):
    """sm_q4_gemv_job (include/summa_amd.h)."""
    _fields_ = [("codes", C.c_void_p), ("scales", C.c_void_p), ("x", C.c_void_p),
                ("y", C.c_void_p), ("N", C.c_int64), ("K", C.c_int64),
                ("epilogue", C.c_int32), ("first_block", C.c_int32)]

vp, i32, i64, u64, f32, f64 = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_float, C.c_double

# name -> (restype, argtypes). Kept in the order of include/summa_amd.h.
SIGNATURES: dict[str, tuple] = {
    "sm_version": (i32, []),
    "sm_last_error": (C.c_char_p, []),
    "sm_ce_rows": (i32, [vp, i32, vp, i64, i64, i64, vp, vp, vp, f32, vp, vp, vp]),
    "sm_linear_cross_entropy_workspace_bytes": (i64, [i64, i64, i64, i64, i32]),
    "sm_linear_cross_entropy": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, i64, i32, vp, vp, vp,
                                      i64, vp]),
    "sm_linear_cross_entropy_backward": (i32, [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i32,
                                               vp, vp, vp, vp, i64, vp]),
    "sm_grpo_loss": (i32, [vp, vp, vp, vp, vp, i64, i64, i64, f64, f64, f64, vp, vp, vp, vp, vp]),
    "sm_grpo_flags_message": (C.c_char_p, [C.c_int32]),
    "sm_q4_quantize": (i32, [vp, i32, i64, vp, vp, vp, vp]),
    "sm_q4_pack": (i32, [vp, vp, i64, i64, vp, vp, vp]),
    "sm_q4_matmul": (i32, [vp, vp, i64, i64, vp, i32, i64, i64, vp, i64, i32, vp]),
    "sm_q4_matmul_workspace_bytes": (i64, [i64, i64, i64, i32]),
    "sm_q4_qkv_rope": (i32, [vp, vp, i64, i64, i64, i64, vp, i32, i64, i64, i64, vp, vp, i64, vp,
                             vp, vp, i32, vp]),
    "sm_q4_matmul_ws": (i32, [vp, vp, i64, i64, vp, i32, i64, i64, vp, i64, i32, vp, i64, vp]),
    "sm_q4_matmul_add_rmsnorm": (i32, [vp, vp, i64, i64, vp, i32, i64, i64, vp, vp, f32, vp, vp,
                                       i64, vp]),
    "sm_q4_matmul_add_rmsnorm_router": (i32, [vp, vp, i64, i64, vp, i32, i64, i64, vp, vp, f32,
                                              vp, vp, i64, vp, vp, vp, vp, i64, vp]),
    "sm_q4_noalloc_scratch_bytes": (i64, []),
    "sm_q4_matmul_noalloc": (i32, [vp, vp, i64, i64, vp, i32, i64, i64, vp, i64, i32, vp]),
    "sm_q4_gemv_multi_plan": (i64, [vp, i64, vp]),
    "sm_q4_gemv_multi": (i32, [vp, i64, vp, i64, i64, i32, vp]),
    "sm_gemm_f32": (i32, [vp, i64, i64, vp, i64, i64, vp, i64, i32, vp]),
    "sm_swiglu_f32": (i32, [vp, i64, i64, vp, vp]),
    "sm_embed": (i32, [vp, i32, vp, i64, i64, i64, f32, vp, vp]),
    "sm_rmsnorm": (i32, [vp, vp, i64, i64, f32, vp, i32, vp]),
    "sm_rope_append": (i32, [vp, vp, vp, i64, i64, i64, i64, i64, i64, vp, i32, vp, vp, i32, vp]),
    "sm_attn_decode": (i32, [vp, vp, vp, vp, vp, i32, i32, i64, i64, i64, i64, i64, vp]),
    "sm_attn_decode_prefix_workspace_bytes": (i64, [i64, i64, i64, i64, i64, i64]),
    "sm_attn_decode_prefix": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, i64, i32, i32, i64, i64, i64,
                                    i64, i64, i64, i64, vp]),
    "sm_attn_prefill": (i32, [vp, vp, vp, vp, vp, i32, i32, i64, i64, i64, i64, i64, i64, vp]),
    "sm_attn_prefill_lse": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, i64, i64, i64, i64, i64, i64, vp]),
    "sm_attention": (i32, [vp, vp, vp, i32, i64, i64, i64, i64, i64, i32, vp, vp, vp]),
    "sm_attention_backward": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i32, vp, vp,
                                    vp, vp, vp]),
    "sm_sample": (i32, [vp, i64, i64, i64, f32, u64, i64, vp, i64, vp, i64, vp, vp]),
    "sm_sample_ex": (i32, [vp, i64, i64, i64, vp, u64, i64, vp, i64, vp, vp, vp, i64, vp, i64, vp,
                           vp]),
    "sm_seen_tokens": (i32, [vp, i64, i64, i64, i64, vp, i64, i32, vp]),
    "sm_moe_plan_words": (i64, [i64, i64, i64]),
    "sm_moe_router_top2": (i32, [vp, i32, vp, i64, i64, i64, vp, vp, vp, vp]),
    "sm_moe_route_plan": (i32, [vp, i64, i64, i64, vp, vp, vp]),
    "sm_moe_route_plan_logits": (i32, [vp, i64, i64, vp, vp, vp, vp, vp]),
    "sm_q4_grouped_matmul": (i32, [vp, vp, i64, i64, i64, vp, i32, i64, i32, vp, i64, i64, vp, i64,
                                   i32, vp]),
    "sm_moe_combine": (i32, [vp, vp, vp, i64, i64, i64, i64, vp, vp]),
    "sm_moe_combine_rmsnorm": (i32, [vp, vp, vp, i64, i64, i64, i64, vp, vp, f32, vp, vp]),
    "sm_moe_gather": (i32, [vp, i32, vp, i64, i64, i64, i64, vp, vp]),
    "sm_moe_gather_backward": (i32, [vp, i32, vp, i64, i64, i64, i64, vp, vp]),
    "sm_moe_combine_backward": (i32, [vp, vp, i32, vp, vp, i64, i64, i64, i64, vp, vp, vp]),
    "sm_swiglu": (i32, [vp, i32, i64, i64, vp, vp]),
    "sm_swiglu_backward": (i32, [vp, vp, i32, i64, i64, vp, vp]),
    "sm_gemm_ex": (i32, [i32, i32, i64, i64, i64, f32, vp, i64, vp, i64, f32, vp, i64, vp]),
    "sm_gemm_mfma": (i32, [i32, i32, i64, i64, i64, f32, vp, i64, vp, i64, f32, vp, i64, vp]),
    "sm_gemm_planes": (i32, [i32, i32, i32, i64, i64, i64, f32, vp, i64, vp, i64, f32, vp, i64,
                             vp]),
    "sm_gemm_planes_scratch_bytes": (i64, [i32, i32, i64, i64, i64]),
    "sm_gemm_planes_ws": (i32, [i32, i32, i32, i32, i64, i64, i64, f32, vp, i64, vp, i64, f32, vp,
                                i64, vp, i64, vp]),
    "sm_rmsnorm_backward": (i32, [vp, vp, vp, i64, i64, f32, i32, vp, vp, vp, vp]),
    "sm_rope_qk": (i32, [vp, vp, vp, i64, i64, i64, i64, i64, i32, vp]),
    "sm_attn_backward_f32": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, vp, vp, vp, vp,
                                   vp]),
    "sm_attn_backward_bf16ops": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, vp, vp, vp,
                                       vp, vp]),
    "sm_attn_prefill_lse_bf16ops": (i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, i64,
                                          vp]),
    "sm_embed_backward": (i32, [vp, vp, i64, i64, i64, vp, vp]),
    "sm_adamw_step": (i32, [vp, vp, vp, vp, i64, f32, f32, f32, f32, f32, i64, vp]),
    "sm_muon_momentum": (i32, [vp, vp, vp, i64, f32, i32, vp]),
    "sm_axpby": (i32, [vp, vp, i64, f32, f32, vp]),
    "sm_frobenius_normalize": (i32, [vp, i64, f32, vp, vp]),
    "sm_model_create": (i32, [vp, vp]),
    "sm_model_destroy": (i32, [vp]),
    "sm_model_weight_bytes": (i64, [vp]),
    "sm_model_set_tensor": (i32, [vp, i32, i32, vp, vp]),
    "sm_model_trace_routes": (i32, [vp, vp, vp, i64]),
    "sm_model_route_trace_count": (i32, [vp, vp, vp]),
    "sm_fnv1a64": (u64, [vp, i64]),
    "sm_hquant_parse": (i32, [vp, i64, vp]),
    "sm_hquant_bytes": (i64, [vp]),
    "sm_hquant_write": (i32, [vp, vp, i64, vp]),
    "sm_hquant_decode": (i32, [vp, vp, i32, vp]),
    "sm_model_load_packed": (i32, [vp, i32, i32, vp, i32, vp]),
    "sm_model_init_random": (i32, [vp, u64, f32, vp]),
    "sm_rl_workspace_bytes": (i64, [vp, i64, i64, i64, i64]),
    "sm_model_bind_workspace": (i32, [vp, vp, i64, i64, i64, i64, i64]),
    "sm_model_set_prompt_groups": (i32, [vp, i64]),
    "sm_rl_generate": (i32, [vp, vp, i64, i64, i64, f32, u64, vp, vp, vp]),
    "sm_rl_generate_ex": (i32, [vp, vp, i64, i64, i64, vp, u64, vp, vp, vp, vp]),
    "sm_completion_mask": (i32, [vp, i64, i64, vp, vp]),
    "sm_rl_logprobs": (i32, [vp, vp, vp, i64, i64, i64, i64, vp, vp]),
    "sm_rl_prepare": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, f64, f64, f64, i64,
                            vp, vp, vp, vp, vp, vp]),
    "sm_row_permute": (i32, [vp, i32, i64, i64, vp, vp, vp]),
    "sm_grouped_linear": (i32, [vp, vp, vp, i64, i64, i64, i64, vp, vp]),
    "sm_grouped_linear_backward": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, vp, vp, vp]),
    "sm_grouped_swiglu_mlp": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, i64, vp, vp, vp, vp]),
    "sm_grouped_swiglu_mlp_backward": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, i64, vp, vp, vp,
                                             vp, vp, vp, vp, vp]),
    "sm_policy_create": (i32, [vp, vp, vp]),
    "sm_policy_destroy": (i32, [vp]),
    "sm_policy_set_matmul_planes": (i32, [vp, i32]),
    "sm_policy_set_tensor": (i32, [vp, i32, i32, vp, vp]),
    "sm_policy_get_tensor": (i32, [vp, i32, i32, vp, i32, vp]),
    "sm_policy_install": (i32, [vp, vp, vp]),
    "sm_policy_prepare": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, f64, f64, f64,
                                vp, vp, vp, vp, vp, vp]),
    "sm_policy_prepare_with_ref": (i32, [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, f64, f64,
                                         f64, vp, vp, vp, vp, vp]),
    "sm_policy_optimizer_step": (i32, [vp, f64, vp, vp]),
    "sm_fill_normal": (i32, [vp, i32, i64, f32, f32, u64, vp]),
    "sm_fill_ce_stress": (i32, [vp, i32, vp, i64, i64, f32, f32, u64, vp]),
}


class SummaError(RuntimeError):
    """Raised when a C-ABI call returns a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m summa_amd.build` (no CPU fallback exists)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != SM_OK:
        msg = lib().sm_last_error().decode(errors="replace")
        raise SummaError(status, msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
