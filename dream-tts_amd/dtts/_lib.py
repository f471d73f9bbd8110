"""ctypes loader for libdtts.so and the call/raise plumbing.

torch is imported before the library is opened: torch ships its own HIP runtime
(``libamdhip64.so.7``) and the dynamic linker then resolves libdtts's dependency to that same
loaded copy, so device pointers and streams are shared. The product path has no fallback: a
missing or unloadable library raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  -- binds the HIP runtime before libdtts loads

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB_PATH = os.path.join(PKG, "libdtts.so")

_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F32 = ctypes.c_float
_F64 = ctypes.c_double
_P = ctypes.c_void_p
_SZ = ctypes.c_size_t

# name -> argtypes (restype is int unless listed in _RESTYPES)
SIGNATURES = {
    "dtts_last_error": [],
    "dtts_version": [],
    "dtts_init": [],
    "dtts_snake_ncl_f32": [_P, _P, _P, _P, _I64, _I64, _I64, _P],
    "dtts_snake_ncl_f16": [_P, _P, _P, _P, _I64, _I64, _I64, _P],
    "dtts_snake_nlc_f32": [_P, _P, _P, _P, _I64, _I64, _P],
    "dtts_snake_nlc_f16": [_P, _P, _P, _P, _I64, _I64, _P],
    "dtts_snake_folded_f32": [_P, _P, _I64, _P],
    "dtts_snake_alpha_f32": [_P, _P, _P, _I64, _I64, _I64, _P],
    "dtts_conv1d_nlc_f16_ex": [_P, _P],
    "dtts_conv1d_nlc_f32_ex": [_P, _P],
    "dtts_conv_split_weight_bytes": [_I64, _I64, _I64],
    "dtts_conv_split_weight": [_P, _I64, _I64, _I64, _P, _P, _P],
    "dtts_conv1d_nlc_f32_split_workspace_bytes": [_P],
    "dtts_conv1d_nlc_f32_split": [_P, _F32, _P, _SZ, _P],
    "dtts_causal_conv1d_nlc_f16": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "dtts_snake_conv_residual_nlc_f16": [_P, _P, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                         _I64, _P],
    "dtts_residual_unit_nlc_f16": [_P, _P],
    "dtts_residual_unit_supported": [_P],
    "dtts_conv1d_ncl_f32_ex": [_P, _P],
    "dtts_im2col_tap_major_f32": [_P, _P, _I64, _I64, _I64, _I64, _I64, _P],
    "dtts_tap_major_weight": [_P, _P, _I64, _I64, _I64, _I64],
    "dtts_tap_weight_to_tap_major": [_P, _P, _I64, _I64, _I64, _I64],
    "dtts_transpose_tap_major_weight": [_P, _P, _I64, _I64, _I64, _I64, _I64],
    "dtts_transpose_bias": [_P, _P, _I64, _I64, _I64],
    "dtts_rms_norm_f32": [_P, _P, _P, _I64, _I64, _F32, _P],
    "dtts_rms_norm_f16": [_P, _P, _P, _I64, _I64, _F32, _P],
    "dtts_rope_table_f32": [_I64, _I64, _F64, _P, _P],
    "dtts_rope_halfsplit_f32": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "dtts_rope_halfsplit_f16": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "dtts_qk_norm_rope_kv_append_f32": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                        _I64, _I64, _F32, _P],
    "dtts_qk_norm_rope_kv_append_f16": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                        _I64, _I64, _F32, _P],
    "dtts_qkrope_apply_f32": [_P, _P, _P, _P, _P, _P, _I64, _I64, _F32, _P, _P, _P, _I64, _I64, _I64, _I64,
                              _I64, _I64, _P],
    "dtts_kv_append_f32": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "dtts_kv_append_f16": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "dtts_decode_attention_workspace_bytes": [_I64, _I64, _I64, _I64, _I64],
    "dtts_decode_attention_f16": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _SZ, _P],
    "dtts_decode_attention_f32": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _SZ, _P],
    "dtts_rvq_lookup_sum_f16": [_P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "dtts_depthwise_layernorm_nlc_f16": [_P, _P, _P, _P, _P, _F32, _P, _I64, _I64, _I64, _I64, _P],
    "dtts_rms_norm_rows_f16": [_P, _P, _P, _I64, _I64, _F32, _P],
    "dtts_swiglu_rows_f16": [_P, _P, _I64, _I64, _P],
    "dtts_window_attention_prefill_f16": [_P, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F32, _P],
    "dtts_codec_front_create": [_P, _P, _P],
    "dtts_codec_front_destroy": [_P],
    "dtts_codec_front_workspace_bytes": [_P, _I64, _I64],
    "dtts_codec_front_decode": [_P, _P, _P, _I64, _I64, _P, _SZ, _P],
    "dtts_codec_document_workspace_bytes": [_P, _P, _I64, _I64, _I64],
    "dtts_codec_decode_document": [_P, _P, _P, _I64, _I64, _I64, _P, _P, _SZ, _P],
    "dtts_checkpoint_open": [ctypes.c_char_p, _P],
    "dtts_checkpoint_close": [_P],
    "dtts_checkpoint_count": [_P],
    "dtts_checkpoint_at": [_P, _I64, _P],
    "dtts_checkpoint_get": [_P, ctypes.c_char_p, _P],
    "dtts_convert_f16": [_P, _I32, _P, _I64, _P],
    "dtts_convert_f32": [_P, _I32, _P, _I64, _P],
    "dtts_convert_f16_cols": [_P, _I32, _P, _I64, _I64, _I64, _I64, _P],
    "dtts_convert_transpose_f16": [_P, _I32, _P, _I64, _I64, _P],
    "dtts_convert_tap_major_f16": [_P, _I32, _P, _I64, _I64, _I64, _P],
    "dtts_convert_transpose_tap_major_f16": [_P, _I32, _P, _I64, _I64, _I64, _I64, _P],
    "dtts_convert_repeat_f16": [_P, _I32, _P, _I64, _I64, _P],
    "dtts_convert_snake_fold": [_P, _P, _I32, _P, _P, _I64, _P],
    "dtts_convert_codebook_fold": [_P, _P, _I32, _F32, _P, _I64, _I64, _P],
    "dtts_convert_q8_0": [_P, _I32, _P, _I64, _I64, _P],
    "dtts_codec_model_load": [_P, _P, _P, _P, _P],
    "dtts_codec_model_destroy": [_P],
    "dtts_codec_model_front": [_P],
    "dtts_codec_model_wave": [_P],
    "dtts_codec_model_bytes": [_P],
    "dtts_convert_f32_scaled": [_P, _I32, _P, _I64, _F32, _P],
    "dtts_stack_model_load": [_P, ctypes.c_char_p, _P, _P, _P],
    "dtts_stack_model_load_as": [_P, ctypes.c_char_p, _P, _I32, _P, _P],
    "dtts_stack_model_destroy": [_P],
    "dtts_stack_model_stack": [_P],
    "dtts_stack_model_bytes": [_P],
    "dtts_gemm_q8_0_workspace_bytes": [_I64, _I64, _I64],
    "dtts_gemm_q8_0_ws": [_P, _P, _P, _I64, _I64, _I64, _I32, _P, _SZ, _P],
    "dtts_q8_0_packed_bytes": [_I64, _I64],
    "dtts_q8_0_repack": [_P, _P, _I64, _I64, _P],
    "dtts_gemm_q8_0_packed": [_P, _P, _P, _I64, _I64, _I64, _I32, _P, _SZ, _P],
    "dtts_gemm_q8_0_f32": [_P, _P, _P, _I64, _I64, _I64, _I32, _P],
    "dtts_gemm_q8_0_ws_f32": [_P, _P, _P, _I64, _I64, _I64, _I32, _P, _SZ, _P],
    "dtts_gemm_q8_0_packed_f32": [_P, _P, _P, _I64, _I64, _I64, _I32, _P, _SZ, _P],
    "dtts_stack_create": [_P, _P, _P, _P],
    "dtts_stack_create_as": [_P, _P, _P, _I32, _P],
    "dtts_gemm_f32_nt_workspace_bytes": [_I64, _I64, _I64],
    "dtts_gemm_f32_nt": [_P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P],
    "dtts_stack_destroy": [_P],
    "dtts_stack_workspace_bytes": [_P, _I64, _I64],
    "dtts_stack_decode": [_P, _P, _P, _P, _I64, _I64, _P, _P, _SZ, _I32, _P],
    "dtts_stack_prefill_workspace_bytes": [_P, _I64, _I64],
    "dtts_stack_prefill": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _SZ, _P],
    "dtts_gemm_f16_skinny": [_P, _P, _P, _I64, _I64, _I64, _P],
    "dtts_gemm_f16_workspace_bytes": [_I64, _I64, _I64, _I32],
    "dtts_gemm_f16_nt": [_P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P],
    "dtts_gemm_f16_nt_noalloc": [_P, _P, _P, _I64, _I64, _I64, _P],
    "dtts_gemm_f16_gateup_silu": [_P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P],
    "dtts_swiglu_mul_f32": [_P, _P, _P, _I64, _P],
    "dtts_q8_0_quantize": [_P, _P, _I64, _I64],
    "dtts_q8_0_dequantize_f32": [_P, _P, _I64, _I64, _P],
    "dtts_gemm_q8_0": [_P, _P, _P, _I64, _I64, _I64, _I32, _P],
    "dtts_codec_create": [_P, _P, _P],
    "dtts_codec_create_f32": [_P, _P, _P],
    "dtts_codec_destroy": [_P],
    "dtts_codec_hop": [_P],
    "dtts_codec_workspace_bytes": [_P, _I64, _I64],
    "dtts_codec_decode": [_P, _P, _P, _I64, _I64, _P, _SZ, _P],
    "dtts_codec_decode_f32": [_P, _P, _P, _I64, _I64, _P, _SZ, _P],
    "dtts_codec_profile": [_P, _P, _P, _I64, _I64, _P, _SZ, _P, _P, _I32, _P],
}
_RESTYPES = {"dtts_last_error": ctypes.c_char_p, "dtts_codec_destroy": None,
             "dtts_codec_hop": ctypes.c_int64, "dtts_codec_workspace_bytes": ctypes.c_size_t,
             "dtts_decode_attention_workspace_bytes": ctypes.c_size_t,
             "dtts_gemm_f16_workspace_bytes": ctypes.c_size_t, "dtts_stack_destroy": None,
             "dtts_stack_workspace_bytes": ctypes.c_size_t, "dtts_gemm_f32_nt_workspace_bytes": ctypes.c_size_t, "dtts_stack_prefill_workspace_bytes": ctypes.c_size_t, "dtts_codec_front_destroy": None,
             "dtts_codec_front_workspace_bytes": ctypes.c_size_t,
             "dtts_codec_document_workspace_bytes": ctypes.c_size_t, "dtts_checkpoint_close": None,
             "dtts_checkpoint_count": ctypes.c_int64, "dtts_codec_model_destroy": None,
             "dtts_codec_model_front": ctypes.c_void_p, "dtts_codec_model_wave": ctypes.c_void_p,
             "dtts_codec_model_bytes": ctypes.c_size_t, "dtts_stack_model_destroy": None,
             "dtts_stack_model_stack": ctypes.c_void_p, "dtts_stack_model_bytes": ctypes.c_size_t,
             "dtts_gemm_q8_0_workspace_bytes": ctypes.c_size_t, "dtts_q8_0_packed_bytes": ctypes.c_size_t,
             "dtts_conv_split_weight_bytes": ctypes.c_size_t,
             "dtts_conv1d_nlc_f32_split_workspace_bytes": ctypes.c_size_t}


class DttsError(RuntimeError):
    pass


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise DttsError(f"libdtts.so is not built ({LIB_PATH}); run dream-tts_amd/build.py")
        handle = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = handle
    return _lib


def call(name: str, *args) -> None:
    status = getattr(lib(), name)(*args)
    if status != 0:
        msg = lib().dtts_last_error().decode(errors="replace")
        raise DttsError(f"{name} failed ({status}): {msg}")


def ptr(t) -> ctypes.c_void_p | None:
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream_handle(device=None) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
