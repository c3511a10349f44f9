"""ctypes binding of libapeiron_hip.so (the C ABI of include/apeiron_hip.h).

Loading fails loudly when the library has not been built: there is no CPU fallback on the
product path.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libapeiron_hip.so")

STATUS = {
    0: "ok", 1: "ShapeMismatch", 2: "RowLength", 3: "ShortPayload", 4: "LengthOverflow",
    5: "UnsupportedQuant", 6: "NonFiniteScale", 7: "FixedOverflow", 8: "AccumulatorOverflow",
    9: "OutputOverflow", 10: "NonFiniteInput", 11: "InputRange", 20: "NoDevice",
    12: "FfnOverflow", 13: "ExpOutOfRange", 14: "ZeroDenominator",
    21: "InvalidArg", 22: "Hip", 23: "OutOfMemory", 24: "ScratchLimit", 25: "SeqTimeout",
}

# Every symbol include/apeiron_hip.h declares.
EXPORTS = [
    "ah_init", "ah_destroy", "ah_status_str", "ah_last_hip_error", "ah_upload_weight",
    "ah_wrap_weight_dev", "ah_free_tensor", "ah_tensor_info", "ah_quant_act_f32_dev",
    "ah_quant_act_q32_dev", "ah_gemv_f32_dev", "ah_gemv_q8_dev", "ah_gemv_plan_create",
    "ah_gemv_plan_run", "ah_gemv_plan_free", "ah_gemm_f32_dev", "ah_gemm_q8_dev",
    "ah_gemv_q8_dots_dev", "ah_sync_status", "ah_matvec_q8act", "ah_matmat_q8act",
    "ah_quant_act", "ah_probe_mfma_peak", "ah_gemm_group_f32_dev", "ah_gemm_group_q8_dev",
    "ah_last_refusal_bits", "ah_gemm_f32_noalloc_dev", "ah_gemm_noalloc_scratch_bytes",
    "ah_set_gemm_design", "ah_ffn_gate_up_dev", "ah_ffn_dev", "ah_ffn_gate_up_prefill_dev",
    "ah_ffn_prefill_dev", "ah_set_ffn_prefill_form", "ah_swiglu_quant_dev", "ah_ffn_q8_dev",
    "ah_ffn_prefill_q8_dev", "ah_dev_alloc", "ah_dev_free", "ah_copy_to_dev", "ah_copy_to_host", "ah_seq_set_spin_limit", "ah_ctx_scratch_bytes",
    "ah_seq_create", "ah_seq_run", "ah_seq_sync_status", "ah_seq_free", "ah_seq_info",
]

_lib = None

P = ctypes.c_void_p


class SeqStage(ctypes.Structure):
    """struct ah_seq_stage of include/apeiron_hip.h."""
    _fields_ = [("kind", ctypes.c_uint32), ("n_parts", ctypes.c_size_t), ("w", ctypes.c_void_p),
                ("x", ctypes.c_void_p), ("codes", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("y", ctypes.c_void_p), ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p),
                ("n", ctypes.c_size_t), ("h_codes", ctypes.c_void_p), ("h_scales", ctypes.c_void_p)]

S = ctypes.c_size_t
I32 = ctypes.c_int32
U32 = ctypes.c_uint32


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m apeiron_amd.build` "
            "(the HIP path has no fallback)")
    L = ctypes.CDLL(LIB_PATH)
    sig = {
        "ah_init": (I32, [I32, ctypes.POINTER(P)]),
        "ah_destroy": (I32, [P]),
        "ah_status_str": (ctypes.c_char_p, [I32]),
        "ah_last_hip_error": (I32, [P]),
        "ah_last_refusal_bits": (I32, [P, ctypes.POINTER(U32)]),
        "ah_upload_weight": (I32, [P, U32, P, S, S, S, ctypes.POINTER(P)]),
        "ah_wrap_weight_dev": (I32, [P, U32, P, S, S, S, ctypes.POINTER(P)]),
        "ah_free_tensor": (I32, [P, P]),
        "ah_tensor_info": (I32, [P, ctypes.POINTER(U32), ctypes.POINTER(S), ctypes.POINTER(S),
                                 ctypes.POINTER(S), ctypes.POINTER(P)]),
        "ah_quant_act_f32_dev": (I32, [P, P, S, S, P, P, P]),
        "ah_quant_act_q32_dev": (I32, [P, P, S, S, P, P, P]),
        "ah_gemv_f32_dev": (I32, [P, P, P, P, P]),
        "ah_gemv_q8_dev": (I32, [P, P, P, P, P, P]),
        "ah_gemv_q8_dots_dev": (I32, [P, P, P, P, P, P, P]),
        "ah_gemv_plan_create": (I32, [P, S, P, P, P, ctypes.POINTER(P)]),
        "ah_gemv_plan_run": (I32, [P, P, P]),
        "ah_gemv_plan_free": (I32, [P, P]),
        "ah_gemm_f32_dev": (I32, [P, P, P, S, P, P]),
        "ah_ffn_gate_up_dev": (I32, [P, P, P, P, P, P, P, P, P]),
        "ah_ffn_dev": (I32, [P, P, P, P, P, P, P, P, P]),
        "ah_ffn_gate_up_prefill_dev": (I32, [P, P, P, P, S, P, P, P, P, P]),
        "ah_ffn_prefill_dev": (I32, [P, P, P, P, P, S, P, P, P, P]),
        "ah_set_ffn_prefill_form": (I32, [P, U32]),
        "ah_swiglu_quant_dev": (I32, [P, P, P, S, S, P, P, P]),
        "ah_ffn_q8_dev": (I32, [P, P, P, P, P, P, P, P, P, P]),
        "ah_ffn_prefill_q8_dev": (I32, [P, P, P, P, P, P, S, P, P, P, P]),
        "ah_dev_alloc": (I32, [P, S, ctypes.POINTER(P)]),
        "ah_dev_free": (I32, [P, P]),
        "ah_copy_to_dev": (I32, [P, P, P, S, P]),
        "ah_copy_to_host": (I32, [P, P, P, S, P]),
        "ah_seq_set_spin_limit": (I32, [P, U32]),
        "ah_ctx_scratch_bytes": (I32, [P, ctypes.POINTER(S)]),
        "ah_gemm_f32_noalloc_dev": (I32, [P, P, P, S, P, P]),
        "ah_gemm_noalloc_scratch_bytes": (I32, [ctypes.POINTER(S)]),
        "ah_set_gemm_design": (I32, [P, U32, U32]),
        "ah_gemm_q8_dev": (I32, [P, P, P, P, S, P, P]),
        "ah_sync_status": (I32, [P, P]),
        "ah_matvec_q8act": (I32, [P, P, P, P, S, P]),
        "ah_matmat_q8act": (I32, [P, P, P, P, S, P]),
        "ah_quant_act": (I32, [P, P, S, P, P]),
        "ah_probe_mfma_peak": (I32, [P, U32, ctypes.POINTER(ctypes.c_double)]),
        "ah_gemm_group_f32_dev": (I32, [P, S, P, P, S, P, P]),
        "ah_gemm_group_q8_dev": (I32, [P, S, P, P, P, S, P, P]),
        "ah_seq_create": (I32, [P, S, P, ctypes.POINTER(P)]),
        "ah_seq_run": (I32, [P, P, P]),
        "ah_seq_sync_status": (I32, [P, P, P, ctypes.POINTER(U32)]),
        "ah_seq_free": (I32, [P, P]),
        "ah_seq_info": (I32, [P, ctypes.POINTER(U32), ctypes.POINTER(U32)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L
