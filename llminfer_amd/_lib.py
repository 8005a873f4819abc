"""ctypes bindings of libllminfer_hip.so (declarations: include/llminfer_hip.h).

The library is loaded from llminfer_amd/lib/ only. There is no fallback: if it
is missing, importing the backend raises, so no caller can silently run a
CPU path in its place.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libllminfer_hip.so"

OK = 0
INVALID_ARGUMENT = 1
UNSUPPORTED = 2
WORKSPACE = 3
LAUNCH_FAILED = 4
NO_DEVICE = 5

OP_KV_APPEND = 0
OP_CAUSAL_GQA = 1
OP_DELTA_UPDATE = 2
OP_KV_APPEND_CAUSAL_GQA = 3
OP_NORM_ROPE = 4
OP_RMS_NORM = 5
OP_PARTIAL_ROPE = 6
OP_SIGMOID_MUL = 7
OP_CAUSAL_CONV = 8
OP_L2_NORM = 9
OP_DELTA_GATES = 10
OP_GATED_RMS_NORM = 11
OP_GATED_ATTENTION = 12
OP_QUANTIZE_ACTIVATION = 13
OP_LINEAR_W8A8 = 14
OP_EMBEDDING_W8 = 15
OP_EMBEDDING = 16
OP_RESIDUAL_ADD = 17
OP_SWIGLU = 18
OP_SILU = 19
OP_MULTIPLY = 20
OP_COPY_HALF_VIEW = 21
OP_LINEAR_F16 = 22
OP_ADD_RMS_NORM_QUANTIZE = 23
OP_ADD_RMS_NORM_LINEAR_W8A8 = 24
NORM_LINEAR_MAX = 4  # LLMI_HIP_NORM_LINEAR_MAX

# LinearEpilogue (ReferenceParams.h:8-16)
LINEAR_NONE, LINEAR_SILU, LINEAR_SILU_MUL, LINEAR_SIGMOID_COLUMNS = 0, 1, 2, 3
LINEAR_SILU_F32, LINEAR_DELTA_BETA, LINEAR_DELTA_DECAY = 4, 5, 6

NOALLOC_SCRATCH_BYTES = 8 << 20  # LLMI_HIP_NOALLOC_SCRATCH_BYTES


class CacheParams(C.Structure):
    _fields_ = [("count", C.c_uint), ("offset", C.c_uint)]


class RowParams(C.Structure):
    _fields_ = [("rows", C.c_uint), ("width", C.c_uint), ("epsilon", C.c_float)]


class ElementParams(C.Structure):
    _fields_ = [("count", C.c_uint)]


class RopeParams(C.Structure):
    _fields_ = [(n, C.c_uint) for n in ("tokens", "heads", "headDim", "rotaryDim",
                                        "headStride", "past", "outputStart")] + \
               [("epsilon", C.c_float), ("theta", C.c_float)]


class PartialRopeParams(C.Structure):
    _fields_ = [(n, C.c_uint) for n in ("rows", "heads", "width", "rotaryWidth", "past")] + \
               [("theta", C.c_float)]


class ConvParams(C.Structure):
    _fields_ = [(n, C.c_uint) for n in ("tokens", "channels", "kernelSize", "applySilu")]


class L2Params(C.Structure):
    _fields_ = [("rows", C.c_uint), ("width", C.c_uint), ("epsilon", C.c_float),
                ("scale", C.c_float)]


class QuantizeParams(C.Structure):
    _fields_ = [(n, C.c_uint) for n in ("rows", "width", "groups")]


class LinearW8Params(C.Structure):
    _fields_ = [(n, C.c_uint) for n in ("outputWidth", "firstRow", "groups", "rows", "columns",
                                        "epilogue", "epilogueBlock")]


class NormProjection(C.Structure):
    _fields_ = [("weight", C.c_void_p), ("weight_scales", C.c_void_p), ("output", C.c_void_p),
                ("aux", C.c_void_p), ("bias", C.c_void_p), ("conv_weight", C.c_void_p),
                ("conv_history", C.c_void_p)]


class NormLinearParams(C.Structure):
    _fields_ = [("norm", RowParams), ("count", C.c_uint),
                ("linear", LinearW8Params * NORM_LINEAR_MAX)]


class GroupedEmbedParams(C.Structure):
    _fields_ = [(n, C.c_uint) for n in ("tokens", "hidden", "firstRow", "rowCount", "groups")]


class EmbedParams(C.Structure):
    _fields_ = [(n, C.c_uint) for n in ("tokens", "hidden", "firstRow", "rowCount")]


class HalfViewParams(C.Structure):
    _fields_ = [("count", C.c_uint), ("offset", C.c_uint), ("dims", C.c_uint * 3),
                ("strides", C.c_uint * 3)]


class LinearParams(C.Structure):
    _fields_ = [(n, C.c_uint) for n in ("tokens", "inputWidth", "outputWidth", "firstRow",
                                        "rowCount", "epilogue", "epilogueBlock")]


class GqaParams(C.Structure):
    _fields_ = [("tokens", C.c_uint), ("queryHeads", C.c_uint),
                ("kvHeads", C.c_uint), ("headDim", C.c_uint), ("past", C.c_uint)]


class GraphDeltaParams(C.Structure):
    _fields_ = [("tokens", C.c_uint), ("keyHeads", C.c_uint), ("keyDim", C.c_uint),
                ("valueHeads", C.c_uint), ("valueDim", C.c_uint)]


class SessionConfig(C.Structure):
    _fields_ = [("capacity", C.c_uint), ("queryHeads", C.c_uint),
                ("kvHeads", C.c_uint), ("headDim", C.c_uint),
                ("keyHeads", C.c_uint), ("keyDim", C.c_uint),
                ("valueHeads", C.c_uint), ("valueDim", C.c_uint)]


class Dispatch(C.Structure):
    """MetalDispatchInfo{opIndex, kernel, epilogue, fusedOpIndex}."""
    _fields_ = [("op_index", C.c_size_t), ("kernel", C.c_char_p),
                ("epilogue", C.c_char_p), ("fused_op_index", C.c_size_t)]


class HipError(RuntimeError):
    """A nonzero llmi_hip status, with the library's message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status})")
        self.status = status


_P = C.c_void_p
_SZ = C.c_size_t

# name -> (restype, argtypes). Every function declared in include/llminfer_hip.h.
SIGNATURES = {
    "llmi_hip_cache_append": (C.c_int, [_P, _P, CacheParams, _P]),
    "llmi_hip_norm_rope": (C.c_int, [_P, _P, _P, RopeParams, _P]),
    "llmi_hip_rms_norm": (C.c_int, [_P, _P, _P, RowParams, _P]),
    "llmi_hip_partial_rope": (C.c_int, [_P, _P, PartialRopeParams, _P]),
    "llmi_hip_sigmoid_mul": (C.c_int, [_P, _P, _P, ElementParams, _P]),
    "llmi_hip_causal_conv": (C.c_int, [_P, _P, _P, _P, ConvParams, _P]),
    "llmi_hip_l2_norm": (C.c_int, [_P, _P, L2Params, _P]),
    "llmi_hip_delta_gates": (C.c_int, [_P, _P, _P, _P, _P, _P, RowParams, _P]),
    "llmi_hip_gated_rms_norm": (C.c_int, [_P, _P, _P, _P, RowParams, _P]),
    "llmi_hip_gated_rms_norm_activated": (C.c_int, [_P, _P, _P, _P, RowParams, _P]),
    "llmi_hip_kv_append": (C.c_int, [_P, _P, _P, _P, CacheParams, _P]),
    "llmi_hip_causal_gqa": (C.c_int, [_P, _P, _P, _P, GqaParams, _P, _SZ, _P]),
    "llmi_hip_gqa_workspace_bytes": (_SZ, [GqaParams]),
    "llmi_hip_kv_append_causal_gqa": (C.c_int, [_P, _P, _P, _P, _P, _P, GqaParams, _P, _SZ,
                                                _P]),
    "llmi_hip_kv_append_causal_gqa_noalloc": (C.c_int, [_P, _P, _P, _P, _P, _P, GqaParams,
                                                        _P]),
    "llmi_hip_gated_attention": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, GqaParams,
                                           C.c_uint, C.c_float, C.c_float, _P, _SZ, _P]),
    "llmi_hip_gated_attention_activated": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, GqaParams,
                                                     C.c_uint, C.c_float, C.c_float, _P, _SZ,
                                                     _P]),
    "llmi_hip_delta_update": (C.c_int, [_P, _P, _P, _P, _P, _P, _P,
                                        GraphDeltaParams, _P, _SZ, _P]),
    "llmi_hip_delta_workspace_bytes": (_SZ, [GraphDeltaParams]),
    "llmi_hip_l2_norm_delta_update": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, GraphDeltaParams,
                                                C.c_float, C.c_float, _P, _SZ, _P]),
    "llmi_hip_l2_norm_delta_gated_norm": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P,
                                                    GraphDeltaParams, C.c_float, C.c_float,
                                                    C.c_float, _P, _SZ, _P]),
    "llmi_hip_l2_norm_delta_gated_norm_status": (C.c_int, [_P, _SZ, GraphDeltaParams, _P]),
    "llmi_hip_l2_norm_delta_gated_norm_activated_quantize": (
        C.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, GraphDeltaParams, C.c_float,
                  C.c_float, C.c_float, _P]),
    "llmi_hip_set_arrival_wait_limit": (C.c_uint, [C.c_uint]),
    "llmi_hip_quantize_activation": (C.c_int, [_P, _P, _P, _P, QuantizeParams, _P]),
    "llmi_hip_linear_w8a8": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, LinearW8Params, _P]),
    "llmi_hip_embedding_w8": (C.c_int, [_P, _P, _P, _P, GroupedEmbedParams, _P]),
    "llmi_hip_embedding": (C.c_int, [_P, _P, _P, EmbedParams, _P]),
    "llmi_hip_residual_add": (C.c_int, [_P, _P, _P, ElementParams, _P]),
    "llmi_hip_swiglu": (C.c_int, [_P, _P, _P, ElementParams, _P]),
    "llmi_hip_silu": (C.c_int, [_P, _P, ElementParams, _P]),
    "llmi_hip_multiply": (C.c_int, [_P, _P, _P, ElementParams, _P]),
    "llmi_hip_copy_half_view": (C.c_int, [_P, _P, HalfViewParams, _P]),
    "llmi_hip_linear_f16": (C.c_int, [_P, _P, _P, _P, _P, LinearParams, _P]),
    "llmi_hip_add_rms_norm_quantize": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, RowParams, _P]),
    "llmi_hip_add_rms_norm_linear_w8a8": (C.c_int, [_P, _P, _P, _P, _P, _P, _P, _P,
                                                    NormLinearParams, _P]),
    "llmi_hip_gated_rms_norm_activated_quantize": (C.c_int, [_P, _P, _P, _P, _P, _P, _P,
                                                             RowParams, _P]),
    "llmi_hip_workspace_init": (C.c_int, [_P, _SZ, _P]),
    "llmi_hip_dispatch_count": (C.c_uint, [C.c_int, _P]),
    "llmi_hip_kernel_name": (C.c_char_p, [C.c_int, _P, C.c_uint]),
    "llmi_hip_status_string": (C.c_char_p, [C.c_int]),
    "llmi_hip_last_error": (C.c_char_p, []),
    "llmi_hip_build_info": (C.c_char_p, []),
    "llmi_hip_session_open": (C.c_int, [C.POINTER(SessionConfig), _P, C.POINTER(_P)]),
    "llmi_hip_session_close": (None, [_P]),
    "llmi_hip_session_reset": (None, [_P]),
    "llmi_hip_session_past": (C.c_uint, [_P]),
    "llmi_hip_session_restore": (C.c_int, [_P, C.c_uint]),
    "llmi_hip_session_check": (C.c_int, [C.POINTER(SessionConfig), C.c_uint, C.c_uint]),
    "llmi_hip_session_invalid": (C.c_int, [_P]),
    "llmi_hip_session_key_cache": (_P, [_P]),
    "llmi_hip_session_value_cache": (_P, [_P]),
    "llmi_hip_session_recurrent_state": (_P, [_P]),
    "llmi_hip_session_step": (C.c_int, [_P, C.c_uint, _P, _P, _P, _P, _P, _P,
                                        _P, _P, _P, _P, C.POINTER(Dispatch), _SZ,
                                        C.POINTER(_SZ)]),
    # whole-graph plan (structs in llminfer_amd/plan.py)
    "llmi_hip_plan_lower": (C.c_int, [_P, _P, _SZ, _P]),
    "llmi_hip_plan_destroy": (None, [_P]),
    "llmi_hip_plan_scratch_bytes": (_SZ, [_P]),
    "llmi_hip_plan_logits": (None, [_P, _P, _P]),
    "llmi_hip_plan_dispatches": (_SZ, [_P, C.POINTER(Dispatch), _SZ]),
    "llmi_hip_plan_launches": (_SZ, [_P]),
    "llmi_hip_plan_execute": (C.c_int, [_P, _P, _SZ, _P, _SZ, _P, _P, _P, _P]),
    # Qwen3.5 graph builder and model session (structs in llminfer_amd/plan.py)
    "llmi_qwen35_build": (C.c_int, [_P, C.c_uint64, C.c_uint64, C.c_uint64, C.c_int, _P]),
    "llmi_qwen35_graph_view": (_P, [_P]),
    "llmi_qwen35_graph_tensor_count": (_SZ, [_P]),
    "llmi_qwen35_graph_tensor": (C.c_char_p, [_P, _SZ]),
    "llmi_qwen35_graph_destroy": (None, [_P]),
    "llmi_hip_model_open": (C.c_int, [_P, _P, _SZ, C.c_uint64, _P, _P]),
    "llmi_hip_model_close": (None, [_P]),
    "llmi_hip_model_reset": (None, [_P]),
    "llmi_hip_model_past": (C.c_uint64, [_P]),
    "llmi_hip_model_invalid": (C.c_int, [_P]),
    "llmi_hip_model_vocabulary": (C.c_uint64, [_P]),
    "llmi_hip_model_step": (C.c_int, [_P, _P, _SZ, C.c_int, _P, _SZ, _P]),
    "llmi_hip_model_dispatches": (_SZ, [_P, C.POINTER(Dispatch), _SZ]),
    "llmi_hip_model_state_count": (_SZ, [_P]),
    "llmi_hip_model_state": (C.c_int, [_P, _SZ, _P, _P, _P]),
    "llmi_hip_model_read_state": (C.c_int, [_P, _SZ, _P, _SZ]),
    "llmi_hip_model_plan": (C.c_int, [_P, C.c_uint64, C.c_uint64, C.c_int, _P]),
    "llmi_hip_model_run": (C.c_int, [_P, _P, _P, _P]),
}

_lib = None


def load() -> C.CDLL:
    """Load the backend library (once). Raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m llminfer_amd.build` "
            "(there is no non-HIP fallback)")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue  # reported by the export test, not at load time
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status: int) -> None:
    if status != OK:
        lib = load()
        raise HipError(status, lib.llmi_hip_last_error().decode())
