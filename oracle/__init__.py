"""numpy front end of the C oracle (oracle.c). TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
the checker / CPU baseline; the product package never imports it. Every
function forwards to the C restatement documented in oracle.h, which cites
the reference file:line it follows.

Synthetic inputs (seeded, reproducible on any host):
  make_gqa_inputs    q [T,Hq,d], caches [cap,Hkv,d] with rows [0,P+T) filled
  make_delta_inputs  the DeltaUpdate operands as the reference graph produces
                     them: L2-normalised fp32 q (x 1/sqrt(dk)) and k, fp16 v,
                     beta = fp16(sigmoid(b)), decay = exp(-softplus(a)).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libllmiref.so"

_lib = None

_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u32 = C.c_uint32
_u64 = C.c_uint64


class Cost(C.Structure):
    _fields_ = [("fp_macs", _u64), ("scalar_ops", _u64), ("exp", _u64),
                ("read_bytes", _u64), ("write_bytes", _u64)]


def build() -> Path:
    """Compile liboracle.so with the committed Makefile (always rebuilds)."""
    subprocess.run(["make", "-s", "-B", "-C", str(HERE), "liboracle.so"], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f32_to_f16_n.argtypes = [_f32p, _u16p, C.c_size_t]
        L.orc_f16_to_f32_n.argtypes = [_u16p, _f32p, C.c_size_t]
        L.orc_fill_normal_f32.argtypes = [_u64, _u64, C.c_size_t, C.c_double, C.c_double, _f32p]
        L.orc_fill_normal_f16.argtypes = [_u64, _u64, C.c_size_t, C.c_double, C.c_double, _u16p]
        L.orc_fill_lcg_f16.argtypes = [C.POINTER(_u32), C.c_size_t, _u16p]
        L.orc_gqa_dense_f64.argtypes = [_u16p, _u16p, _u16p, _f64p] + [_u32] * 5
        L.orc_gqa_eager_f16.argtypes = [_u16p, _u16p, _u16p, _u16p] + [_u32] * 5
        L.orc_gqa_f32.argtypes = [_u16p, _u16p, _u16p, _u16p] + [_u32] * 5 + [C.c_int]
        L.orc_kv_append.argtypes = [_u16p, _u16p] + [_u32] * 4
        L.orc_delta_recurrent_f64.argtypes = [_f32p, _f32p, _u16p, _f32p, _f32p, _f32p,
                                              _f64p, C.c_void_p] + [_u32] * 5
        L.orc_delta_recurrent_f32.argtypes = [_f32p, _f32p, _u16p, _f32p, _f32p, _f32p,
                                              _u16p] + [_u32] * 5 + [C.c_int]
        L.orc_delta_chunked_f64.argtypes = [_f32p, _f32p, _u16p, _f32p, _f32p, _f32p,
                                            _f64p, C.c_void_p] + [_u32] * 6
        L.orc_delta_gates.argtypes = [_u16p, _u16p, _f32p, _f32p, _f32p, _f32p, _u32, _u32]
        L.orc_l2norm_f32.argtypes = [_u16p, _f32p, _u32, _u32, C.c_float, C.c_float]
        L.orc_norm_rope.argtypes = [_u16p, _f32p, _u16p] + [_u32] * 7 + [C.c_float, C.c_float]
        L.orc_sigmoid_mul.argtypes = [_u16p, _u16p, _u16p, C.c_size_t]
        L.orc_causal_conv.argtypes = [_u16p, _u16p, _u16p, _u16p] + [_u32] * 4
        L.orc_gated_rms_norm.argtypes = [_u16p, C.c_void_p, C.c_void_p, _f32p, _u16p,
                                         _u32, _u32, C.c_float]
        L.orc_quantize_activation.argtypes = [_u16p, C.c_void_p, _f32p, C.POINTER(_u32)] + \
            [_u32] * 3
        L.orc_linear_w8a8.argtypes = [C.c_void_p, _f32p, C.c_void_p, _u16p, C.c_void_p,
                                      C.c_void_p, C.c_void_p] + [_u32] * 7
        L.orc_embedding_w8.argtypes = [C.c_void_p, C.c_void_p, _u16p, _u16p] + [_u32] * 5
        L.orc_embedding.argtypes = [C.c_void_p, _u16p, _u16p] + [_u32] * 4
        L.orc_elementwise.argtypes = [_u32, _u16p, _u16p, _u16p, C.c_size_t]
        L.orc_partial_rope.argtypes = [_u16p, _u16p] + [_u32] * 5 + [C.c_float]
        L.orc_copy_half_view.argtypes = [_u16p, _u16p, _u32, _u32, C.POINTER(_u32),
                                         C.POINTER(_u32)]
        L.orc_linear_f16.argtypes = [_u16p, _u16p, C.c_void_p, C.c_void_p, C.c_void_p] + \
            [_u32] * 7
        for name, n in (("orc_cost_kv_append", 3), ("orc_cost_causal_gqa", 5),
                        ("orc_cost_delta_update", 5)):
            fn = getattr(L, name)
            fn.restype = C.c_int
            fn.argtypes = [_u64] * n + [C.POINTER(Cost)]
        L.orc_cpu_count.restype = C.c_int
        _lib = L
    return _lib


# ------------------------------------------------------------------ fp16

def f32_to_f16(x) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().orc_f32_to_f16_n(a.reshape(-1), out.reshape(-1), a.size)
    return out


def f16_to_f32(bits) -> np.ndarray:
    a = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(a.shape, np.float32)
    lib().orc_f16_to_f32_n(a.reshape(-1), out.reshape(-1), a.size)
    return out


# ------------------------------------------------------------------- RNG

def normal_f16(seed: int, stream: int, shape, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(shape, np.uint16)
    lib().orc_fill_normal_f16(seed, stream, out.size, mean, std, out.reshape(-1))
    return out


def normal_f32(seed: int, stream: int, shape, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(shape, np.float32)
    lib().orc_fill_normal_f32(seed, stream, out.size, mean, std, out.reshape(-1))
    return out


def lcg_f16(state: int, n: int) -> tuple[np.ndarray, int]:
    s = _u32(state)
    out = np.empty(n, np.uint16)
    lib().orc_fill_lcg_f16(C.byref(s), n, out)
    return out, s.value


# ------------------------------------------------------------------- GQA

def gqa_dense_f64(q, kc, vc, past: int) -> np.ndarray:
    T, hq, d = q.shape
    hkv = kc.shape[1]
    assert kc.shape[0] >= past + T and vc.shape == kc.shape
    out = np.empty((T, hq, d), np.float64)
    lib().orc_gqa_dense_f64(np.ascontiguousarray(q), np.ascontiguousarray(kc),
                            np.ascontiguousarray(vc), out, T, hq, hkv, d, past)
    return out


def gqa_eager_f16(q, kc, vc, past: int) -> np.ndarray:
    T, hq, d = q.shape
    out = np.empty((T, hq, d), np.uint16)
    lib().orc_gqa_eager_f16(np.ascontiguousarray(q), np.ascontiguousarray(kc),
                            np.ascontiguousarray(vc), out, T, hq, kc.shape[1], d, past)
    return out


def gqa_f32(q, kc, vc, past: int, threads: int = 0) -> np.ndarray:
    T, hq, d = q.shape
    out = np.empty((T, hq, d), np.uint16)
    lib().orc_gqa_f32(np.ascontiguousarray(q), np.ascontiguousarray(kc),
                      np.ascontiguousarray(vc), out, T, hq, kc.shape[1], d, past, threads)
    return out


def kv_append(src, cache, past: int) -> None:
    T, hkv, d = src.shape
    lib().orc_kv_append(np.ascontiguousarray(src), cache, T, hkv, d, past)


@dataclass
class GqaInputs:
    q: np.ndarray         # [T, Hq, d] fp16 bits
    k_new: np.ndarray     # [T, Hkv, d]
    v_new: np.ndarray
    k_cache: np.ndarray   # [cap, Hkv, d], rows [0, P) past, [P, P+T) = k_new
    v_cache: np.ndarray
    past: int


def make_gqa_inputs(seed: int, T: int, hq: int, hkv: int, d: int, past: int,
                    capacity: int | None = None) -> GqaInputs:
    cap = capacity if capacity is not None else past + T
    q = normal_f16(seed, 1, (T, hq, d))
    k_new = normal_f16(seed, 2, (T, hkv, d))
    v_new = normal_f16(seed, 3, (T, hkv, d))
    kc = np.zeros((cap, hkv, d), np.uint16)
    vc = np.zeros((cap, hkv, d), np.uint16)
    if past:
        kc[:past] = normal_f16(seed, 4, (past, hkv, d))
        vc[:past] = normal_f16(seed, 5, (past, hkv, d))
    kc[past:past + T] = k_new
    vc[past:past + T] = v_new
    return GqaInputs(q, k_new, v_new, kc, vc, past)


# -------------------------------------------------------------- DeltaNet

def delta_recurrent_f64(q, k, v, beta, decay, state):
    T = q.shape[0]
    hv, dk, dv = state.shape
    hk = q.shape[1] // dk
    out = np.empty((T, hv * dv), np.float64)
    st = np.empty(state.shape, np.float64)
    lib().orc_delta_recurrent_f64(q, k, v, beta, decay, np.ascontiguousarray(state), st,
                                  out.ctypes.data, T, hk, dk, hv, dv)
    return out, st


def delta_recurrent_f32(q, k, v, beta, decay, state, threads: int = 0):
    """Returns (out fp16 bits, new state); `state` is not modified."""
    T = q.shape[0]
    hv, dk, dv = state.shape
    hk = q.shape[1] // dk
    out = np.empty((T, hv * dv), np.uint16)
    st = np.array(state, np.float32, copy=True)
    lib().orc_delta_recurrent_f32(q, k, v, beta, decay, st, out, T, hk, dk, hv, dv, threads)
    return out, st


def delta_chunked_f64(q, k, v, beta, decay, state, chunk: int = 64):
    T = q.shape[0]
    hv, dk, dv = state.shape
    hk = q.shape[1] // dk
    out = np.empty((T, hv * dv), np.float64)
    st = np.empty(state.shape, np.float64)
    lib().orc_delta_chunked_f64(q, k, v, beta, decay, np.ascontiguousarray(state), st,
                                out.ctypes.data, T, hk, dk, hv, dv, chunk)
    return out, st


def delta_gates(a, b, a_log, dt_bias):
    T, hv = a.shape
    beta = np.empty((T, hv), np.float32)
    decay = np.empty((T, hv), np.float32)
    lib().orc_delta_gates(np.ascontiguousarray(a), np.ascontiguousarray(b),
                          np.ascontiguousarray(a_log, np.float32),
                          np.ascontiguousarray(dt_bias, np.float32), beta, decay, T, hv)
    return beta, decay


def norm_rope(x, weight, tokens: int, heads: int, head_dim: int, rotary_dim: int,
              head_stride: int, past: int, epsilon: float = 1e-6, theta: float = 1e7,
              output=None, output_start: int = 0) -> np.ndarray:
    """normRope (Reference.metal:271-293) on fp16 bits; returns the output rows
    (a new [tokens*heads, head_dim] array, or `output` written from row
    output_start * heads)."""
    a = np.ascontiguousarray(x, np.uint16).reshape(-1)
    w = np.ascontiguousarray(weight, np.float32)
    if output is None:
        output = np.zeros(((output_start + tokens) * heads, head_dim), np.uint16)
    lib().orc_norm_rope(a, w, output.reshape(-1), tokens, heads, head_dim, rotary_dim,
                        head_stride, past, output_start, epsilon, theta)
    return output


def rms_norm(x, weight, epsilon: float = 1e-6) -> np.ndarray:
    """rmsNorm (Reference.metal:105-117) over the last axis: normRope with
    no rotated dims."""
    a = np.ascontiguousarray(x, np.uint16)
    width = a.shape[-1]
    rows = a.size // width
    return norm_rope(a, weight, rows, 1, width, 0, width, 0, epsilon).reshape(a.shape)


def partial_rope(x, rotary_dim: int, past: int, theta: float = 1e7) -> np.ndarray:
    """partialRope (Graph.metal:111-129): x [T, H, width] fp16 bits."""
    a = np.ascontiguousarray(x, np.uint16)
    T, H, width = a.shape
    out = np.empty_like(a)
    lib().orc_partial_rope(a.reshape(-1), out.reshape(-1), T * H, H, width, rotary_dim, past,
                           theta)
    return out


def causal_conv(x, weight, history, apply_silu: bool = True) -> np.ndarray:
    """causalConv (Reference.metal:137-161) on fp16 bits: x [T, C], weight
    [C, k], history [C, k-1] (updated in place); returns the output [T, C]."""
    a = np.ascontiguousarray(x, np.uint16)
    w = np.ascontiguousarray(weight, np.uint16)
    assert history.dtype == np.uint16 and history.flags.c_contiguous
    T, Cn = a.shape
    out = np.empty_like(a)
    lib().orc_causal_conv(a.reshape(-1), w.reshape(-1), history.reshape(-1), out.reshape(-1),
                          T, Cn, w.shape[1], int(apply_silu))
    return out


def gated_rms_norm(x, gate, weight, eps: float = 1e-6) -> np.ndarray:
    """gatedRmsNorm (Reference.metal:228-259): x [rows, width] fp16 bits;
    gate fp16 bits (through SiLU) or float32 (already activated)."""
    a = np.ascontiguousarray(x, np.uint16)
    w = np.ascontiguousarray(weight, np.float32)
    g = np.ascontiguousarray(gate)
    out = np.empty_like(a)
    g16 = g.ctypes.data if g.dtype == np.uint16 else None
    g32 = g.ctypes.data if g.dtype == np.float32 else None
    assert g16 or g32, "gate must be fp16 bits or float32"
    lib().orc_gated_rms_norm(a.reshape(-1), g16, g32, w, out.reshape(-1), a.shape[0],
                             a.shape[1], eps)
    return out


def sigmoid_mul(gate, x) -> np.ndarray:
    """sigmoidMul (Graph.metal:78-85) on fp16 bits."""
    g = np.ascontiguousarray(gate, np.uint16)
    a = np.ascontiguousarray(x, np.uint16)
    out = np.empty(a.shape, np.uint16)
    lib().orc_sigmoid_mul(g.reshape(-1), a.reshape(-1), out.reshape(-1), a.size)
    return out


# ------------------------------------------------------------- W8A8 path

LINEAR_NONE, LINEAR_SILU, LINEAR_SILU_MUL, LINEAR_SIGMOID_COLUMNS = 0, 1, 2, 3
LINEAR_SILU_F32, LINEAR_DELTA_BETA, LINEAR_DELTA_DECAY = 4, 5, 6
F32_EPILOGUES = (LINEAR_SILU_F32, LINEAR_DELTA_BETA, LINEAR_DELTA_DECAY)


def quantize_activation(x) -> tuple[np.ndarray, np.ndarray, int]:
    """quantizeActivation (Graph.metal:33-68) on fp16 bits [rows, width]:
    int8 [rows, groups * 32], float32 scales [rows, groups], invalid flag."""
    a = np.ascontiguousarray(x, np.uint16)
    rows, width = a.shape
    groups = (width + 31) // 32
    q = np.zeros((rows, groups * 32), np.int8)
    sc = np.empty((rows, groups), np.float32)
    invalid = _u32(0)
    lib().orc_quantize_activation(a.reshape(-1), q.ctypes.data, sc.reshape(-1),
                                  C.byref(invalid), rows, width, groups)
    return q, sc, invalid.value


def linear_w8a8(act, act_scales, weight, weight_scales, epilogue: int = LINEAR_NONE,
                block: int = 0, aux=None, bias=None, output=None, first_row: int = 0,
                output_width: int | None = None) -> np.ndarray:
    """linearW8A8Gemv/Gemm (W8A8.metal:28-113) with storeLinear
    (Reference.metal:14-47): act int8 [rows, groups * 32], act_scales float32
    [rows, groups], weight int8 [columns, groups * 32], weight_scales fp16
    bits [columns, groups]. Returns (or writes into `output`, rows x
    output_width) fp16 bits, or float32 for the fp32 epilogues."""
    x = np.ascontiguousarray(act, np.int8)
    w = np.ascontiguousarray(weight, np.int8)
    xs = np.ascontiguousarray(act_scales, np.float32)
    ws = np.ascontiguousarray(weight_scales, np.uint16)
    rows, columns, groups = x.shape[0], w.shape[0], xs.shape[1]
    assert x.shape[1] == w.shape[1] == groups * 32 and ws.shape == (columns, groups)
    width = output_width if output_width is not None else first_row + columns
    if output is None:
        dt = np.float32 if epilogue in F32_EPILOGUES else np.uint16
        output = np.zeros((rows, width), dt)
    ax = np.ascontiguousarray(aux) if aux is not None else None
    bs = np.ascontiguousarray(bias, np.float32) if bias is not None else None
    lib().orc_linear_w8a8(x.ctypes.data, xs.reshape(-1), w.ctypes.data, ws.reshape(-1),
                          output.ctypes.data, ax.ctypes.data if ax is not None else None,
                          bs.ctypes.data if bs is not None else None, width, first_row, groups,
                          rows, columns, epilogue, block)
    return output


def embedding_w8(ids, weight, scales, hidden: int, first_row: int = 0, output=None):
    """embeddingW8 (Graph.metal:16-31): ids uint32 [tokens], weight int8
    [rows, groups * 32], scales fp16 bits [rows, groups]."""
    i = np.ascontiguousarray(ids, np.uint32)
    w = np.ascontiguousarray(weight, np.int8)
    sc = np.ascontiguousarray(scales, np.uint16)
    if output is None:
        output = np.zeros((i.size, hidden), np.uint16)
    lib().orc_embedding_w8(i.ctypes.data, w.ctypes.data, sc.reshape(-1), output.reshape(-1),
                           i.size, hidden, first_row, w.shape[0], sc.shape[1])
    return output


def embedding(ids, weight, first_row: int = 0, output=None):
    """embedding (Reference.metal:49-58): fp16 rows of weight [rows, hidden]."""
    i = np.ascontiguousarray(ids, np.uint32)
    w = np.ascontiguousarray(weight, np.uint16)
    if output is None:
        output = np.zeros((i.size, w.shape[1]), np.uint16)
    lib().orc_embedding(i.ctypes.data, w.reshape(-1), output.reshape(-1), i.size, w.shape[1],
                        first_row, w.shape[0])
    return output


ELEMENTWISE = {"add": 0, "swiglu": 1, "silu": 2, "multiply": 3}


def elementwise(kind: str, a, b=None) -> np.ndarray:
    """residualAdd / swiGlu / siluF16 / multiplyF16 (Reference.metal:119-135,
    Graph.metal:70-95) on fp16 bits."""
    x = np.ascontiguousarray(a, np.uint16)
    y = np.ascontiguousarray(b if b is not None else a, np.uint16)
    assert x.shape == y.shape
    out = np.empty(x.shape, np.uint16)
    lib().orc_elementwise(ELEMENTWISE[kind], x.reshape(-1), y.reshape(-1), out.reshape(-1),
                          x.size)
    return out


def copy_half_view(src, dims, strides, offset: int = 0) -> np.ndarray:
    """copyHalfView (Graph.metal:1-14): a dense copy of the view of fp16 bits
    with at most 3 dims (outermost first), strides and offset in elements."""
    s = np.ascontiguousarray(src, np.uint16).reshape(-1)
    d = [1] * (3 - len(dims)) + list(dims)
    st = [0] * (3 - len(strides)) + list(strides)
    count = int(np.prod(d))
    out = np.empty(count, np.uint16)
    D = (C.c_uint32 * 3)(*d)
    S = (C.c_uint32 * 3)(*st)
    lib().orc_copy_half_view(s, out, count, offset, D, S)
    return out.reshape(dims)


def linear_f16(x, weight, epilogue: int = LINEAR_NONE, block: int = 0, aux=None, bias=None,
               output=None, first_row: int = 0, output_width: int | None = None) -> np.ndarray:
    """linearF16 (Reference.metal:61-103): x fp16 bits [tokens, K], weight
    fp16 bits [columns, K]; one fp32 fma chain per output over k in order,
    then storeLinear."""
    a = np.ascontiguousarray(x, np.uint16)
    w = np.ascontiguousarray(weight, np.uint16)
    tokens, k = a.shape
    columns = w.shape[0]
    assert w.shape[1] == k
    width = output_width if output_width is not None else first_row + columns
    if output is None:
        dt = np.float32 if epilogue in F32_EPILOGUES else np.uint16
        output = np.zeros((tokens, width), dt)
    ax = np.ascontiguousarray(aux) if aux is not None else None
    bs = np.ascontiguousarray(bias, np.float32) if bias is not None else None
    lib().orc_linear_f16(a.reshape(-1), w.reshape(-1), output.ctypes.data,
                         ax.ctypes.data if ax is not None else None,
                         bs.ctypes.data if bs is not None else None, tokens, k, width,
                         first_row, columns, epilogue, block)
    return output


def l2norm_f32(x, width: int, eps: float = 1e-6, scale: float = 1.0) -> np.ndarray:
    a = np.ascontiguousarray(x, np.uint16)
    out = np.empty(a.shape, np.float32)
    lib().orc_l2norm_f32(a.reshape(-1), out.reshape(-1), a.size // width, width, eps, scale)
    return out


@dataclass
class DeltaInputs:
    q: np.ndarray      # [T, Hk*dk] fp32
    k: np.ndarray      # [T, Hk*dk] fp32
    v: np.ndarray      # [T, Hv*dv] fp16 bits
    beta: np.ndarray   # [T, Hv] fp32
    decay: np.ndarray  # [T, Hv] fp32 (linear)
    state: np.ndarray  # [Hv, dk, dv] fp32


def make_delta_inputs(seed: int, T: int, hk: int, dk: int, hv: int, dv: int,
                      state_std: float = 0.0) -> DeltaInputs:
    """cfg4/cfg5 DeltaNet operands, produced the way the reference graph does:
    L2Norm(q, eps 1e-6, scale 1/sqrt(dk)) and L2Norm(k) (Qwen35ModelBuilder.cpp:
    155-156, Graph.metal:96-109), gates via deltaGates with A_log = 0 and
    dt_bias = 0 (Graph.metal:131-144)."""
    qh = normal_f16(seed, 11, (T, hk * dk))
    kh = normal_f16(seed, 12, (T, hk * dk))
    v = normal_f16(seed, 13, (T, hv * dv))
    a = normal_f16(seed, 14, (T, hv))
    b = normal_f16(seed, 15, (T, hv))
    q = l2norm_f32(qh, dk, 1e-6, float(1.0 / np.sqrt(np.float32(dk))))
    k = l2norm_f32(kh, dk, 1e-6, 1.0)
    beta, decay = delta_gates(a, b, np.zeros(hv, np.float32), np.zeros(hv, np.float32))
    if state_std:
        state = normal_f32(seed, 16, (hv, dk, dv), 0.0, state_std)
    else:
        state = np.zeros((hv, dk, dv), np.float32)
    return DeltaInputs(q, k, v, beta, decay, state)


# ------------------------------------------------------------------ cost

def cost(kind: str, *dims: int) -> Cost:
    c = Cost()
    fn = {"kv_append": lib().orc_cost_kv_append,
          "causal_gqa": lib().orc_cost_causal_gqa,
          "delta_update": lib().orc_cost_delta_update}[kind]
    if fn(*dims, C.byref(c)) != 0:
        raise OverflowError(f"{kind} cost overflow")
    return c


def cpu_count() -> int:
    return lib().orc_cpu_count()
