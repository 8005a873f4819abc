"""Torch-tensor front end of the HIP backend (device memory and streams only).

Each function checks dtypes/layouts on the host, fills the reference's
parameter struct and calls the C ABI on torch's current HIP stream. The math
runs in the gfx950 kernels of libllminfer_hip.so; there is no other path.

Layouts follow the reference's op contracts (lib/GraphIR/Graph.cpp:226-279):
  q [T, Hq, d] fp16; caches [capacity, Hkv, d] fp16; out [T, Hq, d] fp16
  DeltaNet q, k [T, Hk*dk] fp32; v [T, Hv*dv] fp16; beta, decay [T, Hv] fp32;
  state [Hv, dk, dv] fp32 (in place); out [T, Hv*dv] fp16
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib

_workspaces: dict[tuple[int, str, int], torch.Tensor] = {}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _require(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def workspace(nbytes: int, device: torch.device | None = None, kind: str = "gqa") -> torch.Tensor:
    """A workspace of at least nbytes, reused per (device, kind, stream).
    Calls on one stream are ordered, so they can share it (its contents
    between calls do not matter); calls on different streams get different
    buffers, so they never write the same partials. Each buffer is
    allocated on its own stream, so when it grows torch's allocator hands
    the old memory only to later work on that same stream, after the
    kernels that used it."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(index)
    key = (index, kind, stream.cuda_stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        with torch.cuda.stream(stream):
            ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _workspaces[key] = ws
    return ws


def cache_append(src: torch.Tensor, cache: torch.Tensor, offset: int) -> None:
    """cache.view(-1)[offset : offset + src.numel()] = src (cacheAppend)."""
    _require(src, torch.float16, "src")
    _require(cache, torch.float16, "cache")
    if offset + src.numel() > cache.numel():
        raise ValueError("append exceeds the cache")
    lib = _lib.load()
    _lib.check(lib.llmi_hip_cache_append(_ptr(src), _ptr(cache),
                                         _lib.CacheParams(src.numel(), offset), _stream()))


def bind_norm_rope(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, past: int,
                   rotary_dim: int, epsilon: float = 1e-6, theta: float = 1e7,
                   head_dim: int | None = None, output_start: int = 0) -> "Bound":
    """normRope (Reference.metal:271-293): x [T, H, stride] fp16 (the first
    head_dim halves of each head are read; stride = 2 * head_dim for the
    projected q with its gate), weight [head_dim] fp32, out [>= output_start
    + T, H, head_dim] fp16, rows written from output_start (the key cache
    with output_start = past)."""
    _require(x, torch.float16, "x")
    _require(weight, torch.float32, "weight")
    _require(out, torch.float16, "out")
    if x.dim() != 3 or out.dim() != 3 or out.shape[1] != x.shape[1]:
        raise ValueError("x is [T, H, stride] and out [rows, H, head_dim]")
    T, H, stride = x.shape
    d = out.shape[2] if head_dim is None else head_dim
    if d != out.shape[2] or d > stride or weight.numel() != d:
        raise ValueError("head_dim must match out and weight and fit the stride")
    if output_start + T > out.shape[0]:
        raise ValueError("output rows exceed out")
    p = _lib.RopeParams(T, H, d, rotary_dim, stride, past, output_start, epsilon, theta)
    return Bound(_lib.load().llmi_hip_norm_rope, (_ptr(x), _ptr(weight), _ptr(out), p, _stream()),
                 kernel_names(_lib.OP_NORM_ROPE, p)[0] if T * H * d else "normRope")


def norm_rope(*args, **kwargs) -> None:
    bind_norm_rope(*args, **kwargs)()


def rms_norm(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor,
             epsilon: float = 1e-6) -> None:
    """rmsNorm (Reference.metal:105-117) over the last dimension."""
    for t, n in ((x, "x"), (out, "out")):
        _require(t, torch.float16, n)
    _require(weight, torch.float32, "weight")
    if x.shape != out.shape or weight.numel() != x.shape[-1]:
        raise ValueError("x, out and weight shapes disagree")
    width = x.shape[-1]
    p = _lib.RowParams(x.numel() // max(width, 1), width, epsilon)
    _lib.check(_lib.load().llmi_hip_rms_norm(_ptr(x), _ptr(weight), _ptr(out), p, _stream()))


def partial_rope(x: torch.Tensor, out: torch.Tensor, past: int, rotary_dim: int,
                 theta: float = 1e7) -> None:
    """partialRope (Graph.metal:111-129): x, out [T, H, width] fp16."""
    for t, n in ((x, "x"), (out, "out")):
        _require(t, torch.float16, n)
    if x.shape != out.shape or x.dim() != 3:
        raise ValueError("x and out are [T, H, width]")
    T, H, width = x.shape
    p = _lib.PartialRopeParams(T * H, H, width, rotary_dim, past, theta)
    _lib.check(_lib.load().llmi_hip_partial_rope(_ptr(x), _ptr(out), p, _stream()))


def bind_sigmoid_mul(gate: torch.Tensor, x: torch.Tensor, out: torch.Tensor) -> "Bound":
    for t, n in ((gate, "gate"), (x, "x"), (out, "out")):
        _require(t, torch.float16, n)
    if gate.numel() != x.numel() or out.numel() != x.numel():
        raise ValueError("gate, x and out must have the same size")
    p = _lib.ElementParams(x.numel())
    return Bound(_lib.load().llmi_hip_sigmoid_mul, (_ptr(gate), _ptr(x), _ptr(out), p, _stream()),
                 kernel_names(_lib.OP_SIGMOID_MUL, p)[0] if x.numel() else "sigmoidMul")


def sigmoid_mul(gate: torch.Tensor, x: torch.Tensor, out: torch.Tensor) -> None:
    """sigmoidMul (Graph.metal:78-85): out = fp16(fp16(sigmoid(gate)) * x)."""
    bind_sigmoid_mul(gate, x, out)()


# ------------------------------------------------------ W8A8 projections

def bind_quantize_activation(x: torch.Tensor, q: torch.Tensor, scales: torch.Tensor,
                             invalid: torch.Tensor | None = None) -> "Bound":
    """quantizeActivation (Graph.metal:33-68): x [rows, width] fp16 -> q [rows,
    groups * 32] int8, scales [rows, groups] fp32; invalid (int32, one
    element) gets bit 0 set by a group holding a non-finite value."""
    _require(x, torch.float16, "x")
    _require(q, torch.int8, "q")
    _require(scales, torch.float32, "scales")
    if x.dim() != 2:
        raise ValueError("x is [rows, width]")
    rows, width = x.shape
    groups = (width + 31) // 32
    if tuple(q.shape) != (rows, groups * 32) or tuple(scales.shape) != (rows, groups):
        raise ValueError("q is [rows, groups * 32] and scales [rows, groups]")
    if invalid is not None:
        _require(invalid, torch.int32, "invalid")
    p = _lib.QuantizeParams(rows, width, groups)
    return Bound(_lib.load().llmi_hip_quantize_activation,
                 (_ptr(x), _ptr(q), _ptr(scales), _ptr(invalid), p, _stream()),
                 "quantizeActivation")


def quantize_activation(*args) -> None:
    bind_quantize_activation(*args)()


_F32_EPILOGUES = (_lib.LINEAR_SILU_F32, _lib.LINEAR_DELTA_BETA, _lib.LINEAR_DELTA_DECAY)


def bind_linear_w8a8(q: torch.Tensor, scales: torch.Tensor, weight: torch.Tensor,
                     weight_scales: torch.Tensor, out: torch.Tensor,
                     epilogue: int = _lib.LINEAR_NONE, block: int = 0,
                     aux: torch.Tensor | None = None, bias: torch.Tensor | None = None,
                     first_row: int = 0) -> "Bound":
    """linearW8A8Gemv / Gemm (W8A8.metal:28-113) with storeLinear
    (Reference.metal:14-47): q [rows, groups * 32] int8, scales [rows, groups]
    fp32, weight [columns, groups * 32] int8, weight_scales [columns, groups]
    fp16; out [rows, width] fp16 (fp32 for the SiluF32, DeltaBeta and
    DeltaDecay epilogues), columns first_row .. first_row + columns - 1
    written. aux: fp16 like out (SiluMul) or fp32 A_log [width]
    (DeltaDecay); bias: fp32 [width] (DeltaDecay)."""
    _require(q, torch.int8, "q")
    _require(scales, torch.float32, "scales")
    _require(weight, torch.int8, "weight")
    _require(weight_scales, torch.float16, "weight_scales")
    _require(out, torch.float32 if epilogue in _F32_EPILOGUES else torch.float16, "out")
    rows, groups = scales.shape
    columns = weight.shape[0]
    if tuple(q.shape) != (rows, groups * 32) or tuple(weight.shape) != (columns, groups * 32) \
            or tuple(weight_scales.shape) != (columns, groups) or out.dim() != 2 \
            or out.shape[0] != rows:
        raise ValueError("q, scales, weight, weight_scales and out shapes disagree")
    if aux is not None:
        _require(aux, aux.dtype, "aux")
    if bias is not None:
        _require(bias, torch.float32, "bias")
    p = _lib.LinearW8Params(out.shape[1], first_row, groups, rows, columns, epilogue, block)
    return Bound(_lib.load().llmi_hip_linear_w8a8,
                 (_ptr(q), _ptr(scales), _ptr(weight), _ptr(weight_scales), _ptr(out), _ptr(aux),
                  _ptr(bias), p, _stream()),
                 "linearW8A8Gemv" if rows == 1 else "linearW8A8Gemm")


def linear_w8a8(*args, **kwargs) -> None:
    bind_linear_w8a8(*args, **kwargs)()


def bind_embedding_w8(ids: torch.Tensor, weight: torch.Tensor, scales: torch.Tensor,
                      out: torch.Tensor, first_row: int = 0) -> "Bound":
    """embeddingW8 (Graph.metal:16-31): ids int32 [tokens] (read as uint32),
    weight [rows, groups * 32] int8, scales [rows, groups] fp16, out [tokens,
    hidden] fp16 (rows of other shards' ids untouched)."""
    _require(ids, torch.int32, "ids")
    _require(weight, torch.int8, "weight")
    _require(scales, torch.float16, "scales")
    _require(out, torch.float16, "out")
    rows, groups = scales.shape
    if out.dim() != 2 or out.shape[0] != ids.numel() or tuple(weight.shape) != (rows, groups * 32):
        raise ValueError("ids, weight, scales and out shapes disagree")
    p = _lib.GroupedEmbedParams(ids.numel(), out.shape[1], first_row, rows, groups)
    return Bound(_lib.load().llmi_hip_embedding_w8,
                 (_ptr(ids), _ptr(weight), _ptr(scales), _ptr(out), p, _stream()), "embeddingW8")


def embedding_w8(*args, **kwargs) -> None:
    bind_embedding_w8(*args, **kwargs)()


def bind_embedding(ids: torch.Tensor, weight: torch.Tensor, out: torch.Tensor,
                   first_row: int = 0) -> "Bound":
    """embedding (Reference.metal:49-58): fp16 weight rows [rows, hidden]."""
    _require(ids, torch.int32, "ids")
    _require(weight, torch.float16, "weight")
    _require(out, torch.float16, "out")
    if out.dim() != 2 or out.shape[0] != ids.numel() or weight.shape[1] != out.shape[1]:
        raise ValueError("ids, weight and out shapes disagree")
    p = _lib.EmbedParams(ids.numel(), out.shape[1], first_row, weight.shape[0])
    return Bound(_lib.load().llmi_hip_embedding, (_ptr(ids), _ptr(weight), _ptr(out), p,
                                                  _stream()), "embedding")


def embedding(*args, **kwargs) -> None:
    bind_embedding(*args, **kwargs)()


# ------------------------------------ elementwise, views, fp16 projections

_ELEMENTWISE = {"add": ("llmi_hip_residual_add", "residualAdd"),
                "swiglu": ("llmi_hip_swiglu", "swiGlu"),
                "multiply": ("llmi_hip_multiply", "multiplyF16")}


def bind_elementwise(kind: str, a: torch.Tensor, b: torch.Tensor | None,
                     out: torch.Tensor) -> "Bound":
    """residualAdd (a + b), swiGlu (fp16(silu(a)) * b), multiplyF16 (a * b)
    or siluF16 (silu(a), kind "silu", b unused): fp16 tensors of one size
    (Reference.metal:119-135, Graph.metal:70-95)."""
    operands = ((a, "a"), (out, "out")) if kind == "silu" else ((a, "a"), (b, "b"), (out, "out"))
    for t, n in operands:
        _require(t, torch.float16, n)
    if out.numel() != a.numel() or (kind != "silu" and b.numel() != a.numel()):
        raise ValueError("operands and out must have the same size")
    p = _lib.ElementParams(a.numel())
    if kind == "silu":
        return Bound(_lib.load().llmi_hip_silu, (_ptr(a), _ptr(out), p, _stream()), "siluF16")
    fn, name = _ELEMENTWISE[kind]
    return Bound(getattr(_lib.load(), fn), (_ptr(a), _ptr(b), _ptr(out), p, _stream()), name)


def elementwise(kind: str, a: torch.Tensor, b: torch.Tensor | None, out: torch.Tensor) -> None:
    bind_elementwise(kind, a, b, out)()


def bind_copy_half_view(src: torch.Tensor, out: torch.Tensor, dims, strides,
                        offset: int = 0) -> "Bound":
    """copyHalfView (Graph.metal:1-14): out (dense, fp16) = the view of src
    with up to 3 dims (outermost first), strides and offset in elements."""
    _require(src, torch.float16, "src")
    _require(out, torch.float16, "out")
    d = [1] * (3 - len(dims)) + [int(x) for x in dims]
    st = [0] * (3 - len(strides)) + [int(x) for x in strides]
    count = d[0] * d[1] * d[2]
    if out.numel() != count:
        raise ValueError("out must hold the view's elements")
    if offset + sum((x - 1) * y for x, y in zip(d, st)) >= src.numel():
        raise ValueError("the view reaches past src")
    p = _lib.HalfViewParams(count, offset, (C.c_uint * 3)(*d), (C.c_uint * 3)(*st))
    return Bound(_lib.load().llmi_hip_copy_half_view, (_ptr(src), _ptr(out), p, _stream()),
                 "copyHalfView")


def copy_half_view(*args, **kwargs) -> None:
    bind_copy_half_view(*args, **kwargs)()


def bind_linear_f16(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor,
                    epilogue: int = _lib.LINEAR_NONE, block: int = 0,
                    aux: torch.Tensor | None = None, bias: torch.Tensor | None = None,
                    first_row: int = 0) -> "Bound":
    """linearF16 (Reference.metal:61-103) with storeLinear: x [tokens, K]
    fp16, weight [columns, K] fp16, out [tokens, width] (fp32 for the fp32
    epilogues), columns first_row .. first_row + columns - 1 written."""
    _require(x, torch.float16, "x")
    _require(weight, torch.float16, "weight")
    _require(out, torch.float32 if epilogue in _F32_EPILOGUES else torch.float16, "out")
    if x.dim() != 2 or weight.dim() != 2 or weight.shape[1] != x.shape[1] or out.dim() != 2 \
            or out.shape[0] != x.shape[0]:
        raise ValueError("x [tokens, K], weight [columns, K] and out [tokens, width] disagree")
    tokens, k = x.shape
    p = _lib.LinearParams(tokens, k, out.shape[1], first_row, weight.shape[0], epilogue, block)
    return Bound(_lib.load().llmi_hip_linear_f16,
                 (_ptr(x), _ptr(weight), _ptr(out), _ptr(aux), _ptr(bias), p, _stream()),
                 "linearF16")


def linear_f16(*args, **kwargs) -> None:
    bind_linear_f16(*args, **kwargs)()


def bind_add_rms_norm_quantize(a: torch.Tensor, b: torch.Tensor | None,
                               sum_out: torch.Tensor | None, weight: torch.Tensor,
                               q: torch.Tensor, scales: torch.Tensor,
                               invalid: torch.Tensor | None = None,
                               epsilon: float = 1e-6) -> "Bound":
    """residualAdd -> rmsNorm -> quantizeActivation in one launch: a, b,
    sum_out [rows, width] fp16 (b None: normalise a); weight [width] fp32;
    q [rows, groups * 32] int8, scales [rows, groups] fp32."""
    _require(a, torch.float16, "a")
    if b is not None:
        _require(b, torch.float16, "b")
        _require(sum_out, torch.float16, "sum_out")
    _require(weight, torch.float32, "weight")
    _require(q, torch.int8, "q")
    _require(scales, torch.float32, "scales")
    rows, width = a.shape
    groups = (width + 31) // 32
    if (b is not None and (b.shape != a.shape or sum_out.shape != a.shape)) or \
            weight.numel() != width or tuple(q.shape) != (rows, groups * 32) or \
            tuple(scales.shape) != (rows, groups):
        raise ValueError("a, b, sum_out [rows, width], weight [width], q, scales disagree")
    if invalid is not None:
        _require(invalid, torch.int32, "invalid")
    p = _lib.RowParams(rows, width, epsilon)
    return Bound(_lib.load().llmi_hip_add_rms_norm_quantize,
                 (_ptr(a), _ptr(b), _ptr(sum_out), _ptr(weight), _ptr(q), _ptr(scales),
                  _ptr(invalid), p, _stream()), "addRmsNormQuantize")


def add_rms_norm_quantize(*args, **kwargs) -> None:
    bind_add_rms_norm_quantize(*args, **kwargs)()


def bind_add_rms_norm_linear_w8a8(a: torch.Tensor, b: torch.Tensor | None,
                                  sum_out: torch.Tensor | None, weight: torch.Tensor,
                                  projections: list, q: torch.Tensor | None = None,
                                  scales: torch.Tensor | None = None,
                                  invalid: torch.Tensor | None = None,
                                  epsilon: float = 1e-6) -> "Bound":
    """add_rms_norm_quantize of one row, then linear_w8a8 of each projection
    on the quantized row, in one launch. a, b, sum_out [1, width] fp16;
    projections: up to 4 dicts with weight, weight_scales, out and optionally
    epilogue, block, aux, bias, first_row (as for linear_w8a8; a SwiGLU
    projection follows its multiplier's projection and takes its out as
    aux) and conv_weight [columns, 4], conv_history [columns, 3] (fp16: the
    row then passes through the one-token causal_conv with SiLU, history
    updated, as causal_conv leaves it); q, scales as for
    add_rms_norm_quantize or None."""
    _require(a, torch.float16, "a")
    if b is not None:
        _require(b, torch.float16, "b")
        _require(sum_out, torch.float16, "sum_out")
    _require(weight, torch.float32, "weight")
    rows, width = a.shape
    groups = (width + 31) // 32
    if (b is not None and (b.shape != a.shape or sum_out.shape != a.shape)) or \
            weight.numel() != width:
        raise ValueError("a, b, sum_out [1, width] and weight [width] disagree")
    if q is not None:
        _require(q, torch.int8, "q")
        _require(scales, torch.float32, "scales")
        if tuple(q.shape) != (rows, groups * 32) or tuple(scales.shape) != (rows, groups):
            raise ValueError("q [rows, groups * 32] and scales [rows, groups] disagree")
    if invalid is not None:
        _require(invalid, torch.int32, "invalid")
    if not 1 <= len(projections) <= _lib.NORM_LINEAR_MAX:
        raise ValueError(f"1 to {_lib.NORM_LINEAR_MAX} projections")
    bufs = (_lib.NormProjection * _lib.NORM_LINEAR_MAX)()
    p = _lib.NormLinearParams()
    p.norm = _lib.RowParams(rows, width, epsilon)
    p.count = len(projections)
    for k, x in enumerate(projections):
        w, ws, out = x["weight"], x["weight_scales"], x["out"]
        epilogue = x.get("epilogue", _lib.LINEAR_NONE)
        _require(w, torch.int8, "weight")
        _require(ws, torch.float16, "weight_scales")
        _require(out, torch.float32 if epilogue in _F32_EPILOGUES else torch.float16, "out")
        columns = w.shape[0]
        if tuple(w.shape) != (columns, groups * 32) or tuple(ws.shape) != (columns, groups) \
                or out.dim() != 2 or out.shape[0] != rows:
            raise ValueError(f"projection {k}: weight, weight_scales and out shapes disagree")
        aux, bias = x.get("aux"), x.get("bias")
        cw, ch = x.get("conv_weight"), x.get("conv_history")
        if cw is not None:
            _require(cw, torch.float16, "conv_weight")
            _require(ch, torch.float16, "conv_history")
            if tuple(cw.shape) != (columns, 4) or tuple(ch.shape) != (columns, 3) or \
                    tuple(out.shape) != (1, columns):
                raise ValueError(f"projection {k}: conv_weight [columns, 4], conv_history "
                                 "[columns, 3] and out [1, columns] disagree")
        bufs[k] = _lib.NormProjection(_ptr(w), _ptr(ws), _ptr(out), _ptr(aux), _ptr(bias),
                                      _ptr(cw), _ptr(ch))
        p.linear[k] = _lib.LinearW8Params(out.shape[1], x.get("first_row", 0), groups, rows,
                                          columns, epilogue, x.get("block", 0))
    bound = Bound(_lib.load().llmi_hip_add_rms_norm_linear_w8a8,
                  (_ptr(a), _ptr(b), _ptr(sum_out), _ptr(weight), _ptr(q), _ptr(scales),
                   _ptr(invalid), C.addressof(bufs), p, _stream()), "addRmsNormLinearW8A8")
    bound.keep = bufs  # the projection table the call points at
    return bound


def add_rms_norm_linear_w8a8(*args, **kwargs) -> None:
    bind_add_rms_norm_linear_w8a8(*args, **kwargs)()


def gated_rms_norm_activated_quantize(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor,
                                      out: torch.Tensor, q: torch.Tensor, scales: torch.Tensor,
                                      invalid: torch.Tensor | None = None,
                                      epsilon: float = 1e-6) -> None:
    """gated_rms_norm_activated of x [rows, width] (gate fp32, weight [width]
    fp32) into out, and quantize_activation of out's flattened rows into q
    [n * 32] int8 and scales [n] fp32, n = rows * width / 32, one launch."""
    _require(x, torch.float16, "x")
    _require(gate, torch.float32, "gate")
    _require(weight, torch.float32, "weight")
    _require(out, torch.float16, "out")
    _require(q, torch.int8, "q")
    _require(scales, torch.float32, "scales")
    rows, width = x.shape
    if gate.shape != x.shape or out.shape != x.shape or weight.numel() != width or \
            q.numel() != rows * width or scales.numel() * 32 != rows * width:
        raise ValueError("x, gate, out [rows, width], weight [width], q, scales disagree")
    if invalid is not None:
        _require(invalid, torch.int32, "invalid")
    _lib.check(_lib.load().llmi_hip_gated_rms_norm_activated_quantize(
        _ptr(x), _ptr(gate), _ptr(weight), _ptr(out), _ptr(q), _ptr(scales), _ptr(invalid),
        _lib.RowParams(rows, width, epsilon), _stream()))


def bind_causal_conv(x: torch.Tensor, weight: torch.Tensor, history: torch.Tensor | None,
                     out: torch.Tensor, silu: bool = True) -> "Bound":
    """causalConv (Reference.metal:137-161): x, out [T, C] fp16; weight [C, k]
    fp16; history [C, k-1] fp16, updated in place."""
    for t, n in ((x, "x"), (weight, "weight"), (out, "out")):
        _require(t, torch.float16, n)
    if x.dim() != 2 or out.shape != x.shape or weight.dim() != 2 or weight.shape[0] != x.shape[1]:
        raise ValueError("x, out are [T, C] and weight [C, k]")
    T, Cn = x.shape
    k = weight.shape[1]
    if k > 1:
        if history is None:
            raise ValueError("history is required for k > 1")
        _require(history, torch.float16, "history")
        if tuple(history.shape) != (Cn, k - 1):
            raise ValueError("history is [C, k-1]")
    p = _lib.ConvParams(T, Cn, k, int(silu))
    return Bound(_lib.load().llmi_hip_causal_conv,
                 (_ptr(x), _ptr(weight), _ptr(history), _ptr(out), p, _stream()), "causalConv")


def causal_conv(*args, **kwargs) -> None:
    bind_causal_conv(*args, **kwargs)()


def bind_l2_norm(x: torch.Tensor, out: torch.Tensor, width: int, epsilon: float = 1e-6,
                 scale: float = 1.0) -> "Bound":
    """l2NormF32 (Graph.metal:96-109): groups of `width` fp16 values -> fp32."""
    _require(x, torch.float16, "x")
    _require(out, torch.float32, "out")
    if out.numel() != x.numel() or width <= 0 or x.numel() % width:
        raise ValueError("x and out must hold whole rows of `width`")
    p = _lib.L2Params(x.numel() // width, width, epsilon, scale)
    return Bound(_lib.load().llmi_hip_l2_norm, (_ptr(x), _ptr(out), p, _stream()),
                 kernel_names(_lib.OP_L2_NORM, p)[0] if x.numel() else "l2Norm")


def l2_norm(*args, **kwargs) -> None:
    bind_l2_norm(*args, **kwargs)()


def bind_delta_gates(a: torch.Tensor, b: torch.Tensor, a_log: torch.Tensor,
                     dt_bias: torch.Tensor, beta: torch.Tensor, decay: torch.Tensor) -> "Bound":
    """deltaGates (Graph.metal:131-144): a, b [T, Hv] fp16; a_log, dt_bias
    [Hv] fp32; beta, decay [T, Hv] fp32."""
    for t, n in ((a, "a"), (b, "b")):
        _require(t, torch.float16, n)
    for t, n in ((a_log, "a_log"), (dt_bias, "dt_bias"), (beta, "beta"), (decay, "decay")):
        _require(t, torch.float32, n)
    if a.dim() != 2 or b.shape != a.shape or beta.shape != a.shape or decay.shape != a.shape \
            or a_log.numel() != a.shape[1] or dt_bias.numel() != a.shape[1]:
        raise ValueError("gate operand shapes disagree")
    p = _lib.RowParams(a.shape[0], a.shape[1], 0.0)
    return Bound(_lib.load().llmi_hip_delta_gates,
                 (_ptr(a), _ptr(b), _ptr(a_log), _ptr(dt_bias), _ptr(beta), _ptr(decay), p,
                  _stream()), "deltaGates")


def delta_gates(*args) -> None:
    bind_delta_gates(*args)()


def bind_gated_rms_norm(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor,
                        out: torch.Tensor, epsilon: float = 1e-6) -> "Bound":
    """gatedRmsNorm (Reference.metal:228-259) over the last dimension: gate
    fp16 (through SiLU) or fp32 (already activated, gatedRmsNormActivated)."""
    _require(x, torch.float16, "x")
    _require(out, torch.float16, "out")
    _require(weight, torch.float32, "weight")
    if gate.dtype not in (torch.float16, torch.float32):
        raise ValueError("gate must be float16 or float32")
    _require(gate, gate.dtype, "gate")
    width = x.shape[-1]
    if gate.shape != x.shape or out.shape != x.shape or weight.numel() != width:
        raise ValueError("x, gate, out and weight shapes disagree")
    p = _lib.RowParams(x.numel() // max(width, 1), width, epsilon)
    lib = _lib.load()
    fn = lib.llmi_hip_gated_rms_norm if gate.dtype == torch.float16 \
        else lib.llmi_hip_gated_rms_norm_activated
    return Bound(fn, (_ptr(x), _ptr(gate), _ptr(weight), _ptr(out), p, _stream()),
                 "gatedRmsNormTile")


def gated_rms_norm(*args, **kwargs) -> None:
    bind_gated_rms_norm(*args, **kwargs)()


def kv_append(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
              v_cache: torch.Tensor, past: int) -> None:
    """KvAppend: rows [past, past+T) of both caches <- k, v ([T, Hkv, d])."""
    for t, n in ((k, "k"), (v, "v"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _require(t, torch.float16, n)
    if k.shape != v.shape or k.dim() != 3 or k_cache.shape != v_cache.shape \
            or k.shape[1:] != k_cache.shape[1:]:
        raise ValueError("new keys and values must match the cache layout")
    T, hkv, d = k.shape
    if past + T > k_cache.shape[0]:
        raise ValueError("append exceeds the cache capacity")
    lib = _lib.load()
    p = _lib.CacheParams(T * hkv * d, past * hkv * d)
    _lib.check(lib.llmi_hip_kv_append(_ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache),
                                      p, _stream()))


def gqa_params(q: torch.Tensor, k_cache: torch.Tensor, past: int) -> _lib.GqaParams:
    T, hq, d = q.shape
    return _lib.GqaParams(T, hq, k_cache.shape[1], d, past)


def causal_gqa(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
               past: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """CausalGqa over cache rows [0, past+T) (the step's rows already appended)."""
    _require(q, torch.float16, "q")
    _require(k_cache, torch.float16, "k_cache")
    _require(v_cache, torch.float16, "v_cache")
    if q.dim() != 3 or k_cache.dim() != 3 or k_cache.shape != v_cache.shape \
            or q.shape[2] != k_cache.shape[2]:
        raise ValueError("invalid attention head shape")
    if past + q.shape[0] > k_cache.shape[0]:
        raise ValueError("past + tokens exceeds the cache capacity")
    if out is None:
        out = torch.empty_like(q)
    _require(out, torch.float16, "out")
    lib = _lib.load()
    p = gqa_params(q, k_cache, past)
    need = lib.llmi_hip_gqa_workspace_bytes(p)
    ws = workspace(need, q.device) if need else None
    _lib.check(lib.llmi_hip_causal_gqa(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out),
                                       p, _ptr(ws), ws.numel() if ws is not None else 0,
                                       _stream()))
    return out


def kv_append_causal_gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         k_cache: torch.Tensor, v_cache: torch.Tensor, past: int,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """KvAppend(k, v) at row `past` then CausalGqa(q), in one call (one launch
    for T == 1: the decode kernel appends while it attends)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _require(t, torch.float16, n)
    if q.dim() != 3 or k.dim() != 3 or k.shape != v.shape or k_cache.shape != v_cache.shape \
            or k.shape[1:] != k_cache.shape[1:] or q.shape[0] != k.shape[0] \
            or q.shape[2] != k_cache.shape[2]:
        raise ValueError("KvAppend/CausalGqa operands do not match the cache layout")
    if past + q.shape[0] > k_cache.shape[0]:
        raise ValueError("past + tokens exceeds the cache capacity")
    if out is None:
        out = torch.empty_like(q)
    _require(out, torch.float16, "out")
    lib = _lib.load()
    p = gqa_params(q, k_cache, past)
    need = lib.llmi_hip_gqa_workspace_bytes(p)
    ws = workspace(need, q.device) if need else None
    _lib.check(lib.llmi_hip_kv_append_causal_gqa(
        _ptr(q), _ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache), _ptr(out), p, _ptr(ws),
        ws.numel() if ws is not None else 0, _stream()))
    return out


def delta_params(q: torch.Tensor, v: torch.Tensor, state: torch.Tensor) -> _lib.GraphDeltaParams:
    hv, dk, dv = state.shape
    return _lib.GraphDeltaParams(q.shape[0], q.shape[1] // dk, dk, hv, dv)


def delta_update(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                 decay: torch.Tensor, state: torch.Tensor,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """DeltaUpdate: gated delta rule over T tokens, state updated in place."""
    for t, n, dt in ((q, "q", torch.float32), (k, "k", torch.float32),
                     (v, "v", torch.float16), (beta, "beta", torch.float32),
                     (decay, "decay", torch.float32), (state, "state", torch.float32)):
        _require(t, dt, n)
    T = q.shape[0]
    hv, dk, dv = state.shape
    if q.dim() != 2 or k.shape != q.shape or q.shape[1] % dk or \
            hv % (q.shape[1] // dk) or v.shape != (T, hv * dv) or \
            beta.shape != (T, hv) or decay.shape != beta.shape:
        raise ValueError("DeltaUpdate operand shapes do not match its recurrent state")
    if out is None:
        out = torch.empty_like(v)
    _require(out, torch.float16, "out")
    lib = _lib.load()
    p = delta_params(q, v, state)
    need = lib.llmi_hip_delta_workspace_bytes(p)
    ws = workspace(need, q.device, "delta") if need else None
    _lib.check(lib.llmi_hip_delta_update(_ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(decay),
                                         _ptr(state), _ptr(out), p, _ptr(ws),
                                         ws.numel() if ws is not None else 0, _stream()))
    return out


def bind_gated_attention(q_proj: torch.Tensor, k_proj: torch.Tensor, v_new: torch.Tensor,
                         q_weight: torch.Tensor, k_weight: torch.Tensor, k_cache: torch.Tensor,
                         v_cache: torch.Tensor, out: torch.Tensor, past: int, rotary_dim: int,
                         epsilon: float = 1e-6, theta: float = 1e7,
                         activated: bool = False) -> "Bound":
    """The attention block around CausalGqa in one call (llmi_hip_gated_attention):
    q_proj [T, Hq, 2d] (per head d query then d gate values), k_proj and v_new
    [T, Hkv, d], norm weights [d] fp32, caches [capacity, Hkv, d], out
    [T, Hq, d]: normRope(q), normRope(k) into the cache at row past, V
    appended, CausalGqa, sigmoid gate. activated: the gate values are already
    fp16(logistic(.)) and the output is their product with the attention
    (llmi_hip_gated_attention_activated)."""
    for t, n in ((q_proj, "q_proj"), (k_proj, "k_proj"), (v_new, "v_new"),
                 (k_cache, "k_cache"), (v_cache, "v_cache"), (out, "out")):
        _require(t, torch.float16, n)
    for t, n in ((q_weight, "q_weight"), (k_weight, "k_weight")):
        _require(t, torch.float32, n)
    if q_proj.dim() != 3 or k_proj.dim() != 3 or v_new.shape != k_proj.shape or \
            k_cache.shape != v_cache.shape or k_cache.shape[1:] != k_proj.shape[1:]:
        raise ValueError("gated attention operands disagree")
    T, hq, d2 = q_proj.shape
    d = d2 // 2
    hkv = k_proj.shape[1]
    if d2 != 2 * d or k_proj.shape[0] != T or k_proj.shape[2] != d or \
            out.shape != (T, hq, d) or q_weight.numel() != d or k_weight.numel() != d or \
            past + T > k_cache.shape[0]:
        raise ValueError("gated attention shapes do not match the cache")
    lib = _lib.load()
    p = _lib.GqaParams(T, hq, hkv, d, past)
    need = lib.llmi_hip_gqa_workspace_bytes(p)
    ws = workspace(need, q_proj.device) if need else None
    args = (_ptr(q_proj), _ptr(k_proj), _ptr(v_new), _ptr(q_weight), _ptr(k_weight),
            _ptr(k_cache), _ptr(v_cache), _ptr(out), p, rotary_dim, epsilon, theta, _ptr(ws),
            ws.numel() if ws is not None else 0, _stream())
    names = kernel_names(_lib.OP_GATED_ATTENTION, p)
    fn = lib.llmi_hip_gated_attention_activated if activated else lib.llmi_hip_gated_attention
    b = Bound(fn, args, "+".join(names))
    b._keep = ws
    return b


def gated_attention(q_proj, k_proj, v_new, q_weight, k_weight, k_cache, v_cache, past: int,
                    rotary_dim: int, epsilon: float = 1e-6, theta: float = 1e7,
                    out: torch.Tensor | None = None, activated: bool = False) -> torch.Tensor:
    """bind_gated_attention, called once."""
    if out is None:
        T, hq, d2 = q_proj.shape
        out = torch.empty((T, hq, d2 // 2), dtype=torch.float16, device=q_proj.device)
    bind_gated_attention(q_proj, k_proj, v_new, q_weight, k_weight, k_cache, v_cache, out,
                         past, rotary_dim, epsilon, theta, activated)()
    return out


def bind_l2_norm_delta_update(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                              beta: torch.Tensor, decay: torch.Tensor, state: torch.Tensor,
                              out: torch.Tensor, epsilon: float = 1e-6,
                              q_scale: float | None = None) -> "Bound":
    """L2Norm(q, epsilon, q_scale), L2Norm(k, epsilon, 1) and DeltaUpdate in one
    call: q, k [T, Hk*dk] fp16 rows (l2NormF32, Graph.metal:96-109, before
    graphDeltaUpdate). q_scale defaults to 1/sqrt(dk) as the builder emits it
    (Qwen35ModelBuilder.cpp:155-156)."""
    for t, n, dt in ((q, "q", torch.float16), (k, "k", torch.float16),
                     (v, "v", torch.float16), (beta, "beta", torch.float32),
                     (decay, "decay", torch.float32), (state, "state", torch.float32),
                     (out, "out", torch.float16)):
        _require(t, dt, n)
    T = q.shape[0]
    hv, dk, dv = state.shape
    if q.dim() != 2 or k.shape != q.shape or q.shape[1] % dk or \
            hv % (q.shape[1] // dk) or v.shape != (T, hv * dv) or \
            beta.shape != (T, hv) or decay.shape != beta.shape or out.shape != v.shape:
        raise ValueError("DeltaUpdate operand shapes do not match its recurrent state")
    if q_scale is None:  # 1.0f / std::sqrt(float(keyDim)), both in fp32
        q_scale = float(np.float32(1.0) / np.sqrt(np.float32(dk)))
    lib = _lib.load()
    p = delta_params(q, v, state)
    need = lib.llmi_hip_delta_workspace_bytes(p)
    ws = workspace(need, q.device, "delta") if need else None
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(decay), _ptr(state), _ptr(out),
            p, epsilon, q_scale, _ptr(ws), ws.numel() if ws is not None else 0, _stream())
    names = kernel_names(_lib.OP_DELTA_UPDATE, p)
    b = Bound(lib.llmi_hip_l2_norm_delta_update, args, "+".join(names))
    b._keep = ws
    return b


def l2_norm_delta_update(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                         decay: torch.Tensor, state: torch.Tensor,
                         out: torch.Tensor | None = None, epsilon: float = 1e-6,
                         q_scale: float | None = None) -> torch.Tensor:
    """The fused L2Norm -> DeltaUpdate pair (bind_l2_norm_delta_update)."""
    if out is None:
        out = torch.empty_like(v)
    bind_l2_norm_delta_update(q, k, v, beta, decay, state, out, epsilon, q_scale)()
    return out


def bind_l2_norm_delta_gated_norm(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                  beta: torch.Tensor, decay: torch.Tensor, state: torch.Tensor,
                                  gate: torch.Tensor, norm_weight: torch.Tensor,
                                  out: torch.Tensor, epsilon: float = 1e-6,
                                  q_scale: float | None = None,
                                  norm_epsilon: float = 1e-6) -> "Bound":
    """L2Norm(q), L2Norm(k), DeltaUpdate and GatedRmsNorm(out, gate,
    norm_weight, norm_epsilon) in one call (Qwen35ModelBuilder.cpp:155-166):
    operands as bind_l2_norm_delta_update, gate fp16 like v, norm_weight fp32
    [dv]; out receives the normalised rows."""
    _require(gate, torch.float16, "gate")
    _require(norm_weight, torch.float32, "norm_weight")
    hv, dk, dv = state.shape
    if gate.shape != v.shape or norm_weight.numel() != dv:
        raise ValueError("gate must match v and norm_weight have dv elements")
    inner = bind_l2_norm_delta_update(q, k, v, beta, decay, state, out, epsilon, q_scale)
    a = inner._args
    lib = _lib.load()
    args = a[:6] + (_ptr(gate), _ptr(norm_weight)) + a[6:10] + (norm_epsilon,) + a[10:]
    b = Bound(lib.llmi_hip_l2_norm_delta_gated_norm, args, inner.what + "+gatedRmsNorm")
    b._keep = inner._keep
    # the chunked form's bounded arrival wait: its give-up, read after a call
    b.status_args = (a[10], a[11], a[7], a[12])
    return b


def gated_norm_status(b: "Bound") -> None:
    """Waits for the stream of a bind_l2_norm_delta_gated_norm call and raises
    HipError (LAUNCH_FAILED) if the chunked scan's arrival wait gave up."""
    _lib.check(_lib.load().llmi_hip_l2_norm_delta_gated_norm_status(*b.status_args))


def l2_norm_delta_gated_norm(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                             beta: torch.Tensor, decay: torch.Tensor, state: torch.Tensor,
                             gate: torch.Tensor, norm_weight: torch.Tensor,
                             out: torch.Tensor | None = None, epsilon: float = 1e-6,
                             q_scale: float | None = None,
                             norm_epsilon: float = 1e-6, check: bool = True) -> torch.Tensor:
    """The fused L2Norm -> DeltaUpdate -> GatedRmsNorm chain
    (bind_l2_norm_delta_gated_norm). With `check` it waits for the call and
    raises if the chunked scan's arrival wait gave up (gated_norm_status)."""
    if out is None:
        out = torch.empty_like(v)
    b = bind_l2_norm_delta_gated_norm(q, k, v, beta, decay, state, gate, norm_weight, out,
                                      epsilon, q_scale, norm_epsilon)
    b()
    if check:
        gated_norm_status(b)
    return out


def bind_l2_norm_delta_gated_norm_activated_quantize(
        q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
        decay: torch.Tensor, state: torch.Tensor, gate: torch.Tensor, norm_weight: torch.Tensor,
        out: torch.Tensor, quantized: torch.Tensor, scales: torch.Tensor,
        invalid: torch.Tensor | None = None, epsilon: float = 1e-6,
        q_scale: float | None = None, norm_epsilon: float = 1e-6) -> "Bound":
    """The W8A8 DeltaNet tail in one call: L2Norm(q), L2Norm(k), DeltaUpdate,
    GatedRmsNorm with the fp32 activated gate (gatedRmsNormActivated) and the
    QuantizeActivation of its rows (Qwen35ModelBuilder.cpp:155-166, then the
    out projection's prepare): operands as bind_l2_norm_delta_update, gate
    fp32 like v, norm_weight fp32 [dv]; out the normalised rows (fp16),
    quantized int8 [T*Hv*dv], scales fp32 [T*Hv*dv/32]. T <= 32."""
    _require(gate, torch.float32, "gate")
    _require(norm_weight, torch.float32, "norm_weight")
    _require(quantized, torch.int8, "quantized")
    _require(scales, torch.float32, "scales")
    if invalid is not None:
        _require(invalid, torch.int32, "invalid")
    hv, dk, dv = state.shape
    if gate.shape != v.shape or norm_weight.numel() != dv or quantized.numel() != v.numel() or \
            scales.numel() * 32 != v.numel():
        raise ValueError("gate must match v, norm_weight have dv elements, quantized and "
                         "scales cover v's elements in 32-wide groups")
    inner = bind_l2_norm_delta_update(q, k, v, beta, decay, state, out, epsilon, q_scale)
    a = inner._args
    lib = _lib.load()
    args = a[:6] + (_ptr(gate), _ptr(norm_weight), a[6], _ptr(quantized), _ptr(scales),
                    _ptr(invalid), a[7], a[8], a[9], norm_epsilon, a[12])
    return Bound(lib.llmi_hip_l2_norm_delta_gated_norm_activated_quantize, args,
                 inner.what + "+gatedRmsNormQuantize")


def l2_norm_delta_gated_norm_activated_quantize(q, k, v, beta, decay, state, gate, norm_weight,
                                                out, quantized, scales, invalid=None,
                                                epsilon: float = 1e-6,
                                                q_scale: float | None = None,
                                                norm_epsilon: float = 1e-6) -> None:
    """bind_l2_norm_delta_gated_norm_activated_quantize, called once."""
    bind_l2_norm_delta_gated_norm_activated_quantize(q, k, v, beta, decay, state, gate,
                                                     norm_weight, out, quantized, scales,
                                                     invalid, epsilon, q_scale,
                                                     norm_epsilon)()


class Bound:
    """One C-ABI call with every argument converted once, for hot loops.

    `bind_*` validate like the functions above and return a Bound whose
    call() re-issues the launch on the same buffers with no per-call host
    work beyond the ctypes call itself. Buffers must stay alive and keep
    their shapes while the Bound is used.
    """

    def __init__(self, fn, args, what: str):
        self._fn = fn
        self._args = args
        self.what = what

    def __call__(self) -> None:
        st = self._fn(*self._args)
        if st != _lib.OK:
            _lib.check(st)


def bind_kv_append(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                   v_cache: torch.Tensor, past: int) -> Bound:
    for t, n in ((k, "k"), (v, "v"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _require(t, torch.float16, n)
    T, hkv, d = k.shape
    if v.shape != k.shape or k_cache.shape != v_cache.shape or \
            k_cache.shape[1:] != k.shape[1:] or past + T > k_cache.shape[0]:
        raise ValueError("KvAppend operands do not match the cache")
    lib = _lib.load()
    args = (_ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache),
            _lib.CacheParams(T * hkv * d, past * hkv * d), _stream())
    return Bound(lib.llmi_hip_kv_append, args, "kvAppend")


def bind_causal_gqa(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    out: torch.Tensor, past: int) -> Bound:
    for t, n in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache"), (out, "out")):
        _require(t, torch.float16, n)
    if q.dim() != 3 or k_cache.shape != v_cache.shape or out.shape != q.shape or \
            q.shape[2] != k_cache.shape[2] or past + q.shape[0] > k_cache.shape[0]:
        raise ValueError("CausalGqa operands do not match the cache")
    lib = _lib.load()
    p = gqa_params(q, k_cache, past)
    need = lib.llmi_hip_gqa_workspace_bytes(p)
    ws = workspace(need, q.device) if need else None
    args = (_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), p, _ptr(ws),
            ws.numel() if ws is not None else 0, _stream())
    b = Bound(lib.llmi_hip_causal_gqa, args, kernel_names(_lib.OP_CAUSAL_GQA, p)[0])
    b._keep = ws
    return b


def bind_kv_append_causal_gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                              k_cache: torch.Tensor, v_cache: torch.Tensor,
                              out: torch.Tensor, past: int) -> Bound:
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (k_cache, "k_cache"), (v_cache, "v_cache"),
                 (out, "out")):
        _require(t, torch.float16, n)
    if q.dim() != 3 or k.shape != v.shape or k_cache.shape != v_cache.shape or \
            k.shape[1:] != k_cache.shape[1:] or q.shape[0] != k.shape[0] or \
            out.shape != q.shape or past + q.shape[0] > k_cache.shape[0]:
        raise ValueError("KvAppend/CausalGqa operands do not match the cache")
    lib = _lib.load()
    p = gqa_params(q, k_cache, past)
    need = lib.llmi_hip_gqa_workspace_bytes(p)
    ws = workspace(need, q.device) if need else None
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache), _ptr(out), p, _ptr(ws),
            ws.numel() if ws is not None else 0, _stream())
    names = kernel_names(_lib.OP_KV_APPEND_CAUSAL_GQA, p)
    b = Bound(lib.llmi_hip_kv_append_causal_gqa, args, "+".join(names))
    b._keep = ws
    return b


def bind_delta_update(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      beta: torch.Tensor, decay: torch.Tensor, state: torch.Tensor,
                      out: torch.Tensor) -> Bound:
    for t, n, dt in ((q, "q", torch.float32), (k, "k", torch.float32),
                     (v, "v", torch.float16), (beta, "beta", torch.float32),
                     (decay, "decay", torch.float32), (state, "state", torch.float32),
                     (out, "out", torch.float16)):
        _require(t, dt, n)
    T = q.shape[0]
    hv, dk, dv = state.shape
    if q.dim() != 2 or k.shape != q.shape or q.shape[1] % dk or \
            hv % (q.shape[1] // dk) or v.shape != (T, hv * dv) or \
            beta.shape != (T, hv) or decay.shape != beta.shape or out.shape != v.shape:
        raise ValueError("DeltaUpdate operand shapes do not match its recurrent state")
    lib = _lib.load()
    p = delta_params(q, v, state)
    need = lib.llmi_hip_delta_workspace_bytes(p)
    ws = workspace(need, q.device, "delta") if need else None
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(decay), _ptr(state), _ptr(out),
            p, _ptr(ws), ws.numel() if ws is not None else 0, _stream())
    names = kernel_names(_lib.OP_DELTA_UPDATE, p)
    b = Bound(lib.llmi_hip_delta_update, args, "+".join(names))
    b._keep = ws
    return b


def kernel_names(op: int, params) -> list[str]:
    lib = _lib.load()
    ref = C.byref(params)
    n = lib.llmi_hip_dispatch_count(op, ref)
    return [lib.llmi_hip_kernel_name(op, ref, i).decode() for i in range(n)]
