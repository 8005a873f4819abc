"""GPU parity of residualAdd, swiGlu, siluF16, multiplyF16, copyHalfView and
linearF16 against the CPU oracle, bit for bit (Reference.metal:61-135,
Graph.metal:1-14, 70-95)."""
import numpy as np
import pytest
import torch

import oracle
from llminfer_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _f16(x):
    return oracle.f32_to_f16(np.asarray(x, np.float32))


def _u16_dev(bits, gpu):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(gpu).view(torch.float16)


def _host_u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _same16(got, want):
    """Bit for bit, except that any NaN matches any NaN: the default NaN of
    an invalid operation (inf * 0, inf - inf) is negative on x86 and
    positive on the GPU, and NaN payloads carry no meaning here."""
    nan = lambda u: ((u & 0x7C00) == 0x7C00) & ((u & 0x03FF) != 0)
    return bool(np.all((got == want) | (nan(got) & nan(want))))


def _operands(seed, n):
    r = np.random.default_rng(seed)
    special = np.array([0x0000, 0x8000, 0x0001, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00], np.uint16)
    a = _f16(r.standard_normal(n) * 8)
    b = _f16(r.standard_normal(n) * 8)
    a[:special.size] = special
    b[:special.size] = special[::-1]
    return a, b


# 4096: the 16-byte path; 4099: one element a lane
@pytest.mark.parametrize("n", [4096, 4099, 8])
@pytest.mark.parametrize("kind", ["add", "swiglu", "silu", "multiply"])
def test_elementwise_bit_exact(gpu, kind, n):
    print(f"elementwise {kind} n={n}", flush=True)
    a, b = _operands(n + len(kind), n)
    out = torch.empty(n, dtype=torch.float16, device=gpu)
    ops.elementwise(kind, _u16_dev(a, gpu), None if kind == "silu" else _u16_dev(b, gpu), out)
    torch.cuda.synchronize()
    assert _same16(_host_u16(out), oracle.elementwise(kind, a, b))


def test_elementwise_offset_views_take_the_scalar_path(gpu):
    a, b = _operands(3, 4104)
    da, db = _u16_dev(a, gpu), _u16_dev(b, gpu)
    out = torch.empty(4096, dtype=torch.float16, device=gpu)
    ops.elementwise("add", da[3:4099], db[5:4101], out)   # 16-byte misaligned operands
    torch.cuda.synchronize()
    assert _same16(_host_u16(out), oracle.elementwise("add", a[3:4099], b[5:4101]))


@pytest.mark.parametrize("shape,axis,begin,length", [
    ((7, 4, 24), 2, 12, 12), ((7, 4, 24), 2, 0, 12),  # the interleaved query / gate halves
    ((5, 300), 1, 128, 100), ((9, 10), 0, 2, 5)])
def test_copy_half_view_bit_exact(gpu, shape, axis, begin, length):
    src = np.random.default_rng(1).integers(0, 65535, shape).astype(np.uint16)
    src[(src & 0x7C00) == 0x7C00] = 0x3C00  # finite values only: bits compare as data
    index = [slice(None)] * len(shape)
    index[axis] = slice(begin, begin + length)
    view = src[tuple(index)]
    strides = [s // 2 for s in view.strides]
    out = torch.empty(view.size, dtype=torch.float16, device=gpu)
    ops.copy_half_view(_u16_dev(src, gpu), out, view.shape, strides, begin * strides[axis])
    torch.cuda.synchronize()
    assert np.array_equal(_host_u16(out).reshape(view.shape), np.ascontiguousarray(view))


@pytest.mark.parametrize("tokens,k,columns", [(1, 2560, 300), (3, 70, 33), (9, 64, 256),
                                              (17, 129, 513), (1, 1, 5)])
def test_linear_f16_bit_exact(gpu, tokens, k, columns):
    print(f"linearF16 tokens={tokens} k={k} columns={columns}", flush=True)
    r = np.random.default_rng(tokens * 1000 + k + columns)
    x = _f16(r.standard_normal((tokens, k)))
    w = _f16(r.standard_normal((columns, k)) * 0.05)
    out = torch.full((tokens, columns), 7.0, dtype=torch.float16, device=gpu)
    ops.linear_f16(_u16_dev(x, gpu), _u16_dev(w, gpu), out)
    torch.cuda.synchronize()
    assert np.array_equal(_host_u16(out), oracle.linear_f16(x, w))


@pytest.mark.parametrize("epilogue", [1, 2, 3, 4, 5, 6])
def test_linear_f16_epilogues_bit_exact(gpu, epilogue):
    r = np.random.default_rng(epilogue)
    tokens, k, columns = 5, 96, 48
    x = _f16(r.standard_normal((tokens, k)) * 2)
    w = _f16(r.standard_normal((columns, k)) * 0.3)
    aux = bias = None
    if epilogue == _lib.LINEAR_SILU_MUL:
        aux = _f16(r.standard_normal((tokens, columns)))
    if epilogue == _lib.LINEAR_DELTA_DECAY:
        aux = (r.standard_normal(columns) * 0.5).astype(np.float32)
        bias = (r.standard_normal(columns) * 0.5).astype(np.float32)
    f32 = epilogue in oracle.F32_EPILOGUES
    out = torch.zeros((tokens, columns), dtype=torch.float32 if f32 else torch.float16, device=gpu)
    aux_d = None
    if aux is not None:
        aux_d = _u16_dev(aux, gpu) if aux.dtype == np.uint16 else torch.from_numpy(aux).to(gpu)
    bias_d = torch.from_numpy(bias).to(gpu) if bias is not None else None
    ops.linear_f16(_u16_dev(x, gpu), _u16_dev(w, gpu), out, epilogue, 8, aux_d, bias_d)
    torch.cuda.synchronize()
    want = oracle.linear_f16(x, w, epilogue, 8, aux, bias)
    got = out.cpu().numpy() if f32 else _host_u16(out)
    if f32:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert np.array_equal(got, want)
