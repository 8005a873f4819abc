"""GPU parity of normRope, rmsNorm, partialRope and sigmoidMul against the
oracle (oracle.c: orc_norm_rope, orc_sigmoid_mul), through the C ABI.

The bar is bit-exact: the kernels evaluate the reference's expressions in
IEEE fp32 in the reference's order (sequential fma sum, correctly rounded
pow/cos/sin/exp, see oracle.h), so every fp16 output equals the oracle's.
Shapes: the Qwen3.5 attention block (q: 16 heads x 256 with the gate
interleaved, stride 512; k: 4 heads into the cache at outputStart = past;
rotary 64 = 0.25 x 256) at decode, chunk and full prefill sizes; the
reference tests' rotary factor 0.5; rows kernels for unaligned shapes and
pointers; positions up to 2^20 (large-argument cos/sin).
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import torch_to_u16, u16_to_torch
from llminfer_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _x(seed, rows, stride, scale=0.7):
    rng = np.random.default_rng(seed)
    return oracle.f32_to_f16((rng.standard_normal((rows, stride)) * scale).astype(np.float32))


def _w(seed, d):
    return (np.random.default_rng(seed + 100).standard_normal(d) * 0.2).astype(np.float32)


def _same(got, ref, what=""):
    """Bit equality, with the mismatching elements named on failure."""
    bad = np.argwhere(got != ref)
    if len(bad):
        r, c = bad[0]
        f = lambda b: float(oracle.f16_to_f32(np.array([b], np.uint16))[0])
        print(f"{what}: {len(bad)} of {got.size} differ; rows {np.unique(bad[:, 0])[:10]} "
              f"cols {np.unique(bad[:, 1])[:20]}; first ({r},{c}) got {f(got[r, c])} "
              f"ref {f(ref[r, c])}", flush=True)
    return len(bad) == 0


def _run_norm_rope(gpu, x, w, T, H, d, rot, stride, past, start=0, cap=None,
                   eps=1e-6, theta=1e7):
    cap = start + T if cap is None else cap
    xt = u16_to_torch(x.reshape(T, H, stride))
    wt = torch.from_numpy(w).to(gpu)
    sentinel = np.full((cap * H, d), 0x7C01, np.uint16)
    out = u16_to_torch(sentinel.reshape(cap, H, d))
    print(f"normRope T={T} H={H} d={d} rot={rot} stride={stride} past={past} start={start}",
          flush=True)
    ops.norm_rope(xt, wt, out, past, rot, eps, theta, head_dim=d, output_start=start)
    torch.cuda.synchronize()
    ref = oracle.norm_rope(x, w, T, H, d, rot, stride, past, eps, theta,
                           output=sentinel.copy(), output_start=start)
    return torch_to_u16(out).reshape(cap * H, d), ref


@pytest.mark.parametrize("T,past", [(1, 0), (1, 4095), (7, 100), (300, 0), (2048, 0),
                                    (64, 1 << 20)])
def test_q_path(gpu, T, past):
    H, d = 16, 256
    x, w = _x(T, T * H, 2 * d), _w(T, d)
    got, ref = _run_norm_rope(gpu, x, w, T, H, d, 64, 2 * d, past)
    assert _same(got, ref, "q")


@pytest.mark.parametrize("T,past", [(1, 37), (50, 900), (2048, 2048)])
def test_k_path_into_cache(gpu, T, past):
    H, d = 4, 256
    x, w = _x(T + 1, T * H, d), _w(T + 1, d)
    got, ref = _run_norm_rope(gpu, x, w, T, H, d, 64, d, past, start=past, cap=past + T + 3)
    assert _same(got, ref, "k")                     # includes untouched sentinel rows


@pytest.mark.parametrize("H,d,rot,stride", [
    (4, 128, 64, 256),     # rotary factor 0.5 of the reference tests
    (2, 256, 256, 256),    # full rotation
    (8, 256, 0, 512),      # no rotation: rmsNorm with a stride
    (3, 64, 16, 64),       # smallest tile rotary half (8)
    (5, 1024, 128, 1024),  # long rows: fewer rows per tile
])
def test_tile_shapes(gpu, H, d, rot, stride):
    T, past = 37, 11
    x, w = _x(d + rot, T * H, stride), _w(d, d)
    got, ref = _run_norm_rope(gpu, x, w, T, H, d, rot, stride, past)
    assert _same(got, ref)


@pytest.mark.parametrize("H,d,rot,stride", [
    (2, 100, 36, 100),     # rows kernel: width and rotary half not multiples of 8
    (3, 256, 24, 260),     # rotary half 12
    (1, 4096, 64, 4096),   # beyond the tile's width
])
def test_rows_kernel_shapes(gpu, H, d, rot, stride):
    T, past = 9, 3
    x, w = _x(d, T * H, stride), _w(d, d)
    got, ref = _run_norm_rope(gpu, x, w, T, H, d, rot, stride, past)
    assert _same(got, ref)


def test_unaligned_pointer_uses_rows_kernel(gpu):
    T, H, d = 5, 4, 256
    x, w = _x(5, T * H, d), _w(5, d)
    flat = u16_to_torch(np.concatenate([np.zeros(1, np.uint16), x.reshape(-1)]))
    xt = flat[1:].view(T, H, d)                     # 2-byte offset
    wt = torch.from_numpy(w).to(gpu)
    out = torch.empty(T, H, d, dtype=torch.float16, device=gpu)
    ops.norm_rope(xt, wt, out, 17, 64)
    torch.cuda.synchronize()
    assert np.array_equal(torch_to_u16(out).reshape(T * H, d),
                          oracle.norm_rope(x, w, T, H, d, 64, d, 17))


def test_extreme_values(gpu):
    """Rows of zeros (scale = 1/sqrt(eps)), huge and subnormal fp16 values."""
    T, H, d = 4, 4, 256
    x = _x(9, T * H, d)
    x[0] = 0
    x[1] = 0x7BFF                                   # 65504 everywhere
    x[2, ::3] = 0x0001                              # smallest subnormal
    x[3, :] = np.where(np.arange(d) % 2, 0x0400, 0x8400)
    w = _w(9, d)
    got, ref = _run_norm_rope(gpu, x, w, T, H, d, 64, d, 5)
    assert np.array_equal(got, ref)


def test_rms_norm_and_in_place(gpu):
    rows, width = 1000, 2048
    x, w = _x(11, rows, width), _w(11, width)
    xt, wt = u16_to_torch(x), torch.from_numpy(w).to(gpu)
    out = torch.empty_like(xt)
    ops.rms_norm(xt, wt, out)
    ops.rms_norm(xt, wt, xt)                        # in place
    torch.cuda.synchronize()
    ref = oracle.norm_rope(x, w, rows, 1, width, 0, width, 0)
    assert np.array_equal(torch_to_u16(out), ref)
    assert np.array_equal(torch_to_u16(xt), ref)


def test_partial_rope(gpu):
    T, H, d, past = 40, 16, 256, 333
    x = _x(12, T * H, d)
    xt = u16_to_torch(x.reshape(T, H, d))
    out = torch.empty_like(xt)
    ops.partial_rope(xt, out, past, 64)
    ops.partial_rope(xt, xt, past, 64)              # in place
    torch.cuda.synchronize()
    # Reference: rotatePair on the raw halves, the rest copied. The oracle's
    # normRope with a unit scale is not that (it normalises), so compare
    # against the oracle rotation of a pre-normalised input: normRope(x)
    # equals partialRope(rmsNorm(x)) (Reference.metal:271-293 rounds the
    # normalised value to fp16 before rotatePair, exactly what rmsNorm stores).
    w = _w(12, d)
    normed = oracle.norm_rope(x, w, T, H, d, 0, d, 0)
    nt = u16_to_torch(normed.reshape(T, H, d))
    rot = torch.empty_like(nt)
    ops.partial_rope(nt, rot, past, 64)
    torch.cuda.synchronize()
    assert np.array_equal(torch_to_u16(rot).reshape(T * H, d),
                          oracle.norm_rope(x, w, T, H, d, 64, d, past))
    got = torch_to_u16(out).reshape(T * H, d)
    assert np.array_equal(got[:, 64:], x[:, 64:])   # copied part
    assert np.array_equal(torch_to_u16(xt).reshape(T * H, d), got)


@pytest.mark.parametrize("count", [16 * 256, 2048 * 16 * 256, 4097, 7])
def test_sigmoid_mul(gpu, count):
    rng = np.random.default_rng(count)
    g = oracle.f32_to_f16((rng.standard_normal(count) * 5).astype(np.float32))
    x = oracle.f32_to_f16(rng.standard_normal(count).astype(np.float32))
    if count > 64:
        g[:6] = [0x7C00, 0xFC00, 0x0000, 0x8000, 0x7BFF, 0xFBFF]   # +-inf, +-0, +-max
    out = torch.empty(count, dtype=torch.float16, device=gpu)
    print(f"sigmoidMul count={count}", flush=True)
    ops.sigmoid_mul(u16_to_torch(g), u16_to_torch(x), out)
    torch.cuda.synchronize()
    assert np.array_equal(torch_to_u16(out), oracle.sigmoid_mul(g, x))


def test_sigmoid_mul_every_gate_value(gpu):
    """All 63488 finite fp16 gates (the slow path's cases included) times 1."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    finite = bits[(bits & 0x7C00) != 0x7C00]
    g = finite[: len(finite) // 8 * 8]
    x = np.full(g.shape, 0x3C00, np.uint16)         # 1.0: output = fp16(logistic)
    out = torch.empty(g.size, dtype=torch.float16, device=gpu)
    ops.sigmoid_mul(u16_to_torch(g), u16_to_torch(x), out)
    torch.cuda.synchronize()
    assert np.array_equal(torch_to_u16(out), oracle.sigmoid_mul(g, x))


def test_kernel_names_match_the_launch():
    assert ops.kernel_names(_lib.OP_NORM_ROPE,
                            _lib.RopeParams(1, 16, 256, 64, 512, 0, 0, 1e-6, 1e7)) == \
        ["normRopeTile"]


@pytest.mark.parametrize("rows,width", [(1, 2560), (37, 2560), (3, 4100), (2, 257)])
def test_rms_norm_wide_rows(gpu, rows, width):
    """Rows past the tile's width (the model's hidden RMSNorms): a workgroup
    per row, the same sequential sum, bit-exact; in place too."""
    print(f"rmsNorm wide rows={rows} width={width}", flush=True)
    x, w = _x(21 + rows, rows, width, 2.0), _w(21, width)
    xt, wt = u16_to_torch(x), torch.from_numpy(w).to(gpu)
    out = torch.empty_like(xt)
    ops.rms_norm(xt, wt, out)
    ops.rms_norm(xt, wt, xt)
    torch.cuda.synchronize()
    ref = oracle.norm_rope(x, w, rows, 1, width, 0, width, 0)
    assert _same(torch_to_u16(out), ref, "wide")
    assert np.array_equal(torch_to_u16(xt), ref)
    assert ops.kernel_names(_lib.OP_RMS_NORM, _lib.RowParams(rows, width, 1e-6)) == \
        ["normRopeWide"]


def test_norm_rope_wide_heads(gpu):
    """normRope and partialRope on heads wider than the tile (64 rotated
    dims of 2600)."""
    T, H, d, past = 3, 2, 2600, 9
    x, w = _x(23, T * H, d), _w(23, d)
    got, ref = _run_norm_rope(gpu, x, w, T, H, d, 64, d, past)
    assert _same(got, ref, "normRope wide")
    normed = oracle.norm_rope(x, w, T, H, d, 0, d, 0)
    nt = u16_to_torch(normed.reshape(T, H, d))
    rot = torch.empty_like(nt)
    ops.partial_rope(nt, rot, past, 64)
    torch.cuda.synchronize()
    assert np.array_equal(torch_to_u16(rot).reshape(T * H, d), ref)
