"""GPU parity of the DeltaNet front end (causalConv + SiLU, l2NormF32,
deltaGates) against the oracle (oracle.c: orc_causal_conv, orc_l2norm_f32,
orc_delta_gates), through the C ABI.

The bar is bit-exact: the kernels evaluate the reference's expressions in
IEEE fp32 in the reference's order, with exp and log correctly rounded (the
oracle's convention). Shapes: Qwen3.5's conv over q, k, v (8192 channels,
k = 4) at prefill 1024 and decode, the L2 norm of 16 + 16 heads of 128 with
q scaled by 1/sqrt(128), gates for 32 value heads; other filter sizes,
widths and unaligned rows; every finite fp16 value through SiLU and the
gate's logistic.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import torch_to_u16, u16_to_torch
from llminfer_amd import ops

pytestmark = pytest.mark.gpu


def _f16(rng, shape, s=1.0):
    return oracle.f32_to_f16((rng.standard_normal(shape) * s).astype(np.float32))


@pytest.mark.parametrize("T,C,k,silu", [(1024, 8192, 4, True), (1, 8192, 4, True),
                                        (37, 300, 4, False), (2, 64, 4, True),
                                        (50, 130, 1, True), (19, 96, 2, True),
                                        (33, 70, 8, False)])
def test_causal_conv(gpu, T, C, k, silu):
    rng = np.random.default_rng(T * 31 + C + k)
    x, w, h = _f16(rng, (T, C)), _f16(rng, (C, k), 0.5), _f16(rng, (C, k - 1))
    print(f"causalConv T={T} C={C} k={k} silu={silu}", flush=True)
    ht = u16_to_torch(h) if k > 1 else None
    out = torch.empty(T, C, dtype=torch.float16, device=gpu)
    ops.causal_conv(u16_to_torch(x), u16_to_torch(w), ht, out, silu)
    torch.cuda.synchronize()
    href = h.copy()
    ref = oracle.causal_conv(x, w, href, silu)
    assert np.array_equal(torch_to_u16(out), ref)
    if k > 1:
        assert np.array_equal(torch_to_u16(ht), href)


def test_causal_conv_split_calls_carry_history(gpu):
    rng = np.random.default_rng(5)
    T, C, k = 40, 256, 4
    x, w, h = _f16(rng, (T, C)), _f16(rng, (C, k), 0.5), _f16(rng, (C, k - 1))
    ht, wt = u16_to_torch(h), u16_to_torch(w)
    outs = []
    for a, b in ((0, 17), (17, 18), (18, 40)):         # includes a one-token step
        o = torch.empty(b - a, C, dtype=torch.float16, device=gpu)
        ops.causal_conv(u16_to_torch(x[a:b]), wt, ht, o, True)
        outs.append(o)
    torch.cuda.synchronize()
    href = h.copy()
    ref = oracle.causal_conv(x, w, href, True)
    assert np.array_equal(torch_to_u16(torch.cat(outs)), ref)
    assert np.array_equal(torch_to_u16(ht), href)


def test_silu_every_fp16_value(gpu):
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = bits[(bits & 0x7C00) != 0x7C00][None, :]       # finite values as channels
    C = x.shape[1]
    w = np.zeros((C, 4), np.uint16)
    w[:, 3] = 0x3C00                                   # acc = x exactly
    h = np.zeros((C, 3), np.uint16)
    out = torch.empty(1, C, dtype=torch.float16, device=gpu)
    ops.causal_conv(u16_to_torch(x), u16_to_torch(w), u16_to_torch(h), out, True)
    torch.cuda.synchronize()
    assert np.array_equal(torch_to_u16(out), oracle.causal_conv(x, w, h.copy(), True))


@pytest.mark.parametrize("rows,width,scale", [(1024 * 16, 128, 128 ** -0.5), (1024 * 16, 128, 1.0),
                                              (77, 256, 1.0), (50, 100, 0.5), (3, 64, 1.0)])
def test_l2_norm(gpu, rows, width, scale):
    rng = np.random.default_rng(rows + width)
    x = _f16(rng, (rows, width))
    x[0] = 0                                           # zero row: eps only
    out = torch.empty(rows, width, dtype=torch.float32, device=gpu)
    print(f"l2Norm rows={rows} width={width}", flush=True)
    ops.l2_norm(u16_to_torch(x), out, width, 1e-6, scale)
    torch.cuda.synchronize()
    ref = oracle.l2norm_f32(x, width, 1e-6, scale)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("T,H", [(1024, 32), (1, 32), (7, 5)])
def test_delta_gates(gpu, T, H):
    rng = np.random.default_rng(T + H)
    a, b = _f16(rng, (T, H), 3.0), _f16(rng, (T, H), 4.0)
    if T > 4:
        a[0, :4] = [0x7BFF, 0xFBFF, 0x0000, 0x8000]
        b[0, :4] = [0x7BFF, 0xFBFF, 0x0000, 0x8000]
    a_log = (rng.standard_normal(H) * 0.5).astype(np.float32)
    dt = (rng.standard_normal(H) * 0.5).astype(np.float32)
    dev = lambda v: torch.from_numpy(v).to(gpu)
    beta = torch.empty(T, H, dtype=torch.float32, device=gpu)
    decay = torch.empty_like(beta)
    ops.delta_gates(u16_to_torch(a), u16_to_torch(b), dev(a_log), dev(dt), beta, decay)
    torch.cuda.synchronize()
    rb, rd = oracle.delta_gates(a, b, a_log, dt)
    assert np.array_equal(beta.cpu().numpy().view(np.uint32), rb.view(np.uint32))
    assert np.array_equal(decay.cpu().numpy().view(np.uint32), rd.view(np.uint32))


def test_gate_beta_every_fp16_value(gpu):
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    b = bits[(bits & 0x7C00) != 0x7C00].reshape(-1, 32)
    a = np.zeros_like(b)
    z = np.zeros(32, np.float32)
    beta = torch.empty(b.shape, dtype=torch.float32, device=gpu)
    decay = torch.empty_like(beta)
    ops.delta_gates(u16_to_torch(a), u16_to_torch(b), torch.from_numpy(z).to(gpu),
                    torch.from_numpy(z).to(gpu), beta, decay)
    torch.cuda.synchronize()
    rb, rd = oracle.delta_gates(a, b, z, z)
    assert np.array_equal(beta.cpu().numpy().view(np.uint32), rb.view(np.uint32))


@pytest.mark.parametrize("rows,width,activated", [(1024 * 32, 128, False), (32, 128, False),
                                                  (1000, 128, True), (45, 256, False),
                                                  (7, 64, True),
                                                  # a thread per row: odd and wide widths
                                                  (37, 5, False), (9, 5, True), (300, 100, False),
                                                  (3, 264, True)])
def test_gated_rms_norm(gpu, rows, width, activated):
    rng = np.random.default_rng(rows + width)
    x = _f16(rng, (rows, width))
    x[0] = 0
    w = (1 + 0.2 * rng.standard_normal(width)).astype(np.float32)
    if activated:
        g = (rng.standard_normal((rows, width)) * 2).astype(np.float32)
        gt = torch.from_numpy(g).to(gpu)
    else:
        g = _f16(rng, (rows, width), 3.0)
        special = [0x7BFF, 0xFBFF, 0x0000, 0x8000, 0xCC00, 0x4C00][:width]
        g[1, :len(special)] = special
        gt = u16_to_torch(g)
    out = torch.empty(rows, width, dtype=torch.float16, device=gpu)
    print(f"gatedRmsNorm rows={rows} width={width} activated={activated}", flush=True)
    ops.gated_rms_norm(u16_to_torch(x), gt, torch.from_numpy(w).to(gpu), out)
    torch.cuda.synchronize()
    assert np.array_equal(torch_to_u16(out), oracle.gated_rms_norm(x, g, w))


def test_gated_rms_norm_every_gate_value(gpu):
    """Every finite fp16 gate value through SiLU, on rows of ones."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    g = bits[(bits & 0x7C00) != 0x7C00].reshape(-1, 128)
    x = np.full(g.shape, 0x3C00, np.uint16)
    w = np.ones(128, np.float32)
    out = torch.empty(g.shape, dtype=torch.float16, device=gpu)
    ops.gated_rms_norm(u16_to_torch(x), u16_to_torch(g), torch.from_numpy(w).to(gpu), out)
    torch.cuda.synchronize()
    assert np.array_equal(torch_to_u16(out), oracle.gated_rms_norm(x, g, w))
