"""GPU parity of the W8A8 projection path against the CPU oracle.

quantizeActivation, linearW8A8Gemv / Gemm with every storeLinear epilogue,
embeddingW8 and embedding: the HIP kernels follow the reference kernels'
integer and fp32 arithmetic order (Graph.metal:16-68, W8A8.metal:28-113,
Reference.metal:14-58), so every output is compared bit for bit with
oracle.c on the same seeded inputs. Shapes include Qwen3.5-4B's decode
projections (hidden 2560, MLP 9216).
"""
import numpy as np
import pytest
import torch

import oracle
from llminfer_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def _f16(x):
    return oracle.f32_to_f16(np.asarray(x, np.float32))


def _u16_dev(bits, gpu):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(gpu).view(torch.float16)


def _host_u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("rows,width", [(1, 2560), (1, 9216), (7, 96), (3, 70), (64, 2560),
                                        (2, 1)])
def test_quantize_bit_exact(gpu, rows, width):
    print(f"quantize rows={rows} width={width}", flush=True)
    x = _f16(np.random.default_rng(rows + width).standard_normal((rows, width)) * 4)
    if width >= 96:
        x[0, 32:64] = 0           # an all-zero group
        x[-1, 1] = 0x7E00         # NaN in group 0 of the last row
        x[0, 127 % width] = 0xFC00  # -inf
        vals = [127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5]
        x[rows // 2, 64:72] = _f16(vals)  # exact ties (the group max is 127)
        x[rows // 2, 72:96] = 0
    q_ref, s_ref, inv_ref = oracle.quantize_activation(x)
    groups = (width + 31) // 32
    q = torch.empty((rows, groups * 32), dtype=torch.int8, device=gpu)
    s = torch.empty((rows, groups), dtype=torch.float32, device=gpu)
    inv = torch.zeros(1, dtype=torch.int32, device=gpu)
    ops.quantize_activation(_u16_dev(x, gpu), q, s, inv)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert int(inv.item()) == inv_ref


def _case(seed, rows, columns, groups, spread=1.0):
    r = np.random.default_rng(seed)
    x16 = _f16(r.standard_normal((rows, groups * 32)) * spread)
    xq, xs, _ = oracle.quantize_activation(x16)
    w = r.integers(-127, 128, (columns, groups * 32), dtype=np.int8)
    ws = _f16(r.random((columns, groups)) * 0.01 + 2e-4)
    return xq, xs, w, ws


def _run_linear(gpu, xq, xs, w, ws, epilogue=0, block=0, aux=None, bias=None, first_row=0,
                width=None):
    rows = xq.shape[0]
    width = width if width is not None else first_row + w.shape[0]
    f32 = epilogue in oracle.F32_EPILOGUES
    out = torch.full((rows, width), 7.0, dtype=torch.float32 if f32 else torch.float16,
                     device=gpu)
    aux_d = None
    if aux is not None:
        aux_d = _u16_dev(aux, gpu) if aux.dtype == np.uint16 else _dev(aux, gpu)
    bias_d = _dev(bias, gpu) if bias is not None else None
    ops.linear_w8a8(_dev(xq, gpu), _dev(xs, gpu), _dev(w, gpu), _u16_dev(ws, gpu), out,
                    epilogue, block, aux_d, bias_d, first_row)
    torch.cuda.synchronize()
    got = out.cpu().numpy() if f32 else _host_u16(out)
    ref_out = np.full((rows, width), 7.0, np.float32) if f32 else \
        np.full((rows, width), 0x4700, np.uint16)
    oracle.linear_w8a8(xq, xs, w, ws, epilogue, block, aux, bias, ref_out, first_row, width)
    return got, ref_out


def _same(got, want):
    if got.dtype == np.float32:
        return np.array_equal(got.view(np.uint32), want.view(np.uint32))
    return np.array_equal(got, want)


@pytest.mark.parametrize("rows,columns,groups", [
    (1, 9216, 80),    # Qwen3.5-4B MLP gate/up, decode
    (1, 2560, 288),   # MLP down, decode
    (1, 2560, 128), (1, 40, 113),  # out projections: 8 steps a lane, the split kernel's 2 a wave
    (1, 37, 5), (1, 16, 1), (1, 33, 17),
    (1, 50, 150), (1, 20, 1024), (1, 12, 1030),   # four waves per column; the limit; past it
    (2, 40, 9), (3, 70, 12), (4, 32, 80), (5, 19, 3), (15, 40, 9),
    # the MFMA kernel (16 rows or more): eight waves per tile, four once the
    # grid has 1024 tiles, and ragged row and column tiles
    (16, 40, 9), (37, 70, 12), (64, 256, 80), (100, 33, 1), (33, 65, 3), (128, 96, 288),
    (32, 32768, 2), (70, 15000, 3), (20, 40, 600)])
def test_linear_bit_exact(gpu, rows, columns, groups):
    print(f"linear rows={rows} columns={columns} groups={groups}", flush=True)
    xq, xs, w, ws = _case(rows * 7 + columns + groups, rows, columns, groups)
    got, want = _run_linear(gpu, xq, xs, w, ws)
    assert _same(got, want)


def test_linear_shard_writes_only_its_columns(gpu):
    xq, xs, w, ws = _case(3, 3, 48, 7)
    got, want = _run_linear(gpu, xq, xs, w, ws, first_row=40, width=100)
    assert _same(got, want)
    assert np.all(got[:, :40] == 0x4700) and np.all(got[:, 88:] == 0x4700)
    got1, want1 = _run_linear(gpu, xq[:1], xs[:1], w, ws, first_row=52, width=100)
    assert _same(got1, want1)
    xq, xs, w, ws = _case(4, 40, 48, 7)
    got2, want2 = _run_linear(gpu, xq, xs, w, ws, first_row=30, width=100)
    assert _same(got2, want2)
    assert np.all(got2[:, :30] == 0x4700) and np.all(got2[:, 78:] == 0x4700)


@pytest.mark.parametrize("rows,groups", [(1, 20), (1, 160), (6, 20), (20, 20), (40, 160)])
@pytest.mark.parametrize("epilogue", [1, 2, 3, 4, 5, 6])
def test_linear_epilogues_bit_exact(gpu, rows, groups, epilogue):
    print(f"linear epilogue {epilogue} rows={rows} groups={groups}", flush=True)
    columns = 96
    # wide activations: projections spread over the epilogues' ranges
    xq, xs, w, ws = _case(100 + epilogue * 10 + rows, rows, columns, groups, spread=6.0)
    r = np.random.default_rng(epilogue)
    aux = bias = None
    if epilogue == oracle.LINEAR_SILU_MUL:
        aux = _f16(r.standard_normal((rows, columns)) * 2)
    if epilogue == oracle.LINEAR_DELTA_DECAY:
        aux = (r.standard_normal(columns) * 0.5).astype(np.float32)
        bias = (r.standard_normal(columns) * 0.5).astype(np.float32)
    got, want = _run_linear(gpu, xq, xs, w, ws, epilogue, 16, aux, bias)
    assert _same(got, want)


def test_embeddings_bit_exact(gpu):
    r = np.random.default_rng(5)
    rows, hidden = 300, 2560
    groups = hidden // 32
    w = r.integers(-127, 128, (rows, groups * 32), dtype=np.int8)
    sc = _f16(r.random((rows, groups)) * 0.02)
    ids = np.array([5, 299, 0, 301, 150, 5, 1000], np.uint32)   # 301, 1000: other shards
    out = torch.full((ids.size, hidden), 3.0, dtype=torch.float16, device=gpu)
    ops.embedding_w8(_dev(ids.view(np.int32), gpu), _dev(w, gpu), _u16_dev(sc, gpu), out)
    want = np.full((ids.size, hidden), 0x4200, np.uint16)
    oracle.embedding_w8(ids, w, sc, hidden, 0, want)
    torch.cuda.synchronize()
    assert np.array_equal(_host_u16(out), want)
    # an odd width takes the one-element path; a shard offset
    hid2 = 70
    w2 = r.integers(-127, 128, (40, 96), dtype=np.int8)
    sc2 = _f16(r.random((40, 3)) * 0.02)
    ids2 = np.array([12, 51, 9, 30], np.uint32)
    out2 = torch.zeros((4, hid2), dtype=torch.float16, device=gpu)
    ops.embedding_w8(_dev(ids2.view(np.int32), gpu), _dev(w2, gpu), _u16_dev(sc2, gpu), out2,
                     first_row=10)
    want2 = np.zeros((4, hid2), np.uint16)
    oracle.embedding_w8(ids2, w2, sc2, hid2, 10, want2)
    torch.cuda.synchronize()
    assert np.array_equal(_host_u16(out2), want2)
    wf = _f16(r.standard_normal((rows, hidden)))
    outf = torch.zeros((ids.size, hidden), dtype=torch.float16, device=gpu)
    ops.embedding(_dev(ids.view(np.int32), gpu), _u16_dev(wf, gpu), outf)
    torch.cuda.synchronize()
    assert np.array_equal(_host_u16(outf), oracle.embedding(ids, wf))


def test_quantize_then_project_decode_step(gpu):
    """One decode-step projection as the plan lowers it: quantizeActivation
    then linearW8A8Gemv with the SwiGLU epilogue (the up projection's output
    as aux), against the oracle chain."""
    r = np.random.default_rng(11)
    hidden, inter = 2560, 9216
    x = _f16(r.standard_normal((1, hidden)))
    groups = hidden // 32
    wg = r.integers(-127, 128, (inter, hidden), dtype=np.int8)
    wu = r.integers(-127, 128, (inter, hidden), dtype=np.int8)
    sg = _f16(r.random((inter, groups)) * 0.002)
    su = _f16(r.random((inter, groups)) * 0.002)
    q = torch.empty((1, hidden), dtype=torch.int8, device=gpu)
    s = torch.empty((1, groups), dtype=torch.float32, device=gpu)
    ops.quantize_activation(_u16_dev(x, gpu), q, s)
    up = torch.empty((1, inter), dtype=torch.float16, device=gpu)
    ops.linear_w8a8(q, s, _dev(wu, gpu), _u16_dev(su, gpu), up)
    act = torch.empty((1, inter), dtype=torch.float16, device=gpu)
    ops.linear_w8a8(q, s, _dev(wg, gpu), _u16_dev(sg, gpu), act, _lib.LINEAR_SILU_MUL, 0, up)
    torch.cuda.synchronize()
    xq, xs, _ = oracle.quantize_activation(x)
    up_ref = oracle.linear_w8a8(xq, xs, wu, su)
    act_ref = oracle.linear_w8a8(xq, xs, wg, sg, oracle.LINEAR_SILU_MUL, 0, up_ref)
    assert np.array_equal(_host_u16(up), up_ref)
    assert np.array_equal(_host_u16(act), act_ref)


@pytest.mark.parametrize("rows,width,add", [(1, 2560, True), (37, 2560, True), (5, 4100, False),
                                            (3, 33, True), (512, 2560, True), (2, 96, False)])
def test_add_rms_norm_quantize_is_the_three_ops(gpu, rows, width, add):
    """residualAdd -> rmsNorm -> quantizeActivation in one launch equals the
    three launches bit for bit: the sum, the int8 rows, the scales and the
    invalid flag."""
    print(f"addRmsNormQuantize rows={rows} width={width} add={add}", flush=True)
    r = np.random.default_rng(rows + width)
    a = _f16(r.standard_normal((rows, width)) * 3)
    b = _f16(r.standard_normal((rows, width)) * 3)
    if rows > 2:
        a[2, 5] = 0x7C00                      # inf: its row's groups flag invalid
    w = (r.standard_normal(width) * 0.2).astype(np.float32)
    groups = (width + 31) // 32
    da, db, dw = _u16_dev(a, gpu), _u16_dev(b, gpu), _dev(w, gpu)
    # three launches
    s3 = torch.empty(rows, width, dtype=torch.float16, device=gpu)
    n3 = torch.empty_like(s3)
    q3 = torch.empty(rows, groups * 32, dtype=torch.int8, device=gpu)
    c3 = torch.empty(rows, groups, dtype=torch.float32, device=gpu)
    i3 = torch.zeros(1, dtype=torch.int32, device=gpu)
    src = s3 if add else da
    if add:
        ops.elementwise("add", da, db, s3)
    ops.rms_norm(src, dw, n3)
    ops.quantize_activation(n3, q3, c3, i3)
    # one launch
    s1 = torch.empty_like(s3)
    q1 = torch.empty_like(q3)
    c1 = torch.empty_like(c3)
    i1 = torch.zeros(1, dtype=torch.int32, device=gpu)
    ops.add_rms_norm_quantize(da, db if add else None, s1 if add else None, dw, q1, c1, i1)
    torch.cuda.synchronize()
    if add:
        assert np.array_equal(_host_u16(s1), _host_u16(s3))
    assert torch.equal(q1, q3)
    assert np.array_equal(c1.cpu().numpy().view(np.uint32), c3.cpu().numpy().view(np.uint32))
    assert int(i1.item()) == int(i3.item())


def _projection_weights(r, columns, groups, gpu):
    w = r.integers(-127, 128, (columns, groups * 32), dtype=np.int8)
    ws = _f16(r.uniform(0.001, 0.02, (columns, groups)))
    return _dev(w, gpu), _u16_dev(ws, gpu)


# (width, add, projections: (columns, epilogue, block)); the shapes of the
# Qwen3.5-4B decode step's input norms: DeltaNet qkv / z / a / b, the MLP's
# up + gate (SwiGLU, its multiplier up's output: computed by up's lanes),
# the attention's q (+ gate columns) / k / v.
_PAIRED = -1  # SwiGLU with the previous projection's output as multiplier
_NORM_LINEAR_CASES = [
    (2560, True, [(8192, _lib.LINEAR_NONE, 0), (4096, _lib.LINEAR_SILU_F32, 0),
                  (32, _lib.LINEAR_DELTA_DECAY, 0), (32, _lib.LINEAR_DELTA_BETA, 0)]),
    (2560, True, [(9216, _lib.LINEAR_NONE, 0), (9216, _PAIRED, 0)]),
    (2560, False, [(8192, _lib.LINEAR_SIGMOID_COLUMNS, 256), (1024, _lib.LINEAR_NONE, 0),
                   (1024, _lib.LINEAR_NONE, 0)]),
    (1000, True, [(100, _lib.LINEAR_SILU, 0), (37, _lib.LINEAR_NONE, 0),
                  (37, _lib.LINEAR_SILU_MUL, 0)]),  # its multiplier computed beforehand
    (4096, False, [(17, _lib.LINEAR_NONE, 0)]),
    (33, True, [(16, _lib.LINEAR_DELTA_BETA, 0), (65, _lib.LINEAR_NONE, 0),
                (65, _PAIRED, 0), (129, _lib.LINEAR_SIGMOID_COLUMNS, 8)]),
    (4000, False, [(61, _lib.LINEAR_NONE, 0), (7, _lib.LINEAR_SILU_MUL, 0)]),
]


@pytest.mark.parametrize("case", range(len(_NORM_LINEAR_CASES)))
@pytest.mark.parametrize("special", [False, True])
def test_add_rms_norm_linear_is_the_separate_ops(gpu, case, special):
    """The norm and its projections in one launch equal add_rms_norm_quantize
    followed by one linear_w8a8 per projection, bit for bit: the sum, the
    quantized row, its scales, the invalid flag and every projection
    output (special: an infinite input quantizes its group to zeros and
    raises the flag)."""
    width, add, projs = _NORM_LINEAR_CASES[case]
    print(f"addRmsNormLinearW8A8 width={width} add={add} projections={projs} "
          f"special={special}", flush=True)
    r = np.random.default_rng(100 + case)
    groups = (width + 31) // 32
    a = _f16(r.standard_normal((1, width)) * 3)
    b = _f16(r.standard_normal((1, width)) * 3)
    if special:
        a[0, width // 2] = 0x7C00
    w = (r.standard_normal(width) * 0.2).astype(np.float32)
    da, db, dw = _u16_dev(a, gpu), _u16_dev(b, gpu), _dev(w, gpu)
    f32 = (_lib.LINEAR_SILU_F32, _lib.LINEAR_DELTA_BETA, _lib.LINEAR_DELTA_DECAY)
    specs, paired = [], []
    for k, (columns, epilogue, block) in enumerate(projs):
        paired.append(epilogue == _PAIRED)
        epilogue = _lib.LINEAR_SILU_MUL if epilogue == _PAIRED else epilogue
        wt, ws = _projection_weights(r, columns, groups, gpu)
        spec = {"weight": wt, "weight_scales": ws, "epilogue": epilogue, "block": block}
        if epilogue == _lib.LINEAR_DELTA_DECAY:
            spec["aux"] = _dev(r.uniform(-2, 1, columns).astype(np.float32), gpu)
            spec["bias"] = _dev(r.uniform(-1, 1, columns).astype(np.float32), gpu)
        if epilogue == _lib.LINEAR_SILU_MUL and not paired[k]:  # computed before the call
            spec["aux"] = _u16_dev(_f16(r.standard_normal((1, columns))), gpu)
        specs.append(spec)

    def outputs():
        outs = []
        for (columns, _, _), spec in zip(projs, specs):
            dtype = torch.float32 if spec["epilogue"] in f32 else torch.float16
            outs.append(torch.full((1, columns), -7.0, dtype=dtype, device=gpu))
        return outs

    # separate launches
    s3 = torch.empty(1, width, dtype=torch.float16, device=gpu)
    q3 = torch.empty(1, groups * 32, dtype=torch.int8, device=gpu)
    c3 = torch.empty(1, groups, dtype=torch.float32, device=gpu)
    i3 = torch.zeros(1, dtype=torch.int32, device=gpu)
    ops.add_rms_norm_quantize(da, db if add else None, s3 if add else None, dw, q3, c3, i3)
    o3 = outputs()
    for k, spec in enumerate(specs):
        aux = o3[k - 1] if paired[k] else spec.get("aux")
        ops.linear_w8a8(q3, c3, spec["weight"], spec["weight_scales"], o3[k], spec["epilogue"],
                        spec["block"], aux, spec.get("bias"))
    # one launch
    s1 = torch.empty_like(s3)
    q1 = torch.zeros_like(q3)
    c1 = torch.zeros_like(c3)
    i1 = torch.zeros(1, dtype=torch.int32, device=gpu)
    o1 = outputs()
    plist = [dict(spec, out=o1[k], **({"aux": o1[k - 1]} if paired[k] else {}))
             for k, spec in enumerate(specs)]
    ops.add_rms_norm_linear_w8a8(da, db if add else None, s1 if add else None, dw, plist, q1, c1,
                                 i1)
    torch.cuda.synchronize()
    if add:
        assert np.array_equal(_host_u16(s1), _host_u16(s3))
    assert torch.equal(q1, q3)
    assert np.array_equal(c1.cpu().numpy().view(np.uint32), c3.cpu().numpy().view(np.uint32))
    assert int(i1.item()) == int(i3.item()) == (1 if special else 0)
    for k in range(len(projs)):
        assert np.array_equal(o1[k].cpu().numpy().view(np.uint8),
                              o3[k].cpu().numpy().view(np.uint8)), f"projection {k}"


@pytest.mark.parametrize("width,columns,second", [(2560, 8192, 4096), (1000, 300, 0),
                                                  (4096, 65, 64)])
def test_add_rms_norm_linear_conv_is_the_separate_ops(gpu, width, columns, second):
    """A projection with the convolution epilogue equals linear_w8a8 of the
    quantized row followed by causal_conv (one token, kernel 4, SiLU) of its
    output, bit for bit: the convolution's output and its updated history,
    twice in a row (the second call convolving over the first's history);
    a projection beside it keeps its own output (second: its columns, 0
    for none)."""
    print(f"addRmsNormLinearW8A8 conv width={width} columns={columns} second={second}",
          flush=True)
    r = np.random.default_rng(width + columns)
    groups = (width + 31) // 32
    w = _dev((r.standard_normal(width) * 0.2).astype(np.float32), gpu)
    wt, ws = _projection_weights(r, columns, groups, gpu)
    cw = _u16_dev(_f16(r.standard_normal((columns, 4)) * 0.5), gpu)
    hist0 = _f16(r.standard_normal((columns, 3)))
    h_ref, h_got = _u16_dev(hist0, gpu), _u16_dev(hist0, gpu)
    extra = _projection_weights(r, second, groups, gpu) if second else None
    for step in range(2):
        a = _u16_dev(_f16(r.standard_normal((1, width)) * 3), gpu)
        b = _u16_dev(_f16(r.standard_normal((1, width)) * 3), gpu)
        # separate launches
        s3 = torch.empty(1, width, dtype=torch.float16, device=gpu)
        q3 = torch.empty(1, groups * 32, dtype=torch.int8, device=gpu)
        c3 = torch.empty(1, groups, dtype=torch.float32, device=gpu)
        ops.add_rms_norm_quantize(a, b, s3, w, q3, c3)
        x = torch.empty(1, columns, dtype=torch.float16, device=gpu)
        ops.linear_w8a8(q3, c3, wt, ws, x)
        want = torch.empty_like(x)
        ops.causal_conv(x, cw, h_ref, want, silu=True)
        if second:
            want2 = torch.empty(1, second, dtype=torch.float16, device=gpu)
            ops.linear_w8a8(q3, c3, extra[0], extra[1], want2)
        # one launch
        s1 = torch.empty_like(s3)
        got = torch.full_like(x, -7.0)
        plist = [{"weight": wt, "weight_scales": ws, "out": got, "conv_weight": cw,
                  "conv_history": h_got}]
        if second:
            got2 = torch.full_like(want2, -7.0)
            plist.append({"weight": extra[0], "weight_scales": extra[1], "out": got2})
        ops.add_rms_norm_linear_w8a8(a, b, s1, w, plist)
        torch.cuda.synchronize()
        g, e = _host_u16(got).reshape(-1), _host_u16(want).reshape(-1)
        assert np.array_equal(g, e), f"step {step}"
        assert np.array_equal(_host_u16(h_got), _host_u16(h_ref)), f"history, step {step}"
        assert np.array_equal(_host_u16(s1), _host_u16(s3))
        if second:
            assert np.array_equal(_host_u16(got2), _host_u16(want2))


def test_add_rms_norm_linear_without_q(gpu):
    """q and scales may be omitted; the projections are the same."""
    print("addRmsNormLinearW8A8 without q", flush=True)
    r = np.random.default_rng(7)
    width, groups = 2560, 80
    a = _u16_dev(_f16(r.standard_normal((1, width))), gpu)
    w = _dev((r.standard_normal(width) * 0.2).astype(np.float32), gpu)
    wt, ws = _projection_weights(r, 300, groups, gpu)
    q = torch.empty(1, groups * 32, dtype=torch.int8, device=gpu)
    c = torch.empty(1, groups, dtype=torch.float32, device=gpu)
    ops.add_rms_norm_quantize(a, None, None, w, q, c)
    want = torch.empty(1, 300, dtype=torch.float16, device=gpu)
    ops.linear_w8a8(q, c, wt, ws, want)
    got = torch.empty_like(want)
    ops.add_rms_norm_linear_w8a8(a, None, None, w,
                                 [{"weight": wt, "weight_scales": ws, "out": got}])
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("rows,width", [(32, 128), (1024 * 32, 128), (5, 256), (3, 32)])
@pytest.mark.parametrize("special", [False, True])
def test_gated_norm_quantize_is_the_two_ops(gpu, rows, width, special):
    """The activated gated RMSNorm and the quantization of its output in one
    launch equal gated_rms_norm (fp32 gate) followed by quantize_activation
    of the flattened rows, bit for bit: the normalised rows, the int8 rows,
    the scales and the invalid flag (special: an infinite input)."""
    print(f"gatedRmsNormQuantize rows={rows} width={width} special={special}", flush=True)
    r = np.random.default_rng(rows + width)
    x = _f16(r.standard_normal((rows, width)) * 2)
    if special:
        x[rows // 2, width // 3] = 0x7C00
    dx = _u16_dev(x, gpu)
    gate = _dev((r.standard_normal((rows, width)) * 1.5).astype(np.float32), gpu)
    w = _dev((r.standard_normal(width) * 0.2).astype(np.float32), gpu)
    n = rows * width
    out2 = torch.empty(rows, width, dtype=torch.float16, device=gpu)
    q2 = torch.empty(1, n, dtype=torch.int8, device=gpu)
    c2 = torch.empty(1, n // 32, dtype=torch.float32, device=gpu)
    i2 = torch.zeros(1, dtype=torch.int32, device=gpu)
    ops.gated_rms_norm(dx, gate, w, out2)
    ops.quantize_activation(out2.view(1, n), q2, c2, i2)
    out1 = torch.empty_like(out2)
    q1, c1 = torch.zeros_like(q2), torch.zeros_like(c2)
    i1 = torch.zeros(1, dtype=torch.int32, device=gpu)
    ops.gated_rms_norm_activated_quantize(dx, gate, w, out1, q1, c1, i1)
    torch.cuda.synchronize()
    assert np.array_equal(_host_u16(out1), _host_u16(out2))
    assert torch.equal(q1, q2)
    assert np.array_equal(c1.cpu().numpy().view(np.uint32), c2.cpu().numpy().view(np.uint32))
    assert int(i1.item()) == int(i2.item()) == (1 if special else 0)
