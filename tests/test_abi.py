"""The C-ABI library loads and exports what include/*.h declares; host-side
validation and plan records work without a GPU (no kernel is launched: every
call below is rejected, or only sizes/names something, before any launch)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from llminfer_amd import _lib

ROOT = Path(__file__).resolve().parent.parent


def declared_functions() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"LLMI_HIP_API\s+[^;{]*?\b(llmi_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_header_declares_the_boundary():
    names = declared_functions()
    for n in ("llmi_hip_kv_append", "llmi_hip_causal_gqa", "llmi_hip_delta_update",
              "llmi_hip_session_step", "llmi_hip_kernel_name"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_bindings_cover_every_declared_symbol():
    assert declared_functions() == set(_lib.SIGNATURES)


def test_param_structs_match_reference_layout():
    # All fields 32-bit unsigned, in the reference's order
    # (ReferenceParams.h:49-55, GraphParams.h:50-52).
    assert C.sizeof(_lib.CacheParams) == 8
    assert C.sizeof(_lib.GqaParams) == 20
    assert C.sizeof(_lib.GraphDeltaParams) == 20
    assert [f[0] for f in _lib.GqaParams._fields_] == \
        ["tokens", "queryHeads", "kvHeads", "headDim", "past"]
    assert [f[0] for f in _lib.GraphDeltaParams._fields_] == \
        ["tokens", "keyHeads", "keyDim", "valueHeads", "valueDim"]


def test_row_param_structs_match_reference_layout():
    # ReferenceParams.h:23-30, :44-47; GraphParams.h:35-38.
    assert C.sizeof(_lib.RowParams) == 12
    assert C.sizeof(_lib.ElementParams) == 4
    assert C.sizeof(_lib.RopeParams) == 36
    assert C.sizeof(_lib.PartialRopeParams) == 24
    assert [f[0] for f in _lib.RopeParams._fields_] == \
        ["tokens", "heads", "headDim", "rotaryDim", "headStride", "past", "outputStart",
         "epsilon", "theta"]
    assert [f[0] for f in _lib.PartialRopeParams._fields_] == \
        ["rows", "heads", "width", "rotaryWidth", "past", "theta"]


def test_invalid_rope_rejected_before_launch():
    lib = _lib.load()
    for p in (_lib.RopeParams(2, 4, 256, 63, 256, 0, 0, 1e-6, 1e7),    # odd rotary
              _lib.RopeParams(2, 4, 64, 128, 64, 0, 0, 1e-6, 1e7),     # rotary > width
              _lib.RopeParams(1 << 16, 16, 256, 64, 8192, 0, 0, 1e-6, 1e7)):  # > 32-bit
        assert lib.llmi_hip_norm_rope(1, 1, 1, p, None) == _lib.INVALID_ARGUMENT
        assert lib.llmi_hip_last_error()
    p = _lib.RopeParams(2, 4, 256, 64, 512, 0, 0, 1e-6, 1e7)
    assert lib.llmi_hip_norm_rope(None, 1, 1, p, None) == _lib.INVALID_ARGUMENT
    assert lib.llmi_hip_norm_rope(1, None, 1, p, None) == _lib.INVALID_ARGUMENT
    # empty shapes launch nothing and succeed
    for q in (_lib.RopeParams(0, 4, 256, 64, 512, 0, 0, 1e-6, 1e7),
              _lib.RopeParams(3, 0, 256, 64, 512, 0, 0, 1e-6, 1e7)):
        assert lib.llmi_hip_norm_rope(None, None, None, q, None) == _lib.OK
        assert lib.llmi_hip_dispatch_count(_lib.OP_NORM_ROPE, C.byref(q)) == 0
    assert lib.llmi_hip_partial_rope(1, 1, _lib.PartialRopeParams(4, 0, 64, 16, 0, 1e4),
                                     None) == _lib.INVALID_ARGUMENT
    assert lib.llmi_hip_partial_rope(1, 1, _lib.PartialRopeParams(4, 2, 64, 15, 0, 1e4),
                                     None) == _lib.INVALID_ARGUMENT
    assert lib.llmi_hip_rms_norm(None, 1, 1, _lib.RowParams(4, 64, 1e-6), None) == \
        _lib.INVALID_ARGUMENT
    assert lib.llmi_hip_sigmoid_mul(1, None, 1, _lib.ElementParams(8), None) == \
        _lib.INVALID_ARGUMENT
    assert lib.llmi_hip_sigmoid_mul(None, None, None, _lib.ElementParams(0), None) == _lib.OK


def test_plan_records_row_ops():
    from llminfer_amd import ops
    assert ops.kernel_names(_lib.OP_NORM_ROPE,
                            _lib.RopeParams(2048, 16, 256, 64, 512, 0, 0, 1e-6, 1e7)) == \
        ["normRopeTile"]
    assert ops.kernel_names(_lib.OP_NORM_ROPE,
                            _lib.RopeParams(3, 2, 100, 36, 100, 0, 0, 1e-6, 1e7)) == \
        ["normRopeRows"]
    # rows wider than the tile take a workgroup each up to 16K halves
    assert ops.kernel_names(_lib.OP_RMS_NORM, _lib.RowParams(7, 4096, 1e-6)) == \
        ["normRopeWide"]
    assert ops.kernel_names(_lib.OP_RMS_NORM, _lib.RowParams(7, 2560, 1e-6)) == \
        ["normRopeWide"]
    assert ops.kernel_names(_lib.OP_RMS_NORM, _lib.RowParams(7, 20000, 1e-6)) == \
        ["normRopeRows"]
    assert ops.kernel_names(_lib.OP_PARTIAL_ROPE,
                            _lib.PartialRopeParams(64, 16, 256, 64, 3, 1e7)) == \
        ["partialRopeTile"]
    assert ops.kernel_names(_lib.OP_SIGMOID_MUL, _lib.ElementParams(4096)) == ["sigmoidMulVec"]
    assert ops.kernel_names(_lib.OP_SIGMOID_MUL, _lib.ElementParams(4097)) == \
        ["sigmoidMulScalar"]


def test_delta_front_abi():
    from llminfer_amd import ops
    assert C.sizeof(_lib.ConvParams) == 16 and C.sizeof(_lib.L2Params) == 16
    lib = _lib.load()
    assert lib.llmi_hip_causal_conv(1, 1, 1, 1, _lib.ConvParams(4, 8, 9, 1), None) == \
        _lib.UNSUPPORTED
    assert lib.llmi_hip_causal_conv(1, 1, None, 1, _lib.ConvParams(4, 8, 4, 1), None) == \
        _lib.INVALID_ARGUMENT
    assert lib.llmi_hip_causal_conv(None, None, None, None, _lib.ConvParams(0, 8, 4, 1),
                                    None) == _lib.OK
    assert lib.llmi_hip_l2_norm(None, 1, _lib.L2Params(4, 128, 1e-6, 1.0), None) == \
        _lib.INVALID_ARGUMENT
    assert lib.llmi_hip_delta_gates(1, 1, 1, None, 1, 1, _lib.RowParams(4, 32, 0), None) == \
        _lib.INVALID_ARGUMENT
    assert ops.kernel_names(_lib.OP_CAUSAL_CONV, _lib.ConvParams(1024, 8192, 4, 1)) == \
        ["causalConv"]
    assert ops.kernel_names(_lib.OP_L2_NORM, _lib.L2Params(64, 128, 1e-6, 1.0)) == ["l2NormTile"]
    assert ops.kernel_names(_lib.OP_L2_NORM, _lib.L2Params(64, 100, 1e-6, 1.0)) == ["l2NormRows"]
    assert ops.kernel_names(_lib.OP_DELTA_GATES, _lib.RowParams(1024, 32, 0)) == ["deltaGates"]
    # gatedRmsNorm: the LDS tile up to width 256 in multiples of 8, else a
    # thread per row
    assert lib.llmi_hip_gated_rms_norm(None, 16, 16, 16, _lib.RowParams(4, 128, 1e-6), None) == \
        _lib.INVALID_ARGUMENT
    assert ops.kernel_names(_lib.OP_GATED_RMS_NORM, _lib.RowParams(32768, 128, 1e-6)) == \
        ["gatedRmsNormTile"]
    assert ops.kernel_names(_lib.OP_GATED_RMS_NORM, _lib.RowParams(4, 100, 1e-6)) == \
        ["gatedRmsNormRows"]


def test_invalid_gqa_rejected_before_launch():
    lib = _lib.load()
    bad = [_lib.GqaParams(0, 16, 4, 256, 0),     # no tokens
           _lib.GqaParams(1, 15, 4, 256, 0),     # Hq % Hkv != 0
           _lib.GqaParams(1, 16, 0, 256, 0),
           _lib.GqaParams(1 << 20, 1 << 10, 4, 256, 0)]  # beyond 32-bit indices
    for p in bad:
        st = lib.llmi_hip_causal_gqa(1, 1, 1, 1, p, None, 0, None)
        assert st == _lib.INVALID_ARGUMENT, p
        assert lib.llmi_hip_last_error()
        assert lib.llmi_hip_gqa_workspace_bytes(p) == 0
        assert lib.llmi_hip_dispatch_count(_lib.OP_CAUSAL_GQA, C.byref(p)) == 0
    # null buffers
    p = _lib.GqaParams(1, 16, 4, 256, 10)
    assert lib.llmi_hip_causal_gqa(None, 1, 1, 1, p, None, 0, None) == _lib.INVALID_ARGUMENT


def test_decode_requires_workspace():
    lib = _lib.load()
    p = _lib.GqaParams(1, 16, 4, 256, 4096)
    need = lib.llmi_hip_gqa_workspace_bytes(p)
    assert need > 4096
    st = lib.llmi_hip_causal_gqa(1, 1, 1, 1, p, None, 0, None)
    assert st == _lib.WORKSPACE
    st = lib.llmi_hip_causal_gqa(1, 1, 1, 1, p, 1, need - 1, None)
    assert st == _lib.WORKSPACE


def test_invalid_delta_rejected_before_launch():
    lib = _lib.load()
    for p in (_lib.GraphDeltaParams(0, 16, 128, 32, 128),
              _lib.GraphDeltaParams(4, 16, 128, 24, 128),   # Hv % Hk != 0
              _lib.GraphDeltaParams(4, 0, 128, 32, 128)):
        st = lib.llmi_hip_delta_update(1, 1, 1, 1, 1, 1, 1, p, None, 0, None)
        assert st == _lib.INVALID_ARGUMENT


def test_append_rejects_index_overflow():
    lib = _lib.load()
    st = lib.llmi_hip_kv_append(1, 1, 1, 1, _lib.CacheParams(16, 0xFFFFFFF8), None)
    assert st == _lib.INVALID_ARGUMENT
    assert lib.llmi_hip_cache_append(None, 1, _lib.CacheParams(4, 0), None) == \
        _lib.INVALID_ARGUMENT


@pytest.mark.parametrize("T,P,names", [
    (1, 4096, ["gqaDecodeSplitK", "gqaDecodeMerge"]),
    (1, 0, ["gqaDecodeSplitK"]),
    (2, 0, ["gqaPrefillMfma"]),
    (2048, 2048, ["gqaPrefillMfma"]),
])
def test_plan_records_gqa(T, P, names):
    from llminfer_amd import ops
    got = ops.kernel_names(_lib.OP_CAUSAL_GQA, _lib.GqaParams(T, 16, 4, 256, P))
    # The split-K decode merges its splits in a second launch or inside its
    # last workgroup, depending on the build's merge mode; one split needs no merge.
    if names[-1] == "gqaDecodeMerge":
        assert got in (names, names[:1])
    else:
        assert got == names


def test_plan_records_generic_shapes():
    from llminfer_amd import ops
    # The reference kernel test's head_dim 12 (FlashAttentionTest.mm:108).
    assert ops.kernel_names(_lib.OP_CAUSAL_GQA, _lib.GqaParams(19, 4, 2, 12, 0)) == \
        ["gqaGeneric"]
    assert ops.kernel_names(_lib.OP_DELTA_UPDATE, _lib.GraphDeltaParams(3, 2, 7, 4, 5)) == \
        ["deltaGeneric"]
    assert ops.kernel_names(_lib.OP_KV_APPEND, _lib.CacheParams(8, 0)) == ["kvAppend"]


def test_status_strings():
    lib = _lib.load()
    for st in range(6):
        assert lib.llmi_hip_status_string(st)
    assert lib.llmi_hip_status_string(99) == b"unknown status"
    assert b"gfx950" in lib.llmi_hip_build_info()


def test_session_open_validates_config():
    lib = _lib.load()
    h = C.c_void_p()
    bad = _lib.SessionConfig(0, 16, 4, 256, 16, 128, 32, 128)
    assert lib.llmi_hip_session_open(C.byref(bad), None, C.byref(h)) == _lib.INVALID_ARGUMENT
    bad = _lib.SessionConfig(64, 16, 5, 256, 16, 128, 32, 128)
    assert lib.llmi_hip_session_open(C.byref(bad), None, C.byref(h)) == _lib.INVALID_ARGUMENT
    assert h.value is None
    assert lib.llmi_hip_session_step(None, 1, *([None] * 10), None, 0, None) == \
        _lib.INVALID_ARGUMENT


def test_noalloc_rejects_partials_beyond_its_scratch():
    """The allocation-free decode refuses, before any launch, a split plan
    whose partials exceed its static scratch (here forced by planning for
    far more resident workgroups than a GPU has)."""
    import subprocess
    import sys
    code = (
        "from llminfer_amd import _lib\n"
        "lib = _lib.load()\n"
        "p = _lib.GqaParams(1, 128, 16, 256, 32768)\n"
        "need = lib.llmi_hip_gqa_workspace_bytes(p)\n"
        "assert need > _lib.NOALLOC_SCRATCH_BYTES, need\n"
        "st = lib.llmi_hip_kv_append_causal_gqa_noalloc(1, 1, 1, 1, 1, 1, p, None)\n"
        "assert st == _lib.WORKSPACE, st\n"
        "assert b'static scratch' in lib.llmi_hip_last_error()\n"
        "assert lib.llmi_hip_kv_append_causal_gqa_noalloc(None, 1, 1, 1, 1, 1, p, None) == "
        "_lib.INVALID_ARGUMENT\n")
    env = dict(__import__("os").environ, LLMI_DECODE_TARGET_WGS="65536")
    r = subprocess.run([sys.executable, "-c", code], cwd=str(ROOT), env=env,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr


def test_l2_norm_delta_update_rejects_shapes_without_kernel():
    """The fused L2Norm+DeltaUpdate has kernels for dk 64/128 only: dk = 7
    is UNSUPPORTED before any launch; a contract violation stays
    INVALID_ARGUMENT."""
    lib = _lib.load()
    p = _lib.GraphDeltaParams(4, 1, 7, 2, 5)
    assert lib.llmi_hip_l2_norm_delta_update(1, 1, 1, 1, 1, 1, 1, p, 1e-6, 1.0, None, 0,
                                             None) == _lib.UNSUPPORTED
    bad = _lib.GraphDeltaParams(4, 16, 128, 24, 128)  # Hv % Hk != 0
    assert lib.llmi_hip_l2_norm_delta_update(1, 1, 1, 1, 1, 1, 1, bad, 1e-6, 1.0, None, 0,
                                             None) == _lib.INVALID_ARGUMENT
    ok = _lib.GraphDeltaParams(1024, 16, 128, 32, 128)
    assert lib.llmi_hip_l2_norm_delta_update(1, 1, 1, 1, 1, 1, 1, ok, 1e-6, 1.0, None, 0,
                                             None) == _lib.WORKSPACE


def test_l2_norm_delta_gated_norm_rejects_shapes_without_kernel():
    """The fused L2Norm+DeltaUpdate+GatedRmsNorm has a chunked kernel (dk 128,
    T >= 32) and a one-workgroup-per-head recurrent kernel (dk 64/128, dv
    64/128, T <= 32): dk 64 at T = 64 and dv 48 at T = 5 are UNSUPPORTED
    before any launch; the chunked form checks its workspace and the 16-byte
    alignment of out and gate; a contract violation stays INVALID_ARGUMENT."""
    lib = _lib.load()
    f = lib.llmi_hip_l2_norm_delta_gated_norm
    for T, dk, dv in ((64, 64, 64), (5, 128, 48)):
        p = _lib.GraphDeltaParams(T, 2, dk, 4, dv)
        assert f(16, 16, 16, 16, 16, 16, 16, 16, 16, p, 1e-6, 0.1, 1e-6, None, 0,
                 None) == _lib.UNSUPPORTED, (T, dk, dv)
    ok = _lib.GraphDeltaParams(1024, 16, 128, 32, 128)
    assert f(16, 16, 16, 16, 16, 16, 16, 16, 16, ok, 1e-6, 0.1, 1e-6, None, 0,
             None) == _lib.WORKSPACE
    assert f(16, 16, 16, 16, 16, 16, 18, 16, 16, ok, 1e-6, 0.1, 1e-6, None, 0,
             None) == _lib.UNSUPPORTED  # gate not 16-byte aligned
    bad = _lib.GraphDeltaParams(4, 16, 128, 24, 128)  # Hv % Hk != 0
    assert f(16, 16, 16, 16, 16, 16, 16, 16, 16, bad, 1e-6, 0.1, 1e-6, None, 0,
             None) == _lib.INVALID_ARGUMENT
    assert f(16, 16, 16, 16, 16, 16, None, 16, 16, ok, 1e-6, 0.1, 1e-6, None, 0,
             None) == _lib.INVALID_ARGUMENT


def test_delta_norm_quantize_rejects_shapes_without_kernel():
    """The W8A8 DeltaNet tail in one call has only the one-workgroup-per-head
    kernel: T 33, dk 96 and dv 48 are UNSUPPORTED before any launch, and so
    are an out or quantized row that is not 16-byte aligned; a contract
    violation (Hv % Hk, a null buffer) stays INVALID_ARGUMENT."""
    lib = _lib.load()
    f = lib.llmi_hip_l2_norm_delta_gated_norm_activated_quantize
    ptrs = [16] * 12
    call = lambda p, ptrs=ptrs: f(*ptrs, p, 1e-6, 0.1, 1e-6, None)
    for T, dk, dv in ((33, 128, 128), (4, 96, 128), (5, 128, 48)):
        assert call(_lib.GraphDeltaParams(T, 2, dk, 4, dv)) == _lib.UNSUPPORTED, (T, dk, dv)
    ok = _lib.GraphDeltaParams(1, 16, 128, 32, 128)
    for at in (8, 9):  # out, quantized
        assert call(ok, [18 if i == at else 16 for i in range(12)]) == _lib.UNSUPPORTED, at
    assert call(_lib.GraphDeltaParams(1, 16, 128, 24, 128)) == _lib.INVALID_ARGUMENT
    for at in range(11):  # every buffer but the optional invalid flag
        assert call(ok, [None if i == at else 16 for i in range(12)]) == \
            _lib.INVALID_ARGUMENT, at


def test_gated_norm_status_host_paths():
    """The status call of the fused chain: the recurrent form (T <= 32) has
    no arrival wait and reports OK without touching the device; the chunked
    form refuses a workspace smaller than the call's; a contract violation
    stays INVALID_ARGUMENT. The wait bound setter returns the previous bound
    (2^22 polls by default)."""
    lib = _lib.load()
    st = lib.llmi_hip_l2_norm_delta_gated_norm_status
    assert st(None, 0, _lib.GraphDeltaParams(1, 16, 128, 32, 128), None) == _lib.OK
    assert st(None, 0, _lib.GraphDeltaParams(1024, 16, 128, 32, 128), None) == _lib.WORKSPACE
    assert st(None, 0, _lib.GraphDeltaParams(4, 16, 128, 24, 128), None) == \
        _lib.INVALID_ARGUMENT
    old = lib.llmi_hip_set_arrival_wait_limit(5)
    assert old == 1 << 22
    assert lib.llmi_hip_set_arrival_wait_limit(old) == 5


def test_w8a8_abi():
    """The W8A8 projection path: GraphParams.h:8-28 / ReferenceParams.h:4-6
    layouts, validation before any launch, plan-record names
    (LinearW8Launch.h:14-21: one row -> linearW8A8Gemv)."""
    from llminfer_amd import ops
    assert C.sizeof(_lib.QuantizeParams) == 12
    assert C.sizeof(_lib.LinearW8Params) == 28
    assert C.sizeof(_lib.GroupedEmbedParams) == 20
    assert C.sizeof(_lib.EmbedParams) == 16
    lib = _lib.load()
    a16 = 16  # a 16-byte-aligned stand-in pointer; nothing is launched
    ok = _lib.LinearW8Params(2560, 0, 80, 1, 2560, _lib.LINEAR_NONE, 0)
    assert lib.llmi_hip_linear_w8a8(None, None, None, None, None, None, None,
                                    _lib.LinearW8Params(2560, 0, 80, 0, 2560, 0, 0), None) == \
        _lib.OK
    bad = [
        _lib.LinearW8Params(2560, 0, 80, 1, 2560, 7, 0),                   # unknown epilogue
        _lib.LinearW8Params(2560, 0, 80, 1, 2560, _lib.LINEAR_SIGMOID_COLUMNS, 0),  # no block
        _lib.LinearW8Params(2560, 1, 80, 1, 2560, 0, 0),                   # past the width
        _lib.LinearW8Params(2560, 0, 0, 1, 2560, 0, 0),                    # no groups
    ]
    for p in bad:
        assert lib.llmi_hip_linear_w8a8(a16, a16, a16, a16, a16, None, None, p, None) == \
            _lib.INVALID_ARGUMENT
    silu_mul = _lib.LinearW8Params(2560, 0, 80, 1, 2560, _lib.LINEAR_SILU_MUL, 0)
    assert lib.llmi_hip_linear_w8a8(a16, a16, a16, a16, a16, None, None, silu_mul, None) == \
        _lib.INVALID_ARGUMENT
    decay = _lib.LinearW8Params(32, 0, 80, 4, 32, _lib.LINEAR_DELTA_DECAY, 0)
    assert lib.llmi_hip_linear_w8a8(a16, a16, a16, a16, a16, a16, None, decay, None) == \
        _lib.INVALID_ARGUMENT
    assert lib.llmi_hip_linear_w8a8(a16 + 1, a16, a16, a16, a16, None, None, ok, None) == \
        _lib.UNSUPPORTED
    assert lib.llmi_hip_quantize_activation(a16, a16, a16, None,
                                            _lib.QuantizeParams(4, 100, 3), None) == \
        _lib.INVALID_ARGUMENT
    assert lib.llmi_hip_embedding_w8(a16, a16, a16, a16,
                                     _lib.GroupedEmbedParams(4, 100, 0, 10, 3), None) == \
        _lib.INVALID_ARGUMENT
    assert lib.llmi_hip_embedding(None, a16, a16, _lib.EmbedParams(4, 100, 0, 10), None) == \
        _lib.INVALID_ARGUMENT
    assert ops.kernel_names(_lib.OP_LINEAR_W8A8, ok) == ["linearW8A8Gemv"]
    assert ops.kernel_names(_lib.OP_LINEAR_W8A8,
                            _lib.LinearW8Params(9216, 0, 80, 64, 9216, 2, 0)) == ["linearW8A8Gemm"]
    assert ops.kernel_names(_lib.OP_LINEAR_W8A8, bad[0]) == []
    assert ops.kernel_names(_lib.OP_QUANTIZE_ACTIVATION, _lib.QuantizeParams(4, 100, 4)) == \
        ["quantizeActivation"]
    assert ops.kernel_names(_lib.OP_EMBEDDING_W8,
                            _lib.GroupedEmbedParams(4, 100, 0, 10, 4)) == ["embeddingW8"]
    assert ops.kernel_names(_lib.OP_EMBEDDING, _lib.EmbedParams(4, 100, 0, 10)) == ["embedding"]


def test_norm_linear_abi():
    """The decode norm + projections launch: its parameter layout, the shapes
    it takes (one row of at most 4096, 1-4 projections of that row's
    groups, at most 4096 workgroups of 60 columns) and a SwiGLU multiplier
    computed in the same call only as the previous projection's output (the
    pair computed by the same lanes), a convolution epilogue only on the
    whole row of a projection with no epilogue that is no multiplier, all
    rejected before any launch."""
    from llminfer_amd import ops
    assert C.sizeof(_lib.NormProjection) == 56
    assert C.sizeof(_lib.NormLinearParams) == 12 + 4 + 4 * 28
    lib = _lib.load()
    a16 = 16  # a 16-byte-aligned stand-in pointer; nothing is launched

    def params(width, *linears, rows=1):
        p = _lib.NormLinearParams()
        p.norm = _lib.RowParams(rows, width, 1e-6)
        p.count = len(linears)
        for k, (cols, ep) in enumerate(linears):
            p.linear[k] = _lib.LinearW8Params(cols, 0, (width + 31) // 32, 1, cols, ep, 0)
        return p

    op = _lib.OP_ADD_RMS_NORM_LINEAR_W8A8
    good = params(2560, (8192, 0), (4096, _lib.LINEAR_SILU_F32), (32, _lib.LINEAR_DELTA_DECAY),
                  (32, _lib.LINEAR_DELTA_BETA))
    assert ops.kernel_names(op, good) == ["addRmsNormLinearW8A8"]
    for bad in (params(8192, (16, 0)), params(2560, (16, 0), rows=2), params(2560),
                params(2560, (0, 0)), params(40, (300000, 0))):
        assert ops.kernel_names(op, bad) == []
    wrong_groups = params(2560, (16, 0))
    wrong_groups.linear[0].groups = 79
    assert ops.kernel_names(op, wrong_groups) == []
    # a SwiGLU projection whose multiplier is computed in the call but is not
    # the previous projection's output, or is too wide to pair
    bufs = (_lib.NormProjection * _lib.NORM_LINEAR_MAX)()
    bufs[0] = _lib.NormProjection(a16, a16, 4096, None, None)
    bufs[1] = _lib.NormProjection(a16, a16, 8192, None, None)
    bufs[2] = _lib.NormProjection(a16, a16, 12288, 4096, None)
    p = params(2560, (64, 0), (64, 0), (64, _lib.LINEAR_SILU_MUL))
    assert lib.llmi_hip_add_rms_norm_linear_w8a8(a16, None, None, a16, None, None, None,
                                                 C.addressof(bufs), p, None) == _lib.UNSUPPORTED
    bufs[1] = _lib.NormProjection(a16, a16, 8192, 4096, None)
    for p in (params(4096, (64, 0), (64, _lib.LINEAR_SILU_MUL)),
              params(2560, (64, 0), (32, _lib.LINEAR_SILU_MUL)),
              params(2560, (64, _lib.LINEAR_SILU), (64, _lib.LINEAR_SILU_MUL))):
        assert lib.llmi_hip_add_rms_norm_linear_w8a8(a16, None, None, a16, None, None, None,
                                                     C.addressof(bufs), p, None) == \
            _lib.UNSUPPORTED
    bufs[1] = _lib.NormProjection(a16, a16, 8192, None, None)
    p = params(2560, (64, 0), (64, _lib.LINEAR_SILU_MUL))
    assert lib.llmi_hip_add_rms_norm_linear_w8a8(a16, None, None, a16, None, None, None,
                                                 C.addressof(bufs), p, None) == \
        _lib.INVALID_ARGUMENT
    # the convolution epilogue: weight and history together, on the whole
    # row of a projection with no epilogue that is no SwiGLU multiplier
    call = lambda p: lib.llmi_hip_add_rms_norm_linear_w8a8(
        a16, None, None, a16, None, None, None, C.addressof(bufs), p, None)
    bufs[0] = _lib.NormProjection(a16, a16, 4096, None, None, a16, None)
    assert call(params(2560, (64, 0))) == _lib.INVALID_ARGUMENT
    bufs[0] = _lib.NormProjection(a16, a16, 4096, None, None, a16, 8192)
    assert call(params(2560, (64, _lib.LINEAR_SILU))) == _lib.UNSUPPORTED
    split = params(2560, (64, 0))
    split.linear[0].firstRow = 32
    split.linear[0].columns = 32
    assert call(split) == _lib.UNSUPPORTED
    bufs[1] = _lib.NormProjection(a16, a16, 12288, 4096, None)
    assert call(params(2560, (64, 0), (64, _lib.LINEAR_SILU_MUL))) == _lib.UNSUPPORTED
