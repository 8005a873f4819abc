"""Op-contract parity with the reference's GraphIR (lib/GraphIR/Graph.cpp).

The session's pre-launch checks (llmi_hip_session_check, the same function
llmi_hip_session_step runs before it allocates or launches) are compared with
the reference's own Graph.cpp, compiled from its sources into oracle/_ref, on
the same shapes:

  * StepShape: 0 < tokens <= capacity - past (Graph.cpp:382-387);
  * KvAppend / CausalGqa (Graph.cpp:248-279): q [T, Hq, d], k/v [T, Hkv, d],
    caches [capacity, Hkv, d] fp16, Hq % Hkv == 0, positive dimensions
    (Graph.cpp:23-26); KvAppend writes rows [past, past + T) (version 0 -> 1)
    and CausalGqa reads [0, past + T) at version 1;
  * DeltaUpdate (Graph.cpp:226-246): q, k [T, Hk*dk] f32, v [T, Hv*dv] f16,
    beta, decay [T, Hv] f32, state [Hv, dk, dv] f32, Hv % Hk == 0;
  * graph order: CausalGqa without the KvAppend before it is rejected.

Where the two differ by design the test says so: the reference's Metal
lowering caps every tensor at 2^32 elements (MetalExecutionPlan.cpp:32-40),
which the backend enforces at the same point (the graph itself accepts
such shapes), and a valid op with no HIP kernel is UNSUPPORTED, not invalid.
No GPU is needed: nothing here launches.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from llminfer_amd import _lib
from llminfer_amd.session import HipSession

F16, F32 = 2, 3


@pytest.fixture(scope="module")
def ref():
    if not oracle.REF_PATH.exists():
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    lib = C.CDLL(str(oracle.REF_PATH))
    u64p = C.POINTER(C.c_uint64)
    lib.ref_gqa_graph.restype = C.c_int
    lib.ref_gqa_graph.argtypes = [C.c_uint64] * 3 + [u64p] * 4 + [C.c_int] * 3 + \
        [u64p, u64p, C.c_char_p, C.c_size_t]
    lib.ref_delta_graph.restype = C.c_int
    lib.ref_delta_graph.argtypes = [C.c_uint64, C.POINTER(C.c_int), u64p, C.POINTER(C.c_int),
                                    u64p, C.c_int, u64p, C.c_char_p, C.c_size_t]
    return lib


def _arr(vals):
    return (C.c_uint64 * len(vals))(*vals)


def ref_gqa(ref, T, P, cap, hq, hkv, d, skip_append=False):
    """(KvAppend accepted, CausalGqa accepted, effects) from Graph.cpp."""
    cost = (C.c_uint64 * 6)()
    eff = (C.c_uint64 * 6)()
    msg = C.create_string_buffer(256)
    mask = ref.ref_gqa_graph(T, P, cap, _arr([T, hq, d]), _arr([T, hkv, d]),
                             _arr([T, hkv, d]), _arr([cap, hkv, d]), F16, F16,
                             2 if skip_append else 0, cost, eff, msg, 256)
    return bool(mask & 2), bool(mask & 4), tuple(eff), msg.value.decode()


def ref_delta(ref, T, hk, dk, hv, dv):
    ranks = (C.c_int * 5)(2, 2, 2, 2, 2)
    dims = _arr([T, hk * dk, 0, 0, T, hk * dk, 0, 0, T, hv * dv, 0, 0,
                 T, hv, 0, 0, T, hv, 0, 0])
    elems = (C.c_int * 5)(F32, F32, F16, F32, F32)
    cost = (C.c_uint64 * 4)()
    return ref.ref_delta_graph(T, ranks, dims, elems, _arr([hv, dk, dv]), F32, cost,
                               None, 0) == 1


def ours(T, P, cap, hq, hkv, d, hk, dk, hv, dv):
    cfg = _lib.SessionConfig(cap, hq, hkv, d, hk, dk, hv, dv)
    return HipSession.check(cfg, P, T)


def _fits32(*dims):
    return int(np.prod([int(x) for x in dims], dtype=object)) < 2 ** 32


def test_step_contract_matches_graph_cpp(ref):
    rng = np.random.default_rng(8)
    seen = {"accept": 0, "reject": 0}
    for i in range(3000):
        T = int(rng.integers(0, 40))
        P = int(rng.integers(0, 300))
        cap = max(0, P + T + int(rng.integers(-4, 6)))
        hkv = int(rng.integers(0, 5))
        hq = hkv * int(rng.integers(1, 5)) + (int(rng.integers(1, 3)) if i % 7 == 0 else 0)
        d = int(rng.choice([0, 8, 12, 64, 128, 256, 320]))
        hk = int(rng.integers(0, 4))
        hv = hk * int(rng.integers(1, 4)) + (1 if i % 11 == 0 else 0)
        dk = int(rng.choice([0, 4, 64, 128]))
        dv = int(rng.choice([0, 4, 48, 128]))
        app, gqa, _, _ = ref_gqa(ref, T, P, cap, hq, hkv, d)
        want = app and gqa and ref_delta(ref, T, hk, dk, hv, dv)
        got = ours(T, P, cap, hq, hkv, d, hk, dk, hv, dv)
        case = (T, P, cap, hq, hkv, d, hk, dk, hv, dv)
        if want:
            assert got == _lib.OK, (case, _lib.load().llmi_hip_last_error())
        else:
            assert got == _lib.INVALID_ARGUMENT, case
        seen["accept" if want else "reject"] += 1
    assert min(seen.values()) > 300, seen


@pytest.mark.parametrize("T,P,cap", [(1, 4096, 8192), (2048, 2048, 4096), (1, 32768, 32800),
                                     (128, 0, 128), (17, 0, 160)])
def test_configs_accepted_and_effects(ref, T, P, cap):
    """The north-star configurations pass both; the reference records the
    effects the session's kernels produce (KvAppend writes [P, P+T) and moves
    the caches to version 1; CausalGqa reads [0, P+T) at version 1). The GPU
    session tests check that exactly those cache rows change."""
    app, gqa, eff, _ = ref_gqa(ref, T, P, cap, 16, 4, 256)
    assert app and gqa and ref_delta(ref, T, 16, 128, 32, 128)
    assert eff == (P, T, 1, 0, P + T, 1)
    assert ours(T, P, cap, 16, 4, 256, 16, 128, 32, 128) == _lib.OK


def test_attention_requires_the_append(ref):
    """Graph order: CausalGqa on caches no KvAppend has written this step is
    rejected by the reference (Graph.cpp:264-267). The session cannot issue
    it: every step records KvAppend (op 1) before CausalGqa (op 2)."""
    app, gqa, _, msg = ref_gqa(ref, 1, 10, 16, 16, 4, 256, skip_append=True)
    assert not app and not gqa and "appended KV version" in msg


def test_index_limit_is_the_lowerings(ref):
    """A cache of more than 2^32 elements is a valid graph (Graph.cpp has no
    such limit) but no Metal lowering accepts it (MetalExecutionPlan.cpp:
    32-40); the backend rejects it at the same point, before any launch."""
    cap, hkv, d = 1 << 21, 8, 512
    assert not _fits32(cap, hkv, d)
    app, gqa, _, _ = ref_gqa(ref, 1, 0, cap, 16, hkv, d)
    assert app and gqa
    assert ours(1, 0, cap, 16, hkv, d, 16, 128, 32, 128) == _lib.INVALID_ARGUMENT
    assert "32-bit" in _lib.load().llmi_hip_last_error().decode()


def test_headdim_without_kernel_is_unsupported(ref):
    """head_dim 1024 is a valid graph, but no HIP kernel takes it: UNSUPPORTED,
    a status distinct from a contract violation."""
    app, gqa, _, _ = ref_gqa(ref, 3, 5, 8, 4, 2, 1024)
    assert app and gqa
    assert ours(3, 5, 8, 4, 2, 1024, 1, 4, 1, 4) == _lib.UNSUPPORTED
