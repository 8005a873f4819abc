"""llmi_hip_kv_append_causal_gqa_noalloc: the allocation-free variant of
llmi_hip_kv_append_causal_gqa (its split partials in a static device array)
gives the same output bits and the same appended cache rows as the
workspace entry point, called through the C ABI, on two calls in a row --
the second on a smaller context -- and both are within the north-star 2e-3
of the double-precision oracle."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from llminfer_amd import _lib
from tests.conftest import torch_to_u16, u16_to_torch

pytestmark = pytest.mark.gpu


def _call(fn, q, kn, vn, kc, vc, out, p, ws=None):
    stream = torch.cuda.current_stream().cuda_stream
    if ws is None:
        return fn(q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                  out.data_ptr(), p, stream)
    return fn(q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kc.data_ptr(), vc.data_ptr(),
              out.data_ptr(), p, ws.data_ptr(), ws.numel(), stream)


@pytest.mark.parametrize("pasts", [(32768, 4096), (4096, 33)])
def test_noalloc_matches_workspace_entry(gpu, pasts):
    lib = _lib.load()
    for past in pasts:
        print(f"noalloc decode past={past}", flush=True)
        x = oracle.make_gqa_inputs(70 + past, 1, 16, 4, 256, past, capacity=past + 3)
        p = _lib.GqaParams(1, 16, 4, 256, past)
        need = lib.llmi_hip_gqa_workspace_bytes(p)
        assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES
        q, kn, vn = (u16_to_torch(a, gpu) for a in (x.q, x.k_new, x.v_new))
        outs, caches = [], []
        for variant in ("workspace", "noalloc"):
            kc = u16_to_torch(x.k_cache, gpu)
            vc = u16_to_torch(x.v_cache, gpu)
            kc[past:] = 0
            vc[past:] = 0
            out = torch.empty_like(q)
            if variant == "workspace":
                ws = torch.empty(need, dtype=torch.uint8, device=gpu)
                st = _call(lib.llmi_hip_kv_append_causal_gqa, q, kn, vn, kc, vc, out, p, ws)
            else:
                st = _call(lib.llmi_hip_kv_append_causal_gqa_noalloc, q, kn, vn, kc, vc, out, p)
            _lib.check(st)
            torch.cuda.synchronize()
            outs.append(torch_to_u16(out))
            caches.append((torch_to_u16(kc), torch_to_u16(vc)))
        assert np.array_equal(outs[0], outs[1])
        for a, b, want in ((caches[0][0], caches[1][0], x.k_cache),
                           (caches[0][1], caches[1][1], x.v_cache)):
            assert np.array_equal(a, b) and np.array_equal(b, want)
        got = oracle.f16_to_f32(outs[1]).astype(np.float64)
        err = np.max(np.abs(got - oracle.gqa_dense_f64(x.q, x.k_cache, x.v_cache, past)))
        assert err <= 2e-3, err


def test_noalloc_prefill_needs_no_scratch(gpu):
    """T > 1 runs append + the MFMA prefill, which take no workspace: the
    same bits as the workspace entry point."""
    lib = _lib.load()
    x = oracle.make_gqa_inputs(5, 40, 16, 4, 256, 24)
    p = _lib.GqaParams(40, 16, 4, 256, 24)
    q, kn, vn = (u16_to_torch(a, gpu) for a in (x.q, x.k_new, x.v_new))
    res = []
    for noalloc in (False, True):
        kc, vc = u16_to_torch(x.k_cache, gpu), u16_to_torch(x.v_cache, gpu)
        out = torch.empty_like(q)
        if noalloc:
            st = _call(lib.llmi_hip_kv_append_causal_gqa_noalloc, q, kn, vn, kc, vc, out, p)
        else:
            st = _call(lib.llmi_hip_kv_append_causal_gqa, q, kn, vn, kc, vc, out, p,
                       torch.empty(1, dtype=torch.uint8, device=gpu))
        _lib.check(st)
        torch.cuda.synchronize()
        res.append(torch_to_u16(out))
    assert np.array_equal(res[0], res[1])
