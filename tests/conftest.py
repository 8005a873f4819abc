import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    # GPU tests are not silently skipped: without a device they fail in
    # their fixture, so `-m gpu` on a GPU-less host is a visible failure.
    pass


def u16_to_torch(a, device="cuda"):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.float16)
    return t.to(device)


def torch_to_u16(t):
    return t.detach().cpu().contiguous().view(__import__("torch").int16).numpy().view(np.uint16)


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    import llminfer_amd._lib as L
    L.load()  # the HIP library must be there; no fallback exists
    return torch.device("cuda", 0)


def p_rounding_bound(q, k, v, P):
    """First-order bound of rounding every softmax weight to fp16 before the
    PV product: |dO| <= u * sum_j p_j |v_j| / l with u = 2^-11 (fp16 unit
    roundoff). Zero for kernels that keep P in fp32. q [T,Hq,d], k/v
    [>=P+T, Hkv, d] as fp16 bits."""
    import oracle
    qf, kf, vf = (oracle.f16_to_f32(a).astype(np.float64) for a in (q, k, v))
    T, hq, d = q.shape
    g = hq // k.shape[1]
    bound = np.zeros((T, hq, d))
    for t in range(T):
        for h in range(hq):
            n = P + t + 1
            s = kf[:n, h // g] @ qf[t, h] / np.sqrt(d)
            p = np.exp(s - s.max())
            bound[t, h] = 2.0 ** -11 * (p @ np.abs(vf[:n, h // g])) / p.sum()
    return bound
