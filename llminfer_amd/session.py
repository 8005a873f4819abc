"""HipSession: the reference's session contract over the C ABI.

Mirrors MetalSession (include/llminfer/Backend/Metal/MetalSession.h:28-50,
lib/Backend/Metal/MetalExecutor.mm:230-298) for one hybrid layer pair -- a
DeltaNet layer and a GQA layer. The session owns the device state (K/V
caches [capacity, Hkv, d] fp16, recurrent state [Hv, dk, dv] fp32); step()
validates before launching, advances `past` only on success and leaves the
session invalid after a failure that happened after a launch; reset() zeroes
the state.

    s = HipSession.open(capacity=8192)        # cfg shapes by default
    res = s.step(delta_q, delta_k, delta_v, beta, decay, q, k, v)
    res.delta_out, res.gqa_out, res.dispatches  # plan records {op_index, kernel}
    HipSession.check(cfg, past, tokens)         # the step's checks, no device
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib


@dataclass
class StepResult:
    """MetalStepResult (MetalSession.h:18-25) without the logits."""
    past: int
    delta_out: torch.Tensor
    gqa_out: torch.Tensor
    dispatches: list[dict]


class HipSession:
    def __init__(self, handle: int, cfg: _lib.SessionConfig, device: torch.device):
        self._h = handle
        self.cfg = cfg
        self.device = device

    @classmethod
    def open(cls, capacity: int, query_heads: int = 16, kv_heads: int = 4,
             head_dim: int = 256, key_heads: int = 16, key_dim: int = 128,
             value_heads: int = 32, value_dim: int = 128,
             device: torch.device | None = None) -> "HipSession":
        dev = device or torch.device("cuda", torch.cuda.current_device())
        lib = _lib.load()
        cfg = _lib.SessionConfig(capacity, query_heads, kv_heads, head_dim, key_heads,
                                 key_dim, value_heads, value_dim)
        h = C.c_void_p()
        with torch.cuda.device(dev):
            _lib.check(lib.llmi_hip_session_open(C.byref(cfg),
                                                 torch.cuda.current_stream().cuda_stream,
                                                 C.byref(h)))
        return cls(h.value, cfg, dev)

    @staticmethod
    def check(cfg: _lib.SessionConfig, past: int, tokens: int) -> int:
        """The status a step of `tokens` at `past` would get from its checks
        (llmi_hip_session_check; host only)."""
        return _lib.load().llmi_hip_session_check(C.byref(cfg), past, tokens)

    def close(self) -> None:
        if self._h:
            _lib.load().llmi_hip_session_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self) -> None:
        _lib.load().llmi_hip_session_reset(self._h)

    @property
    def past(self) -> int:
        return _lib.load().llmi_hip_session_past(self._h)

    @property
    def invalid(self) -> bool:
        return bool(_lib.load().llmi_hip_session_invalid(self._h))

    def _view(self, ptr_fn, shape, dtype) -> torch.Tensor:
        """A copy of a session-owned device buffer (for inspection and tests)."""
        ptr = getattr(_lib.load(), ptr_fn)(self._h)
        torch.cuda.synchronize(self.device)
        return torch.as_tensor(_DeviceArray(ptr, shape, dtype), device=self.device).clone()

    def restore(self, past: int) -> None:
        """Declare cache rows [0, past) and the recurrent state as written
        through the writable views (a restored checkpoint, a seeded test)."""
        _lib.check(_lib.load().llmi_hip_session_restore(self._h, past))

    def writable_views(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Zero-copy tensors over the session-owned K cache, V cache and
        recurrent state, for seeding them before restore()."""
        c = self.cfg
        lib = _lib.load()
        kv = (c.capacity, c.kvHeads, c.headDim)
        mk = lambda fn, shape, dt: torch.as_tensor(
            _DeviceArray(getattr(lib, fn)(self._h), shape, dt), device=self.device)
        return (mk("llmi_hip_session_key_cache", kv, torch.float16),
                mk("llmi_hip_session_value_cache", kv, torch.float16),
                mk("llmi_hip_session_recurrent_state",
                   (c.valueHeads, c.keyDim, c.valueDim), torch.float32))

    def key_cache(self) -> torch.Tensor:
        c = self.cfg
        return self._view("llmi_hip_session_key_cache",
                          (c.capacity, c.kvHeads, c.headDim), torch.float16)

    def value_cache(self) -> torch.Tensor:
        c = self.cfg
        return self._view("llmi_hip_session_value_cache",
                          (c.capacity, c.kvHeads, c.headDim), torch.float16)

    def recurrent_state(self) -> torch.Tensor:
        c = self.cfg
        return self._view("llmi_hip_session_recurrent_state",
                          (c.valueHeads, c.keyDim, c.valueDim), torch.float32)

    def step(self, dq, dk, dv, beta, decay, q, k, v) -> StepResult:
        """One step of T tokens: DeltaUpdate, KvAppend, CausalGqa (graph order)."""
        c = self.cfg
        T = q.shape[0]
        want = ((dq, torch.float32), (dk, torch.float32), (dv, torch.float16),
                (beta, torch.float32), (decay, torch.float32), (q, torch.float16),
                (k, torch.float16), (v, torch.float16))
        for t, dt in want:
            if not t.is_cuda or t.dtype != dt or not t.is_contiguous():
                raise ValueError("session step operands must be contiguous device tensors "
                                 "of the op contract's dtypes")
        if dq.shape != (T, c.keyHeads * c.keyDim) or dk.shape != dq.shape or \
                dv.shape != (T, c.valueHeads * c.valueDim) or \
                beta.shape != (T, c.valueHeads) or decay.shape != beta.shape or \
                q.shape != (T, c.queryHeads, c.headDim) or \
                k.shape != (T, c.kvHeads, c.headDim) or v.shape != k.shape:
            raise ValueError("session step operand shapes do not match the session")
        delta_out = torch.empty_like(dv)
        gqa_out = torch.empty_like(q)
        recs = (_lib.Dispatch * 16)()
        n = C.c_size_t()
        lib = _lib.load()
        _lib.check(lib.llmi_hip_session_step(
            self._h, T, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), beta.data_ptr(),
            decay.data_ptr(), delta_out.data_ptr(), q.data_ptr(), k.data_ptr(),
            v.data_ptr(), gqa_out.data_ptr(), recs, len(recs), C.byref(n)))
        # Records as tools/run/Main.cpp:244-255 prints them: epilogue and
        # fused_op_index only for a record with a non-empty epilogue.
        plan = []
        for i in range(min(n.value, len(recs))):
            rec = {"op_index": int(recs[i].op_index), "kernel": recs[i].kernel.decode()}
            if recs[i].epilogue:
                rec["epilogue"] = recs[i].epilogue.decode()
                rec["fused_op_index"] = int(recs[i].fused_op_index)
            plan.append(rec)
        return StepResult(self.past, delta_out, gqa_out, plan)


class _DeviceArray:
    """__cuda_array_interface__ over a raw device pointer (zero-copy import)."""

    _TYPES = {torch.float16: "<f2", torch.float32: "<f4"}

    def __init__(self, ptr: int, shape, dtype):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": self._TYPES[dtype],
                                         "data": (int(ptr), False), "version": 2}
