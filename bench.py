#!/usr/bin/env python3
"""Benchmark of the llminfer attention hot path on one MI355X (gfx950).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only-headline]
                    [--cpu-seconds S] [--no-cpu] [--only KEY,...]

`--only` runs just the named configurations (`headline` names the headline):
a profile of one configuration then holds that configuration's launches and
no other's. Without the headline the line carries only `configs`.

Prints ONE compact JSON line on stdout (under 7.5 KB: the contract's fields,
the headline's roofline and CPU baseline, and a short summary per
configuration); the full record of every leg goes to stderr as one
`[bench-detail] KEY {...}` line per leg, and to `--detail FILE` when given.
The headline workload is the GQA single-token decode
of the reference's decode path (KvAppend + CausalGqa, T=1, 4096 past rows,
capacity 8192, 16 query / 4 KV heads, head_dim 256, fp16): one "step" is one
attention layer's decode -- KvAppend + CausalGqa, which the backend runs as
one split-K launch that also appends the new row -- over inputs already
resident in HBM. `value` is GPU microseconds
per layer step (time-like, lower is better). The K/V caches rotate over 32
independent sets (1.07 GB) so that every step reads its 16.8 MB of K/V from
HBM rather than from the 256 MB Infinity Cache.

Timing. Warmup W steps, synchronize, then a spin kernel holds the GPU while
the host enqueues all K steps, so the GPU runs them back to back and the
measurement is device time, not Python launch latency. Start/end HIP events
on the launch stream bracket exactly the K steps (ms_per_step). The headline
step is one op -- the fused append+attention call -- so the same time is
the op's time per call for the roofline; the kernels it launches and their
rocprofv3 durations are listed in profiles/. (Events around every single
launch were avoided: each pair adds several microseconds to a kernel of
ten.) For the other configurations the dominant op is also timed in its own
back-to-back loop the same way.

`roofline`: algorithmic bytes of one decode launch (K and V rows [0, P+1)
plus q and out -- the reference cost model's traffic for CausalGqa,
lib/GraphIR/Cost.cpp:56-94 -- plus the 4 KB KvAppend cache write the launch
performs) / its average event-timed duration, against MI355X's 8 TB/s.
`traffic` is the HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE, read from profiles/traffic.json when that summary
exists for this kernel and workload.

`cpu_baseline`: the C oracle (oracle/liboracle.so, the same CPU restatement
the parity tests use) timed on this host's cores on the same inputs; it also
reports the GPU-vs-CPU max-abs output difference of the same step.

`configs`: the other BASELINE configurations measured the same way (prefill
128, chunked prefill 2048+2048, DeltaNet prefill 1024, hybrid 32K decode),
each with its roofline fraction and a bounded CPU sample.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = ("attn µs/layer + % HBM roofline (decode) / % MFMA peak (prefill), 1 GPU")
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s
CPU_THREAD_CAP = 16         # the GPU box's CPU share per GPU


# --------------------------------------------------------------- helpers

def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gqa_flops(T: int, P: int, hq: int, d: int) -> int:
    """2 x MACs of lib/GraphIR/Cost.cpp:188-201."""
    return 4 * hq * d * (T * P + T * (T + 1) // 2)


def gqa_bytes(T: int, P: int, hq: int, hkv: int, d: int) -> int:
    """q + visible K and V rows + out, fp16 (Cost.cpp:56-94 traffic)."""
    return 2 * (2 * T * hq * d + 2 * (P + T) * hkv * d)


def append_bytes(T: int, hkv: int, d: int) -> int:
    """KvAppend's cache write (its reads are the new K/V rows the attention
    reads anyway)."""
    return 2 * T * hkv * d * 2


def delta_flops(T: int, hv: int, dk: int, dv: int) -> int:
    """2 x MACs of Cost.cpp:180-187 (3 T Hv dk dv MACs)."""
    return 6 * T * hv * dk * dv


def delta_bytes(T: int, hk: int, dk: int, hv: int, dv: int) -> int:
    """f32 q, k; fp16 v; f32 beta, decay; f32 state in and out; fp16 out."""
    return (8 * T * hk * dk + 2 * T * hv * dv + 8 * T * hv
            + 8 * hv * dk * dv + 2 * T * hv * dv)


def rows_bytes(T: int, hq: int, hkv: int, d: int) -> dict:
    """Algorithmic HBM bytes of the attention block's row ops per call: each
    reads its fp16 input rows once and writes its output rows once (the
    gate half of the projected q is not read; the weights are 1 KB)."""
    return {"q_norm_rope": 2 * T * hq * d * 2 + d * 4,
            "k_norm_rope": 2 * T * hkv * d * 2 + d * 4,
            "gate": 3 * T * hq * d * 2}


def cpu_threads() -> int:
    import oracle
    return max(1, min(CPU_THREAD_CAP, oracle.cpu_count()))


def host_cores() -> int:
    """CPUs this process may run on (the box's share), not the thread cap."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def host_u16(t):
    import numpy as np
    import torch
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def host_f32(t):
    import numpy as np
    return t.detach().contiguous().cpu().numpy().astype(np.float32, copy=False)


def time_cpu(fn, budget_s: float, min_runs: int = 1) -> tuple[float, int]:
    """Mean seconds per fn() call, repeating until budget_s is spent."""
    runs, t0 = 0, time.perf_counter()
    while True:
        fn()
        runs += 1
        el = time.perf_counter() - t0
        if runs >= min_runs and el >= budget_s:
            return el / runs, runs
        if runs >= 10000:
            return el / runs, runs


# ------------------------------------------------------------- workloads

class Workload:
    """A repeatable step on resident device inputs.

    op(label, i) enqueues one op of step i (one C-ABI call: one or two
    launches); launch(i) enqueues the whole step, its ops in graph order.
    `dominant` labels the op the roofline is computed for.
    """
    name = ""
    tokens = 1
    dominant = "gqa"
    labels: tuple = ("gqa",)
    bound = "hbm"

    def op(self, label: str, i: int) -> None:
        raise NotImplementedError

    def launch(self, i: int) -> None:
        for label in self.labels:
            self.op(label, i)

    def kernels(self) -> str:
        """Kernel names of the dominant op (plan-record names)."""
        raise NotImplementedError

    def work(self, i: int) -> int:  # algorithmic bytes or flops of the dominant launch
        raise NotImplementedError

    def config(self) -> dict:
        raise NotImplementedError

    def cpu(self, budget_s: float) -> dict:
        raise NotImplementedError


def _randn16(gen, shape, dev):
    import torch
    return torch.randn(shape, generator=gen, device=dev, dtype=torch.float32).half()


class GqaDecode(Workload):
    """configs[1] (and the GQA half of configs[4]): KvAppend + split-K decode."""
    bound = "hbm"

    def __init__(self, dev, seed=2, past=4096, cap=8192, sets=32, hq=16, hkv=4, d=256):
        import torch
        from llminfer_amd import ops
        self.P, self.cap, self.sets, self.hq, self.hkv, self.d = past, cap, sets, hq, hkv, d
        self.name = f"gqa_decode_{past // 1024}k"
        g = torch.Generator(device=dev).manual_seed(seed)
        self.kc = [_randn16(g, (cap, hkv, d), dev) for _ in range(sets)]
        self.vc = [_randn16(g, (cap, hkv, d), dev) for _ in range(sets)]
        self.q = _randn16(g, (1, hq, d), dev)
        self.kn = _randn16(g, (1, hkv, d), dev)
        self.vn = _randn16(g, (1, hkv, d), dev)
        self.out = torch.empty_like(self.q)
        # KvAppend + CausalGqa as one fused launch (the append rides along).
        self.att = [ops.bind_kv_append_causal_gqa(self.q, self.kn, self.vn, self.kc[s],
                                                  self.vc[s], self.out, past)
                    for s in range(sets)]

    def op(self, label, i):
        self.att[i % self.sets]()

    def launch_warm(self, i):
        self.att[0]()

    def kernels(self):
        return self.att[0].what

    def work(self, i):
        return gqa_bytes(1, self.P, self.hq, self.hkv, self.d) + append_bytes(1, self.hkv, self.d)

    def config(self):
        return {"workload": self.name, "tokens": 1, "past": self.P, "capacity": self.cap,
                "query_heads": self.hq, "kv_heads": self.hkv, "head_dim": self.d,
                "kv_sets": self.sets,
                "kv_bytes_resident": 2 * self.sets * self.cap * self.hkv * self.d * 2,
                "cache_state": "cold: K/V rotate over independent sets larger than the MALL"}

    def cpu(self, budget_s):
        import numpy as np
        import oracle
        import torch
        s = 0
        torch.cuda.synchronize()
        kc, vc, q = host_u16(self.kc[s]), host_u16(self.vc[s]), host_u16(self.q)
        kn, vn = host_u16(self.kn), host_u16(self.vn)
        # Re-run the GPU step on set 0 so `out` belongs to these inputs.
        self.att[s]()
        torch.cuda.synchronize()
        gpu_out = oracle.f16_to_f32(host_u16(self.out))
        thr = cpu_threads()

        def step(threads):
            oracle.kv_append(kn, kc, self.P)
            oracle.kv_append(vn, vc, self.P)
            return oracle.gqa_f32(q, kc, vc, self.P, threads)

        want = step(thr)
        err = float(np.max(np.abs(gpu_out - oracle.f16_to_f32(want))))
        sec, runs = time_cpu(lambda: step(thr), budget_s)
        sec1, runs1 = time_cpu(lambda: step(1), budget_s / 4)
        return {"value": sec * 1e6, "unit": "µs/layer", "cores": thr, "kind": "port",
                "sample": f"the full step (KvAppend + CausalGqa, P={self.P}, 16/4 heads, d=256) "
                          f"on one cache set, {runs} runs, fp32 online softmax "
                          "(oracle orc_gqa_f32)",
                "single_thread_value": sec1 * 1e6, "single_thread_runs": runs1,
                "cpu_model": cpu_model(), "gpu_vs_cpu_max_abs": err}


class GqaPrefill(Workload):
    """configs[0] (T=128, P=0) and configs[2] (T=2048 after P=2048)."""
    bound = "mfma"
    labels = ("append", "gqa")

    def __init__(self, dev, T, P, cap, seed, hq=16, hkv=4, d=256):
        import torch
        from llminfer_amd import ops
        self.T, self.P, self.cap, self.hq, self.hkv, self.d = T, P, cap, hq, hkv, d
        self.name = f"gqa_prefill_{T}_past{P}"
        self.tokens = T
        g = torch.Generator(device=dev).manual_seed(seed)
        self.kc = _randn16(g, (cap, hkv, d), dev)
        self.vc = _randn16(g, (cap, hkv, d), dev)
        self.q = _randn16(g, (T, hq, d), dev)
        self.kn = _randn16(g, (T, hkv, d), dev)
        self.vn = _randn16(g, (T, hkv, d), dev)
        self.out = torch.empty_like(self.q)
        self.app = ops.bind_kv_append(self.kn, self.vn, self.kc, self.vc, P)
        self.att = ops.bind_causal_gqa(self.q, self.kc, self.vc, self.out, P)

    def op(self, label, i):
        (self.app if label == "append" else self.att)()

    def kernels(self):
        return self.att.what

    def work(self, i):
        return gqa_flops(self.T, self.P, self.hq, self.d)

    def config(self):
        return {"workload": self.name, "tokens": self.T, "past": self.P, "capacity": self.cap,
                "query_heads": self.hq, "kv_heads": self.hkv, "head_dim": self.d}

    def cpu(self, budget_s):
        import numpy as np
        import oracle
        import torch
        torch.cuda.synchronize()
        self.app()
        self.att()
        torch.cuda.synchronize()
        kc, vc, q = host_u16(self.kc), host_u16(self.vc), host_u16(self.q)
        gpu_out = oracle.f16_to_f32(host_u16(self.out))
        thr = cpu_threads()
        # Sample: a contiguous block of query rows centred on T/2, whose mean
        # visible length equals the whole chunk's (P + T/2); scaled by T/rows.
        rows = min(self.T, 64)
        t0 = (self.T - rows) // 2
        qs = np.ascontiguousarray(q[t0:t0 + rows])
        want = oracle.gqa_f32(qs, kc, vc, self.P + t0, thr)
        err = float(np.max(np.abs(gpu_out[t0:t0 + rows] - oracle.f16_to_f32(want))))
        sec, runs = time_cpu(lambda: oracle.gqa_f32(qs, kc, vc, self.P + t0, thr), budget_s)
        scale = self.T / rows
        return {"value": sec * scale * 1e6, "unit": "µs/layer", "cores": thr,
                "kind": "port",
                "sample": f"{rows} query rows [{t0}, {t0 + rows}) of {self.T} "
                          f"(mean visible length = the chunk's), x{scale:g}, {runs} runs",
                "gpu_vs_cpu_max_abs": err}


class AttnRows(Workload):
    """The attention block's row work on either side of CausalGqa
    (Qwen35ModelBuilder.cpp:175-197, lowered as MetalReferenceGraph.mm:307-330):
    q RmsNorm + PartialRoPE from the projected q with its gate interleaved
    (stride 2 * head_dim), k RmsNorm + PartialRoPE written straight into the
    key cache at row `past`, and the sigmoidMul output gate. Inputs rotate
    over independent sets larger than the MALL."""
    bound = "hbm"
    labels = ("q_norm_rope", "k_norm_rope", "gate")
    dominant = "q_norm_rope"

    def __init__(self, dev, T, past, sets, seed, hq=16, hkv=4, d=256, rot=64):
        import torch
        from llminfer_amd import ops
        self.T, self.P, self.sets, self.hq, self.hkv, self.d, self.rot = T, past, sets, hq, hkv, d, rot
        self.tokens = T
        self.name = f"attn_rows_T{T}"
        g = torch.Generator(device=dev).manual_seed(seed)
        self.qg = [_randn16(g, (T, hq, 2 * d), dev) for _ in range(sets)]
        self.k = [_randn16(g, (T, hkv, d), dev) for _ in range(sets)]
        self.attn = [_randn16(g, (T, hq, d), dev) for _ in range(sets)]
        self.qw = (0.2 * torch.randn(d, generator=g, device=dev)).float()
        self.kw = (0.2 * torch.randn(d, generator=g, device=dev)).float()
        self.qout = [torch.empty(T, hq, d, dtype=torch.float16, device=dev) for _ in range(sets)]
        self.out = [torch.empty(T, hq, d, dtype=torch.float16, device=dev) for _ in range(sets)]
        self.kc = torch.zeros(past + T, hkv, d, dtype=torch.float16, device=dev)
        # the gate is the second half of each projected q head, made dense
        self.gate = [x[:, :, d:].contiguous() for x in self.qg]
        self.bound_ops = {
            "q_norm_rope": [ops.bind_norm_rope(self.qg[s], self.qw, self.qout[s], past, rot,
                                               head_dim=d) for s in range(sets)],
            "k_norm_rope": [ops.bind_norm_rope(self.k[s], self.kw, self.kc, past, rot,
                                               output_start=past) for s in range(sets)],
            "gate": [ops.bind_sigmoid_mul(self.gate[s], self.attn[s], self.out[s])
                     for s in range(sets)],
        }
        self.bytes = rows_bytes(T, hq, hkv, d)

    def op(self, label, i):
        self.bound_ops[label][i % self.sets]()

    def kernels(self):
        return self.bound_ops["q_norm_rope"][0].what

    def work(self, i):
        return self.bytes["q_norm_rope"]

    def config(self):
        return {"workload": self.name, "tokens": self.T, "past": self.P,
                "query_heads": self.hq, "kv_heads": self.hkv, "head_dim": self.d,
                "rotary_dim": self.rot, "theta": 1e7, "epsilon": 1e-6, "sets": self.sets,
                "ops": "q normRope (stride 2d) + k normRope into the cache + sigmoidMul"}

    def cpu(self, budget_s):
        import numpy as np
        import oracle
        import torch
        s = 0
        T, hq, hkv, d, P, rot = self.T, self.hq, self.hkv, self.d, self.P, self.rot
        for label in self.labels:
            self.op(label, s)
        torch.cuda.synchronize()
        qg, k = host_u16(self.qg[s]).reshape(T * hq, 2 * d), host_u16(self.k[s]).reshape(T * hkv, d)
        gate, attn = host_u16(self.gate[s]), host_u16(self.attn[s])
        qw, kw = host_f32(self.qw), host_f32(self.kw)
        kc = np.zeros(((P + T) * hkv, d), np.uint16)

        def step():
            q = oracle.norm_rope(qg, qw, T, hq, d, rot, 2 * d, P)
            oracle.norm_rope(k, kw, T, hkv, d, rot, d, P, output=kc, output_start=P)
            return q, oracle.sigmoid_mul(gate, attn)

        q, o = step()
        exact = bool(np.array_equal(q.reshape(-1), host_u16(self.qout[s]).reshape(-1))
                     and np.array_equal(kc[P * hkv:], host_u16(self.kc[P:]).reshape(-1, d))
                     and np.array_equal(o.reshape(-1), host_u16(self.out[s]).reshape(-1)))
        sec, runs = time_cpu(step, budget_s)
        return {"value": sec * 1e6, "unit": "µs/layer", "cores": 1, "kind": "port",
                "sample": f"the three ops on one input set (T={T}, P={P}), {runs} runs, "
                          "scalar C oracle (orc_norm_rope, orc_sigmoid_mul)",
                "gpu_bit_exact": exact}


def front_bytes(T: int, hk: int, dk: int, hv: int, dv: int, k: int = 4) -> dict:
    """Algorithmic HBM bytes of the DeltaNet front end per call: the conv
    reads and writes [T, C] fp16 (C = 2 hk dk + hv dv) plus its weights and
    history; each L2 norm reads [T, hk dk] fp16 and writes it as fp32; the
    gates read a, b fp16 and write beta, decay fp32; the gated norm after
    DeltaUpdate reads the output and the gate z and writes fp16."""
    C = 2 * hk * dk + hv * dv
    return {"conv": 2 * T * C * 2 + C * k * 2 + 2 * C * (k - 1) * 2,
            "l2norm_q": T * hk * dk * 6, "l2norm_k": T * hk * dk * 6,
            "gates": T * hv * 12 + hv * 8,
            "gated_norm": T * hv * dv * 6 + dv * 4}


class DeltaFront(Workload):
    """The DeltaNet layer's front end ahead of DeltaUpdate
    (Qwen35ModelBuilder.cpp:146-160): causalConv + SiLU over q, k, v
    (8192 channels, 4 taps, history carried), the L2 norms of q (scaled by
    1/sqrt(dk)) and k to fp32, and the gates; and the gatedRmsNorm that
    follows DeltaUpdate (z gate through SiLU). Inputs rotate over sets
    larger than the MALL."""
    bound = "hbm"
    labels = ("conv", "l2norm_q", "l2norm_k", "gates", "gated_norm")
    dominant = "conv"

    def __init__(self, dev, T, sets, seed, hk=16, dk=128, hv=32, dv=128, k=4):
        import torch
        from llminfer_amd import ops
        self.T, self.sets, self.shape = T, sets, (hk, dk, hv, dv)
        self.tokens = T
        self.name = f"delta_front_T{T}"
        C = 2 * hk * dk + hv * dv
        g = torch.Generator(device=dev).manual_seed(seed)
        self.x = [_randn16(g, (T, C), dev) for _ in range(sets)]
        self.w = (0.5 * torch.randn(C, k, generator=g, device=dev)).half()
        self.hist = [_randn16(g, (C, k - 1), dev) for _ in range(sets)]
        self.y = [torch.empty(T, C, dtype=torch.float16, device=dev) for _ in range(sets)]
        self.qn = [torch.empty(T, hk * dk, dtype=torch.float32, device=dev) for _ in range(sets)]
        self.kn = [torch.empty(T, hk * dk, dtype=torch.float32, device=dev) for _ in range(sets)]
        self.a = [_randn16(g, (T, hv), dev) for _ in range(sets)]
        self.b = [_randn16(g, (T, hv), dev) for _ in range(sets)]
        self.a_log = (0.5 * torch.randn(hv, generator=g, device=dev)).float()
        self.dt = (0.5 * torch.randn(hv, generator=g, device=dev)).float()
        self.beta = [torch.empty(T, hv, dtype=torch.float32, device=dev) for _ in range(sets)]
        self.mixed = [_randn16(g, (T * hv, dv), dev) for _ in range(sets)]
        self.z = [_randn16(g, (T * hv, dv), dev) for _ in range(sets)]
        self.nw = (1 + 0.2 * torch.randn(dv, generator=g, device=dev)).float()
        self.gated = [torch.empty(T * hv, dv, dtype=torch.float16, device=dev) for _ in range(sets)]
        self.decay = [torch.empty(T, hv, dtype=torch.float32, device=dev) for _ in range(sets)]
        q_of = lambda s: self.y[s][:, :hk * dk]
        k_of = lambda s: self.y[s][:, hk * dk:2 * hk * dk]
        convs = [ops.bind_causal_conv(self.x[s], self.w, self.hist[s], self.y[s], True)
                 for s in range(sets)]
        for c in convs:
            c()
        torch.cuda.synchronize()
        # The norms take dense [T, hk*dk] inputs: copies of the conv output's
        # q and k column blocks, made once, outside the timed region.
        self.qin = [q_of(s).contiguous() for s in range(sets)]
        self.kin = [k_of(s).contiguous() for s in range(sets)]
        self.bound_ops = {
            "conv": convs,
            "l2norm_q": [ops.bind_l2_norm(self.qin[s], self.qn[s], dk, 1e-6, dk ** -0.5)
                         for s in range(sets)],
            "l2norm_k": [ops.bind_l2_norm(self.kin[s], self.kn[s], dk, 1e-6, 1.0)
                         for s in range(sets)],
            "gates": [ops.bind_delta_gates(self.a[s], self.b[s], self.a_log, self.dt,
                                           self.beta[s], self.decay[s]) for s in range(sets)],
            "gated_norm": [ops.bind_gated_rms_norm(self.mixed[s], self.z[s], self.nw,
                                                   self.gated[s]) for s in range(sets)],
        }
        self.bytes = front_bytes(T, hk, dk, hv, dv, k)

    def op(self, label, i):
        self.bound_ops[label][i % self.sets]()

    def kernels(self):
        return "causalConv"

    def work(self, i):
        return self.bytes["conv"]

    def config(self):
        hk, dk, hv, dv = self.shape
        return {"workload": self.name, "tokens": self.T, "key_heads": hk, "key_dim": dk,
                "value_heads": hv, "value_dim": dv, "conv_channels": 2 * hk * dk + hv * dv,
                "conv_kernel": 4, "sets": self.sets,
                "ops": "causalConv+SiLU, l2NormF32 (q scaled 1/sqrt(dk), k), deltaGates, "
                       "gatedRmsNorm (after DeltaUpdate)"}

    def cpu(self, budget_s):
        import numpy as np
        import oracle
        import torch
        s = 0
        hk, dk, hv, dv = self.shape
        x, w = host_u16(self.x[s]), host_u16(self.w)
        h0 = host_u16(self.hist[s]).copy()
        for label in self.labels:
            self.op(label, s)
        torch.cuda.synchronize()
        qin, kin = host_u16(self.qin[s]), host_u16(self.kin[s])
        a, b = host_u16(self.a[s]), host_u16(self.b[s])
        a_log, dt = host_f32(self.a_log), host_f32(self.dt)

        mixed, z, nw = host_u16(self.mixed[s]), host_u16(self.z[s]), host_f32(self.nw)

        def step():
            y = oracle.causal_conv(x, w, h0.copy(), True)
            qn = oracle.l2norm_f32(qin, dk, 1e-6, dk ** -0.5)
            kn = oracle.l2norm_f32(kin, dk, 1e-6, 1.0)
            return (y, qn, kn, oracle.delta_gates(a, b, a_log, dt),
                    oracle.gated_rms_norm(mixed, z, nw))

        y, qn, kn, (beta, decay), gn = step()
        exact = bool(np.array_equal(y, host_u16(self.y[s]))
                     and np.array_equal(qn.view(np.uint32), host_f32(self.qn[s]).view(np.uint32))
                     and np.array_equal(kn.view(np.uint32), host_f32(self.kn[s]).view(np.uint32))
                     and np.array_equal(beta.view(np.uint32), host_f32(self.beta[s]).view(np.uint32))
                     and np.array_equal(decay.view(np.uint32), host_f32(self.decay[s]).view(np.uint32))
                     and np.array_equal(gn, host_u16(self.gated[s])))
        sec, runs = time_cpu(step, budget_s)
        return {"value": sec * 1e6, "unit": "µs/layer", "cores": 1, "kind": "port",
                "sample": f"the five ops on one input set (T={self.T}), {runs} runs, scalar C "
                          "oracle (orc_causal_conv, orc_l2norm_f32, orc_delta_gates, "
                          "orc_gated_rms_norm)",
                "gpu_bit_exact": exact}


def w8_bytes(rows: int, columns: int, groups: int, out_bytes: int = 2) -> int:
    """HBM bytes of one linearW8A8 call: int8 weights and fp16 weight scales
    (read once), int8 activations and fp32 activation scales, the output."""
    return (columns * groups * (32 + 2) + rows * groups * (32 + 4) +
            rows * columns * out_bytes)


def quantize_bytes(rows: int, width: int) -> int:
    """quantizeActivation: fp16 in, int8 and fp32 scales out."""
    groups = (width + 31) // 32
    return rows * width * 2 + rows * groups * (32 + 4)


class W8A8Mlp(Workload):
    """The SwiGLU MLP of a Qwen3.5-4B layer (hidden 2560, intermediate 9216,
    docs/architecture.md:115) on the W8A8 path as the plan lowers it
    (MetalExecutionPlan.cpp:464-510, 566-580): quantizeActivation of the
    hidden rows, the up projection, the gate projection with the SwiGLU
    epilogue (the up output as its multiplier), quantizeActivation of the
    product, the down projection. Random int8 weights and fp16 scales of
    those shapes (75 MB a set) rotate over sets larger than the MALL."""
    bound = "hbm"
    labels = ("quantize_in", "up", "gate_swiglu", "quantize_mid", "down")
    dominant = "up"

    def __init__(self, dev, T, sets, seed, hidden=2560, inter=9216):
        import torch
        from llminfer_amd import _lib, ops
        self.T, self.sets, self.hidden, self.inter = T, sets, hidden, inter
        self.tokens = T
        self.name = f"w8a8_mlp_T{T}"
        g = torch.Generator(device=dev).manual_seed(seed)
        gh, gi = hidden // 32, inter // 32

        def weights(cols, groups):
            w = torch.randint(-127, 128, (cols, groups * 32), generator=g, device=dev,
                              dtype=torch.int8)
            sc = (torch.rand(cols, groups, generator=g, device=dev) * 2e-3 + 1e-4).half()
            return w, sc

        self.wu, self.wg, self.wd = [], [], []
        for _ in range(sets):
            self.wu.append(weights(inter, gh))
            self.wg.append(weights(inter, gh))
            self.wd.append(weights(hidden, gi))
        self.x = [_randn16(g, (T, hidden), dev) for _ in range(sets)]
        self.qx = [torch.empty(T, gh * 32, dtype=torch.int8, device=dev) for _ in range(sets)]
        self.sx = [torch.empty(T, gh, dtype=torch.float32, device=dev) for _ in range(sets)]
        self.up = [torch.empty(T, inter, dtype=torch.float16, device=dev) for _ in range(sets)]
        self.act = [torch.empty(T, inter, dtype=torch.float16, device=dev) for _ in range(sets)]
        self.qa = [torch.empty(T, gi * 32, dtype=torch.int8, device=dev) for _ in range(sets)]
        self.sa = [torch.empty(T, gi, dtype=torch.float32, device=dev) for _ in range(sets)]
        self.out = [torch.empty(T, hidden, dtype=torch.float16, device=dev) for _ in range(sets)]
        S = range(sets)
        self.bound_ops = {
            "quantize_in": [ops.bind_quantize_activation(self.x[s], self.qx[s], self.sx[s])
                            for s in S],
            "up": [ops.bind_linear_w8a8(self.qx[s], self.sx[s], *self.wu[s], self.up[s]) for s in S],
            "gate_swiglu": [ops.bind_linear_w8a8(self.qx[s], self.sx[s], *self.wg[s], self.act[s],
                                                 _lib.LINEAR_SILU_MUL, 0, self.up[s]) for s in S],
            "quantize_mid": [ops.bind_quantize_activation(self.act[s], self.qa[s], self.sa[s])
                             for s in S],
            "down": [ops.bind_linear_w8a8(self.qa[s], self.sa[s], *self.wd[s], self.out[s])
                     for s in S],
        }
        self.bytes = {
            "quantize_in": quantize_bytes(T, hidden),
            "up": w8_bytes(T, inter, gh),
            "gate_swiglu": w8_bytes(T, inter, gh) + T * inter * 2,
            "quantize_mid": quantize_bytes(T, inter),
            "down": w8_bytes(T, hidden, gi),
        }

    def launch(self, i):
        for label in self.labels:
            self.op(label, i)

    def op(self, label, i):
        self.bound_ops[label][i % self.sets]()

    def kernels(self):
        return "linearW8A8Gemv" if self.T == 1 else "linearW8A8Gemm"

    def work(self, i):
        return self.bytes["up"]

    def config(self):
        return {"workload": self.name, "tokens": self.T, "hidden": self.hidden,
                "intermediate": self.inter, "group": 32, "sets": self.sets,
                "ops": "quantizeActivation, linearW8A8 up, linearW8A8 gate + SwiGLU epilogue, "
                       "quantizeActivation, linearW8A8 down"}

    def cpu(self, budget_s):
        import numpy as np
        import oracle
        import torch
        s = 0
        self.launch(s)
        torch.cuda.synchronize()
        x = host_u16(self.x[s])
        wu, su = self.wu[s][0].cpu().numpy(), host_u16(self.wu[s][1])
        wg, sg = self.wg[s][0].cpu().numpy(), host_u16(self.wg[s][1])
        wd, sd = self.wd[s][0].cpu().numpy(), host_u16(self.wd[s][1])

        def step():
            qx, sx, _ = oracle.quantize_activation(x)
            up = oracle.linear_w8a8(qx, sx, wu, su)
            act = oracle.linear_w8a8(qx, sx, wg, sg, oracle.LINEAR_SILU_MUL, 0, up)
            qa, sa, _ = oracle.quantize_activation(act)
            return up, act, oracle.linear_w8a8(qa, sa, wd, sd)

        up, act, out = step()
        exact = bool(np.array_equal(up, host_u16(self.up[s])) and
                     np.array_equal(act, host_u16(self.act[s])) and
                     np.array_equal(out, host_u16(self.out[s])))
        sec, runs = time_cpu(step, budget_s)
        return {"value": sec * 1e6, "unit": "µs/layer", "cores": 1, "kind": "port",
                "sample": f"the five ops on one weight set (T={self.T}), {runs} runs, scalar C "
                          "oracle (orc_quantize_activation, orc_linear_w8a8)",
                "gpu_bit_exact": exact}


class Qwen35Model(Workload):
    """Qwen3.5-4B with W8A8 weights (random, of the model's shapes) through
    the whole-graph HIP plan (llminfer_amd.plan.ModelSession): the graph of
    each step lowered once before timing, then one step a call. Decode:
    step i runs at past = P + i after an untimed P-token prefill, one token
    and the last row's logits; prefill: T tokens from past 0, the last
    row's logits (the reference's llmi-benchmark: prefill then decode,
    docs/architecture.md:145)."""
    labels = ("step",)
    dominant = "step"

    def __init__(self, dev, T, past, plans=64, seed=30):
        import torch
        from llminfer_amd.graph import qwen35_4b
        from llminfer_amd.plan import ModelSession, random_weights
        self.c = c = qwen35_4b()
        self.T, self.P = T, past
        self.tokens = T
        self.decode = T == 1
        self.bound = "hbm" if self.decode else "mfma"
        self.name = f"qwen35_4b_w8a8_decode_P{past}" if self.decode else \
            f"qwen35_4b_w8a8_prefill_{T}"
        weights = random_weights(c, True, dev, seed)
        self.session = s = ModelSession(c, weights, past + plans + T + 8, True, dev)
        g = torch.Generator().manual_seed(seed)
        if self.decode and past:
            s.step(torch.randint(0, c.vocabulary, (past,), generator=g).numpy(), "none")
        self.plans = [s.plan(T, "last")]
        if self.decode:   # the graphs of the next positions (no step run)
            self.plans += [s.plan(1, "last", past=past + i) for i in range(1, plans)]
        self.ids = torch.randint(0, c.vocabulary, (T,), generator=g, dtype=torch.int32).to(dev)
        self.logits = torch.empty(1, c.vocabulary, dtype=torch.float16, device=dev)
        s.run(self.plans[-1], self.ids, self.logits)   # size the scratch arena once
        torch.cuda.synchronize()

    def op(self, label, i):
        self.session.run(self.plans[i % len(self.plans)], self.ids, self.logits)

    def kernels(self):
        return f"whole-graph plan ({self.plans[0].launches} launches a step)"

    def weight_bytes(self):
        from llminfer_amd.graph import EMBEDDING_ID, Element, qwen35_tensors
        total = 0
        for tid, (element, shape) in qwen35_tensors(self.c, True).items():
            if tid == EMBEDDING_ID:
                continue  # gathered rows here; the tied head below reads it whole
            n = 1
            for d in shape:
                n *= d
            total += n * (1 if element == Element.I8 else 2 if element == Element.F16 else 4)
            if element == Element.I8:
                total += shape[0] * ((shape[1] + 31) // 32) * 2
        rows, width = self.c.vocabulary, self.c.hidden
        return total + rows * width + rows * ((width + 31) // 32) * 2

    def work(self, i):
        c = self.c
        gqa = sum(k == "gqa" for k in c.layers)
        delta = len(c.layers) - gqa
        if self.decode:
            past = self.P + i % len(self.plans)
            kv = gqa * 2 * (past + 1) * c.kv_heads * c.head_dim * 2
            state = delta * 2 * c.value_heads * c.key_dim * c.value_dim * 4
            return self.weight_bytes() + kv + state
        # prefill: two flops per weight per token (the projections and the
        # head on the last row), attention's QK and PV, the delta rule's
        # recurrent count (4 dk dv per head and token)
        proj = (self.weight_bytes() - c.vocabulary * c.hidden) * 2 * self.T
        head = 2 * c.vocabulary * c.hidden
        att = gqa * 2 * 2 * c.q_heads * c.head_dim * self.T * (self.T + 1) // 2
        rec = delta * 4 * c.value_heads * c.key_dim * c.value_dim * self.T
        return proj + head + att + rec

    def config(self):
        c = self.c
        return {"workload": self.name, "model": "Qwen3.5-4B (random weights of its shapes)",
                "precision": "W8A8", "tokens": self.T, "past": self.P,
                "layers": len(c.layers), "vocabulary": c.vocabulary,
                "launches_per_step": self.plans[0].launches,
                "records_per_step": len(self.plans[0].dispatches),
                "scratch_bytes": self.plans[0].scratch_bytes,
                "reference_m2_tok_s": 9.82 if self.decode else 20.81}

    def cpu(self, budget_s):
        """The whole step on the CPU oracle (oracle/graph_runner.py, scalar C,
        one thread), from a bounded sample: one DeltaNet and one GQA layer of
        the model's widths and the head over 8192 of its 248,320 rows, at the
        leg's past (the caches and states hold random values: the time does
        not depend on them); prefill runs 16 of the 512 tokens. Scaled: 24
        DeltaNet + 8 GQA layers, the head to the full vocabulary, and for the
        prefill the per-token work x 512/16 (the head reads one row; the
        quadratic attention term is then undercounted, ~2 % of the step)."""
        import dataclasses
        import time as _time
        import numpy as np
        import oracle
        from llminfer_amd.graph import (EMBEDDING_ID, Element, OpKind, build_qwen35,
                                        qwen35_tensors)
        from oracle.graph_runner import GraphRunner
        c = self.c
        sample_vocab, T = 8192, (1 if self.decode else 16)
        cs = dataclasses.replace(c, layers=("delta", "gqa"), vocabulary=sample_vocab)
        r = np.random.default_rng(7)
        weights = {}
        for tid, (element, shape) in qwen35_tensors(cs, True).items():
            if element == Element.I8:
                rows, width = shape
                groups = (width + 31) // 32
                data = np.zeros((rows, groups * 32), np.int8)
                data[:, :width] = r.integers(-127, 128, (rows, width), dtype=np.int8)
                scale = (0.25 if tid == EMBEDDING_ID else 0.6 / np.sqrt(width)) / 127
                weights[tid] = (data, oracle.f32_to_f16(
                    (r.random((rows, groups)) * 2 * scale).astype(np.float32)))
            elif element == Element.F16:
                weights[tid] = (oracle.f32_to_f16(
                    (r.standard_normal(shape) * 0.12).astype(np.float32)), None)
            else:
                v = (r.standard_normal(shape) * 0.1).astype(np.float32)
                weights[tid] = (v + 1 if tid.endswith("linear_attn.norm.weight") else v, None)
        past = self.P
        g = build_qwen35(cs, T, past, past + T, "last", True)
        states = []
        for st in g.states:
            if st.element == Element.F32:
                states.append((r.standard_normal(st.shape) * 0.1).astype(np.float32))
            else:
                states.append(oracle.f32_to_f16(
                    r.standard_normal(st.shape).astype(np.float32)))
        ids = r.integers(0, sample_vocab, T).astype(np.uint32)
        head_op = max(i for i, op in enumerate(g.ops) if op.kind == OpKind.LINEAR_W8A8)
        tot = {"delta": 0.0, "gqa": 0.0, "head": 0.0, "rest": 0.0}

        def account(i, op, dt):
            part = "head" if i == head_op else {0: "delta", 1: "gqa"}.get(op.layer, "rest")
            tot[part] += dt

        runs, t0 = 0, _time.perf_counter()
        while runs == 0 or _time.perf_counter() - t0 < budget_s:
            run = GraphRunner(g, weights, states)
            run.op_hook = account
            run.run(ids)
            runs += 1
        per = {k: v / runs for k, v in tot.items()}
        n_gqa = sum(k == "gqa" for k in c.layers)
        n_delta = len(c.layers) - n_gqa
        scale_t = self.T / T
        step_s = scale_t * (n_delta * per["delta"] + n_gqa * per["gqa"] + per["rest"]) + \
            per["head"] * c.vocabulary / sample_vocab
        return {"value": step_s * 1e6, "unit": "µs/step", "cores": 1, "kind": "port",
                "tokens_per_s": round(self.T / step_s, 3),
                "sample": f"oracle graph runner, 1 thread: one DeltaNet + one GQA layer and "
                          f"the head over {sample_vocab} rows at T={T}, past={past}, "
                          f"{runs} runs, scaled to {n_delta}+{n_gqa} layers, "
                          f"{c.vocabulary} rows" + ("" if self.decode else
                                                    f", x{self.T // T} tokens"),
                "per_layer_us": {k: round(v * 1e6, 1) for k, v in per.items()}}


def _delta_inputs(g, dev, T, hk, dk, hv, dv):
    """DeltaUpdate operands as the reference graph produces them: L2-normalised
    fp32 q (x 1/sqrt(dk)) and k from fp16 N(0,1) (Graph.metal:96-109), fp16 v,
    beta = fp16(sigmoid(N(0,1))), decay = exp(-softplus(N(0,1)))."""
    import torch
    qh = _randn16(g, (T, hk, dk), dev).float()
    kh = _randn16(g, (T, hk, dk), dev).float()
    q = qh * (torch.rsqrt((qh * qh).sum(-1, keepdim=True) + 1e-6) / math.sqrt(dk))
    k = kh * torch.rsqrt((kh * kh).sum(-1, keepdim=True) + 1e-6)
    v = _randn16(g, (T, hv * dv), dev)
    beta = torch.sigmoid(_randn16(g, (T, hv), dev).float()).half().float()
    decay = torch.exp(-torch.nn.functional.softplus(_randn16(g, (T, hv), dev).float()))
    return (q.reshape(T, hk * dk).contiguous(), k.reshape(T, hk * dk).contiguous(),
            v, beta.contiguous(), decay.contiguous())


class DeltaPrefill(Workload):
    """DeltaUpdate over 1024 tokens from a zero state. The timed
    calls rotate over `sets` independent operand sets (q, k, v, gates, state,
    out: 34 MB each, 272 MB in all, past the 256 MB MALL); `warm_op` repeats
    one set. Each timed call continues from the state its set holds (the
    work per call does not depend on the state's values)."""
    bound = "hbm"
    dominant = "delta"
    labels = ("delta",)
    cache_state = ("cold: 8 operand sets (272 MB) rotate past the MALL; warm: one set "
                   "repeated")

    def __init__(self, dev, T=1024, hk=16, dk=128, hv=32, dv=128, seed=4, sets=8):
        import torch
        from llminfer_amd import ops
        self.T, self.hk, self.dk, self.hv, self.dv = T, hk, dk, hv, dv
        self.name = f"delta_prefill_{T}"
        self.tokens = T
        self.sets = sets
        g = torch.Generator(device=dev).manual_seed(seed)
        self.x = []
        for _ in range(sets):
            q, k, v, beta, decay = _delta_inputs(g, dev, T, hk, dk, hv, dv)
            state = torch.zeros((hv, dk, dv), dtype=torch.float32, device=dev)
            out = torch.empty_like(v)
            self.x.append(dict(q=q, k=k, v=v, beta=beta, decay=decay, state=state, out=out,
                               upd=ops.bind_delta_update(q, k, v, beta, decay, state, out)))
        self.state0 = torch.zeros((hv, dk, dv), dtype=torch.float32, device=dev)
        self.upd = self.x[0]["upd"]

    def op(self, label, i):
        self.x[i % self.sets]["upd"]()

    def warm_op(self, i):
        self.upd()

    def kernels(self):
        return self.upd.what

    def work(self, i):
        return delta_bytes(self.T, self.hk, self.dk, self.hv, self.dv)

    def config(self):
        return {"workload": self.name, "tokens": self.T, "key_heads": self.hk,
                "key_dim": self.dk, "value_heads": self.hv, "value_dim": self.dv,
                "operand_sets": self.sets, "cache_state": self.cache_state}

    def cpu(self, budget_s):
        import numpy as np
        import oracle
        import torch
        x = self.x[0]
        torch.cuda.synchronize()
        x["state"].copy_(self.state0)
        self.upd()
        torch.cuda.synchronize()
        q, k, beta, decay = (host_f32(x[n]) for n in ("q", "k", "beta", "decay"))
        v = host_u16(x["v"])
        s0 = host_f32(self.state0)
        gpu_out = oracle.f16_to_f32(host_u16(x["out"]))
        gpu_state = host_f32(x["state"])
        thr = cpu_threads()
        want, wstate = oracle.delta_recurrent_f32(q, k, v, beta, decay, s0, thr)
        err = float(np.max(np.abs(gpu_out - oracle.f16_to_f32(want))))
        serr = float(np.max(np.abs(gpu_state - wstate)) / max(1e-30, np.max(np.abs(wstate))))
        sec, runs = time_cpu(lambda: oracle.delta_recurrent_f32(q, k, v, beta, decay, s0, thr),
                             budget_s)
        return {"value": sec * 1e6, "unit": "µs/layer", "cores": thr, "kind": "port",
                "sample": f"the full {self.T}-token DeltaUpdate, {runs} runs, fp32 "
                          "recurrence (oracle orc_delta_recurrent_f32)",
                "gpu_vs_cpu_max_abs": err, "gpu_vs_cpu_state_rel": serr}


class GatedAttention(Workload):
    """The attention block around CausalGqa fused into one call
    (llmi_hip_gated_attention: q and k normRope, V append, attention, sigmoid
    gate; Qwen35ModelBuilder.cpp:175-197), next to the same block as five
    standalone calls (q normRope, k normRope into the cache, cacheAppend of
    V, CausalGqa, sigmoidMul). Decode rotates cache sets past the MALL; the
    roofline is the attention's (bytes at decode, FLOPs at prefill)."""
    labels = ("fused", "unfused")
    dominant = "fused"

    def __init__(self, dev, T, past, cap, sets, seed, hq=16, hkv=4, d=256, rot=64):
        import torch
        from llminfer_amd import ops
        self.T, self.P, self.sets, self.hq, self.hkv, self.d, self.rot = T, past, sets, hq, hkv, d, rot
        self.tokens = T
        self.bound = "hbm" if T == 1 else "mfma"
        self.name = f"gated_attention_T{T}_past{past}"
        g = torch.Generator(device=dev).manual_seed(seed)
        self.qw = (0.2 * torch.randn(d, generator=g, device=dev)).float()
        self.kw = (0.2 * torch.randn(d, generator=g, device=dev)).float()
        self.x = []
        for _ in range(sets):
            x = dict(qp=_randn16(g, (T, hq, 2 * d), dev), kp=_randn16(g, (T, hkv, d), dev),
                     vn=_randn16(g, (T, hkv, d), dev), kc=_randn16(g, (cap, hkv, d), dev),
                     vc=_randn16(g, (cap, hkv, d), dev),
                     out=torch.empty(T, hq, d, dtype=torch.float16, device=dev),
                     qn=torch.empty(T, hq, d, dtype=torch.float16, device=dev),
                     attn=torch.empty(T, hq, d, dtype=torch.float16, device=dev),
                     out2=torch.empty(T, hq, d, dtype=torch.float16, device=dev))
            x["gate"] = x["qp"][:, :, d:].contiguous()
            x["fused"] = ops.bind_gated_attention(x["qp"], x["kp"], x["vn"], self.qw, self.kw,
                                                  x["kc"], x["vc"], x["out"], past, rot)
            x["unfused"] = [
                ops.bind_norm_rope(x["qp"], self.qw, x["qn"], past, rot, head_dim=d),
                ops.bind_norm_rope(x["kp"], self.kw, x["kc"], past, rot, output_start=past),
                ops.Bound(*_append_call(x["vn"], x["vc"], past * hkv * d), "cacheAppend"),
                ops.bind_causal_gqa(x["qn"], x["kc"], x["vc"], x["attn"], past),
                ops.bind_sigmoid_mul(x["gate"], x["attn"], x["out2"])]
            self.x.append(x)

    def op(self, label, i):
        x = self.x[i % self.sets]
        if label == "fused":
            x["fused"]()
        else:
            for b in x["unfused"]:
                b()

    def kernels(self):
        return self.x[0]["fused"].what

    def work(self, i):
        if self.bound == "hbm":
            return gqa_bytes(1, self.P, self.hq, self.hkv, self.d)
        return gqa_flops(self.T, self.P, self.hq, self.d)

    def config(self):
        return {"workload": self.name, "tokens": self.T, "past": self.P,
                "query_heads": self.hq, "kv_heads": self.hkv, "head_dim": self.d,
                "rotary_dim": self.rot, "sets": self.sets}

    def cpu(self, budget_s):
        import torch
        x = self.x[0]
        for label in self.labels:
            self.op(label, 0)
        torch.cuda.synchronize()
        return {"value": None, "unit": "µs/layer", "cores": 0, "kind": "port",
                "sample": "none: the block's parts have their own CPU samples "
                          "(attention legs, next_attn_rows_*)",
                "gpu_fused_equals_unfused": bool(torch.equal(x["out"], x["out2"]))}


def _append_call(src, cache, offset):
    """cacheAppend as a Bound-ready (fn, args) pair."""
    from llminfer_amd import _lib
    return (_lib.load().llmi_hip_cache_append,
            (src.data_ptr(), cache.data_ptr(), _lib.CacheParams(src.numel(), offset),
             __import__("torch").cuda.current_stream().cuda_stream))


def norm_delta_bytes(T: int, hk: int, dk: int, hv: int, dv: int) -> int:
    """The fused L2Norm -> DeltaUpdate pair: fp16 q, k instead of fp32."""
    return delta_bytes(T, hk, dk, hv, dv) - 4 * T * hk * dk


class DeltaNormUpdate(Workload):
    """The L2Norm(q), L2Norm(k) -> DeltaUpdate pair of a DeltaNet layer
    (Qwen35ModelBuilder.cpp:155-156) fused into one call
    (llmi_hip_l2_norm_delta_update: fp16 q/k normalised in the update's own
    loads), next to the same pair unfused (two l2NormF32 launches and
    DeltaUpdate on fp32 q/k). Operand sets rotate past the MALL."""
    bound = "hbm"
    labels = ("fused", "unfused")
    dominant = "fused"

    def __init__(self, dev, T, sets, seed, hk=16, dk=128, hv=32, dv=128):
        import numpy as np
        import torch
        from llminfer_amd import ops
        self.T, self.sets, self.shape = T, sets, (hk, dk, hv, dv)
        self.tokens = T
        self.name = f"l2norm_delta_T{T}"
        qs = float(np.float32(1.0) / np.sqrt(np.float32(dk)))
        g = torch.Generator(device=dev).manual_seed(seed)
        self.x = []
        for _ in range(sets):
            _, _, v, beta, decay = _delta_inputs(g, dev, T, hk, dk, hv, dv)
            x = dict(q16=_randn16(g, (T, hk * dk), dev), k16=_randn16(g, (T, hk * dk), dev),
                     v=v, beta=beta, decay=decay,
                     qf=torch.empty((T, hk * dk), dtype=torch.float32, device=dev),
                     kf=torch.empty((T, hk * dk), dtype=torch.float32, device=dev),
                     s1=torch.randn((hv, dk, dv), generator=g, device=dev) * 0.1,
                     o1=torch.empty_like(v), o2=torch.empty_like(v))
            x["s2"] = x["s1"].clone()
            x["fused"] = ops.bind_l2_norm_delta_update(x["q16"], x["k16"], v, beta, decay,
                                                       x["s1"], x["o1"], 1e-6, qs)
            x["unfused"] = [ops.bind_l2_norm(x["q16"], x["qf"], dk, 1e-6, qs),
                            ops.bind_l2_norm(x["k16"], x["kf"], dk, 1e-6, 1.0),
                            ops.bind_delta_update(x["qf"], x["kf"], v, beta, decay, x["s2"],
                                                  x["o2"])]
            self.x.append(x)
        self.bytes = {"fused": norm_delta_bytes(T, hk, dk, hv, dv),
                      "unfused": norm_delta_bytes(T, hk, dk, hv, dv)}

    def op(self, label, i):
        x = self.x[i % self.sets]
        if label == "fused":
            x["fused"]()
        else:
            for b in x["unfused"]:
                b()

    def kernels(self):
        return self.x[0]["fused"].what

    def work(self, i):
        return self.bytes["fused"]

    def config(self):
        hk, dk, hv, dv = self.shape
        return {"workload": self.name, "tokens": self.T, "key_heads": hk, "key_dim": dk,
                "value_heads": hv, "value_dim": dv, "operand_sets": self.sets}

    def cpu(self, budget_s):
        import numpy as np
        import oracle
        import torch
        hk, dk, hv, dv = self.shape
        x = self.x[0]
        torch.cuda.synchronize()
        s0 = host_f32(x["s1"])
        x["fused"]()
        torch.cuda.synchronize()
        gpu_out = oracle.f16_to_f32(host_u16(x["o1"]))
        q16, k16, v = host_u16(x["q16"]), host_u16(x["k16"]), host_u16(x["v"])
        beta, decay = host_f32(x["beta"]), host_f32(x["decay"])
        qs = float(np.float32(1.0) / np.sqrt(np.float32(dk)))
        thr = cpu_threads()

        def run():
            q = oracle.l2norm_f32(q16, dk, 1e-6, qs)
            k = oracle.l2norm_f32(k16, dk, 1e-6, 1.0)
            return oracle.delta_recurrent_f32(q, k, v, beta, decay, s0, thr)

        want, _ = run()
        err = float(np.max(np.abs(gpu_out - oracle.f16_to_f32(want))))
        sec, runs = time_cpu(run, budget_s)
        return {"value": sec * 1e6, "unit": "µs/layer", "cores": thr, "kind": "port",
                "sample": f"L2Norm q, k + the {self.T}-token DeltaUpdate on one set, {runs} runs "
                          "(oracle orc_l2norm_f32 + orc_delta_recurrent_f32)",
                "gpu_vs_cpu_max_abs": err}


def norm_delta_gated_bytes(T: int, hk: int, dk: int, hv: int, dv: int) -> int:
    """The fused L2Norm -> DeltaUpdate -> GatedRmsNorm chain: the pair's
    bytes plus the fp16 gate z and the fp32 norm weight (the un-normalised
    rows never leave the kernel)."""
    return norm_delta_bytes(T, hk, dk, hv, dv) + 2 * T * hv * dv + 4 * dv


class DeltaGatedNorm(Workload):
    """The L2Norm -> DeltaUpdate -> GatedRmsNorm chain of a DeltaNet layer
    (Qwen35ModelBuilder.cpp:155-166) in one call
    (llmi_hip_l2_norm_delta_gated_norm: the chunked scan normalises the
    head's rows at its end, the decode kernel in its workgroup), next to the
    same chain as the fused pair plus the standalone gatedRmsNorm launch.
    Operand sets rotate past the MALL."""
    bound = "hbm"
    labels = ("fused", "unfused")
    dominant = "fused"

    def __init__(self, dev, T, sets, seed, hk=16, dk=128, hv=32, dv=128):
        import numpy as np
        import torch
        from llminfer_amd import ops
        self.T, self.sets, self.shape = T, sets, (hk, dk, hv, dv)
        self.tokens = T
        self.name = f"l2norm_delta_gatednorm_T{T}"
        qs = float(np.float32(1.0) / np.sqrt(np.float32(dk)))
        g = torch.Generator(device=dev).manual_seed(seed)
        self.weight = (torch.randn((dv,), generator=g, device=dev) * 0.2 + 1.0)
        self.x = []
        for _ in range(sets):
            _, _, v, beta, decay = _delta_inputs(g, dev, T, hk, dk, hv, dv)
            x = dict(q16=_randn16(g, (T, hk * dk), dev), k16=_randn16(g, (T, hk * dk), dev),
                     z=_randn16(g, (T, hv * dv), dev), v=v, beta=beta, decay=decay,
                     s1=torch.randn((hv, dk, dv), generator=g, device=dev) * 0.1,
                     o1=torch.empty_like(v), o2=torch.empty_like(v), o3=torch.empty_like(v))
            x["s2"] = x["s1"].clone()
            x["fused"] = ops.bind_l2_norm_delta_gated_norm(
                x["q16"], x["k16"], v, beta, decay, x["s1"], x["z"], self.weight, x["o1"],
                1e-6, qs, 1e-6)
            x["unfused"] = [ops.bind_l2_norm_delta_update(x["q16"], x["k16"], v, beta, decay,
                                                          x["s2"], x["o2"], 1e-6, qs),
                            ops.bind_gated_rms_norm(x["o2"].view(T * hv, dv),
                                                    x["z"].view(T * hv, dv), self.weight,
                                                    x["o3"].view(T * hv, dv), 1e-6)]
            self.x.append(x)
        self.bytes = {"fused": norm_delta_gated_bytes(T, hk, dk, hv, dv),
                      "unfused": norm_delta_gated_bytes(T, hk, dk, hv, dv)}

    def op(self, label, i):
        x = self.x[i % self.sets]
        if label == "fused":
            x["fused"]()
        else:
            for b in x["unfused"]:
                b()

    def kernels(self):
        return self.x[0]["fused"].what

    def work(self, i):
        return self.bytes["fused"]

    def config(self):
        hk, dk, hv, dv = self.shape
        return {"workload": self.name, "tokens": self.T, "key_heads": hk, "key_dim": dk,
                "value_heads": hv, "value_dim": dv, "operand_sets": self.sets}

    def cpu(self, budget_s):
        import numpy as np
        import oracle
        import torch
        hk, dk, hv, dv = self.shape
        T = self.T
        x = self.x[0]
        torch.cuda.synchronize()
        s0 = host_f32(x["s1"])
        x["fused"]()
        torch.cuda.synchronize()
        gpu_out = host_u16(x["o1"])
        q16, k16, v, z = (host_u16(x[n]) for n in ("q16", "k16", "v", "z"))
        beta, decay, w = host_f32(x["beta"]), host_f32(x["decay"]), host_f32(self.weight)
        qs = float(np.float32(1.0) / np.sqrt(np.float32(dk)))
        thr = cpu_threads()

        def run():
            q = oracle.l2norm_f32(q16, dk, 1e-6, qs)
            k = oracle.l2norm_f32(k16, dk, 1e-6, 1.0)
            y, _ = oracle.delta_recurrent_f32(q, k, v, beta, decay, s0, thr)
            return oracle.gated_rms_norm(y.reshape(T * hv, dv), z.reshape(T * hv, dv), w)

        want = run()
        err = float(np.max(np.abs(oracle.f16_to_f32(gpu_out).reshape(-1)
                                  - oracle.f16_to_f32(want).reshape(-1))))
        sec, runs = time_cpu(run, budget_s)
        return {"value": sec * 1e6, "unit": "µs/layer", "cores": thr, "kind": "port",
                "sample": f"L2Norm q, k + the {T}-token DeltaUpdate + gatedRmsNorm on one set, "
                          f"{runs} runs (oracle orc_l2norm_f32 + orc_delta_recurrent_f32 + "
                          "orc_gated_rms_norm)",
                "gpu_vs_cpu_max_abs": err}


class HybridDecode(Workload):
    """DeltaNet decode step + KvAppend + GQA decode at 32K context,
    32 positions per layer; `layers` independent layer pairs rotate so that
    the 134 MB of K/V a decode reads come from HBM."""
    bound = "hbm"
    labels = ("delta", "gqa")

    def __init__(self, dev, past=32768, positions=32, layers=4, seed=5,
                 hq=16, hkv=4, d=256, hk=16, dk=128, hv=32, dv=128):
        import torch
        from llminfer_amd import ops
        self.P0, self.n, self.L = past, positions, layers
        self.cap = past + positions
        self.hq, self.hkv, self.d = hq, hkv, d
        self.dshape = (hk, dk, hv, dv)
        self.name = f"hybrid_decode_{past // 1024}k"
        g = torch.Generator(device=dev).manual_seed(seed)
        self.kc = [_randn16(g, (self.cap, hkv, d), dev) for _ in range(layers)]
        self.vc = [_randn16(g, (self.cap, hkv, d), dev) for _ in range(layers)]
        self.state = [torch.randn((hv, dk, dv), generator=g, device=dev) * 0.1
                      for _ in range(layers)]
        self.inp = []
        for j in range(positions):
            dq, dkk, dvv, b, a = _delta_inputs(g, dev, 1, hk, dk, hv, dv)
            self.inp.append(dict(dq=dq, dk=dkk, dv=dvv, beta=b, decay=a,
                                 q=_randn16(g, (1, hq, d), dev),
                                 kn=_randn16(g, (1, hkv, d), dev),
                                 vn=_randn16(g, (1, hkv, d), dev)))
        self.dout = torch.empty((1, hv * dv), dtype=torch.float16, device=dev)
        self.gout = torch.empty((1, hq, d), dtype=torch.float16, device=dev)
        self.ops = {}
        for l in range(layers):
            for j in range(positions):
                x = self.inp[j]
                P = past + j
                self.ops[l, j] = (
                    ops.bind_delta_update(x["dq"], x["dk"], x["dv"], x["beta"], x["decay"],
                                          self.state[l], self.dout),
                    ops.bind_kv_append_causal_gqa(x["q"], x["kn"], x["vn"], self.kc[l],
                                                  self.vc[l], self.gout, P))
        self.tokens = 1

    def pos(self, i):
        return i % self.L, (i // self.L) % self.n

    def op(self, label, i):
        delta, att = self.ops[self.pos(i)]
        (delta if label == "delta" else att)()

    def kernels(self):
        return self.ops[0, 0][1].what

    def work(self, i):
        _, j = self.pos(i)
        return gqa_bytes(1, self.P0 + j, self.hq, self.hkv, self.d) + \
            append_bytes(1, self.hkv, self.d)

    def config(self):
        return {"workload": self.name, "past": self.P0, "positions": self.n,
                "layers": self.L, "capacity": self.cap}

    def cpu(self, budget_s):
        import numpy as np
        import oracle
        import torch
        hk, dk, hv, dv = self.dshape
        thr = cpu_threads()
        torch.cuda.synchronize()
        kc, vc = host_u16(self.kc[0]), host_u16(self.vc[0])
        st = host_f32(self.state[0])
        xs = [{k: (host_u16(v) if v.dtype == torch.float16 else host_f32(v))
               for k, v in x.items()} for x in self.inp]

        def run(n, outs=None):
            s = st
            for j in range(n):
                x = xs[j]
                dout, s = oracle.delta_recurrent_f32(x["dq"], x["dk"], x["dv"], x["beta"],
                                                     x["decay"], s, thr)
                oracle.kv_append(x["kn"], kc, self.P0 + j)
                oracle.kv_append(x["vn"], vc, self.P0 + j)
                gout = oracle.gqa_f32(x["q"], kc, vc, self.P0 + j, thr)
                if outs is not None:
                    outs.append((dout, gout, s))

        # The GPU steps of layer 0 from the state it holds now, position by
        # position, against the oracle from the same state.
        gpu = []
        for j in range(self.n):
            for fn in self.ops[0, j]:
                fn()
            torch.cuda.synchronize()
            gpu.append((host_u16(self.dout), host_u16(self.gout), host_f32(self.state[0])))
        want = []
        run(self.n, want)
        f = oracle.f16_to_f32
        err_d = max(float(np.max(np.abs(f(a[0]) - f(b[0])))) for a, b in zip(gpu, want))
        err_g = max(float(np.max(np.abs(f(a[1]) - f(b[1])))) for a, b in zip(gpu, want))
        rel = float(np.max(np.abs(gpu[-1][2] - want[-1][2])) / np.max(np.abs(want[-1][2])))
        sec, runs = time_cpu(lambda: run(self.n), budget_s)
        return {"value": sec / self.n * 1e6, "unit": "µs/layer-pair", "cores": thr,
                "kind": "port",
                "sample": f"{self.n} hybrid steps (DeltaNet decode + KvAppend + GQA decode "
                          f"at P={self.P0}..{self.P0 + self.n - 1}) of one layer pair, "
                          f"{runs} runs",
                "gpu_vs_cpu_max_abs": max(err_d, err_g),
                "gpu_vs_cpu": {"delta_out_max_abs": err_d, "gqa_out_max_abs": err_g,
                               "final_state_rel": rel, "positions": self.n}}


# ---------------------------------------------------------------- timing

def sleep_cycles_per_ms() -> float:
    import torch
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(1000)  # load the kernel
    torch.cuda.synchronize()
    n = 1 << 22
    a.record()
    torch.cuda._sleep(n)
    b.record()
    b.synchronize()
    ms = a.elapsed_time(b)
    return n / max(ms, 1e-3)


class Timing(float):
    """ms per call (the mean over the K timed calls), with the median and
    10th percentile of the per-chunk means and the host enqueue time."""
    median_ms: float
    p10_ms: float
    host_ms: float

    def summary(self) -> dict:
        return {"mean_us": round(self * 1e3, 3), "median_us": round(self.median_ms * 1e3, 3),
                "p10_us": round(self.p10_ms * 1e3, 3)}


def run_timed(fn, steps: int, warmup: int, cyc_per_ms: float, chunk: int = 10) -> Timing:
    """Device time per call of fn(i), i = warmup .. warmup+steps-1.

    A spin kernel holds the GPU while the host enqueues the K calls, so the
    events on the launch stream time the GPU running them back to back, not
    Python. An event after every `chunk` calls splits the K calls into
    back-to-back chunks; the mean is first to last event, and the median and
    p10 are over the chunk means. If the host still fell behind (its enqueue
    outlasted the hold), the measurement is repeated with a longer hold.
    """
    import statistics
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    n = min(8, max(1, warmup))
    t0 = time.perf_counter()
    for i in range(n):
        fn(i)
    host_ms = (time.perf_counter() - t0) * 1e3 / n
    torch.cuda.synchronize()

    chunk = max(1, min(chunk, steps))
    hold_ms = 10.0 + 3.0 * host_ms * steps
    for _attempt in range(4):
        marks = [torch.cuda.Event(enable_timing=True)]
        torch.cuda.synchronize()
        torch.cuda._sleep(int(min(hold_ms, 8000.0) * cyc_per_ms))
        t0 = time.perf_counter()
        marks[0].record()
        counts = []
        for i in range(steps):
            fn(warmup + i)
            if (i + 1) % chunk == 0 or i + 1 == steps:
                ev = torch.cuda.Event(enable_timing=True)
                ev.record()
                marks.append(ev)
                counts.append((i + 1) - sum(counts))
        enq_ms = (time.perf_counter() - t0) * 1e3
        torch.cuda.synchronize()
        if enq_ms < 0.8 * hold_ms or hold_ms >= 8000.0:
            break
        hold_ms = 2.0 * enq_ms + 10.0
    per = sorted(marks[j].elapsed_time(marks[j + 1]) / counts[j] for j in range(len(counts)))
    t = Timing(marks[0].elapsed_time(marks[-1]) / steps)
    t.median_ms = statistics.median(per)
    t.p10_ms = per[int(0.1 * (len(per) - 1))]
    t.host_ms = enq_ms / steps
    return t


def roofline(w: Workload, op_ms: float, steps: int, warmup: int, traffic) -> dict:
    """Roofline of the dominant op from its back-to-back time per call."""
    import statistics
    avg_s = op_ms * 1e-3
    work = statistics.fmean(w.work(warmup + i) for i in range(steps))
    if w.bound == "hbm":
        achieved, peak, unit = work / avg_s / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        achieved, peak, unit = work / avg_s / 1e12, MFMA_F16_PEAK_TFS, "TFLOP/s"
    return {"bound": w.bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic,
            "kernel": w.kernels(), "kernel_us_avg": round(avg_s * 1e6, 3),
            "work_per_launch": int(work),
            "work_unit": "bytes" if w.bound == "hbm" else "flop"}


COMPACT_LIMIT = 7500  # bytes of the final stdout line; the driver keeps a bounded tail


def _r(x, nd=3):
    return None if x is None else round(float(x), nd)


def compact(result: dict) -> dict:
    """The final stdout line: the contract's fields, the headline's roofline and
    CPU baseline, and a short summary per configuration. The full per-leg
    record goes to stderr (one `[bench-detail]` line per leg) and to --detail."""
    keep = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
            "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
            "tokens_per_s")
    out = {k: result[k] for k in keep if k in result}
    if "timing" in result:
        t = result["timing"]
        out["timing"] = {"cold_median_us": t["cold"]["median_us"],
                         "cold_p10_us": t["cold"]["p10_us"],
                         "warm_mean_us": t["warm"]["mean_us"]}
    if "roofline" in result:
        rl = result["roofline"]
        out["roofline"] = {k: rl[k] for k in ("bound", "achieved", "peak", "unit", "frac",
                                               "traffic", "kernel", "kernel_us_avg",
                                               "work_per_launch", "work_unit") if k in rl}
    if "cpu_baseline" in result:
        cb = result["cpu_baseline"]
        out["cpu_baseline"] = {k: cb[k] for k in (
            "value", "unit", "cores", "host_cores", "kind", "sample", "cpu_model",
            "single_thread_value", "gpu_vs_cpu_max_abs") if k in cb}
        if isinstance(out["cpu_baseline"].get("sample"), str):
            out["cpu_baseline"]["sample"] = out["cpu_baseline"]["sample"][:160]
    confs = {}
    for key, e in result.get("configs", {}).items():
        rl = e.get("roofline", {})
        c = {"us": e.get("us_per_step"), "kernel_us": rl.get("kernel_us_avg"),
             "bound": rl.get("bound"), "frac": rl.get("frac"), "kernel": rl.get("kernel")}
        if "hbm_frac" in e and e["hbm_frac"] is not None:
            c["hbm_frac"] = e["hbm_frac"]
        for k in ("mfma_frac_recurrent_flops", "delta_hbm_frac", "gqa_hbm_frac"):
            if k in e:
                c[k] = e[k]
        cb = e.get("cpu_baseline")
        if cb:
            c["cpu_us"] = _r(cb.get("value"), 1)
            c["cpu_threads"] = cb.get("cores")
            for k in ("gpu_vs_cpu_max_abs", "gpu_vs_cpu_state_rel", "gpu_bit_exact"):
                if k in cb:
                    c[k] = cb[k]
        confs[key] = c
    if confs:
        out["configs"] = confs
    return out


def load_traffic(workload: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary."""
    path = ROOT / "profiles" / "traffic.json"
    try:
        data = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    entry = data.get(workload)
    return entry.get("bytes_per_launch") if isinstance(entry, dict) else None


def headline(dev, args, cyc) -> dict:
    """The headline, configs[1]: its JSON fields."""
    import torch
    w = GqaDecode(dev)
    log(f"headline {w.name}: warmup {args.warmup}, steps {args.steps}")
    ms = run_timed(w.launch, args.steps, args.warmup, cyc)
    host_ms = ms.host_ms
    # The same step on one cache set over and over: its 16.8 MB stay in the
    # 256 MB MALL (warm), next to the rotating sets above (cold).
    warm = run_timed(w.launch_warm, args.steps, args.warmup, cyc)
    # The headline step is the dominant op alone (one fused append+attention
    # call), so its back-to-back time is the op's time.
    rl = roofline(w, ms, args.steps, args.warmup, load_traffic(w.name))
    log(f"headline {ms * 1e3:.2f} us/step, kernel {rl['kernel_us_avg']} us, "
        f"{rl['achieved']} GB/s ({rl['frac']:.1%})")
    result = {
        "metric": METRIC, "value": round(ms * 1e3, 3), "unit": "µs/layer",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": w.config(), "tokens_per_s": round(1e3 / ms, 1),
        "host_enqueue_ms_per_step": round(host_ms, 4),
        "timing": {"cold": ms.summary(), "warm": warm.summary(),
                   "chunks": "median and p10 over back-to-back chunks of 10 steps"},
        "roofline": rl,
    }
    if not args.no_cpu:
        log("cpu baseline (headline)")
        result["cpu_baseline"] = w.cpu(args.cpu_seconds)
        result["cpu_baseline"]["host_cores"] = host_cores()
    del w
    torch.cuda.empty_cache()
    return result


# ------------------------------------------------------------------ main

def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="llminfer attention hot path benchmark")
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only-headline", action="store_true",
                    help="skip the other BASELINE configurations")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="CPU-baseline time budget of the headline (others get half)")
    ap.add_argument("--no-cpu", action="store_true", help="skip every CPU baseline")
    ap.add_argument("--only", default="",
                    help="comma-separated keys of the configurations to run, "
                         "'headline' for the headline (default: all)")
    ap.add_argument("--detail", default="",
                    help="also write the full per-leg record as JSON to this file")
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(this build's hot path runs on a single MI355X; see the sharding notes "
              "in the design document)", file=sys.stderr)
        return 2

    import torch
    from llminfer_amd import _lib
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (no HIP device visible)", file=sys.stderr)
        return 1
    _lib.load()  # raises if the HIP library is missing; there is no fallback
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cyc = sleep_cycles_per_ms()
    log(f"device {torch.cuda.get_device_name(dev)}; spin {cyc:.0f} cycles/ms")

    only = {k for k in args.only.split(",") if k}
    builders = [
        ("cfg0_gqa_prefill_128", lambda: GqaPrefill(dev, 128, 0, 128, seed=1)),
        ("cfg2_gqa_chunked_prefill", lambda: GqaPrefill(dev, 2048, 2048, 4096, seed=3)),
        ("cfg3_delta_prefill_1024", lambda: DeltaPrefill(dev)),
        ("cfg4_hybrid_decode_32k", lambda: HybridDecode(dev)),
        ("next_attn_rows_prefill_2048", lambda: AttnRows(dev, 2048, 2048, 6, seed=6)),
        ("next_attn_rows_decode_4k", lambda: AttnRows(dev, 1, 4096, 64, seed=7)),
        ("next_delta_front_1024", lambda: DeltaFront(dev, 1024, 8, seed=8)),
        ("next_delta_front_decode", lambda: DeltaFront(dev, 1, 64, seed=9)),
        ("next_gated_attention_prefill", lambda: GatedAttention(dev, 2048, 2048, 4096, 2,
                                                                 seed=12)),
        ("next_gated_attention_decode_4k", lambda: GatedAttention(dev, 1, 4096, 8192, 24,
                                                                  seed=13)),
        ("next_l2norm_delta_1024", lambda: DeltaNormUpdate(dev, 1024, 8, seed=10)),
        ("next_l2norm_delta_decode", lambda: DeltaNormUpdate(dev, 1, 128, seed=11)),
        ("next_l2norm_delta_gatednorm_1024", lambda: DeltaGatedNorm(dev, 1024, 8, seed=12)),
        ("next_l2norm_delta_gatednorm_decode", lambda: DeltaGatedNorm(dev, 1, 128, seed=13)),
        ("next_w8a8_mlp_decode", lambda: W8A8Mlp(dev, 1, 4, seed=20)),
        ("next_w8a8_mlp_prefill_128", lambda: W8A8Mlp(dev, 128, 4, seed=21)),
        ("next_qwen35_decode", lambda: Qwen35Model(dev, 1, 512)),
        ("next_qwen35_prefill_512", lambda: Qwen35Model(dev, 512, 0, plans=1)),
    ]
    unknown = only - {k for k, _ in builders} - {"headline"}
    if unknown:
        print(f"unknown configuration(s): {sorted(unknown)}", file=sys.stderr)
        return 2
    result = {"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "data": "synthetic"}
    if not only or "headline" in only:
        result = headline(dev, args, cyc)
    only.discard("headline")

    # ---- the other configurations
    if not args.only_headline and (only or not args.only):
        extra = {}
        steps = max(10, min(args.steps, 50))
        for key, make in builders:
            if only and key not in only:
                continue
            x = make()
            log(f"{key}: {x.name}")
            n = steps if key != "cfg4_hybrid_decode_32k" else max(steps, 128)
            wu = min(args.warmup, 10)
            ms_x = run_timed(x.launch, n, wu, cyc)
            op_ms = {l: run_timed(lambda i, l=l: x.op(l, i), n, wu, cyc) for l in x.labels}
            entry = {"config": x.config(), "us_per_step": round(ms_x * 1e3, 3),
                     "tokens_per_s": round(x.tokens * 1e3 / ms_x, 1), "steps": n,
                     "op_us": {l: round(v * 1e3, 3) for l, v in op_ms.items()},
                     "timing": {"step": ms_x.summary(),
                                "dominant_op": op_ms[x.dominant].summary()},
                     "roofline": roofline(x, op_ms[x.dominant], n, wu, load_traffic(x.name))}
            if hasattr(x, "warm_op"):
                warm = run_timed(x.warm_op, n, wu, cyc)
                entry["timing"]["dominant_op_warm"] = warm.summary()
                entry["timing"]["cache_state"] = x.cache_state
            if x.bound == "mfma":
                entry["hbm_frac"] = None
            if isinstance(x, DeltaPrefill):
                kern_s = entry["roofline"]["kernel_us_avg"] * 1e-6
                entry["mfma_frac_recurrent_flops"] = round(
                    delta_flops(x.T, x.hv, x.dk, x.dv) / kern_s / 1e12 / MFMA_F16_PEAK_TFS, 5)
            if isinstance(x, (AttnRows, DeltaFront, DeltaNormUpdate, W8A8Mlp)):
                entry["op_roofline"] = {
                    l: {"bytes": x.bytes[l],
                        "achieved_GBs": round(x.bytes[l] / (op_ms[l] * 1e-3) / 1e9, 1),
                        "frac": round(x.bytes[l] / (op_ms[l] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
                    for l in x.labels}
            if isinstance(x, HybridDecode):
                hk, dk, hv, dv = x.dshape
                entry["delta_hbm_frac"] = round(
                    delta_bytes(1, hk, dk, hv, dv) / (op_ms["delta"] * 1e-3) / 1e9
                    / HBM_PEAK_GBS, 4)
            if not args.no_cpu:
                entry["cpu_baseline"] = x.cpu(args.cpu_seconds / 2)
                entry["cpu_baseline"]["host_cores"] = host_cores()
            log(f"{key}: {entry['us_per_step']} us/step, kernel "
                f"{entry['roofline']['kernel_us_avg']} us, frac {entry['roofline']['frac']}")
            extra[key] = entry
            print(f"[bench-detail] {key} {json.dumps(entry)}", file=sys.stderr, flush=True)
            del x
            torch.cuda.empty_cache()
        result["configs"] = extra

    if args.detail:
        Path(args.detail).parent.mkdir(parents=True, exist_ok=True)
        Path(args.detail).write_text(json.dumps(result, indent=1) + "\n")
    line = json.dumps(compact(result))
    if len(line) > COMPACT_LIMIT:  # never expected; keep the record parseable
        log(f"compact line {len(line)} B over {COMPACT_LIMIT}: dropping per-config fields")
        slim = compact(result)
        slim["configs"] = {k: {"us": v.get("us"), "frac": v.get("frac")}
                           for k, v in slim.get("configs", {}).items()}
        line = json.dumps(slim)
    print(line, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
