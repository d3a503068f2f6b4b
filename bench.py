"""Delivered-form throughput of the HIP executor on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--forms c1,c2,c3,c4,c5,aff,omd,copy,read]
                    [--cpu-budget SECONDS] [--no-cpu]

One "step" is one forward of a delivered form over one batch of synthetic
input that is already resident in HBM (the five benchmark configurations
C1-C5 at their full shapes, seeded with ``torch.manual_seed(0)``).  The
headline workload is C2 (the
SwiGLU MLP block with RMSNorm: rms_norm -> gate/up GEMM with the silu*mul
epilogue -> down GEMM); its whole-step TFLOP/s is ``value``.  Every other
config is measured the same way and reported under ``forms``, and so are
the dense affine scan (``aff``: a batched LTI recurrence delivered as
``apply(<aff_compose tree>, h)``) and the deferred-affine attention over a
scan's states (``omd``), which are not among C1-C5.

Per form:
  * ``ms_per_step``  — HIP events on torch's current stream (the stream the
    kernels are launched on) around K back-to-back steps, after W warmup
    steps, bracketed by ``torch.cuda.synchronize()``; the form's setup ends
    with about 100 ms of its own steps (``settle``) so the clocks are level
    under the load before the warm-up starts;
  * ``roofline``     — the form's dominant kernel timed alone the same way:
    algorithmic flops (MFMA-bound) or bytes (HBM-bound) per launch divided by
    its average launch duration, against MI355X's published peak;
  * ``cpu_baseline`` — the delivered form's op sequence as eager torch ops on
    the host CPU (``oracle/torch_cpu.py``, the reference's own execution
    style, pinned against the numpy oracle), with torch's pool set to every
    CPU this process may use, timed on a bounded sample of the same inputs:
    median and IQR per the reference's timing contract (``timing.py:54-80``);
    its outputs double as a parity check of the GPU outputs on that sample
    (``parity_max_rel``).

Only rank 0 of one process prints, one JSON line on stdout.  ``--gpus`` above
1 exits with a message: this build measures one GPU.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "delivered-kernel TFLOP/s & HBM GB/s (% of MI355X peak) per lowered form"
PEAK = {"bf16_tflops": 2500.0, "fp32_tflops": 157.3, "hbm_gbs": 8000.0}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# --------------------------------------------------------------------- timing


def time_events(fn, steps: int, warmup: int) -> float:
    """Average ms per call of ``fn`` over ``steps`` calls (HIP events)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        fn()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


SETTLE_MS = 100.0


def settle(fn, ms: float, max_steps: int = 10000) -> int:
    """Run ``fn`` until about ``ms`` of device time has passed (untimed):
    the steps that bring the clocks to their level under this load."""
    import torch

    n, t0 = 0, time.perf_counter()
    while n < max_steps:
        fn()
        n += 1
        if n & 7 == 0:
            torch.cuda.synchronize()
            if (time.perf_counter() - t0) * 1e3 >= ms:
                break
    torch.cuda.synchronize()
    return n


def time_graph_replays(fn, n: int = 30, warmup: int = 5) -> dict:
    """One call of ``fn`` recorded into a hipGraph and replayed: median and
    interquartile range (ms) of ``n`` replays timed one by one with HIP
    events after ``warmup`` untimed replays (the reference's timing contract,
    timing.py:54-80: warmup >= 5, n >= 30, median / IQR)."""
    import statistics

    import torch

    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(n):
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        g.replay()
        t1.record()
        t1.synchronize()
        ts.append(t0.elapsed_time(t1))
    q = statistics.quantiles(ts, n=4)
    # the same n replays issued back to back between two events, as the eager
    # step is timed: no host round trip between steps
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(n):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    b2b = t0.elapsed_time(t1) / n
    del g
    return {"median_ms": round(statistics.median(ts), 5), "iqr_ms": round(q[2] - q[0], 5), "n": n,
            "warmup": warmup, "back_to_back_ms": round(b2b, 5)}


def time_graph(fn, reps: int = 50) -> float:
    """Average ms per call of ``fn`` recorded ``reps`` times into one hipGraph
    (launches back to back on the GPU, no host gap between them)."""
    import torch

    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(3):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / (3 * reps)


def _blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        n = [int(i.get("num_threads", 1)) for i in threadpool_info() if i.get("user_api") == "blas"]
        return max(n) if n else 1
    except Exception:  # pragma: no cover - threadpoolctl missing
        return 1


def host_provenance() -> dict:
    """What the CPU baseline ran on: CPU model, the CPUs this process may
    use, the BLAS pool, and the library versions."""
    import numpy
    import torch

    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:  # pragma: no cover
        pass
    return {"cpu_model": model, "affinity_cpus": len(os.sched_getaffinity(0)), "os_cpu_count": os.cpu_count(),
            "blas_threads": _blas_threads(), "torch_threads": len(os.sched_getaffinity(0)),
            "torch": torch.__version__, "numpy": numpy.__version__,
            "python": sys.version.split()[0]}


def time_cpu(fn, budget_s: float, min_reps: int = 4) -> tuple[float, tuple[float, float], int, object]:
    """Median and (first, third) quartiles of seconds per call of ``fn``
    (≥ ``min_reps`` calls, about ``budget_s`` in all, at most 50), the
    reference's timing contract (``timing.py:54-80``: median, and the IQR
    from quartiles at n = 4; no spread below 4 samples)."""
    times, out = [], None
    t_start = time.perf_counter()
    while len(times) < min_reps or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        out = fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    med = statistics.median(times)
    quart = (med, med)
    if len(times) >= 4:
        q1, _, q3 = statistics.quantiles(times, n=4)
        quart = (q1, q3)
    return med, quart, len(times), out


def rate_iqr(work: float, quart: tuple[float, float]) -> float:
    """IQR of the rate work / t from the quartiles of t (the rate falls as t
    grows, so its quartiles are work / q3 and work / q1)."""
    return work / quart[0] - work / quart[1]


class host_threads:
    """torch's intra-op pool set to every CPU this process may run on, for
    the CPU baseline (restored afterwards)."""

    def __enter__(self):
        import torch

        self.prev = torch.get_num_threads()
        self.n = len(os.sched_getaffinity(0))
        torch.set_num_threads(self.n)
        return self

    def __exit__(self, *exc):
        import torch

        torch.set_num_threads(self.prev)


def cpu_record(value: float, iqr_value: float, unit: str, cores: int, sample: str, reps: int,
               rel: float) -> dict:
    return {"value": value, "iqr": iqr_value, "unit": unit, "cores": cores, "kind": "port",
            "impl": "torch (the delivered form's eager ops on the host CPU, oracle/torch_cpu.py)",
            "sample": f"{sample}, median of {reps} reps", "parity_max_rel": rel}


# --------------------------------------------------------------------- traffic

#: rocprofv3 counter calibration, from a 2 GiB device copy on the MI355X box:
#: FETCH_SIZE reads half the bytes copied, WRITE_SIZE all of them.
FETCH_SCALE, WRITE_SCALE = 2.0, 1.0
TRAFFIC_TABLE = ROOT / "profiles" / "pmc_traffic_all_forms.md"


def traffic_bytes(kernel_key) -> float | None:
    """HBM bytes per launch of a kernel from the committed counter summary:
    (FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0) KiB per dispatch, averaged over
    its dispatches (rows ``| key | fetch KiB | write KiB | ... |``).  A tuple
    of keys (a dominant unit of several launches) sums its rows."""
    if isinstance(kernel_key, tuple):
        parts = [traffic_bytes(k) for k in kernel_key]
        return None if any(p is None for p in parts) else sum(parts)
    if not kernel_key or not TRAFFIC_TABLE.exists():
        return None
    for line in TRAFFIC_TABLE.read_text().splitlines():
        cells = [c.strip().strip("`") for c in line.strip().strip("|").split("|")]
        if len(cells) >= 3 and cells[0] == kernel_key:
            try:
                return round((float(cells[1]) * FETCH_SCALE + float(cells[2]) * WRITE_SCALE) * 1024.0)
            except ValueError:
                return None
    return None


# ---------------------------------------------------------------------- forms


class Form:
    """One benchmark configuration: inputs, one delivered step, its dominant kernel."""

    name = ""
    workload = ""
    dtype = ""
    unit = ""          # the form's headline unit: "TFLOP/s" or "GB/s"
    bound = ""         # "mfma" | "hbm" for the dominant kernel
    peak = 0.0
    work = 0.0         # algorithmic flops or bytes per step
    dom_name = ""
    dom_key = ""       # the dominant kernel's row in the counter summary
    dom_work = 0.0     # algorithmic flops or bytes per dominant-kernel launch

    def setup(self, dev) -> None: ...
    def step(self) -> None: ...
    def dominant(self) -> None: ...
    def cpu(self, budget: float) -> dict | None: return None
    def free(self) -> None:
        for k in list(vars(self)):
            if not k.startswith("_"):
                delattr(self, k)

    def throughput(self, ms: float) -> float:
        scale = 1e12 if self.unit == "TFLOP/s" else 1e9
        return self.work / (ms * 1e-3) / scale


def _gen(seed=0):
    import torch

    return torch.Generator(device="cuda").manual_seed(seed)


_SINKS: dict = {}


def _sink(dev):
    """The drop-in sink (one per device): every form below is delivered
    through its executor table exactly as catopt routes a term."""
    from catopt_amd.sink import HipSink

    key = str(dev)
    if key not in _SINKS:
        _SINKS[key] = HipSink(device=dev)
    return _SINKS[key]


class C1WeightChain(Form):
    name, dtype, unit, bound = "c1", "f32", "TFLOP/s", "mfma"
    workload = "C1 deep linear weight chain: 8x nn.Linear(512,512)+bias folded to one GEMM+bias, x[64,512] fp32"
    peak = PEAK["fp32_tflops"]
    work = dom_work = 2.0 * 64 * 512 * 512
    dom_name = "gemm_f32_skinny<BIAS>"
    dom_key = "gemm_f32_skinny<1>"

    def setup(self, dev):
        import torch

        from catopt_amd import forms
        from catopt_amd import kernels as K
        from catopt_amd.sink import deliver

        torch.manual_seed(0)
        layers = [torch.nn.Linear(512, 512) for _ in range(8)]
        self.x_cpu = torch.randn(64, 512)
        self.Ws_cpu = [l.weight.detach().numpy() for l in layers]
        self.bs_cpu = [l.bias.detach().numpy() for l in layers]
        vals = {}
        for i, l in enumerate(layers):
            vals[f"W{i + 1}"], vals[f"b{i + 1}"] = l.weight.detach(), l.bias.detach()
        self.x = self.x_cpu.to(dev)
        # the delivered term through the sink: construction folds the chain on
        # the device (7 GEMMs + bias mat-vecs); a step is the one remaining
        # GEMM + bias, launched eagerly (a hipGraph replay costs more host
        # time on this stack than the eager launch it replaces)
        ir, _ = forms.weight_chain_form(8, 512, 64)
        res = deliver(ir, vals, _sink(dev), (self.x,))
        self.mod, self.stats = res.module, res.stats
        # the construction fold, timed on its own (a second delivery of the
        # same term: planning, the weight-product GEMMs and the bias
        # mat-vecs on the device; 7·2·512³ flop of products)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        deliver(ir, vals, _sink(dev), (self.x,))
        torch.cuda.synchronize()
        fold_ms = (time.perf_counter() - t0) * 1e3
        self.extras = {"construction": {"ms": round(fold_ms, 3), "fold_flop": 7 * 2 * 512 ** 3,
                                        "note": "one delivery: plan, fold and first checks, host clock"}}
        (_, refs, _), = self.mod._tape.steps
        p = self.mod._param_map
        self.W_eff, self.c = p[refs[1][1]], p[refs[2][1]]
        self.K = K

    def step(self):
        self.y = self.mod(self.x)

    def dominant(self):
        self.K.linear(self.x, self.W_eff, self.c)

    # the kernel runs ~5 us: time it inside a graph of back-to-back launches
    # so the host's per-call launch gap is not counted as kernel time
    dominant_in_graph = True

    def cpu(self, budget):
        import oracle

        x, W, c = (t.detach().float().cpu() for t in (self.x, self.W_eff, self.c))
        with host_threads() as ht:
            sec, iqr, reps, out = time_cpu(lambda: oracle.torch_cpu.weight_chain(x, W, c), budget)
        self.step()
        rel = oracle.verify_equiv(out.double().numpy(), self.y.cpu().double().numpy())["max_rel"]
        return cpu_record(self.work / sec / 1e12, rate_iqr(self.work, iqr) / 1e12, "TFLOP/s", ht.n,
                          "full C1 forward (the folded linear, fp32)", reps, rel)

class C2SwiGLU(Form):
    name, dtype, unit, bound = "c2", "bf16", "TFLOP/s", "mfma"
    workload = ("C2 SwiGLU MLP block with RMSNorm: x[8,2048,4096] bf16, rms_norm(eps=1e-6) -> "
                "gate/up GEMM [4096->2x11008] with fused silu*mul -> down GEMM [11008->4096]")
    peak = PEAK["bf16_tflops"]
    M, D, F = 8 * 2048, 4096, 11008
    work = 2.0 * M * D * 2 * F + 2.0 * M * F * D
    dom_name = "gemm_bf16_nt<SILU_MUL>"
    dom_key = "gemm_bf16_nt<3>"
    dom_work = 2.0 * M * D * 2 * F

    def setup(self, dev):
        import torch

        from catopt_amd import _lib as L
        from catopt_amd import kernels as K

        from catopt_amd import forms
        from catopt_amd.sink import deliver

        g = _gen(0)
        bf = torch.bfloat16
        self.L = L
        self.x = torch.randn(8, 2048, self.D, device=dev, generator=g).to(bf)
        vals = {
            "gamma": (1 + 0.02 * torch.randn(self.D, device=dev, generator=g)).to(bf),
            "W_gate": (0.02 * torch.randn(self.F, self.D, device=dev, generator=g)).to(bf),
            "W_up": (0.02 * torch.randn(self.F, self.D, device=dev, generator=g)).to(bf),
            "W_down": (0.02 * torch.randn(self.D, self.F, device=dev, generator=g)).to(bf),
        }
        # delivered term: rms_norm -> linear(concat(W_gate, W_up)) -> chunk/silu/mul
        # -> linear(W_down); construction folds the concat and fuses the
        # gate into the GEMM epilogue (tape: rms_norm, hip_swiglu, hip_linear)
        ir, _ = forms.swiglu_block_form((8, 2048), self.D, self.F)
        res = deliver(ir, vals, _sink(dev), (self.x,))
        self.mod, self.stats = res.module, res.stats
        del vals
        steps = self.mod._tape.steps
        assert [s[0] for s in steps] == ["rms_norm", "hip_swiglu", "hip_linear"], steps
        p = self.mod._param_map
        self.gamma = p[steps[0][1][1][1]]
        self.w_cat = p[steps[1][1][1][1]]
        self.w_down = p[steps[2][1][1][1]]
        self.K = K
        self.h = K.rmsnorm(self.x, self.gamma, 1e-6)

    def step(self):
        self.y = self.mod(self.x)

    def dominant(self):
        self.K.linear(self.h, self.w_cat, epilogue=self.L.EPI_SILU_MUL)

    def cpu(self, budget):
        import oracle

        rows = 2048
        x = self.x.reshape(-1, self.D)[:rows].cpu()
        gam, wcat, wd = (t.cpu() for t in (self.gamma, self.w_cat, self.w_down))
        wg, wu = wcat[: self.F], wcat[self.F:]
        with host_threads() as ht:
            sec, iqr, reps, out = time_cpu(lambda: oracle.torch_cpu.swiglu_block(x, gam, wg, wu, wd, 1e-6), budget)
        self.step()
        rel = oracle.verify_equiv(out.double().numpy(), self.y.reshape(-1, self.D)[:rows].cpu().double().numpy())["max_rel"]
        flops = self.work * rows / self.M
        return cpu_record(flops / sec / 1e12, rate_iqr(flops, iqr) / 1e12, "TFLOP/s", ht.n,
                          f"first {rows} of {self.M} rows: rms_norm, fused gate/up linear, silu*mul, down linear (bf16)",
                          reps, rel)

class C3Attention(Form):
    name, dtype, unit, bound = "c3", "bf16", "TFLOP/s", "mfma"
    B, H, T, Dh = 4, 32, 4096, 128
    workload = "C3 causal MHA (om_apply(om_elem) online softmax): q,k,v[4,32,4096,128] bf16, scale 1/sqrt(128)"
    peak = PEAK["bf16_tflops"]
    work = dom_work = 4.0 * B * H * T * T * Dh / 2  # causal half of the square
    dom_name = "attn_q64_kernel<CAUSAL>"
    dom_key = "attn_q64_kernel<1>"

    def setup(self, dev):
        import torch

        from catopt_amd import kernels as K

        g = _gen(0)
        shp = (self.B, self.H, self.T, self.Dh)
        self.q = torch.randn(shp, device=dev, generator=g).to(torch.bfloat16)
        self.k = torch.randn(shp, device=dev, generator=g).to(torch.bfloat16)
        self.v = torch.randn(shp, device=dev, generator=g).to(torch.bfloat16)
        self.scale = 1.0 / math.sqrt(self.Dh)
        self.K = K
        from catopt_amd import forms
        from catopt_amd.sink import deliver

        # delivered term: om_apply(om_elem(masked_fill(q k^T / sqrt(d), !mask, -inf), v))
        # with the lower-triangular bool mask as a Param; the OM executor finds
        # the triangle bit-exactly at construction and runs the causal kernel
        ir, _ = forms.causal_attention_form(self.B, self.H, self.T, self.Dh, mask="param")
        mask = torch.ones(self.T, self.T, dtype=torch.bool, device=dev).tril()
        res = deliver(ir, {"mask": mask}, _sink(dev), (self.q, self.k, self.v))
        self.mod, self.stats = res.module, res.stats
        assert self.mod._plan["leaves"][0]["mask_kind"] == "causal"

    def step(self):
        self.o = self.mod(self.q, self.k, self.v)

    def dominant(self):
        self.K.attention(self.q, self.k, self.v, self.scale, causal=True)

    def cpu(self, budget):
        import oracle

        nh = 4  # heads (b = 0, h = 0..3) of the 128; heads are independent
        q, k, v = (t[0, :nh].cpu() for t in (self.q, self.k, self.v))
        with host_threads() as ht:
            sec, iqr, reps, out = time_cpu(lambda: oracle.torch_cpu.causal_attention(q, k, v, self.scale), budget)
        self.step()
        rel = oracle.verify_equiv(out.double().numpy(), self.o[0, :nh].cpu().double().numpy())["max_rel"]
        flops = self.work * nh / (self.B * self.H)
        return cpu_record(flops / sec / 1e12, rate_iqr(flops, iqr) / 1e12, "TFLOP/s", ht.n,
                          f"{nh} of {self.B * self.H} heads, T={self.T}: matmul, masked_fill, softmax, matmul (bf16; "
                          "work counted as the causal half)", reps, rel)

class C4Retention(Form):
    name, dtype, unit, bound = "c4", "bf16", "GB/s", "hbm"
    B, H, T, Dh, C = 4, 16, 8192, 128, 64
    workload = ("C4 chunked decayed retention (om_decayed K-way, C=64): q,k,v[4,16,8192,128] bf16 "
                "~N(0,1)/sqrt(128), gamma_h = 1-2^(-5-h/2) fp32")
    peak = PEAK["hbm_gbs"]
    work = dom_work = 4.0 * B * H * T * Dh * 2  # q, k, v read + o written, bf16
    flops = B * H * (T / C) * (4 * C * C * Dh + 4 * C * Dh * Dh)
    # the dominant unit is one retention call: the state pass (the start
    # states of the T-segments) and the output pass, back to back
    dom_name = "retention_state + retention_out"
    dom_key = ("retention_state", "retention_out")

    def setup(self, dev):
        import torch

        from catopt_amd import kernels as K

        g = _gen(0)
        shp = (self.B, self.H, self.T, self.Dh)
        s = 1.0 / math.sqrt(self.Dh)
        self.q = (torch.randn(shp, device=dev, generator=g) * s).to(torch.bfloat16)
        self.k = (torch.randn(shp, device=dev, generator=g) * s).to(torch.bfloat16)
        self.v = (torch.randn(shp, device=dev, generator=g) * s).to(torch.bfloat16)
        self.gamma = torch.tensor([1 - 2.0 ** (-5 - h / 2) for h in range(self.H)],
                                  dtype=torch.float32, device=dev)
        self.K = K
        from catopt_amd import forms
        from catopt_amd.sink import deliver

        # delivered term: the K-way chunked form (K = T/C = 128 arms, 8128
        # cross blocks), parsed once into (q, k, v, gamma, scale) by the
        # chunked-decay executor
        ir, _ = forms.retention_kway_form(self.B, self.H, self.T, self.Dh, self.C)
        res = deliver(ir, {"gamma": self.gamma}, _sink(dev), (self.q, self.k, self.v))
        self.mod, self.stats = res.module, res.stats
        assert self.mod.n_chunks == self.T // self.C

    def step(self):
        self.o = self.mod(self.q, self.k, self.v)

    def dominant(self):
        self.K.retention(self.q, self.k, self.v, self.gamma, 1.0)

    def cpu(self, budget):
        import oracle

        Ts = 2048  # every head of batch 0, the first 2048 steps (causal: a prefix is exact)
        q, k, v = (t[:1, :, :Ts].cpu() for t in (self.q, self.k, self.v))
        g = self.gamma.cpu()
        with host_threads() as ht:
            sec, iqr, reps, out = time_cpu(lambda: oracle.torch_cpu.retention_chunked(q, k, v, g, self.C, 1.0), budget)
        self.step()
        rel = oracle.verify_equiv(out.double().numpy(), self.o[:1, :, :Ts].cpu().double().numpy())["max_rel"]
        nbytes = 4.0 * self.H * Ts * self.Dh * 2
        return cpu_record(nbytes / sec / 1e9, rate_iqr(nbytes, iqr) / 1e9, "GB/s", ht.n,
                          f"b=0, all {self.H} heads, first {Ts} of {self.T} steps: the chunked decayed form, C={self.C} "
                          "(bf16 operands, fp32 arithmetic)", reps, rel)

class C5SSM(Form):
    name, dtype, unit, bound = "c5", "f32", "GB/s", "hbm"
    B, D, N, T = 16, 2048, 16, 16384
    workload = ("C5 diagonal selective SSM scan, all y_t: B=16 D=2048 N=16 T=16384 fp32, "
                "a_t (B,T,D,N) = exp(-softplus(N(0,1))), b_t,c_t (B,T,N), x_t (B,T,D)")
    peak = PEAK["hbm_gbs"]
    work = dom_work = 4.0 * (B * T * D * N + 2 * B * T * N + 2 * B * T * D)
    dom_name = "ssm_stream_reg<16>"
    dom_key = "ssm_stream_reg<16>"

    def setup(self, dev):
        import torch

        from catopt_amd import forms
        from catopt_amd.sink import deliver

        g = _gen(0)
        B, D, N, T = self.B, self.D, self.N, self.T
        a = torch.randn((B, T, D, N), device=dev, generator=g)
        self.a = a.neg_().sigmoid_()  # exp(-softplus(z)) == sigmoid(-z), in place
        self.bx = torch.randn((B, T, N), device=dev, generator=g)
        self.c = torch.randn((B, T, N), device=dev, generator=g)
        self.x = torch.randn((B, T, D), device=dev, generator=g)
        self.h = torch.zeros((B, D, N), device=dev)
        self.ins = (self.a, self.bx, self.c, self.x, self.h)
        # delivered term: sum(mul(applyd(<stacked prefix maps>, h), c), -1) over
        # T = 16384 leaves aff_diag(a_t, x_t ⊗ bx_t); the scan executor runs it
        # as one fused scan + read-out launch over the blocked-prefix chunk plan
        ir, _ = forms.diag_ssm_form(B, T, D, N)
        res = deliver(ir, {}, _sink(dev), self.ins)
        self.mod, self.stats = res.module, res.stats
        assert self.mod.is_batched and self.mod._plan["factors"] is not None

    def step(self):
        self.y = self.mod(*self.ins)

    dominant = step

    def cpu(self, budget):
        import oracle

        Ts = 512  # every lane (all batches, channels, states), the first 512 steps (a prefix is exact)
        a = self.a[:, :Ts].cpu()
        bx, c, x = (t[:, :Ts].cpu() for t in (self.bx, self.c, self.x))
        h0 = self.h.cpu()
        with host_threads() as ht:
            sec, iqr, reps, out = time_cpu(lambda: oracle.torch_cpu.ssm_scan(a, bx, c, x, h0), budget)
        del a
        self.step()
        rel = oracle.verify_equiv(out.double().numpy(), self.y[:, :Ts].cpu().double().numpy())["max_rel"]
        nbytes = self.work * Ts / self.T
        return cpu_record(nbytes / sec / 1e9, rate_iqr(nbytes, iqr) / 1e9, "GB/s", ht.n,
                          f"all {self.B}x{self.D}x{self.N} lanes, first {Ts} of {self.T} steps: the serial recurrence "
                          "and read-out, each step over every lane (fp32)", reps, rel)

class DenseScan(Form):
    """The dense affine monoid (not one of C1-C5): a batched LTI
    ``LinearRecurrence`` h_t = A h_{t-1} + x_t over many independent
    sequences, delivered as ``apply(<balanced aff_compose tree>, h)`` with one
    shared map; the kernel runs each step as one fp32 MFMA product over all
    sequences' state columns."""

    name, dtype, unit, bound = "aff", "f32", "TFLOP/s", "mfma"
    B, d, T = 16384, 64, 1024
    workload = ("dense affine scan apply(aff_compose tree, h): shared A (64x64), B=16384 sequences, "
                "T=1024 steps, offsets b_t (T,B,64,1), final state (B,64,1), fp32")
    peak = PEAK["fp32_tflops"]
    work = dom_work = 2.0 * T * B * d * d
    dom_name = dom_key = "aff_dense_scan<4, false, true, 0>"

    def setup(self, dev):
        import torch

        from catopt_amd import forms
        from catopt_amd.sink import deliver

        g = _gen(0)
        B, d, T = self.B, self.d, self.T
        self.A = torch.randn((d, d), device=dev, generator=g) * (0.9 / math.sqrt(d))
        self.b = torch.randn((T, B, d, 1), device=dev, generator=g)
        self.h = torch.randn((B, d, 1), device=dev, generator=g)
        ir, _ = forms.dense_scan_form(T, d, (B,), 1)
        res = deliver(ir, {}, _sink(dev), (self.A, self.b, self.h))
        self.mod, self.stats = res.module, res.stats
        assert self.mod.is_batched and self.mod._plan["a_shared"]

    def step(self):
        self.out = self.mod(self.A, self.b, self.h)

    dominant = step  # one kernel launch per step

    def cpu(self, budget):
        import oracle

        Bs = 2048  # 2048 of the 16384 sequences (independent: a subset is exact), all steps
        A = self.A.cpu()
        b = self.b[:, :Bs, :, 0].cpu()
        h = self.h[:Bs, :, 0].cpu()
        with host_threads() as ht:
            sec, iqr, reps, out = time_cpu(lambda: oracle.torch_cpu.dense_scan(A, b, h), budget)
        self.step()
        rel = oracle.verify_equiv(out.double().numpy(), self.out[:Bs, :, 0].cpu().double().numpy())["max_rel"]
        flops = 2.0 * self.T * Bs * self.d * self.d
        return cpu_record(flops / sec / 1e12, rate_iqr(flops, iqr) / 1e12, "TFLOP/s", ht.n,
                          f"{Bs} of {self.B} sequences, all {self.T} steps: one batched matmul + add per step (fp32)",
                          reps, rel)

class OmdScanAttention(Form):
    """Deferred-affine attention (not one of C1-C5): softmax attention of
    Tq queries over the T states of a diagonal scan, delivered as
    ``omd_apply(<omd_compose tree of omd_elem(q·k_iᵀ, stack(affd_a f_j),
    stack(affd_b f_j))>, h)`` over 16 key blocks of the prefix chain f_j."""

    name, dtype, unit, bound = "omd", "f32", "TFLOP/s", "mfma"
    T, d, Tq, blocks, dk = 4096, 64, 4096, 16, 64
    workload = ("omd attention over scan states: T=4096 keys/steps, state d=64, Tq=4096 queries, dk=64, "
                "16 key blocks, diagonal scan a_t,x_t (T,64), fp32")
    peak = PEAK["fp32_tflops"]
    work = 2.0 * Tq * T * (dk + 2 * d)  # scores + the two numerator parts
    dom_name = dom_key = "attn_carrier_f32<64, 4, 0>"
    dom_work = work  # one launch computes every leaf's carrier

    def setup(self, dev):
        import torch

        from catopt_amd import forms
        from catopt_amd import kernels as K
        from catopt_amd.sink import deliver

        g = _gen(0)
        self.q = torch.randn((self.Tq, self.dk), device=dev, generator=g) * 0.125
        self.k = torch.randn((self.T, self.dk), device=dev, generator=g) * 0.125
        self.a = torch.rand((self.T, self.d), device=dev, generator=g) * 0.4 + 0.6
        self.x = torch.randn((self.T, self.d), device=dev, generator=g)
        self.h = torch.randn((self.d,), device=dev, generator=g)
        ir, _ = forms.omd_scan_attention_form(self.T, self.d, self.Tq, self.blocks, self.dk)
        self.ins = (self.q, self.k, self.a, self.x, self.h)
        res = deliver(ir, {}, _sink(dev), self.ins)
        self.mod, self.stats = res.module, res.stats
        assert self.mod.map_mode == "chain"
        C = self.T // self.blocks
        # the dominant launch on the same shapes: all 16 leaves' carriers at once
        self.kb = self.k.reshape(self.blocks, C, self.dk)
        self.V = torch.randn((self.blocks, C, 2 * self.d), device=dev, generator=g)
        self.K = K

    def step(self):
        self.out = self.mod(*self.ins)

    def dominant(self):
        self.K.attn_carrier_f32(self.q, self.kb, self.V, 1.0)

    def cpu(self, budget):
        import oracle

        q, k, a, x, h = (t.cpu() for t in self.ins)
        with host_threads() as ht:
            sec, iqr, reps, out = time_cpu(lambda: oracle.torch_cpu.omd_attention(q, k, a, x, h), budget)
        self.step()
        rel = oracle.verify_equiv(out.double().numpy(), self.out.double().cpu().numpy())["max_rel"]
        flops = 2.0 * self.Tq * self.T * (self.dk + self.d)
        return cpu_record(flops / sec / 1e12, rate_iqr(flops, iqr) / 1e12, "TFLOP/s", ht.n,
                          f"the full form: {self.Tq} queries over all {self.T} scan states (serial scan, dense "
                          "softmax, fp32)", reps, rel)

class CopyStream(Form):
    """STREAM-style device copy of 2 GiB fp32: the measured-achievable HBM
    figure reported beside the vendor peak, and the known-size kernel the
    ``FETCH_SIZE`` / ``WRITE_SIZE`` counters are calibrated against."""

    name, dtype, unit, bound = "copy", "f32", "GB/s", "hbm"
    NBYTES = 2 << 30
    workload = "device-to-device copy of 2 GiB fp32 (torch copy_ kernel), read + write"
    peak = PEAK["hbm_gbs"]
    work = dom_work = 2.0 * NBYTES
    dom_name = "torch copy kernel"
    dom_key = "__amd_rocclr_copyBuffer (2 GiB)"

    def setup(self, dev):
        import torch

        self.src = torch.ones(self.NBYTES // 4, dtype=torch.float32, device=dev)
        self.dst = torch.empty_like(self.src)

    def step(self):
        self.dst.copy_(self.src)

    dominant = step


class ReadStream(Form):
    """Read-only HBM stream over 2 GiB (``catopt_hip_hbm_read``): the
    achievable read rate, the ceiling for the read-dominated scans (C5 reads
    94% of its bytes), beside the copy's read + write figure."""

    name, dtype, unit, bound = "read", "u32", "GB/s", "hbm"
    NBYTES = 2 << 30
    workload = "read-only stream over 2 GiB (catopt_hip_hbm_read), every byte read once"
    peak = PEAK["hbm_gbs"]
    work = dom_work = float(NBYTES)
    dom_name = "hbm_read_kernel"
    dom_key = "hbm_read_kernel (2 GiB)"

    def setup(self, dev):
        import torch

        from catopt_amd import kernels as K

        self.K = K
        self.src = torch.ones(self.NBYTES // 4, dtype=torch.float32, device=dev)
        self.sink = torch.zeros(1, dtype=torch.int32, device=dev)

    def step(self):
        self.K.hbm_read(self.src, self.sink)

    dominant = step


FORMS = {f.name: f for f in (C1WeightChain, C2SwiGLU, C3Attention, C4Retention, C5SSM, DenseScan,
                                OmdScanAttention, CopyStream, ReadStream)}
HEADLINE = "c2"


def measure(form: Form, dev, steps: int, warmup: int, cpu_budget: float | None,
            settle_ms: float = SETTLE_MS) -> dict:
    import torch

    log(f"{form.name}: setup")
    form.setup(dev)
    torch.cuda.synchronize()
    # end the setup with about SETTLE_MS of the form's own steps, so the
    # clocks have settled under this load before the W warm-up steps and the
    # K timed ones (a few warm-up steps of a sub-millisecond step leave the
    # first timed steps up to 10% slow)
    settle_steps = settle(form.step, settle_ms) if settle_ms > 0 else 0
    log(f"{form.name}: timing {steps} steps after {warmup} warmup")
    w0 = time.perf_counter()
    ms = time_events(form.step, steps, warmup)
    wall_ms = (time.perf_counter() - w0) * 1e3
    fb = int(getattr(getattr(form, "mod", None), "fallbacks", 0) or 0)
    if fb:  # a step that left the HIP kernels would time the generic module
        raise RuntimeError(f"{form.name}: {fb} step(s) ran the generic module instead of the HIP path")
    dom_steps = max(steps, 10)
    if getattr(form, "dominant_in_graph", False):
        dom_ms = time_graph(form.dominant)
    else:
        dom_ms = time_events(form.dominant, dom_steps, 2)
    achieved = form.dom_work / (dom_ms * 1e-3) / (1e12 if form.bound == "mfma" else 1e9)
    rec = {
        "workload": form.workload,
        "dtype": form.dtype,
        "ms_per_step": round(ms, 5),
        "value": round(form.throughput(ms), 3),
        "unit": form.unit,
        "work_per_step": form.work,
        "roofline": {
            "kernel": form.dom_name,
            "bound": form.bound,
            "achieved": round(achieved, 3),
            "peak": form.peak,
            "unit": "TFLOP/s" if form.bound == "mfma" else "GB/s",
            "frac": round(achieved / form.peak, 4),
            "traffic": traffic_bytes(form.dom_key),
            "avg_launch_us": round(dom_ms * 1e3, 3),
            "work_per_launch": form.dom_work,
        },
        "wall_ms_incl_warmup": round(wall_ms, 2),
        "settle": {"ms": settle_ms, "steps": settle_steps},
    }
    # the step replayed from a hipGraph (median / IQR over 30 replays)
    try:
        rec["graph_replay"] = time_graph_replays(form.step)
    except Exception as exc:  # a step that cannot be captured is reported, not fatal
        rec["graph_replay"] = {"error": f"{type(exc).__name__}: {exc}"[:200]}
    if getattr(form, "stats", None) is not None:
        rec["delivery"] = {k: (v.value if hasattr(v, "value") else v) for k, v in form.stats.items()}
    if isinstance(form, C4Retention):
        rec["tflops_chunked_form"] = round(form.flops / (ms * 1e-3) / 1e12, 3)
    rec.update(getattr(form, "extras", None) or {})
    if cpu_budget:
        log(f"{form.name}: cpu baseline (~{cpu_budget:.0f}s)")
        try:
            rec["cpu_baseline"] = form.cpu(cpu_budget)
        except MemoryError as exc:  # pragma: no cover
            rec["cpu_baseline"] = {"error": str(exc)}
        if rec["cpu_baseline"] is not None:
            rec["cpu_baseline"]["host"] = host_provenance()
    form.free()
    torch.cuda.empty_cache()
    return rec


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--forms", default="c1,c2,c3,c4,c5,aff,omd,copy,read")
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU oracle work for the headline form (others get a third)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="untimed steps of each form before its warm-up (0: none; counter passes)")
    args = ap.parse_args(argv)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} (WORLD_SIZE={world}) is not "
              "supported; every config runs on one MI355X and reports that GPU's throughput.",
              file=sys.stderr)
        return 2
    if int(os.environ.get("RANK", "0")) != 0:
        return 0

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    from catopt_amd import _lib

    _lib.load()  # loud if the HIP library is missing
    dev = torch.device("cuda", 0)
    names = [n.strip() for n in args.forms.split(",") if n.strip()]
    for n in names:
        if n not in FORMS:
            print(f"unknown form {n!r}; choose from {sorted(FORMS)}", file=sys.stderr)
            return 2
    forms = {}
    for n in names:
        budget = None if args.no_cpu else (args.cpu_budget if n == HEADLINE else args.cpu_budget / 3)
        forms[n] = measure(FORMS[n](), dev, args.steps, args.warmup, budget, args.settle_ms)
        log(f"{n}: {forms[n]['value']} {forms[n]['unit']} ({forms[n]['ms_per_step']} ms/step, "
            f"roofline frac {forms[n]['roofline']['frac']})")

    head = forms.get(HEADLINE) or forms[names[0]]
    head_name = HEADLINE if HEADLINE in forms else names[0]
    line = {
        "metric": METRIC,
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic (seeded N(0,1) inputs and random-init weights of the config shapes)",
        "config": {"workload": head["workload"], "form": head_name,
                   "device": torch.cuda.get_device_name(0)},
        "roofline": head["roofline"],
        "cpu_baseline": head.get("cpu_baseline"),
        "forms": forms,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
