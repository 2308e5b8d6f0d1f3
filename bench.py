"""Benchmark of the MI355X packed 4-bit affine quantized matmul (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only c0,c1,...] [--no-cpu]

Headline (the JSON `value`): the decode gate+up workload — x bf16 [M, 5120] for M = 1, 2 and 4
batched requests against packed 4-bit weights [34816, 5120] (group 64). One step = the three
quantized matmuls (M = 1, 2, 4), each on its own copy of the weights; copies rotate so the
256 MB Infinity Cache cannot serve them (>= 640 MB of distinct weights). value = algorithmic
bytes of the K timed steps / their GPU time (HIP events around the whole region), in GB/s.

Also measured (the `workloads` object): every benchmark workload's kernel time per call (median
of >= 20 single-launch HIP-event samples on rotating weight copies), achieved HBM GB/s and MFMA
TFLOP/s against MI355X peaks (8 TB/s; 2.5 PFLOP/s dense bf16). The `roofline` object is the
dominant kernel of the headline: algorithmic bytes per launch / mean launch duration, measured
with per-launch HIP events on the launch stream in a second pass of K steps.

cpu_baseline: the oracle's C restatement (OpenMP, fp32 accumulation) on the host cores, on a
bounded, time-boxed sample of the same decode steps.
"""

from __future__ import annotations

import argparse
import importlib.util
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mlx-tree-spec_amd"))

METRIC = "qmm µs + HBM GB/s (% of peak) at M=1–64; TFLOP/s at M=4096 prefill"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 << 20
ROTATE_BYTES = 640e6
WARM_S = 0.25  # seconds of back-to-back calls before a workload is timed

WORKLOADS = {
    # name: (config index, rows, K, N, sigma)
    "c0": (0, (16,), 5120, 5120, 1.0),
    "c1": (1, (1, 2, 4), 5120, 34816, 1.0),
    "c2": (2, (64,), 17408, 5120, 0.5),
    "c3": (3, (32,), 5120, 151936, 1.0),
    "c4": (4, (4096,), 5120, 17408, 1.0),
}
# Mid-size M (a short prompt tail, more than 64 tree nodes): the model's up and down projections at
# 65 to 2048 rows. name: (seed, rows, K, N, sigma)
MID = {
    "up": (6, (65, 80, 96, 112, 128, 256, 512, 1024, 2048), 5120, 17408, 1.0),
    "down": (7, (65, 80, 96, 112, 128, 256, 512, 1024, 2048), 17408, 5120, 0.5),
}
# Every eligible linear of the target model (its seven (K, N) shapes) and its two vocabulary heads
# (lm_head 5120 -> 248320, the drafter's 5120 -> 65984) at the decode (1, 4) and tree-verify
# (16, 64, 96, 128) row counts. name: (seed, rows, K, N, sigma)
MODEL = {f"{k}->{n}": (10 + i, (1, 4, 16, 64, 96, 128), k, n, 0.5 if k > 6144 else 1.0)
         for i, (k, n) in enumerate([(5120, 17408), (17408, 5120), (5120, 10240), (5120, 6144), (6144, 5120),
                                     (5120, 12288), (5120, 1024), (5120, 248320), (5120, 65984)])}
# Shapes that reach the two fallback kernels (no shape of the target model does): the K-split verify
# kernel (5-16 rows over a small N with K too long for the row-phase split to fill half the CUs)
# and the stream-K skinny kernel (up to 4 rows where the row-split planner refuses: tiny K and N).
# name: (seed, rows, K, N, sigma)
FALLBACK = {
    "verify 17408->256": (20, (12, 16), 17408, 256, 0.5),
    "skinny 128->16": (21, (1, 4), 128, 16, 1.0),
    "skinny 256->48": (22, (3,), 256, 48, 1.0),
}
# One GPU's share of an 8-way split by output columns (the way the path would shard): the decode
# gate+up and the vocab head at N / 8 columns. name: (seed, rows, K, N / 8, sigma)
SHARD8 = {
    "c1/8": (1, (1, 2, 4), 5120, 34816 // 8, 1.0),
    "c3/8": (3, (32,), 5120, 151936 // 8, 1.0),
}
# The dominant kernel of the headline workload and the committed rocprofv3 summaries the roofline
# record reads (the traffic figure is used only if its summary names this kernel).
HEAD_KERNEL = "rowsplit_kernel<4, 4, false, false, false, false, 0, false>"
TRACE_PROFILE = "qmm4_bench_workloads_kernel_trace.txt"
TRAFFIC_PROFILE = "rowsplit_decode_gate_up_traffic.txt"
DESCR = {
    "c0": "tree-verify qmm: x bf16 [16, 5120] @ packed 4-bit [5120, 5120]",
    "c1": "decode gate+up: x bf16 [M=1,2,4, 5120] @ packed 4-bit [34816, 5120]",
    "c2": "batched verify down proj: x bf16 [64, 17408] @ packed 4-bit [5120, 17408]",
    "c3": "vocab head: x bf16 [32, 5120] @ packed 4-bit [151936, 5120]",
    "c4": "chunked prefill: x bf16 [4096, 5120] @ packed 4-bit [17408, 5120]",
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def bytes_per_call(m: int, k: int, n: int) -> int:
    return n * k // 2 + 2 * 2 * n * (k // 64) + 2 * m * k + 2 * m * n


def _bf16_rne(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (the inputs drawn here are finite)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def synthetic_inputs(m: int, k: int, n: int, sigma: float = 1.0, seed: int = 0):
    """The workloads' seeded synthetic inputs (numpy PCG64(seed), drawn in this order): x =
    bf16(N(0, 1) * sigma) [m, k]; packed words uniform over uint32 [n, k / 8] (every 4-bit code iid
    uniform 0..15); scales = bf16(|N(0, 1)| * 0.004 + 1e-4) and biases = bf16(-8 * scale +
    N(0, 1) * 1e-3), [n, k / 64] each. Returns bf16 bit arrays (uint16) and the words (uint32)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    x = _bf16_rne(rng.standard_normal((m, k), dtype=np.float32) * np.float32(sigma))
    w = rng.integers(0, 2**32, size=(n, k // 8), dtype=np.uint32)
    s = _bf16_rne(np.abs(rng.standard_normal((n, k // 64), dtype=np.float32)) * np.float32(0.004) + np.float32(1e-4))
    sf = (s.astype(np.uint32) << 16).view(np.float32)
    b = _bf16_rne(np.float32(-8.0) * sf + rng.standard_normal((n, k // 64), dtype=np.float32) * np.float32(1e-3))
    return x, w, s, b


class Workload:
    """Device-resident inputs of one benchmark workload with rotating weight copies."""

    def __init__(self, name: str, torch, lib, dev, spec=None):
        idx, rows, k, n, sigma = spec if spec is not None else WORKLOADS[name]
        self.name, self.rows, self.k, self.n = name, rows, k, n
        x, w, s, b = synthetic_inputs(max(rows), k, n, sigma=sigma, seed=idx)
        wbytes = n * k // 2 + 4 * n * (k // 64)
        # (at most 4096 copies: the fallback shapes' weights are a few kilobytes)
        self.copies = max(2, min(4096, int(np.ceil(ROTATE_BYTES / wbytes))))
        t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a).view(dt)).to(dev)
        w0, s0, b0 = t(w, np.int32), t(s, np.int16), t(b, np.int16)
        self.w = [w0] + [w0.clone() for _ in range(self.copies - 1)]
        self.s = [s0] + [s0.clone() for _ in range(self.copies - 1)]
        self.b = [b0] + [b0.clone() for _ in range(self.copies - 1)]
        self.x = t(x, np.int16)
        self.y = {m: torch.empty((m, n), dtype=torch.int16, device=dev) for m in rows}
        self.lib = lib
        self.torch = torch
        self.stream = torch.cuda.current_stream(dev).cuda_stream
        self.i = 0

    def launch(self, m: int, copy: int | None = None) -> None:
        c = self.i % self.copies if copy is None else copy
        self.i += 1
        rc = self.lib.qmm4_affine_bf16(self.x.data_ptr(), self.w[c].data_ptr(), self.s[c].data_ptr(),
                                       self.b[c].data_ptr(), self.y[m].data_ptr(), m, self.n, self.k, 64, 4, 1,
                                       self.stream)
        if rc != 0:
            raise RuntimeError(f"qmm4_affine_bf16 failed ({rc}): {self.lib.qmm4_last_error().decode()}")

    def step(self) -> None:
        for m in self.rows:
            self.launch(m)

    def warm(self, seconds: float = WARM_S) -> None:
        """Back-to-back calls at every row count for at least `seconds` of wall time, so that the
        GPU's clocks have ramped up again after the host built this workload's inputs (the first
        ~100 ms of work after an idle spell run at lower clocks)."""
        t0 = time.perf_counter()
        while True:
            for _ in range(8):
                self.step()
            self.torch.cuda.synchronize()
            if time.perf_counter() - t0 >= seconds:
                break

    def step_bytes(self) -> int:
        return sum(bytes_per_call(m, self.k, self.n) for m in self.rows)


def time_graph(torch, call, reps: int = 20, replays: int = 5) -> float:
    """Kernel time per call (s) without host dispatch: `reps` calls captured into a HIP graph,
    replayed `replays` times between one event pair. call(i, stream) enqueues call i on `stream`
    (it must not allocate: each op was called once before capture)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(3):
            call(i, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    # Captured on the warmed-up stream: the library's workspaces are per stream, and a call that
    # would need one to grow during capture is refused.
    with torch.cuda.graph(g, stream=side):
        st = torch.cuda.current_stream().cuda_stream
        for i in range(reps):
            call(i, st)
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / (replays * reps)


def measure_fused(torch, lib, dev, wl: Workload) -> dict:
    """The ops either side of the projection: the fused gate+up with its SiLU·mul epilogue on the c1
    weights (the gate and up projections stacked; decode rows, and 16- and 64-row verify batches:
    the row-split kernel's and the row-phase kernel's fused forms), and the
    residual add + RMS norm at the model
    width for decode (4 rows) and a prefill chunk (4096 rows). Timed as graph replays of 20
    back-to-back calls on rotating inputs (no host dispatch in the figure). HBM-bound; bytes are the
    algorithmic ones (weights, scales and biases, x, y; for the norm x, r, h, n and the weight row)."""
    out = {}
    n2 = wl.n // 2
    # Decode rows on the workload's x, and 16- and 64-row tree-verify batches.
    g16 = torch.Generator(device="cpu").manual_seed(16)
    xv = {r: torch.randn(r, wl.k, generator=g16).to(torch.bfloat16).to(dev) for r in (16, 64)}
    for m in (*wl.rows, 16, 64):
        y = torch.empty((m, n2), dtype=torch.int16, device=dev)
        xm = wl.x if m <= max(wl.rows) else xv[m]

        def call(i, stream, m=m, y=y, xm=xm):
            c = i % wl.copies
            rc = lib.qmm4_gate_up_silu_bf16(xm.data_ptr(), wl.w[c].data_ptr(), wl.s[c].data_ptr(),
                                            wl.b[c].data_ptr(), y.data_ptr(), m, wl.n, wl.k, 64, 4, 1, stream)
            if rc != 0:
                raise RuntimeError(f"qmm4_gate_up_silu_bf16 failed ({rc}): {lib.qmm4_last_error().decode()}")

        med = time_graph(torch, call)
        byt = wl.n * wl.k // 2 + 4 * wl.n * (wl.k // 64) + 2 * m * wl.k + 2 * m * n2
        out[f"gate_up_silu M={m}"] = {"us": round(med * 1e6, 2), "gbs": round(byt / med / 1e9, 1),
                                      "hbm_frac": round(byt / med / 1e9 / HBM_PEAK_GBS, 4), "bytes": byt}
        log(f"[bench]   gate_up_silu M={m}: {med * 1e6:8.2f} us  {byt / med / 1e9:7.1f} GB/s")
    d = wl.k
    g = torch.Generator(device="cpu").manual_seed(3)
    w = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(dev)
    for rows in (4, 4096):
        copies = max(2, int(np.ceil(ROTATE_BYTES / (8 * rows * d))))
        xs = [torch.randn(rows, d, generator=g).to(torch.bfloat16).to(dev) for _ in range(min(copies, 8))]
        rs = [torch.randn(rows, d, generator=g).to(torch.bfloat16).to(dev) for _ in range(len(xs))]
        h, nn = torch.empty_like(xs[0]), torch.empty_like(xs[0])

        def call(i, stream, rows=rows, xs=xs, rs=rs, h=h, nn=nn):
            c = i % len(xs)
            rc = lib.qmm4_add_rms_norm_bf16(xs[c].data_ptr(), rs[c].data_ptr(), w.data_ptr(), h.data_ptr(),
                                            nn.data_ptr(), rows, d, 1e-6, stream)
            if rc != 0:
                raise RuntimeError(f"qmm4_add_rms_norm_bf16 failed ({rc}): {lib.qmm4_last_error().decode()}")

        med = time_graph(torch, call)
        byt = 8 * rows * d + 2 * d
        out[f"add_rms_norm rows={rows} D={d}"] = {"us": round(med * 1e6, 2), "gbs": round(byt / med / 1e9, 1),
                                                  "hbm_frac": round(byt / med / 1e9 / HBM_PEAK_GBS, 4), "bytes": byt}
        log(f"[bench]   add_rms_norm {rows}x{d}: {med * 1e6:8.2f} us  {byt / med / 1e9:7.1f} GB/s")
    # The norm folded into the gate+up kernel (one launch) against the two calls it replaces
    # (add_rms_norm, then gate_up_silu on its n); the same bits either way.
    for m in wl.rows:
        xs = [torch.randn(m, d, generator=g).to(torch.bfloat16).to(dev) for _ in range(4)]
        rs = [torch.randn(m, d, generator=g).to(torch.bfloat16).to(dev) for _ in range(4)]
        h, nn = torch.empty_like(xs[0]), torch.empty_like(xs[0])
        y = torch.empty((m, n2), dtype=torch.int16, device=dev)

        def pair(i, stream, m=m, xs=xs, rs=rs, h=h, nn=nn, y=y):
            c, j = i % wl.copies, i % len(xs)
            rc = lib.qmm4_add_rms_norm_bf16(xs[j].data_ptr(), rs[j].data_ptr(), w.data_ptr(), h.data_ptr(),
                                            nn.data_ptr(), m, d, 1e-6, stream)
            rc = rc or lib.qmm4_gate_up_silu_bf16(nn.data_ptr(), wl.w[c].data_ptr(), wl.s[c].data_ptr(),
                                                  wl.b[c].data_ptr(), y.data_ptr(), m, wl.n, wl.k, 64, 4, 1, stream)
            if rc != 0:
                raise RuntimeError(f"add_rms_norm + gate_up_silu failed ({rc}): {lib.qmm4_last_error().decode()}")

        def fold(i, stream, m=m, xs=xs, rs=rs, h=h, nn=nn, y=y):
            c, j = i % wl.copies, i % len(xs)
            rc = lib.qmm4_add_rms_norm_qmm_bf16(xs[j].data_ptr(), rs[j].data_ptr(), w.data_ptr(), 1e-6, h.data_ptr(),
                                                nn.data_ptr(), wl.w[c].data_ptr(), wl.s[c].data_ptr(),
                                                wl.b[c].data_ptr(), y.data_ptr(), m, wl.n, wl.k, 64, 4, 1, 1, stream)
            if rc != 0:
                raise RuntimeError(f"qmm4_add_rms_norm_qmm_bf16 failed ({rc}): {lib.qmm4_last_error().decode()}")

        tp, tf = time_graph(torch, pair), time_graph(torch, fold)
        out[f"add_rms_norm+gate_up_silu M={m}"] = {"two_calls_us": round(tp * 1e6, 2), "folded_us": round(tf * 1e6, 2),
                                                   "saved_us": round((tp - tf) * 1e6, 2), "launches": "2 -> 1"}
        log(f"[bench]   add_rms_norm + gate_up_silu M={m}: two calls {tp * 1e6:8.2f} us  folded {tf * 1e6:8.2f} us")
    return out


def measure_layer_tail(torch, dev, rows_list=(4, 64), n_layers: int = 2, samples: int = 20) -> dict:
    """The MLP half of n_layers decoder layers at the model's sizes (D = 5120, H = 17408: the c1 gate+up
    and c2 down projection shapes), per forward: eager calls from Python against one replay of the
    same layers captured in a HIP graph. Random weights; the same layers for every sample. Up to 4
    rows a layer is 3 kernels (the norm folded into the gate+up, the down projection, the next
    norm); 16 rows (a tree-verify batch) run the norm, the gate+up with its epilogue fused, the
    down projection and its reduce, and the next norm; 64 rows run the norm, the gate+up
    projection, its SiLU·mul pass, the down projection and its reduce, and the next norm."""
    from mlx_tree_spec_amd import GraphedTail, MLPLayer, QuantizedLinear, QuantizedMLP, stack_tail

    d, h = 5120, 17408
    g = torch.Generator(device="cpu").manual_seed(11)

    def lin(n, k):
        w = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), generator=g, dtype=torch.int32)
        s = (torch.rand(n, k // 64, generator=g) * 0.004 + 1e-4).to(torch.bfloat16)
        b = (-8 * s.float() + 1e-3 * torch.randn(n, k // 64, generator=g)).to(torch.bfloat16)
        return QuantizedLinear.from_quantized(w.to(dev), s.to(dev), b.to(dev))

    def norm():
        m = torch.nn.RMSNorm(d, eps=1e-6, device=dev, dtype=torch.bfloat16)
        with torch.no_grad():
            m.weight.copy_((1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16))
        return m

    layers = [MLPLayer(norm(), QuantizedMLP(lin(h, d), lin(h, d), lin(d, h))) for _ in range(n_layers)]
    final = norm()
    out = {}
    for rows in rows_list:
        hs = (torch.randn(rows, d, generator=g)).to(torch.bfloat16).to(dev)
        rs = [(0.5 * torch.randn(rows, d, generator=g)).to(torch.bfloat16).to(dev) for _ in layers]
        for _ in range(3):
            stack_tail(hs, rs, layers, final)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(samples):
            stack_tail(hs, rs, layers, final)
        b.record()
        torch.cuda.synchronize()
        eager = a.elapsed_time(b) * 1e-3 / samples
        gt = GraphedTail(layers, final, rows, d, dev)
        gt(hs, rs)
        torch.cuda.synchronize()
        a.record()
        for _ in range(samples):
            gt.graph.replay()
        b.record()
        torch.cuda.synchronize()
        graphed = a.elapsed_time(b) * 1e-3 / samples
        out[f"rows={rows}"] = {"layers": n_layers, "eager_us": round(eager * 1e6, 1),
                               "graph_us": round(graphed * 1e6, 1)}
        log(f"[bench]   layer tail x{n_layers}, {rows} rows: eager {eager * 1e6:8.1f} us  graph {graphed * 1e6:8.1f} us")
        del gt
    return out


def measure_rows(torch, lib, dev, samples: int, table: dict, floors: dict | None = None) -> dict:
    """Per-call medians (HIP events per launch, rotating weight copies) of each shape of `table` at
    its row counts, with HBM and bf16-MFMA fractions of peak: the up and down projections at 65 to
    2048 rows (MID), every linear and head of the model at decode and verify rows (MODEL), the
    shapes that reach the fallback kernels (FALLBACK)."""
    out = {}
    for name, spec in table.items():
        wl = Workload(name, torch, lib, dev, spec=spec)
        wl.warm()
        for m in wl.rows:
            ts = time_launches(torch, wl, m, samples)
            med = statistics.median(ts)
            byt, fl = bytes_per_call(m, wl.k, wl.n), 2 * m * wl.n * wl.k
            hf, mf = byt / med / 1e9 / HBM_PEAK_GBS, fl / med / 1e12 / MFMA_BF16_PEAK_TFLOPS
            out[f"{name} M={m}"] = {"shape": f"{m}x{wl.k}->{wl.n}", "us": round(med * 1e6, 2),
                                    "hbm_frac": round(hf, 4), "mfma_frac": round(mf, 4),
                                    "max_frac": round(max(hf, mf), 4), "samples": len(ts)}
            if floors is not None:
                attach_floor(out[f"{name} M={m}"], byt, med * 1e6, floors, f"{floors['cus']}x1024")
            log(f"[bench]   {name} M={m}: {med * 1e6:8.2f} us  HBM {hf:.1%}  MFMA {mf:.1%}")
        del wl
        torch.cuda.empty_cache()
    return out


def measure_shard8(torch, lib, dev, samples: int) -> dict:
    """Per-call medians (HIP events per launch, rotating weight copies) of the decode gate+up and
    vocab head at one GPU's share of an 8-way column split, with HBM fractions of peak."""
    out = {}
    for name, spec in SHARD8.items():
        wl = Workload(name, torch, lib, dev, spec=spec)
        wl.warm()
        for m in wl.rows:
            ts = time_launches(torch, wl, m, samples)
            med = statistics.median(ts)
            byt = bytes_per_call(m, wl.k, wl.n)
            hf = byt / med / 1e9 / HBM_PEAK_GBS
            out[f"{name} M={m}"] = {"shape": f"{m}x{wl.k}->{wl.n}", "us": round(med * 1e6, 2),
                                    "gbs": round(byt / med / 1e9, 1), "hbm_frac": round(hf, 4),
                                    "samples": len(ts)}
            log(f"[bench]   {name} M={m}: {med * 1e6:8.2f} us  HBM {hf:.1%}")
        del wl
        torch.cuda.empty_cache()
    return out


def profile_figures() -> dict:
    """The committed rocprofv3 figures for the headline kernel: its average duration in the kernel
    trace of the default bench run, and its HBM bytes per launch from the counter passes (null
    when the summary is absent or names another kernel)."""
    out = {"trace_mean_us": None, "traffic": None, "traffic_kernel": None}
    tpath = os.path.join(ROOT, "profiles", TRACE_PROFILE)
    if os.path.exists(tpath):
        with open(tpath) as f:
            for ln in f:
                if ln.startswith(f"head_kernel_mean_us {HEAD_KERNEL}:"):
                    out["trace_mean_us"] = float(ln.rsplit(":", 1)[1])
    cpath = os.path.join(ROOT, "profiles", TRAFFIC_PROFILE)
    if os.path.exists(cpath):
        kernel, traffic = None, None
        with open(cpath) as f:
            for ln in f:
                if ln.startswith("Kernel:"):
                    kernel = ln.split(":", 1)[1].strip()
                if ln.startswith("hbm_bytes_per_launch:"):
                    traffic = int(float(ln.split(":", 1)[1]))
        out["traffic_kernel"] = kernel
        if kernel is not None and HEAD_KERNEL in kernel:
            out["traffic"] = traffic
    return out


def time_launches(torch, wl: Workload, m: int, samples: int) -> list[float]:
    """Per-launch kernel time (s) from HIP event pairs on the launch stream."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(samples)]
    for a, b in evs:
        a.record()
        wl.launch(m)
        b.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) * 1e-3 for a, b in evs]


def load_floor_lib():
    """libqmm4_floor.so (built beside libqmm4.so by build()): an empty kernel and a streaming read."""
    import ctypes

    from mlx_tree_spec_amd import build as kbuild

    lib = ctypes.CDLL(kbuild.FLOOR_PATH)
    lib.qmm4_floor_empty.restype = ctypes.c_int
    lib.qmm4_floor_empty.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.qmm4_floor_read.restype = ctypes.c_int
    lib.qmm4_floor_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    return lib


def measure_floors(torch, dev, samples: int = 30) -> dict:
    """What one GPU can do at best, timed the way the workloads are (HIP events per launch, after a
    warm-up): an empty kernel launched with the grids the quantized-matmul kernels use (one
    workgroup per CU of 1024 or 512 threads; four per CU), a 512 MiB device-to-device copy
    (torch's, read + write bytes: `hbm_ceiling_gbs`), and a 1 GiB streaming read by a plain kernel
    (16-byte loads, four in flight per thread: `hbm_read_ceiling_gbs`, the pattern of the weight
    streams). Each HBM-bound workload is then reported against `hbm_read_ceiling_gbs` and against
    a floor of one empty launch plus its bytes at that rate."""
    fl = load_floor_lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    cus = torch.cuda.get_device_properties(dev).multi_processor_count

    def event_times(fn, n):
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        for a, b in evs:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        return [a.elapsed_time(b) * 1e-3 for a, b in evs]

    def check(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed (hipError {rc})")

    out = {"cus": cus, "empty_launch_us": {}}
    for blocks, threads in ((cus, 1024), (cus, 512), (4 * cus, 256)):
        fn = lambda: check(fl.qmm4_floor_empty(blocks, threads, 0, stream), "empty launch")
        for _ in range(200):
            fn()
        med = statistics.median(event_times(fn, samples))
        out["empty_launch_us"][f"{blocks}x{threads}"] = round(med * 1e6, 2)
        log(f"[bench]   empty launch {blocks} x {threads}: {med * 1e6:6.2f} us")
    n = (512 << 20) // 4
    src = torch.empty(n, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    src.fill_(7)
    for _ in range(5):
        dst.copy_(src)
    med = statistics.median(event_times(lambda: dst.copy_(src), samples))
    out["hbm_ceiling_gbs"] = round(2 * src.numel() * 4 / med / 1e9, 1)
    out["copy"] = {"bytes": 2 * src.numel() * 4, "us": round(med * 1e6, 2), "what": "torch copy_ of 512 MiB, read + write"}
    log(f"[bench]   512 MiB device-to-device copy: {med * 1e6:8.1f} us  {out['hbm_ceiling_gbs']:7.1f} GB/s (read + write)")
    del src, dst
    rb = 1 << 30
    buf = torch.empty(rb // 4, dtype=torch.int32, device=dev)
    buf.fill_(3)
    blocks = 8 * cus
    sink = torch.zeros(blocks * 4, dtype=torch.int32, device=dev)
    fn = lambda: check(fl.qmm4_floor_read(buf.data_ptr(), rb, sink.data_ptr(), blocks, stream), "streaming read")
    for _ in range(5):
        fn()
    med = statistics.median(event_times(fn, samples))
    out["hbm_read_ceiling_gbs"] = round(rb / med / 1e9, 1)
    out["read"] = {"bytes": rb, "us": round(med * 1e6, 2), "workgroups": blocks,
                   "what": "plain kernel, 16-byte loads, 4 in flight per thread"}
    log(f"[bench]   1 GiB streaming read: {med * 1e6:8.1f} us  {out['hbm_read_ceiling_gbs']:7.1f} GB/s")
    del buf, sink
    torch.cuda.empty_cache()
    return out


def attach_floor(entry: dict, byt: int, us: float, floors: dict, empty_key: str) -> None:
    """Adds the workload's fraction of the measured read ceiling and its achievable floor (one empty
    launch of the kernel's grid plus its algorithmic bytes at the read ceiling)."""
    rc = floors["hbm_read_ceiling_gbs"]
    empty = floors["empty_launch_us"][empty_key]
    floor_us = empty + byt / (rc * 1e9) * 1e6
    entry["ceiling_frac"] = round(byt / (us * 1e-6) / 1e9 / rc, 4)
    entry["floor_us"] = round(floor_us, 2)
    entry["floor_frac"] = round(floor_us / us, 4)


def cpu_baseline(wl_rows, k, n, budget_s: float = 10.0) -> dict:
    from oracle import cpu
    from oracle import qmm4_oracle as O

    x, w, s, b = O.make_inputs(max(wl_rows), k, n, seed=1)
    threads = cpu.num_threads()
    cpu.qmm(x[:1], w, s, b)  # warm-up
    t0 = time.perf_counter()
    steps = 0
    while True:
        for m in wl_rows:
            cpu.qmm(x[:m], w, s, b)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or steps >= 5000:
            break
    total = steps * sum(bytes_per_call(m, k, n) for m in wl_rows)
    host = host_cpu_facts()
    return {"value": round(total / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{steps} decode steps (M=1,2,4 x 5120 -> 34816) in {el:.1f} s, {threads} OpenMP threads, "
                      f"oracle/qmm4_cpu.c (fp32 accumulation), CPU: {host['model']}",
            "ms_per_step": round(el / steps * 1e3, 2),
            "threads_used": threads, "host_cpus_visible": host["visible"], "host_logical_cpus": host["logical"],
            "host_physical_cores": host["physical"],
            "mlx_cpu": ("mlx importable but not timed" if importlib.util.find_spec("mlx") is not None
                        else "mx.quantized_matmul on mx.cpu: mlx is not installed on this host and cannot be "
                             "installed offline; unavailable")}


def host_cpu_facts() -> dict:
    """The host's CPU model, logical CPUs, CPUs this process may run on, and physical cores
    (distinct (physical id, core id) pairs of /proc/cpuinfo)."""
    model, cores, phys, core = "", set(), None, None
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                key, _, val = ln.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name" and not model:
                    model = val
                elif key == "physical id":
                    phys = val
                elif key == "core id":
                    core = val
                elif not key and phys is not None and core is not None:
                    cores.add((phys, core))
                    phys = core = None
            if phys is not None and core is not None:
                cores.add((phys, core))
    except OSError:
        pass
    return {"model": model, "logical": os.cpu_count(), "visible": len(os.sched_getaffinity(0)),
            "physical": len(cores) or None}


def profile_mode(torch, lib, dev, args) -> int:
    """Launches only, for counter collection: the workload's steps, then a copy of known size whose
    FETCH_SIZE / WRITE_SIZE calibrate the counters against bytes that are certainly moved once."""
    wl = Workload(args.profile, torch, lib, dev)
    for _ in range(args.steps):
        wl.step()
    torch.cuda.synchronize()
    n = (args.copy_mib << 20) // 4
    src = torch.empty(n, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    src.fill_(7)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] profile {args.profile}: {args.steps} steps of M={list(wl.rows)}, "
        f"5 copies of {args.copy_mib} MiB; done")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", default="c0,c1,c2,c3,c4", help="workloads to measure (c1 is the headline)")
    ap.add_argument("--samples", type=int, default=30, help="single-launch samples per workload")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-mid", action="store_true", help="skip the mid-size M rows")
    ap.add_argument("--no-model", action="store_true", help="skip the model's linears and heads")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--profile", default=None, metavar="WORKLOAD",
                    help="launch-only mode for rocprofv3: run WORKLOAD's steps --steps times, then a plain "
                         "device-to-device copy of --copy-mib MiB five times (counter calibration); no timing")
    ap.add_argument("--copy-mib", type=int, default=512)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        log("bench.py measures one GPU: there is no multi-GPU path (the kernel is per-GPU; the "
            "path would shard over output columns, which is not built). Run with --gpus 1.")
        return 2

    import torch

    from mlx_tree_spec_amd import _lib

    if not torch.cuda.is_available():
        log("no HIP device visible")
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _lib.load()
    if args.profile:
        return profile_mode(torch, lib, dev, args)
    only = [s.strip() for s in args.only.split(",") if s.strip()]
    if "c1" not in only:
        only = ["c1"] + only

    log("[bench] floors: empty launches, HBM copy and streaming-read ceilings")
    floors = measure_floors(torch, dev, args.samples)
    empty_key = f"{floors['cus']}x1024"

    out_workloads = {}
    head = None
    for name in only:
        log(f"[bench] {name}: {DESCR[name]}")
        wl = Workload(name, torch, lib, dev)
        wl.warm()
        res = {"descr": DESCR[name], "weight_copies": wl.copies, "per_m": {}}
        for m in wl.rows:
            ts = time_launches(torch, wl, m, args.samples)
            med = statistics.median(ts)
            byt = bytes_per_call(m, wl.k, wl.n)
            fl = 2 * m * wl.n * wl.k
            res["per_m"][str(m)] = {
                "us": round(med * 1e6, 2), "gbs": round(byt / med / 1e9, 1),
                "hbm_frac": round(byt / med / 1e9 / HBM_PEAK_GBS, 4),
                "tflops": round(fl / med / 1e12, 2), "mfma_frac": round(fl / med / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                "bytes": byt, "flops": fl, "samples": len(ts)}
            attach_floor(res["per_m"][str(m)], byt, med * 1e6, floors, empty_key)
            log(f"[bench]   M={m}: {med * 1e6:8.2f} us  {byt / med / 1e9:7.1f} GB/s  {fl / med / 1e12:7.1f} TFLOP/s"
                f"  (floor {res['per_m'][str(m)]['floor_us']:.2f} us)")
        out_workloads[name] = res
        if name == "c1":
            head = (wl, res)
        else:
            del wl
            torch.cuda.empty_cache()

    wl, res = head
    mid = {}
    if not args.no_mid:
        log("[bench] mid-size M: up and down projections at 65 to 2048 rows")
        mid = measure_rows(torch, lib, dev, args.samples, MID, floors)
    model = {}
    if not args.no_model:
        log("[bench] the model's linears and heads at decode and verify rows")
        model = measure_rows(torch, lib, dev, args.samples, MODEL, floors)
    fallback = {}
    if not args.no_model:
        log("[bench] the fallback kernels (shapes no model linear has)")
        fallback = measure_rows(torch, lib, dev, args.samples, FALLBACK, floors)
    log("[bench] one GPU's share of an 8-way column split")
    shard8 = measure_shard8(torch, lib, dev, args.samples)
    log("[bench] fused ops either side of the projection")
    fused = measure_fused(torch, lib, dev, wl)
    log("[bench] verify-forward layer tails (MLP half), eager and graph-captured")
    fused["layer_tail"] = measure_layer_tail(torch, dev, rows_list=(4, 16, 64))
    # Timed region: exactly K steps, synchronized on both sides.
    for _ in range(args.warmup):
        wl.step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        wl.step()
    end.record()
    torch.cuda.synchronize()
    total_s = start.elapsed_time(end) * 1e-3
    value = wl.step_bytes() * args.steps / total_s / 1e9

    # Second pass: per-launch durations of the dominant kernel (same steps, events per launch).
    durs, byts = [], []
    evs = []
    for _ in range(args.steps):
        for m in wl.rows:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            wl.launch(m)
            b.record()
            evs.append((a, b, m))
    torch.cuda.synchronize()
    for a, b, m in evs:
        durs.append(a.elapsed_time(b) * 1e-3)
        byts.append(bytes_per_call(m, wl.k, wl.n))
    achieved = sum(byts) / sum(durs) / 1e9
    # HBM bytes per launch of the dominant kernel, from the committed rocprofv3 FETCH_SIZE and
    # WRITE_SIZE passes (scaled by a copy of known size), and its trace duration.
    prof = profile_figures()
    mean_bytes = statistics.mean(byts)
    trace_frac = (round(mean_bytes / (prof["trace_mean_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                  if prof["trace_mean_us"] else None)

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(total_s / args.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "decode gate+up projection: x bf16 [M, 5120] for M = 1, 2, 4 batched requests @ "
                               "packed 4-bit affine [34816, 5120] (group 64, bf16 scales/biases), bf16 out; one step "
                               "= the three calls", "M": [1, 2, 4], "K": 5120, "N": 34816, "group_size": 64,
                   "weight_copies": wl.copies},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": prof["traffic"],
                     "frac_step": round(value / HBM_PEAK_GBS, 4),
                     "hbm_ceiling": floors["hbm_ceiling_gbs"], "hbm_read_ceiling": floors["hbm_read_ceiling_gbs"],
                     "frac_of_read_ceiling": round(achieved / floors["hbm_read_ceiling_gbs"], 4),
                     "kernel": f"qmm4::{HEAD_KERNEL} (rows <= 4, one workgroup per CU owning 136 weight rows)",
                     "mean_launch_us": round(statistics.mean(durs) * 1e6, 3),
                     "bytes_per_launch": round(mean_bytes),
                     "trace_mean_us": prof["trace_mean_us"], "frac_trace": trace_frac,
                     "event_overhead_us": (round(statistics.mean(durs) * 1e6 - prof["trace_mean_us"], 3)
                                           if prof["trace_mean_us"] else None),
                     "note": "achieved/frac: HIP events around each launch on the launch stream (they include "
                             "the dispatch); frac_step: the timed steps' value over the peak; "
                             "trace_mean_us/frac_trace: the kernel's average duration in the "
                             "committed rocprofv3 kernel trace of the default bench run; traffic: the committed "
                             "FETCH_SIZE/WRITE_SIZE passes, null unless they name this kernel; hbm_ceiling: a "
                             "512 MiB device-to-device copy in this run (read + write bytes); hbm_read_ceiling: "
                             "a plain streaming-read kernel over 1 GiB in this run"},
        "floors": floors,
        "workloads": out_workloads,
        "mid_m": mid,
        "model_linears": model,
        "fallback_kernels": fallback,
        "shard8": shard8,
        "fused": fused,
    }
    if not args.no_cpu:
        log("[bench] cpu baseline")
        line["cpu_baseline"] = cpu_baseline(wl.rows, wl.k, wl.n, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
