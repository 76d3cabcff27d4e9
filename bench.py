"""Benchmark of the gfx950 small/irregular-shape GEMM path (one JSON line).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2]
                    [--detail FILE] [--no-cpu]

A step is one pass of the hot path over one batch of synthetic input.  The
headline workload is config C2 (the configuration the headline metric is
quoted on): fp32 C = A B + C for M in {2,3,5,7} x N in {1009,4099,11003},
K = 2048, alpha = beta = 1, A, B ~ N(0, 0.02), C ~ U[-1, 1).  One step runs
all twelve shapes once; its rate is `value`.  The default run also times the
other configs -- C1, C3, C4 through the bf16-storage entry and through the
fp32-input gemm_bf16 (c4f), C5, and C5's shapes through the fp32-API
gemm_int8 (c5f) -- each as its own workload, and reports every timed
workload's step rate, dominant kernel and per-shape GB/s, TFLOP/s and
roofline fractions under `configs` (C2's own per-shape figures included).  `--workload NAME` times one workload (its rate
becomes `value`); `--workload all` adds the oneDNN-hook workload;
`--detail FILE` appends the full per-workload records.  `--yardstick` instead
times the vendor library (torch.mm / torch._int_mm, hipBLASLt or rocBLAS)
beside this library on the configs' shapes (`--yardstick dnn`: on DNN
inference shapes, BERT and ResNet-50 GEMMs), one JSON line per shape.

`value` is the algorithmic bytes of a step (sA*M*K + sB*K*N + sC*M*N*(1 +
[beta != 0]), each operand counted once) divided by the wall time of the
timed steps, measured with HIP events on the stream the kernels run on.
Operands are resident in HBM before timing starts; every buffer of a step is
touched once per step and a step's working set exceeds the 256 MB Infinity
Cache (extra copies are rotated when it would not), so nothing is served from
the cache between two launches of the same shape.

Timing uses HIP graphs on one stream: the K timed steps are recorded as one
graph and replayed once between the two events, so host-side launch cost
does not enter (a step of one small GEMM is shorter than a graph launch).  `roofline` is for the kernel with the
largest share of the step time: achieved = its algorithmic bytes (or flops)
per launch / its mean launch time, from HIP events around replays of a graph
of 16 back-to-back launches of each shape (inter-kernel gaps included).  `traffic` is filled from
profiles/<kernel>_<workload>_traffic.json when a rocprofv3 --pmc summary has
been committed for it.

`cpu_baseline` times the oracle's restatement of the reference's CPU path
(oracle/liboracle.so) on the host, on the workload's shapes of at most 2^30
multiply-adds, each once per run (2 warmup runs, 5 timed runs, median -- the
reference's dnnopt::benchmark method -- fewer when a run is long).  `cpu_reference` times the reference's literal
portable fallback (its naive loops, built from its own sources into
oracle/_ref) on a bounded sample, when that build is present.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
PEAKS_TFLOPS = {"f32": 157.3, "bf16": 2500.0, "s8": 5000.0}
METRIC = "GB/s (% HBM peak) at M=1-7; TFLOPS (% MFMA peak) tall-skinny"
SEED = 42


def _binding():
    import importlib.util

    spec = importlib.util.spec_from_file_location("dnnopt_hip", os.path.join(ROOT, "dnn-opt_amd", "python",
                                                                             "dnnopt_hip.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


# ---------------------------------------------------------------- workloads
class Case:
    def __init__(self, name, kind, M, N, K, alpha=1.0, beta=0.0, ta=0, init=None, dtype="f32"):
        self.name, self.kind = name, kind
        self.M, self.N, self.K = M, N, K
        self.alpha, self.beta, self.ta = alpha, beta, ta
        self.init = init or {}
        self.dtype = dtype

    def sizes(self):
        sa, sb = {"f32": (4, 4), "bf16": (2, 2), "f2b": (4, 4), "s8": (1, 1), "s8s": (1, 1), "hf32": (4, 4),
                  "hbf16": (2, 2), "i8f": (4, 4)}[self.kind]
        sc = 4
        # per-column scale (int8) or bias (hook) vector
        extra = 4 * self.N if self.kind == "s8s" or (self.kind == "hf32" and self.init.get("bias")) else 0
        return sa, sb, sc, extra

    def bytes_alg(self):
        sa, sb, sc, extra = self.sizes()
        M, N, K = self.M, self.N, self.K
        return sa * M * K + sb * K * N + sc * M * N * (1 + (1 if self.beta != 0.0 else 0)) + extra

    def flops_alg(self):
        return 2.0 * self.M * self.N * self.K


def workload(name):
    if name == "c1":
        return ("C1: fp32 M=1 N=4096 K=4096, alpha=1 beta=0, A,B ~ U[-1,1)",
                [Case("c1", "f32", 1, 4096, 4096, init={"A": ("u", -1, 1), "B": ("u", -1, 1)})])
    if name == "c2":
        cs = []
        for M in (2, 3, 5, 7):
            for N in (1009, 4099, 11003):
                cs.append(Case(f"c2_m{M}_n{N}", "f32", M, N, 2048, 1.0, 1.0,
                               init={"A": ("n", 0, 0.02), "B": ("n", 0, 0.02), "C": ("u", -1, 1)}))
        return ("C2: fp32 M in {2,3,5,7} x N in {1009,4099,11003} x K=2048, alpha=1 beta=1, "
                "A,B ~ N(0,0.02), C ~ U[-1,1), row-major", cs)
    if name == "c3":
        u = {"A": ("u", -1, 1), "B": ("u", -1, 1)}
        return ("C3: fp32 tall-skinny 65536x{16,64}x256 and 64x64x262144 (A stored KxM), beta=0", [
            Case("c3_n16", "f32", 65536, 16, 256, init=u), Case("c3_n64", "f32", 65536, 64, 256, init=u),
            Case("c3_splitk_tn", "f32", 64, 64, 262144, ta=1, init=u)])
    if name == "c4":
        return ("C4: bf16 storage, fp32 accumulate/output, M in {1,4,32,256} x N=11008 x K=4096, "
                "weights ~ N(0,0.02), activations ~ N(0,1)", [
                    Case(f"c4_m{M}", "bf16", M, 11008, 4096, init={"A": ("n", 0, 1), "B": ("n", 0, 0.02)},
                         dtype="bf16") for M in (1, 4, 32, 256)])
    if name == "c4f":
        # the same shapes through the fp32-input gemm_bf16 (operands stored
        # fp32, rounded to bf16 in registers; src/gemm/gemm.cpp:379-416)
        return ("C4 via fp32-input gemm_bf16: fp32 storage rounded to bf16, fp32 accumulate/output, "
                "M in {1,4,32,256} x N=11008 x K=4096, weights ~ N(0,0.02), activations ~ N(0,1)", [
                    Case(f"c4f_m{M}", "f2b", M, 11008, 4096, init={"A": ("n", 0, 1), "B": ("n", 0, 0.02)},
                         dtype="bf16") for M in (1, 4, 32, 256)])
    if name == "c5":
        cs = []
        for M in (1, 8, 128):
            for N in (4096, 4093):
                cs.append(Case(f"c5_m{M}_n{N}", "s8", M, N, 4096, init={"A": ("i",), "B": ("i",)}, dtype="s8"))
        cs.append(Case("c5_m128_n4093_scale", "s8s", 128, 4093, 4096, init={"A": ("i",), "B": ("i",)}, dtype="s8"))
        return ("C5: int8 s8 x s8 -> s32 (B as N x K), M in {1,8,128} x N in {4096,4093} x K=4096; "
                "+ per-column fp32 scale", cs)
    if name == "c5f":
        # fp32-API gemm_int8 at C5's shapes: dynamic per-tensor quantization
        # of both fp32 operands, exact int8 GEMM, dequantized fp32 C
        # (src/gemm/gemm.cpp:418-455)
        cs = [Case(f"c5f_m{M}_n4096", "i8f", M, 4096, 4096, init={"A": ("u", -1, 1), "B": ("n", 0, 0.02)},
                   dtype="s8") for M in (1, 8, 128)]
        return ("C5 via the fp32-API gemm_int8: fp32 A, B quantized per tensor to int8, exact int32 "
                "accumulation, fp32 C, M in {1,8,128} x N=4096 x K=4096", cs)
    if name == "hook":
        # oneDNN inner product through the column-major hook: extended_sgemm
        # ('T', 'N', OC, MB, IC, W, IC, X, IC, dst, OC, bias).  The case's
        # M, N, K are the row-major view: M = MB, N = OC, K = IC; B = W is
        # stored N x K (weights as PyTorch/oneDNN keep them).
        f = {"A": ("n", 0, 1), "B": ("n", 0, 0.02), "bias": True}
        cs = [Case("hook_f32_mb1_oc4096_ic4096", "hf32", 1, 4096, 4096, init=f),
              Case("hook_f32_mb7_oc11003_ic2048", "hf32", 7, 11003, 2048, init=f)]
        cs += [Case(f"hook_bf16_mb{mb}_oc11008_ic4096", "hbf16", mb, 11008, 4096,
                    init={"A": ("n", 0, 1), "B": ("n", 0, 0.02)}, dtype="bf16") for mb in (1, 32, 256)]
        return ("oneDNN hook: column-major extended_sgemm / gemm_bf16bf16f32 ('T','N', M=OC, N=MB, K=IC), "
                "weights OC x IC, fp32 with bias, beta=0", cs)
    raise SystemExit(f"unknown workload {name}")


# ---------------------------------------------------------------- GPU side
class Buffers:
    def __init__(self, torch, lib, case, copies, dev):
        self.case = case
        M, N, K = case.M, case.N, case.K
        tA = {"f32": torch.float32, "f2b": torch.float32, "bf16": torch.int16, "s8": torch.int8,
              "s8s": torch.int8, "hf32": torch.float32, "hbf16": torch.int16, "i8f": torch.float32}[case.kind]
        dt_code = {torch.float32: 0, torch.int16: 1, torch.int8: 2}[tA]
        a_elems = M * K
        b_elems = K * N
        self.A, self.B, self.C, self.S = [], [], [], []
        for r in range(copies):
            A = torch.empty(a_elems, dtype=tA, device=dev)
            B = torch.empty(b_elems, dtype=tA, device=dev)
            cdt = torch.int32 if case.kind == "s8" else torch.float32
            C = torch.empty(M * N, dtype=cdt, device=dev)
            for t, key, tid in ((A, "A", 1), (B, "B", 2)):
                spec = case.init.get(key, ("u", -1, 1))
                if spec[0] == "i":
                    lib.fill(t, t.numel(), 2, 2, SEED + r, tid, -127, 127)
                else:
                    lib.fill(t, t.numel(), dt_code, 0 if spec[0] == "u" else 1, SEED + r, tid, spec[1], spec[2])
            if case.kind != "s8":
                spec = case.init.get("C", ("u", -1, 1))
                lib.fill(C, C.numel(), 0, 0, SEED + r, 3, spec[1], spec[2])
            self.A.append(A)
            self.B.append(B)
            self.C.append(C)
            if case.kind == "s8s" or (case.kind == "hf32" and case.init.get("bias")):
                S = torch.empty(N, dtype=torch.float32, device=dev)
                lo, hi = (0.001, 0.01) if case.kind == "s8s" else (-1.0, 1.0)
                lib.fill(S, N, 0, 0, SEED + r, 4, lo, hi)
                self.S.append(S)

    def launch(self, lib, r, stream):
        c = self.case
        M, N, K = c.M, c.N, c.K
        A, B, C = self.A[r], self.B[r], self.C[r]
        if c.kind == "f32":
            lda = M if c.ta else K
            lib.sgemm(M, N, K, c.alpha, A, lda, B, N, c.beta, C, N, transA=c.ta, stream=stream)
        elif c.kind == "bf16":
            lib.gemm_bf16(M, N, K, c.alpha, A, K, B, N, c.beta, C, N, stream=stream)
        elif c.kind == "f2b":
            lib.gemm_bf16_f32in(M, N, K, c.alpha, A, K, B, N, c.beta, C, N, stream=stream)
        elif c.kind == "s8":
            lib.gemm_s8s8s32(M, N, K, A, K, B, K, C, N, stream=stream)
        elif c.kind == "i8f":
            lib.gemm_int8_f32(M, N, K, c.alpha, A, K, B, N, c.beta, C, N, stream=stream)
        elif c.kind == "hf32":
            lib.ext_sgemm("T", "N", N, M, K, c.alpha, B, K, A, K, c.beta, C, N,
                          bias=self.S[r] if self.S else None, stream=stream)
        elif c.kind == "hbf16":
            lib.ext_gemm_bf16bf16f32("T", "N", N, M, K, c.alpha, B, K, A, K, c.beta, C, N, stream=stream)
        else:
            lib.gemm_s8s8f32_colscale(M, N, K, A, K, B, K, self.S[r], C, N, stream=stream)


def kernel_key(lib, case):
    """Kernel template instance as rocprof names it (family<params>)."""
    if case.kind in ("f32",):
        p = lib.plan_sgemm(case.M, case.N, case.K, transA=case.ta)
    elif case.kind == "hf32":
        p = lib.plan_sgemm(case.M, case.N, case.K, transB=1)
    elif case.kind == "hbf16":
        p = lib.plan_bf16_ex(case.M, case.N, case.K, transB=1)
    elif case.kind in ("bf16", "f2b"):
        p = lib.plan_bf16(case.M, case.N, case.K, fp32_inputs=int(case.kind == "f2b"))
    elif case.kind == "i8f":
        p = lib.plan_int8_f32(case.M, case.N, case.K)
        if p["name"] == "dnnopt_skinny_q8":
            return f"dnnopt_skinny_q8<{case.M}>", p
        if p["name"] == "dnnopt_s8_lds_q8b":
            return "dnnopt_s8_lds<2, 1, 2, 2, 3, 1, 128, 1>", p
    else:
        p = lib.plan_s8(case.M, case.N, case.K, with_scale=int(case.kind == "s8s"))
    if p["name"] == "dnnopt_skinny":
        mode = {"f32": 0, "bf16": 1, "f2b": 2, "hf32": 0, "hbf16": 1}[case.kind]
        return f"dnnopt_skinny<{case.M}, {p['block'] // 64}, {mode}>", p
    return f"{p['name']}[{p['rows']}x{p['cols']}]", p


def run_gpu(args, wl_name):
    """Time the workload with HIP graphs replayed on one stream.

    Host-side launch cost (Python, ctypes, planning) would otherwise dominate
    kernels of a few microseconds; a captured graph replays a whole step with
    one host call.  The library's workspace for the stream is created by a
    warm-up pass on that same stream before capture.
    """
    import torch

    b = _binding()
    lib = b.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    desc, cases = workload(wl_name)
    if args.cases:
        keep = set(args.cases.split(","))
        cases = [c for c in cases if c.name in keep]
        if not cases:
            raise SystemExit(f"bench.py: no case of {wl_name} is named in --cases {args.cases}")
    step_bytes = sum(c.bytes_alg() for c in cases)
    # Rotate copies so that one pass over the buffers a graph touches exceeds
    # 2x the 256 MB Infinity Cache: the step graphs rotate `copies` copies of
    # every case, the per-case graphs rotate that case's own copies, so each
    # case gets enough copies for its own rotation to exceed 600 MB as well.
    copies = max(1, -(-(600 << 20) // step_bytes))
    case_copies = [max(copies, -(-(600 << 20) // c.bytes_alg())) for c in cases]
    bufs = [Buffers(torch, lib, c, cc, dev) for c, cc in zip(cases, case_copies)]
    keys = [kernel_key(lib, c) for c in cases]
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=dev)  # default priority
    sp = stream.cuda_stream

    with torch.cuda.stream(stream):
        for w in range(max(1, args.warmup)):
            for bf in bufs:
                bf.launch(lib, w % copies, sp)
    torch.cuda.synchronize()

    def capture(launches):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for fn in launches:
                fn()
        return g

    # one graph per buffer copy: a full step
    step_graphs = [capture([lambda bf=bf, r=r: bf.launch(lib, r, sp) for bf in bufs]) for r in range(copies)]
    # one graph per case: back-to-back launches over all of the case's copies
    # (at least 16 launches)
    reps = [max(16, cc) for cc in case_copies]
    case_graphs = [capture([lambda bf=bf, i=i, cc=cc: bf.launch(lib, i % cc, sp) for i in range(rp)])
                   for bf, cc, rp in zip(bufs, case_copies, reps)]
    torch.cuda.synchronize()

    with torch.cuda.stream(stream):
        for w in range(args.warmup):
            step_graphs[w % copies].replay()
    torch.cuda.synchronize()

    # The K timed steps are recorded as one graph: a step of a small workload
    # (C1 is one GEMM, ~17 us of GPU work) is shorter than the host's cost of
    # launching a graph, so replaying one graph per step would time the host.
    # The graph's first launch is inside the timed region (it can only add).
    timed_graph = capture([lambda bf=bf, r=(args.warmup + st) % copies: bf.launch(lib, r, sp)
                           for st in range(args.steps) for bf in bufs])
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        t0.record(stream)
        timed_graph.replay()
        t1.record(stream)
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    ms_per_step = total_ms / args.steps

    # per-case kernel time: events around graph replays on the launch stream
    reps_timed = max(3, min(args.steps, 10))
    per_case, launch_ms = [], []
    for i, c in enumerate(cases):
        samples = []
        with torch.cuda.stream(stream):
            case_graphs[i].replay()
            for _ in range(reps_timed):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                case_graphs[i].replay()
                e1.record(stream)
                samples.append((e0, e1))
        torch.cuda.synchronize()
        d = [a.elapsed_time(bb) / reps[i] for a, bb in samples]
        med = statistics.median(d)
        launch_ms.append(sum(d) / len(d))
        t_hbm = c.bytes_alg() / (HBM_PEAK_GBS * 1e9)
        t_mfma = c.flops_alg() / (PEAKS_TFLOPS.get(c.dtype, 157.3) * 1e12)
        per_case.append({
            "case": c.name, "M": c.M, "N": c.N, "K": c.K, "kernel": keys[i][0], "plan": keys[i][1],
            "us_median": med * 1e3, "us_mean": launch_ms[-1] * 1e3,
            "GBps": c.bytes_alg() / (med * 1e-3) / 1e9, "TFLOPs": c.flops_alg() / (med * 1e-3) / 1e12,
            "bound": "hbm" if t_hbm >= t_mfma else "mfma",
            "roofline_frac": max(t_hbm, t_mfma) / (med * 1e-3),
        })
    # dominant kernel instance: largest share of the per-launch time
    groups = {}
    for i, c in enumerate(cases):
        g = groups.setdefault(keys[i][0], {"ms": 0.0, "bytes": 0.0, "flops": 0.0, "launches": 0,
                                           "dtype": c.dtype})
        g["ms"] += launch_ms[i]
        g["bytes"] += c.bytes_alg()
        g["flops"] += c.flops_alg()
        g["launches"] += 1
    dom_key, dom = max(groups.items(), key=lambda kv: kv[1]["ms"])
    mean_s = dom["ms"] / dom["launches"] * 1e-3
    bytes_per = dom["bytes"] / dom["launches"]
    flops_per = dom["flops"] / dom["launches"]
    # bound: HBM unless the shape's arithmetic intensity exceeds the ridge
    ai = flops_per / bytes_per
    peak_t = PEAKS_TFLOPS.get(dom["dtype"], 157.3)
    ridge = peak_t * 1e12 / (HBM_PEAK_GBS * 1e9)
    if ai > ridge:
        achieved = flops_per / mean_s / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 3), "peak": peak_t, "unit": "TFLOP/s",
                "frac": round(achieved / peak_t, 4)}
    else:
        achieved = bytes_per / mean_s / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4)}
    roof["kernel"] = dom_key
    roof["launch_us"] = round(mean_s * 1e6, 3)
    roof["bytes_per_launch"] = int(bytes_per)
    roof["traffic"] = read_traffic(dom_key, wl_name)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    return {
        "desc": desc, "value": value, "ms_per_step": ms_per_step, "step_bytes": step_bytes,
        "step_flops": sum(c.flops_alg() for c in cases), "copies": copies, "roofline": roof,
        "per_case": per_case, "cases": cases,
    }


def _traffic_file_stem(kernel):
    return kernel.replace("<", "_").replace(">", "").replace(", ", "_").replace("[", "_").replace("]", "")


def read_traffic(kernel, wl):
    path = os.path.join(ROOT, "profiles", f"{_traffic_file_stem(kernel)}_{wl}_traffic.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


# ---------------------------------------------------------------- CPU baseline
def cpu_reference(cases, budget_s=10.0):
    """Time the reference's literal portable fallback on the host: its own
    naive loops (src/gemm/gemm.cpp:88-100 for fp32, the scalar loop of
    src/gemm/gemm_int8_native.cpp:239-247 for int8), compiled from the
    reference sources into oracle/_ref/libref.so.  None when that build is
    absent.  Single-threaded, as the loops are."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import _util as u

    ref = u.load_ref()
    if ref is None:
        return None
    orc = u.load_oracle()
    prepared = []
    for c in cases:
        M, N, K = c.M, c.N, c.K
        if c.kind == "f32":
            A, B, C = u.uniform(orc, M * K, 1), u.uniform(orc, K * N, 2), u.uniform(orc, M * N, 3)

            def run(A=A, B=B, C=C, c=c):
                ref.ref_gemm_naive_f32(c.M, c.N, c.K, c.alpha, u.ptr(A), c.K, u.ptr(B), c.N, c.beta, u.ptr(C), c.N)
        elif c.kind in ("s8", "s8s"):
            A, B = u.ints8(orc, M * K, 1), u.ints8(orc, N * K, 2)
            C = np.empty(M * N, np.int32)

            def run(A=A, B=B, C=C, c=c):
                ref.ref_gemm_s8s8s32(c.M, c.N, c.K, u.ptr(A), c.K, u.ptr(B), c.K, u.ptr(C), c.N)
        else:
            continue
        prepared.append((c, run))
    if not prepared:
        return None
    # bounded sample: whole passes over the shapes while they fit the budget,
    # else the first shapes that fit
    times, used = [], []
    t_all = time.perf_counter()
    for c, run in prepared:
        t = time.perf_counter()
        run()
        times.append(time.perf_counter() - t)
        used.append(c)
        if time.perf_counter() - t_all > budget_s:
            break
    total_bytes = sum(c.bytes_alg() for c in used)
    med = sum(times)
    return {
        "value": round(total_bytes / med / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "reference",
        "sample": (f"{len(used)} of {len(prepared)} shapes of the workload once ({total_bytes / 1e6:.0f} MB "
                   f"algorithmic, {med:.1f} s): the reference's own naive loops built from its sources "
                   f"(oracle/_ref), single-threaded"),
    }


def cpu_baseline(cases, budget_s=20.0):
    """Time the oracle's restatement of the reference CPU path on the host."""
    import ctypes

    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import _util as u

    orc = u.load_oracle()
    nthreads = os.cpu_count() or 1
    os.environ.setdefault("OMP_NUM_THREADS", str(nthreads))
    kMaxMacs = 1 << 30  # larger M > 8 shapes are left out of the sample
    prepared = []
    for c in cases:
        M, N, K = c.M, c.N, c.K
        if c.kind == "f32" and c.M <= 8:
            A = (u.normal if c.init["A"][0] == "n" else u.uniform)(orc, M * K, 1, *c.init["A"][1:])
            B = (u.normal if c.init["B"][0] == "n" else u.uniform)(orc, K * N, 2, *c.init["B"][1:])
            C = u.uniform(orc, M * N, 3)

            def run(A=A, B=B, C=C, c=c):
                cc = C.copy()
                rc = orc.orc_gemm_f32_smallm(c.M, c.N, c.K, c.alpha, u.ptr(A), c.K, u.ptr(B), c.N, c.beta,
                                             u.ptr(cc), c.N, nthreads)
                if rc != 0:
                    raise RuntimeError("shape outside the restated small-M path")
        elif c.kind in ("s8", "s8s"):
            A, B = u.ints8(orc, M * K, 1), u.ints8(orc, N * K, 2)
            C = np.empty(M * N, np.int32)

            def run(A=A, B=B, C=C, c=c):
                orc.orc_gemm_s8s8s32(c.M, c.N, c.K, u.ptr(A), c.K, u.ptr(B), c.K, u.ptr(C), c.N)
        elif c.kind == "bf16" and (c.M <= 8 or M * N * K <= kMaxMacs):
            A = u.bf16_bits(orc, u.normal(orc, M * K, 1))
            B = u.bf16_bits(orc, u.normal(orc, K * N, 2, 0, 0.02))
            C = np.zeros(M * N, np.float32)

            def run(A=A, B=B, C=C, c=c):
                orc.orc_gemm_bf16(c.M, c.N, c.K, 1.0, u.ptr(A), c.K, u.ptr(B), c.N, 0.0, u.ptr(C), c.N)
        elif c.kind == "f32" and M * N * K <= kMaxMacs:
            # M > 8 fp32 (tall-skinny, TransA): the restated cblas row-major path
            A = u.uniform(orc, M * K, 1)
            B = u.uniform(orc, K * N, 2)
            C = np.zeros(M * N, np.float32)

            def run(A=A, B=B, C=C, c=c):
                orc.orc_cblas_sgemm(101, 112 if c.ta else 111, 111, c.M, c.N, c.K, c.alpha, u.ptr(A),
                                    c.M if c.ta else c.K, u.ptr(B), c.N, c.beta, u.ptr(C), c.N)
        else:
            continue
        prepared.append((c, run))
    if not prepared:
        return None
    # bounded sample: scale repetitions to the budget
    t = time.perf_counter()
    for _, run in prepared:
        run()
    one = time.perf_counter() - t
    runs = []
    total_bytes = sum(c.bytes_alg() for c, _ in prepared)
    warm = one * 3 < budget_s
    if not warm:
        # a long pass (seconds of scalar loops) is its own sample
        reps, runs = 1, [one]
    else:
        reps = 5 if one * 7 < budget_s else max(1, int(budget_s / max(one, 1e-9)) - 2)
        for _ in range(min(2, reps)):
            for _, run in prepared:
                run()
        for _ in range(reps):
            t = time.perf_counter()
            for _, run in prepared:
                run()
            runs.append(time.perf_counter() - t)
    med = statistics.median(runs)
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    del ctypes
    threaded = any(c.kind == "f32" and c.M in (5, 7) and c.N * c.K > 4 * 1024 * 1024 for c, _ in prepared)
    return {
        "value": round(total_bytes / med / 1e9, 3), "unit": "GB/s",
        "cores": nthreads if threaded else 1, "kind": "port",
        "sample": (f"{len(prepared)} of {len(cases)} shapes of the workload once ({total_bytes / 1e6:.0f} MB "
                   f"algorithmic; shapes above 2^30 multiply-adds left out), median of {reps} runs"
                   f"{' after warmup' if warm else ''}; "
                   f"oracle restatement of the reference CPU path (GEMV / wide driver single-threaded, adaptive "
                   f"tiles on {nthreads} OpenMP threads, other shapes its single-threaded row-major loops); "
                   f"host CPU: {cpu_model}"),
    }


def _short_kernel_name(name):
    """'void dnnopt_hip::dnnopt_skinny<7, 8, 0, 1, 0>(dnnopt_hip::SkinnyArgs)' -> 'dnnopt_skinny<7, 8, 0, 1, 0>'."""
    name = name.strip().replace("(anonymous namespace)::", "")
    if name.startswith("void "):
        name = name[5:]
    depth, cut = 0, len(name)
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            cut = i
            break
    return name[:cut].replace("dnnopt_hip::", "")


def rocprof_summary(kernel, workload, trace_csv, pmc=None):
    """Summarise rocprofv3 CSV output for one kernel instance.

    trace_csv: *_kernel_trace.csv of `rocprofv3 --kernel-trace --stats -f csv`.
    pmc: optional (fetch_csv, write_csv, copy_fetch_csv, copy_write_csv) from
    `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE` runs of the same command
    and of `bench.py --copy-calibration`.  Each launch of `kernel` (a name
    prefix, e.g. 'dnnopt_skinny<7, 8, 0') is counted together with a reduce
    kernel dispatched right after it.  Returns (text, traffic dict or None).
    """
    import csv

    def rows(path):
        with open(path, newline="") as f:
            return list(csv.DictReader(f))

    lines = []
    tr = rows(trace_csv)
    tr.sort(key=lambda r: int(r["Start_Timestamp"]))
    groups = {}
    for r in tr:
        nm = _short_kernel_name(r["Kernel_Name"])
        key = (nm, int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"])), int(r["Grid_Size_Y"]),
               int(r["Grid_Size_Z"]), int(r["Workgroup_Size_X"]))
        groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    lines.append(f"{'kernel':<44} {'grid (workgroups x,y,z)':>24} {'block':>5} {'calls':>6} {'avg_us':>8} "
                 f"{'min_us':>8} {'max_us':>8}")
    for (nm, gx, gy, gz, bs), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"{nm:<44} {f'{gx},{gy},{gz}':>24} {bs:>5} {len(d):>6} {sum(d) / len(d):8.2f} {min(d):8.2f} "
                     f"{max(d):8.2f}")
    dom = [sum(d) / len(d) for (nm, *_), d in groups.items() if nm.startswith(kernel)]
    traffic = None
    if pmc:
        fetch_csv, write_csv, cfetch_csv, cwrite_csv = pmc

        def per_launch(path):
            rr = rows(path)
            rr.sort(key=lambda r: int(r["Dispatch_Id"]))
            vals = []
            for i, r in enumerate(rr):
                if _short_kernel_name(r["Kernel_Name"]).startswith(kernel):
                    v = float(r["Counter_Value"])
                    if i + 1 < len(rr) and "reduce" in rr[i + 1]["Kernel_Name"]:
                        v += float(rr[i + 1]["Counter_Value"])
                    vals.append(v)
            return sum(vals) / len(vals) if vals else None, len(vals)

        def calib(path):
            rr = [r for r in rows(path) if "copy" in r["Kernel_Name"].lower()]
            return sum(float(r["Counter_Value"]) for r in rr) / len(rr) if rr else None

        fk, nf = per_launch(fetch_csv)
        wk, nw = per_launch(write_csv)
        copy_kib = (1 << 30) / 1024.0  # bench.py --copy-calibration 1024
        cf, cw = calib(cfetch_csv), calib(cwrite_csv)
        if fk is not None and wk is not None and cf and cw:
            fs, ws = copy_kib / cf, copy_kib / cw
            traffic = {
                "kernel": kernel, "workload": workload, "launches_fetch": nf, "launches_write": nw,
                "fetch_kib_per_launch": round(fk, 1), "write_kib_per_launch": round(wk, 1),
                "copy_1gib_fetch_kib": round(cf, 1), "copy_1gib_write_kib": round(cw, 1),
                "fetch_scale": round(fs, 4), "write_scale": round(ws, 4),
                "traffic_bytes_per_launch": int(round((fk * fs + wk * ws) * 1024)),
            }
            lines.append("")
            lines.append(f"HBM traffic of {kernel}* (+ its reduce kernel) per launch, mean of {nf}/{nw} launches:")
            lines.append(f"  FETCH_SIZE {fk:.1f} KiB x {fs:.4f} + WRITE_SIZE {wk:.1f} KiB x {ws:.4f} = "
                         f"{traffic['traffic_bytes_per_launch'] / 1e6:.2f} MB")
            lines.append(f"  (scales: a 1 GiB device copy reads FETCH_SIZE {cf:.1f} KiB, WRITE_SIZE {cw:.1f} KiB)")
    if dom:
        lines.append("")
        lines.append(f"rocprof mean duration of {kernel}* launches: "
                     + ", ".join(f"{x:.2f} us" for x in dom))
        # A split-K launch is followed by its reduce kernel; the bench times both
        # (one GEMM call), so also give the pair: summed durations, and the span
        # from the kernel's start to the reduce kernel's end.
        pairs = []
        for i, r in enumerate(tr[:-1]):
            nxt = tr[i + 1]
            if _short_kernel_name(r["Kernel_Name"]).startswith(kernel) and "reduce" in nxt["Kernel_Name"]:
                d0 = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
                d1 = int(nxt["End_Timestamp"]) - int(nxt["Start_Timestamp"])
                pairs.append(((d0 + d1) / 1000.0, (int(nxt["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0))
        if pairs:
            lines.append(f"with its reduce kernel ({len(pairs)} pairs): durations summed "
                         f"{sum(p[0] for p in pairs) / len(pairs):.2f} us, start to end "
                         f"{sum(p[1] for p in pairs) / len(pairs):.2f} us")
    # Every split-K launch of the run (any kernel followed by a reduce kernel),
    # grouped by kernel and grid: the main kernel's duration, the gap from its
    # end to the reduce kernel's start, and the reduce kernel's duration.
    split = {}
    for i, r in enumerate(tr[:-1]):
        nxt = tr[i + 1]
        if "reduce" in r["Kernel_Name"] or "reduce" not in nxt["Kernel_Name"]:
            continue
        key = (_short_kernel_name(r["Kernel_Name"]), int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"])),
               _short_kernel_name(nxt["Kernel_Name"]))
        t0, t1 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        t2, t3 = int(nxt["Start_Timestamp"]), int(nxt["End_Timestamp"])
        split.setdefault(key, []).append(((t1 - t0) / 1000.0, (t2 - t1) / 1000.0, (t3 - t2) / 1000.0))
    if split:
        lines.append("")
        lines.append("split-K launches: main kernel, gap to the reduce kernel's start, reduce kernel (mean us)")
        lines.append(f"{'kernel':<36} {'wgs':>5} {'reduce':<26} {'pairs':>6} {'main':>7} {'gap':>6} {'reduce':>7} "
                     f"{'min_red':>7}")
        for (nm, gx, rn), v in sorted(split.items(), key=lambda kv: (kv[0][0], kv[0][1])):
            n = len(v)
            lines.append(f"{nm:<36} {gx:>5} {rn:<26} {n:>6} {sum(x[0] for x in v) / n:7.2f} "
                         f"{sum(x[1] for x in v) / n:6.2f} {sum(x[2] for x in v) / n:7.2f} "
                         f"{min(x[2] for x in v):7.2f}")
    return "\n".join(lines) + "\n", traffic


def _graph_time_us(torch, stream, launches, reps=5):
    """Median time of one launch: a graph of the launches (back to back on
    one stream) is replayed between HIP events, `reps` times."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for fn in launches:
            fn()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        g.replay()
    torch.cuda.synchronize()
    out = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            g.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) * 1e3 / len(launches))
    return statistics.median(out)


def vendor_yardstick_dnn():
    """The vendor library beside this library on DNN_SHAPES: fp32 and bf16
    storage with B stored K x N and N x K, int8 (B stored N x K), under the
    same harness as vendor_yardstick (graphs of back-to-back calls over
    operand copies rotated through at least 600 MB, median of 5 replays;
    torch.mm on bf16 writes a bf16 C, this library an fp32 C; beta = 0)."""
    import torch

    b = _binding()
    lib = b.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    s = torch.cuda.Stream(device=dev)
    rows = []
    cs = lambda: s.cuda_stream  # noqa: E731

    def both(name, torch_fns, ours_fns):
        with torch.cuda.stream(s):
            for f in torch_fns[:2] + ours_fns[:2]:
                f()
        torch.cuda.synchronize()
        t = _graph_time_us(torch, s, torch_fns)
        o = _graph_time_us(torch, s, ours_fns)
        row = {"shape": name, "torch_us": round(t, 2), "ours_us": round(o, 2), "torch_over_ours": round(t / o, 3)}
        rows.append(row)
        print(json.dumps(row), flush=True)

    for M, N, K in DNN_SHAPES:
        for dt, es in ((torch.float32, 4), (torch.bfloat16, 2)):
            n = max(2, min(64, -(-(600 << 20) // ((M * K + K * N) * es))))
            A = [torch.randn(M, K, device=dev).to(dt) for _ in range(n)]
            B = [(torch.randn(K, N, device=dev) * 0.05).to(dt) for _ in range(n)]
            Bt = [x.t().contiguous() for x in B]
            C = torch.empty(M, N, device=dev)
            tag = "fp32" if es == 4 else "bf16"
            if es == 4:
                ours = lambda k, tb: lib.sgemm(M, N, K, 1.0, A[k], K, Bt[k] if tb else B[k], K if tb else N, 0.0, C, N,  # noqa: E731
                                               transB=tb, stream=cs())
            else:
                ours = lambda k, tb: lib.gemm_bf16_ex(M, N, K, 1.0, A[k], K, Bt[k] if tb else B[k], K if tb else N,  # noqa: E731
                                                      0.0, C, N, transB=tb, stream=cs())
            both(f"{tag} {M}x{N}x{K}, B K x N", [lambda k=k: torch.mm(A[k], B[k]) for k in range(n)],
                 [lambda k=k: ours(k, 0) for k in range(n)])
            both(f"{tag} {M}x{N}x{K}, B N x K", [lambda k=k: torch.mm(A[k], Bt[k].t()) for k in range(n)],
                 [lambda k=k: ours(k, 1) for k in range(n)])
            del A, B, Bt, C
        if M > 16:
            n = max(2, min(64, -(-(600 << 20) // (M * K + K * N))))
            A8 = [torch.randint(-127, 128, (M, K), device=dev, dtype=torch.int8) for _ in range(n)]
            B8 = [torch.randint(-127, 128, (N, K), device=dev, dtype=torch.int8) for _ in range(n)]
            C8 = torch.empty(M, N, device=dev, dtype=torch.int32)
            both(f"int8 {M}x{N}x{K}", [lambda k=k: torch._int_mm(A8[k], B8[k].t()) for k in range(n)],
                 [lambda k=k: lib.gemm_s8s8s32(M, N, K, A8[k], K, B8[k], K, C8, N, stream=cs()) for k in range(n)])
            del A8, B8, C8
        torch.cuda.empty_cache()
    _yardstick_summary(torch, rows, "DNN inference shapes")


def vendor_yardstick():
    """The vendor library on the configs' shapes, timed beside this library
    under one harness: torch.mm / torch._int_mm (hipBLASLt / rocBLAS on this
    image) against the library's C-ABI, each a graph of back-to-back calls
    over operand copies rotated through at least 600 MB, median of 5
    replays.  Differences of the calls: torch.mm on bf16 operands writes a
    bf16 C (the library an fp32 C, 2 more bytes per output); torch._int_mm
    needs M > 16 (the int8 rows use M = 17 and 128); beta = 0 throughout.
    One JSON line per shape, then a summary line."""
    import torch

    b = _binding()
    lib = b.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    s = torch.cuda.Stream(device=dev)
    rows = []

    def copies(nbytes):
        return max(16, -(-(600 << 20) // nbytes))

    def both(name, torch_fns, ours_fns):
        with torch.cuda.stream(s):
            for f in torch_fns[:2] + ours_fns[:2]:
                f()
        torch.cuda.synchronize()
        t = _graph_time_us(torch, s, torch_fns)
        o = _graph_time_us(torch, s, ours_fns)
        row = {"shape": name, "torch_us": round(t, 2), "ours_us": round(o, 2), "torch_over_ours": round(t / o, 3)}
        rows.append(row)
        print(json.dumps(row), flush=True)

    cs = lambda: s.cuda_stream  # noqa: E731
    for M in (1, 4, 32, 256):
        N, K = 11008, 4096
        n = copies(N * K * 2)
        A = [torch.randn(M, K, device=dev).to(torch.bfloat16) for _ in range(n)]
        B = [(torch.randn(K, N, device=dev) * 0.02).to(torch.bfloat16) for _ in range(n)]
        C = torch.empty(M, N, device=dev, dtype=torch.float32)
        both(f"bf16 {M}x{N}x{K}, B K x N", [lambda k=k: torch.mm(A[k], B[k]) for k in range(n)],
             [lambda k=k: lib.gemm_bf16(M, N, K, 1.0, A[k], K, B[k], N, 0.0, C, N, stream=cs()) for k in range(n)])
        Bt = [x.t().contiguous() for x in B]
        del B
        both(f"bf16 {M}x{N}x{K}, B N x K", [lambda k=k: torch.mm(A[k], Bt[k].t()) for k in range(n)],
             [lambda k=k: lib.gemm_bf16_ex(M, N, K, 1.0, A[k], K, Bt[k], K, 0.0, C, N, transB=1, stream=cs())
              for k in range(n)])
        del A, Bt, C
        torch.cuda.empty_cache()
    for M in (17, 128):
        N, K = 4096, 4096
        n = copies(N * K)
        A = [torch.randint(-127, 128, (M, K), device=dev, dtype=torch.int8) for _ in range(n)]
        B = [torch.randint(-127, 128, (N, K), device=dev, dtype=torch.int8) for _ in range(n)]
        C = torch.empty(M, N, device=dev, dtype=torch.int32)
        both(f"int8 {M}x{N}x{K}", [lambda k=k: torch._int_mm(A[k], B[k].t()) for k in range(n)],
             [lambda k=k: lib.gemm_s8s8s32(M, N, K, A[k], K, B[k], K, C, N, stream=cs()) for k in range(n)])
        del A, B, C
        torch.cuda.empty_cache()
    fp32 = [(M, N, 2048) for M in (1, 7) for N in (1009, 4099, 11003)] + [(65536, 16, 256), (65536, 64, 256)]
    for M, N, K in fp32:
        n = copies((M * K if M > N else K * N) * 4)
        A = [torch.randn(M, K, device=dev) for _ in range(n if M > N else 1)]
        B = [torch.randn(K, N, device=dev) * 0.02 for _ in range(1 if M > N else n)]
        C = torch.empty(M, N, device=dev)
        a = lambda k: A[k % len(A)]  # noqa: E731
        bb = lambda k: B[k % len(B)]  # noqa: E731
        both(f"fp32 {M}x{N}x{K}", [lambda k=k: torch.mm(a(k), bb(k)) for k in range(n)],
             [lambda k=k: lib.sgemm(M, N, K, 1.0, a(k), K, bb(k), N, 0.0, C, N, stream=cs()) for k in range(n)])
        del A, B, C
        torch.cuda.empty_cache()
    _yardstick_summary(torch, rows, "the configs' shapes")


# DNN inference GEMMs outside the configs: BERT-base encoder layers at 128 /
# 384 / 32 tokens (hidden 768, MLP 3072), ResNet-50 convolutions as im2col
# GEMMs (56x56x64 3x3, 28x28x128 3x3, 14x14x256 3x3, 7x7x512 3x3, 56x56x256
# 1x1), two square-ish blocks, and a 4096-wide projection at 512 tokens.
DNN_SHAPES = [(128, 768, 768), (128, 3072, 768), (128, 768, 3072), (384, 768, 768), (384, 3072, 768),
              (384, 768, 3072), (32, 768, 768), (3136, 64, 576), (784, 128, 1152), (196, 256, 2304),
              (49, 512, 4608), (3136, 256, 64), (64, 1024, 1024), (200, 512, 512), (512, 4096, 4096)]


def _yardstick_summary(torch, rows, what):
    wins = sum(1 for r in rows if r["torch_over_ours"] >= 1.0)
    geo = statistics.geometric_mean([r["torch_over_ours"] for r in rows])
    print(json.dumps({"yardstick": f"torch (hipBLASLt/rocBLAS) vs this library, {what}", "shapes": len(rows),
                      "library_faster": wins, "geomean_torch_over_ours": round(geo, 3),
                      "torch": torch.__version__}), flush=True)


def copy_calibration(mib):
    """Plain copies of a known size: what FETCH_SIZE / WRITE_SIZE read for
    them scales the counters of the GEMM kernels to bytes."""
    import torch

    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    src.fill_(1)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": n, "launches": 5}), flush=True)


def config_summary(r):
    """Per-config figures of the JSON line: the step's GB/s and TFLOP/s, the
    dominant kernel's roofline, and each shape's time, GB/s, TFLOP/s and
    roofline fraction t_roof / t (t_roof = max(bytes / HBM peak, flops / MFMA
    peak))."""
    ms = r["ms_per_step"]
    rf = r["roofline"]
    return {
        "workload": r["desc"], "GBps_step": round(r["value"], 1),
        "TFLOPs_step": round(r["step_flops"] / (ms * 1e-3) / 1e12, 3), "us_per_step": round(ms * 1e3, 2),
        "dominant": {"kernel": rf["kernel"], "bound": rf["bound"], "achieved": rf["achieved"], "unit": rf["unit"],
                     "frac": rf["frac"], "launch_us": rf["launch_us"], "traffic": rf["traffic"]},
        "cases": [{"case": c["case"], "kernel": c["kernel"], "us": round(c["us_median"], 2),
                   "GBps": round(c["GBps"], 1), "TFLOPs": round(c["TFLOPs"], 2), "bound": c["bound"],
                   "roofline_frac": round(c["roofline_frac"], 4)} for c in r["per_case"]],
    }


# ---------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="default",
                    choices=["default", "c1", "c2", "c3", "c4", "c4f", "c5", "c5f", "hook", "all"],
                    help="default: C2 is `value`, C1, C3, C4 (bf16 storage and fp32 inputs) and C5 are timed too "
                         "and reported under `configs`; a single workload makes it `value`; all adds the "
                         "oneDNN-hook workload")
    ap.add_argument("--detail", default=None, help="append per-shape results (JSON lines) to this file")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cases", default=None, help="comma-separated case names of the workload to run (profiling)")
    ap.add_argument("--yardstick", nargs="?", const="configs", choices=("configs", "dnn"),
                    help="only time the vendor library (torch.mm / torch._int_mm) beside this library on the "
                         "configs' shapes (default) or on DNN inference shapes, one JSON line per shape")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device-to-device copies of MIB MiB (scale for HBM byte counters)")
    ap.add_argument("--rocprof-summary", nargs="+", metavar="ARG",
                    help="KERNEL WORKLOAD TRACE_CSV [FETCH_CSV WRITE_CSV COPY_FETCH_CSV COPY_WRITE_CSV]: print a "
                         "summary of rocprofv3 CSV output (no GPU use); with the counter files also write "
                         "profiles/<kernel>_<workload>_traffic.json")
    args = ap.parse_args()
    if args.yardstick:
        vendor_yardstick() if args.yardstick == "configs" else vendor_yardstick_dnn()
        return
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.rocprof_summary:
        a = args.rocprof_summary
        text, traffic = rocprof_summary(a[0], a[1], a[2], tuple(a[3:7]) if len(a) >= 7 else None)
        print(text, end="")
        if traffic:
            path = os.path.join(ROOT, "profiles", f"{_traffic_file_stem(a[0])}_{a[1]}_traffic.json")
            os.makedirs(os.path.dirname(path), exist_ok=True)
            with open(path, "w") as f:
                json.dump(traffic, f, indent=1)
                f.write("\n")
        return
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              "(sharding across GPUs is not built).", file=sys.stderr)
        sys.exit(2)

    if args.workload in ("default", "all"):
        names = ["c2", "c1", "c3", "c4", "c4f", "c5", "c5f"] + (["hook"] if args.workload == "all" else [])
        main_name = "c2"
    else:
        names = [args.workload]
        main_name = args.workload
    results = {}
    for wl in names:
        r = run_gpu(args, wl)
        results[wl] = r
        print(f"[bench] {wl}: {r['value']:.1f} GB/s per step, {r['ms_per_step'] * 1e3:.1f} us/step, "
              f"dominant {r['roofline']['kernel']} frac {r['roofline']['frac']}", file=sys.stderr, flush=True)
    r = results[main_name]
    cpu = None if args.no_cpu else cpu_baseline(r["cases"])
    cpu_ref = None if args.no_cpu else cpu_reference(r["cases"])
    line = {
        "metric": METRIC, "value": round(r["value"], 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(r["ms_per_step"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": {"c4": "bf16", "c5": "s8"}.get(main_name, "f32"),
        "data": "synthetic: SplitMix64 seed 42 (device generator), distributions of the workload description",
        "config": {"workload": r["desc"], "shapes": len(r["cases"]), "bytes_per_step": r["step_bytes"],
                   "hbm_frac": round(r["value"] / HBM_PEAK_GBS, 4), "buffer_copies": r["copies"],
                   "parallelism": "1 GPU"},
        "roofline": {k: r["roofline"][k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic")},
        "roofline_kernel": {k: r["roofline"][k] for k in ("kernel", "launch_us", "bytes_per_launch")},
        "cpu_baseline": cpu,
        "cpu_reference": cpu_ref,
        # every workload timed in this run, the `value` workload included
        # (its per-case figures)
        "configs": {wl: config_summary(rr) for wl, rr in results.items()},
    }
    if args.detail:
        os.makedirs(os.path.dirname(os.path.abspath(args.detail)), exist_ok=True)
        with open(args.detail, "a") as f:
            for wl, rr in results.items():
                f.write(json.dumps({"workload": wl, "desc": rr["desc"], "GBps_step": rr["value"],
                                    "ms_per_step": rr["ms_per_step"], "roofline": rr["roofline"],
                                    "per_case": rr["per_case"]}) + "\n")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
