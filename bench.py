"""Benchmark of the quantized-matmul path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload cfg2]

A step is one Linear/MatMul compute() through the C facade over one batch of
seeded synthetic input already resident in HBM. Default workload: BASELINE
config 2 (s8 x s8 -> s8, M = N = K = 4096, per-channel weight scales, s32 bias,
Relu, requantized), the configuration the headline s8-GEMM TOPS is quoted on.
The GEMV lines of the metric (int8 config 3 and Q4_1 config 4 at M = 1) are
reported under "secondary", each with rotated weight buffers larger than the
256 MB MALL so HBM, not cache, is measured.

Prints ONE JSON line. `roofline` is for the dominant kernel of the workload;
`cpu_baseline` times the CPU oracle (or the reference's compiled oracle when
present) on a bounded sample of the same workload on this host.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_INT8_TOPS = 5000.0      # MI355X dense int8 MFMA, TOPS
PEAK_F16_TFLOPS = 2500.0     # dense f16
PEAK_F32_TFLOPS = 157.3      # dense f32 MFMA
PEAK_HBM_GBS = 8000.0        # HBM3E
METRIC = "s8 GEMM TOPS @4096³; int8/Q4_1 GEMV GB/s @M=1; % of roofline"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", default="cfg2", choices=["cfg2", "cfg1", "cfg3", "cfg4", "cfg4_gemm", "cfg5",
                                                           "gated_ffn", "dense", "copy", "ceilings", "vendor"])
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline of the headline config")
    p.add_argument("--cpu-seconds-each", type=float, default=2.0, help="CPU baseline of each secondary line")
    return p.parse_args()


class Timer:
    """Times K steps with HIP events on the stream the kernels run on, two ways:

    - eager: the K calls issued back to back, one event pair around all of
      them (the device queue stays ahead as long as a call's host cost is
      below its kernel time);
    - graph: the K calls captured once into a HIP graph and replayed, which
      removes the Python/ctypes launch cost of this harness for the short
      kernels (a C++ caller launches in microseconds).

    The step time is the faster of the two; both are reported. Per-call events
    (eager, host launch included) are kept as the call-to-call spread.
    """

    def __init__(self, stream):
        import torch
        self.torch = torch
        self.stream = stream

    def _span(self, body):
        torch = self.torch
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(self.stream)
        body()
        e1.record(self.stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    def time(self, fn, steps, warmup, per_launch=False):
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                fn()
        torch.cuda.synchronize()

        def eager_all():
            with torch.cuda.stream(self.stream):
                for _ in range(steps):
                    fn()
        t0 = time.perf_counter()
        out = {"eager_ms": self._span(eager_all) / steps}
        out["wall_s"] = time.perf_counter() - t0
        try:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=self.stream):
                for _ in range(steps):
                    fn()
            g.replay()
            torch.cuda.synchronize()

            def replay():
                with torch.cuda.stream(self.stream):
                    g.replay()
            t0 = time.perf_counter()
            out["graph_ms"] = self._span(replay) / steps
            out["wall_s"] += time.perf_counter() - t0
        except Exception as exc:  # capture unsupported: eager only
            out["graph_error"] = type(exc).__name__
        if out.get("graph_ms", float("inf")) < out["eager_ms"]:
            out["mean_ms"], out["timing"] = out["graph_ms"], "hip-graph of K steps (faster than eager)"
        else:
            out["mean_ms"], out["timing"] = out["eager_ms"], "K eager steps back to back (faster than the graph)"
        out["eager_mean_ms"] = out["eager_ms"]
        if per_launch:
            out["launch_ms"] = self.per_launch(fn, steps)
        return out

    def per_launch(self, fn, steps):
        """Mean duration of one call's (first) kernel: before each of K
        back-to-back calls the library is armed (nnops_hip_time_next_launch)
        to attach an event pair to that kernel's own dispatch packet, so each
        pair brackets the kernel's execution alone -- the figure rocprofv3's
        kernel trace reports -- without the dispatch gap that events recorded
        on the stream around the call would add."""
        torch = self.torch
        import nnops_amd as na
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        with torch.cuda.stream(self.stream):
            for e0, e1 in ev:      # torch creates an event's HIP handle at its first record
                e0.record(self.stream)
                e1.record(self.stream)
        torch.cuda.synchronize()
        with torch.cuda.stream(self.stream):
            for e0, e1 in ev:
                rc = na.lib().nnops_hip_time_next_launch(C.c_void_p(e0.cuda_event), C.c_void_p(e1.cuda_event))
                assert rc == 0, rc
                fn()
        na.lib().nnops_hip_time_next_launch(None, None)
        torch.cuda.synchronize()
        return sum(e0.elapsed_time(e1) for e0, e1 in ev) / steps


_MEMO = {}


def memo(key, make):
    """Host operands shared by several bench lines (generated once)."""
    if key not in _MEMO:
        _MEMO[key] = make()
    return _MEMO[key]


def cpu_time(fn, seconds):
    """Repeat fn until `seconds` have passed (at least once); seconds per call."""
    reps = 0
    t0 = time.perf_counter()
    while reps == 0 or time.perf_counter() - t0 < seconds:
        fn()
        reps += 1
    return (time.perf_counter() - t0) / reps, reps


def cpu_cores():
    return max(1, min(16, len(os.sched_getaffinity(0))))


def nnops_cpu():
    """nnops' own CPU MatMul (compiled from the reference sources into
    oracle/_ref/libnnops_cpu.so), or None where this host cannot load it."""
    import oracle
    return oracle.cpu_lib()


def make_cfg2(torch, dg, na, M=4096, N=4096, K=4096):
    import numpy as np
    x = torch.from_numpy(dg.act_s8(201, (M, K))).cuda()
    w = torch.from_numpy(dg.ints(202, (N, K), -127, 127)).cuda()
    sb = torch.from_numpy(dg.uniform(203, (N,), 0.001, 0.01)).cuda()
    bias = torch.from_numpy(dg.ints(204, (N,), -5000, 5000, np.int32)).cuda()
    y = torch.zeros((M, N), dtype=torch.int8, device="cuda")
    op = na.Linear(output_dtype=na.DT_S8, act=na.EP_RELU)
    ins = [na.tensor(x, scale=0.02), na.tensor(w, scale_data=sb, granularity=2), na.tensor(bias)]
    outs = [na.tensor(y, scale=0.05)]
    ws_n = op.workspace_size(ins, outs)
    ws = torch.empty(max(ws_n, 1), dtype=torch.uint8, device="cuda")
    return op, ins, outs, ws, (x, w, sb, bias, y)


def run_cfg2(args, torch, dg, na, stream):
    M = N = K = 4096
    op, ins, outs, ws, keep = make_cfg2(torch, dg, na, M, N, K)
    s = stream.cuda_stream

    def step():
        rc = op.compute(outs, ins, stream=s, workspace=ws)
        if rc != 0:
            raise RuntimeError(f"compute failed: {rc}")

    t = Timer(stream).time(step, args.steps, args.warmup, per_launch=True)
    ops = 2.0 * M * N * K
    tops = ops / (t["mean_ms"] * 1e-3) / 1e12
    # the roofline of the kernel: its own average launch duration (one kernel per step)
    k_tops = ops / (t["launch_ms"] * 1e-3) / 1e12
    return {
        "value": tops, "unit": "TOPS", "ms": t["mean_ms"], "t": t,
        "eager_ms_per_step": t["eager_mean_ms"], "timing": t["timing"],
        "config": {"workload": "cfg2: QuantLinear s8xs8->s8 M=N=K=4096, per-channel w scale, s32 bias, "
                               "relu, requant (half away from zero)", "M": M, "N": N, "K": K,
                   "weight_layout": "[N,K]"},
        "roofline": {"bound": "mfma", "achieved": k_tops, "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                     "frac": k_tops / PEAK_INT8_TOPS, "traffic": measured_traffic("gemm_i8_ring_cfg2"),
                     "launch_us": t["launch_ms"] * 1e3,
                     "kernel": "gemm_i8_ring<256,256,2,4,BK=128,NS=2,RING_S8>", "algorithmic_ops_per_launch": ops,
                     "algorithmic_bytes_per_launch": float(M * K + N * K + M * N + N * 8)},
        "dtype": "int8 (s32 accumulate)",
    }


def gemv_i8_case(torch, dg, na, stream, steps, warmup, M=1, K=4096, N=11008, nbuf=8, trans_b=False,
                 prepacked=False, out_s8=False, cpu_seconds=0.0):
    """Config 3: int8 GEMV with `nbuf` rotated weight buffers (> MALL).
    `prepacked`: each weight goes through prepackWeights first (outside the
    timed region, once at load time), and the call reads the packed form.
    `out_s8`: the requantizing variant (per-channel scales as config 2).
    `cpu_seconds` > 0: nnops' own CPU MatMul on the same problem beside it."""
    import numpy as np
    a_h = dg.ints(301, (M, K), -127, 127)
    w_h = memo(("w", trans_b, K, N), lambda: dg.ints(302, (N, K) if trans_b else (K, N), -127, 127))
    sb_h = dg.uniform(303, (N,), 0.001, 0.01)
    a = torch.from_numpy(a_h).cuda()
    ws_list = []
    base = torch.from_numpy(w_h).cuda()
    for i in range(nbuf):
        ws_list.append(base if i == 0 else torch.roll(base, shifts=i, dims=1).contiguous())
    if prepacked:
        kp = (K + 127) // 128 * 128
        packed = []
        for w in ws_list:
            blob = torch.empty(na.lib().nnops_hip_prepack_i8_bytes(K, N), dtype=torch.uint8, device="cuda")
            rc = na.lib().nnops_hip_prepack_i8(w.data_ptr(), K, N, w.stride(0), int(trans_b), blob.data_ptr(),
                                               stream.cuda_stream)
            assert rc == 0, rc
            packed.append(blob[:N * kp].view(torch.int8).view(N, kp))
        stream.synchronize()
        ws_list = packed
    kern_tb = trans_b or prepacked
    c = torch.zeros((M, N), dtype=torch.int8 if out_s8 else torch.int32, device="cuda")
    sb = torch.from_numpy(sb_h).cuda()
    s = stream.cuda_stream
    probe = na.GemmI8Args()
    probe.m, probe.n, probe.k, probe.trans_b = M, N, K, int(kern_tb)
    probe.out_kind = na.OUT_S8 if out_s8 else na.OUT_S32
    need = na.lib().nnops_hip_gemm_i8_workspace_size(C.byref(probe))
    wsp = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    it = [0]
    kw = dict(out_kind=na.OUT_S8, s_a=0.02, s_b=sb, s_out=0.05) if out_s8 else {}

    def step():
        b = ws_list[it[0] % nbuf]
        it[0] += 1
        na.gemm_i8(a, b, c, trans_b=kern_tb, workspace=wsp, stream=s, **kw)

    t = Timer(stream).time(step, steps, warmup)
    nbytes = K * N + K * M + N * M * (1 if out_s8 else 4) + (4 * N if out_s8 else 0)
    gbs = nbytes / (t["mean_ms"] * 1e-3) / 1e9
    out = {"gbs": gbs, "frac_hbm": gbs / PEAK_HBM_GBS, "us": t["mean_ms"] * 1e3,
           "bytes": nbytes, "M": M, "K": K, "N": N, "out": "s8 (requant)" if out_s8 else "s32",
           "weight_layout": "prepacked [K,N] -> [N][kp]" if prepacked else ("[N,K]" if trans_b else "[K,N]"),
           "rotated_weight_bytes": nbuf * K * N, "timing": t["timing"]}
    if cpu_seconds > 0 and prepacked:
        out["cpu_baseline"] = cpu_i8_packed(a_h, w_h, trans_b, nbytes, cpu_seconds,
                                            f"config 3 M={M} (s32 out, weight {'[N,K]' if trans_b else '[K,N]'} "
                                            f"prepacked)")
    elif cpu_seconds > 0:
        out["cpu_baseline"] = cpu_i8(a_h, w_h, trans_b, out_s8, sb_h, nbytes, cpu_seconds, "GB/s",
                                     f"config 3 M={M} ({'s8' if out_s8 else 's32'} out, weight "
                                     f"{'[N,K]' if trans_b else '[K,N]'})")
    return out


def cpu_i8(a, w, trans_b, out_s8, sb, nbytes, seconds, unit, what):
    """nnops' CPU MatMul on one int8 problem, timed in full; `unit` GB/s (the
    GPU line's algorithmic bytes per second) or TOPS."""
    import numpy as np
    cpu = nnops_cpu()
    if cpu is None:
        return {"value": None, "unit": unit, "cores": 0, "kind": "reference",
                "sample": "n/a: oracle/_ref/libnnops_cpu.so not loadable on this host (no AVX-512 VNNI)"}
    M, K = a.shape
    N = w.shape[0] if trans_b else w.shape[1]
    c = np.zeros((M, N), np.int8 if out_s8 else np.int32)
    cores = cpu_cores()

    def call():
        rc = cpu.ref_cpu_matmul_i8(a.ctypes.data, w.ctypes.data, None, c.ctypes.data, M, N, K, int(trans_b),
                                   int(out_s8), 0.02, sb.ctypes.data if out_s8 else None, 0.05, 0, 0, cores)
        if rc != 0:
            raise RuntimeError(f"nnops CPU MatMul failed: status {rc}")
    sec, reps = cpu_time(call, seconds)
    v = nbytes / sec / 1e9 if unit == "GB/s" else 2.0 * M * N * K / sec / 1e12
    return {"value": v, "unit": unit, "cores": cores, "kind": "reference", "us": sec * 1e6,
            "sample": f"{what} in full, {reps} calls; nnops' CPU MatMul (src/backend/cpu/matmul, AVX-512-VNNI) "
                      f"compiled from source, {cores} threads"}


def _cpu_na(unit):
    return {"value": None, "unit": unit, "cores": 0, "kind": "reference",
            "sample": "n/a: oracle/_ref/libnnops_cpu.so not loadable on this host (no AVX-512 VNNI)"}


def cpu_i8_packed(a, w, trans_b, nbytes, seconds, what):
    """nnops' CPU MatMul over its own prepacked s8 weight (MatMul::
    prepackWeights, src/ops/matmul.cpp:96-141, packed once outside the timed
    calls), s32 out; GB/s of the GPU line's algorithmic bytes."""
    import numpy as np
    cpu = nnops_cpu()
    if cpu is None:
        return _cpu_na("GB/s")
    M, K = a.shape
    N = w.shape[0] if trans_b else w.shape[1]
    cores = cpu_cores()
    h = cpu.ref_cpu_prepack_i8(w.ctypes.data, N, K, int(trans_b), 0, None, cores)
    if not h:
        return {"value": None, "unit": "GB/s", "cores": cores, "kind": "reference",
                "sample": "n/a: nnops' prepackWeights gave no packed form for this weight"}
    c = np.zeros((M, N), np.int32)

    def call():
        rc = cpu.ref_cpu_matmul_i8_packed(a.ctypes.data, h, None, c.ctypes.data, M, N, K, 1.0, None, 1.0, 0, 0,
                                          cores)
        if rc != 0:
            raise RuntimeError(f"nnops CPU packed MatMul failed: status {rc}")
    try:
        sec, reps = cpu_time(call, seconds)
    finally:
        cpu.ref_cpu_packed_free(h)
    return {"value": nbytes / sec / 1e9, "unit": "GB/s", "cores": cores, "kind": "reference", "us": sec * 1e6,
            "sample": f"{what} in full, {reps} calls over nnops' own prepacked weight (MatMul::prepackWeights, "
                      f"once, outside the timing); nnops' CPU MatMul (AVX-512-VNNI) compiled from source, "
                      f"{cores} threads"}


def cpu_call(call, seconds, work, unit, what):
    """Times one nnops CPU call (a closure returning its status) in full;
    `work` is the GPU line's algorithmic bytes (GB/s) or ops (TOPS/TFLOPS)."""
    cpu = nnops_cpu()
    if cpu is None:
        return _cpu_na(unit)
    cores = cpu_cores()

    def once():
        rc = call(cpu, cores)
        if rc != 0:
            raise RuntimeError(f"nnops CPU call failed: status {rc}")
    sec, reps = cpu_time(once, seconds)
    scale = 1e9 if unit == "GB/s" else 1e12
    return {"value": work / sec / scale, "unit": unit, "cores": cores, "kind": "reference", "us": sec * 1e6,
            "sample": f"{what} in full, {reps} calls; compiled from the nnops sources, {cores} threads"}


def cpu_q4_1(a, blk, N, trans_b, nbytes, seconds, what):
    """nnops' CPU fp x q4_1 MatMul (f16 A -> f16 C: its output dtype follows A,
    src/ops/matmul.cpp:49-58; matmul_qblock_fused at small M) on one problem."""
    import numpy as np
    cpu = nnops_cpu()
    unit = "GB/s" if a.shape[0] <= 16 else "TFLOPS"
    if cpu is None:
        return {"value": None, "unit": unit, "cores": 0, "kind": "reference",
                "sample": "n/a: oracle/_ref/libnnops_cpu.so not loadable on this host (no AVX-512 VNNI)"}
    M, K = a.shape
    c = np.zeros((M, N), np.float16)
    cores = cpu_cores()

    def call():
        rc = cpu.ref_cpu_matmul_q4_1(a.ctypes.data, blk.ctypes.data, c.ctypes.data, M, N, K, int(trans_b), cores)
        if rc != 0:
            raise RuntimeError(f"nnops CPU q4_1 MatMul failed: status {rc}")
    sec, reps = cpu_time(call, seconds)
    v = nbytes / sec / 1e9 if unit == "GB/s" else 2.0 * M * N * K / sec / 1e12
    return {"value": v, "unit": unit, "cores": cores, "kind": "reference", "us": sec * 1e6,
            "sample": f"{what} in full, {reps} calls; nnops' CPU fp x q4_1 MatMul with f16 output (its route for "
                      f"an f16 A) compiled from source, {cores} threads"}


def gemv_q41_case(torch, dg, na, stream, steps, warmup, M=1, K=4096, N=14336, nbuf=8, trans_b=True,
                  cpu_seconds=0.0):
    a_h = dg.normal(401, (M, K)).astype("float16")
    b_h = dg.q4_1_blocks(402, N, K) if trans_b else dg.q4_1_blocks(402, K, N)
    a = torch.from_numpy(a_h).cuda()
    base = torch.from_numpy(b_h).cuda()
    bufs = [base if i == 0 else torch.roll(base, shifts=20 * i, dims=1).contiguous() for i in range(nbuf)]
    c = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    s = stream.cuda_stream
    it = [0]

    def step():
        b = bufs[it[0] % nbuf]
        it[0] += 1
        na.gemm_q4_1(a, b, c, n=N, trans_b=trans_b, workspace=wsp, stream=s)

    probe = na.GemmQ41Args()
    probe.m, probe.n, probe.k, probe.trans_b, probe.a_f16 = M, N, K, int(trans_b), 1
    probe.out_kind = na.OUT_F32
    need = na.lib().nnops_hip_gemm_q4_1_workspace_size(C.byref(probe))
    wsp = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    t = Timer(stream).time(step, steps, warmup)
    nbytes = N * (K // 32) * 20 + K * M * 2 + N * M * 4
    gbs = nbytes / (t["mean_ms"] * 1e-3) / 1e9
    out = {"gbs": gbs, "frac_hbm": gbs / PEAK_HBM_GBS, "us": t["mean_ms"] * 1e3, "bytes": nbytes,
           "M": M, "K": K, "N": N, "weight_layout": "[N][K/32 blocks]" if trans_b else "[K][N/32 blocks]",
           "rotated_weight_bytes": nbuf * N * (K // 32) * 20, "timing": t["timing"]}
    if cpu_seconds > 0:
        out["cpu_baseline"] = cpu_q4_1(a_h, b_h, N, trans_b, N * (K // 32) * 20 + K * M * 2 + N * M * 2,
                                       cpu_seconds, f"config 4 M={M} (weight {out['weight_layout']})")
    return out


def q41_gemm_case(torch, dg, na, stream, steps, warmup, M=512, K=4096, N=14336, trans_b=True, cpu_seconds=0.0,
                  a_f32=False):
    """Config 4's GEMM; trans_b=False times the literal [K][N/32] layout
    (blocks along N) instead of the GGUF/Linear [N][K/32] one; a_f32 an f32
    A (nnops computes that product in f32; here the split-f16 ring past the
    skinny rows, blocks along K)."""
    import numpy as np
    a_h = dg.normal(403, (M, K)).astype("float32" if a_f32 else "float16")
    b_h = dg.q4_1_blocks(404, N, K) if trans_b else dg.q4_1_blocks(404, K, N)
    a = torch.from_numpy(a_h).cuda()
    b = torch.from_numpy(b_h).cuda()
    # a few rows of A stream the weight: rotate over 8 copies (more than the
    # MALL) so HBM is measured
    nb = 8 if M <= 48 else 1
    bs = [b] + [torch.roll(b, shifts=i, dims=0).contiguous() for i in range(1, nb)]
    c = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    s = stream.cuda_stream
    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    it = [0]

    def step():
        na.gemm_q4_1(a, bs[it[0] % nb], c, n=N, trans_b=trans_b, workspace=ws, stream=s)
        it[0] += 1
    t = Timer(stream).time(step, steps, warmup)
    fl = 2.0 * M * N * K
    tf = fl / (t["mean_ms"] * 1e-3) / 1e12
    out = {"tflops": tf, "us": t["mean_ms"] * 1e3,
           "M": M, "K": K, "N": N, "weight_layout": "[N][K/32 blocks]" if trans_b else "[K][N/32 blocks]",
           "timing": t["timing"]}
    if a_f32 and trans_b and M > 48 and K % 64 == 0:
        # the split-f16 ring: A as two f16 parts, two f16 products per decoded
        # weight on the f16 matrix cores (the fraction counts the algorithmic
        # 2 M N K flops against the f16 peak)
        out["a"] = "f32 (split into two f16 parts)"
        out["frac_f16_mfma"] = tf / PEAK_F16_TFLOPS
    elif a_f32:
        out["a"] = "f32"
        out["frac_f32_mfma"] = tf / PEAK_F32_TFLOPS
    else:
        out["frac_f16_mfma"] = tf / PEAK_F16_TFLOPS
    if M <= 48:
        # a few rows of A: bound by the weight stream, not the matrix cores
        by = N * (K // 32) * 20 + M * K * (4 if a_f32 else 2) + M * N * 4
        out["gbs"] = by / (t["mean_ms"] * 1e-3) / 1e9
        out["frac_hbm"] = out["gbs"] / PEAK_HBM_GBS
    if cpu_seconds > 0 and a_f32:
        # nnops' f32 x q4_1 MatMul (f32 output, its FpRoute<float>)
        cf = np.zeros((M, N), np.float32)
        out["cpu_baseline"] = cpu_call(
            lambda cpu, cores: cpu.ref_cpu_matmul_q4_1_ep(a_h.ctypes.data, 0, b_h.ctypes.data, None, cf.ctypes.data,
                                                          M, N, K, int(trans_b), 1.0, 0.0, 0, 0, 0.0, 1.0,
                                                          -math.inf, math.inf, cores),
            cpu_seconds, fl, "TFLOPS", f"config 4 M={M} with an f32 A (nnops' f32 x q4_1 MatMul, f32 out)")
    elif cpu_seconds > 0:
        by = N * (K // 32) * 20 + M * K * 2 + M * N * 2
        out["cpu_baseline"] = cpu_q4_1(a_h, b_h, N, trans_b, by, cpu_seconds,
                                       f"config 4 M={M} (weight {out['weight_layout']})")
    return out


def gated_ffn_case(torch, dg, na, stream, steps, warmup, M=1, K=4096, N=14336, nbuf=4, cpu_seconds=0.0):
    """Linear's gated form (SwiGLU) over a q4_1 [2N, K] weight (blocks along
    K, the GGUF form) with bias, f16 X [M, K] -> f16 [M, N], through the
    operator API: the Q4_1 GEMM / GEMV into the workspace and the combine.
    M=1 rotates over nbuf weights (more than the MALL) so HBM is measured."""
    import numpy as np
    x_h = dg.normal(420 + M, (M, K)).astype("float16")
    x = torch.from_numpy(x_h).cuda()
    nb = nbuf if M <= 48 else 1
    w0_h = dg.q4_1_blocks(421, 2 * N, K)
    ws_ = [torch.from_numpy(w0_h if i == 0 else dg.q4_1_blocks(421 + i, 2 * N, K)).cuda() for i in range(nb)]
    bias_h = (0.1 * dg.normal(425, (2 * N,))).astype("float16")
    bias = torch.from_numpy(bias_h).cuda()
    y = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    op = na.Linear(gated=True, gate_activation=na.EP_SILU)
    ins = [[na.tensor(x), na.tensor(w, dtype=na.DT_Q4_1, shape=[2 * N, K]), na.tensor(bias)] for w in ws_]
    outs = [na.tensor(y)]
    wsn = op.workspace_size(ins[0], outs)
    wsb = torch.empty(max(wsn, 1), dtype=torch.uint8, device="cuda")
    s = stream.cuda_stream
    it = [0]

    def step():
        rc = op.compute(outs, ins[it[0] % nb], stream=s, workspace=wsb)
        it[0] += 1
        if rc != 0:
            raise RuntimeError(f"gated Linear failed: {rc}")
    t = Timer(stream).time(step, steps, warmup)
    wbytes = 2 * N * (K // 32) * 20
    by = wbytes + M * K * 2 + M * N * 2 + 2 * N * 2
    fl = 2.0 * M * 2 * N * K
    out = {"us": t["mean_ms"] * 1e3, "gbs": by / (t["mean_ms"] * 1e-3) / 1e9, "bytes": by,
           "tflops": fl / (t["mean_ms"] * 1e-3) / 1e12,
           "M": M, "K": K, "N": N, "weight_layout": "[2N][K/32 blocks] (gate rows, then value rows)",
           "op": "Linear gated (SwiGLU) + bias, f16", "timing": t["timing"]}
    if M > 48:
        # the matrix cores bound it (the weight is read once per 128 rows)
        out["frac_f16_mfma"] = out["tflops"] / PEAK_F16_TFLOPS
    else:
        out["frac_hbm"] = out["gbs"] / PEAK_HBM_GBS
    if cpu_seconds > 0:
        yc = np.zeros((M, N), np.float16)
        # nnops' linear_cpu, gated (src/backend/cpu/matmul/linear.cpp:84-170, 199-309), Silu gate
        out["cpu_baseline"] = cpu_call(
            lambda cpu, cores: cpu.ref_cpu_linear_q4_1(x_h.ctypes.data, 1, w0_h.ctypes.data, bias_h.ctypes.data,
                                                       yc.ctypes.data, M, 2 * N, K, 0, 0.0, 1.0, -math.inf,
                                                       math.inf, 0, 0, 1, 6, 1.0, 0.0, math.inf, cores),
            cpu_seconds, by if M <= 16 else fl, "GB/s" if M <= 16 else "TFLOPS",
            f"gated FFN M={M} (nnops' linear_cpu, gated SwiGLU over the q4_1 [2N,K] weight, f16)")
    return out


def q41_packed_case(torch, dg, na, stream, steps, warmup, M, K=4096, N=14336, nbuf=8, cpu_seconds=0.0):
    """Config 4 with the [K][N/32] weight prepacked (MatMul.prepackWeights:
    the nibble and d|m planes), through the operator API. Up to 48 rows of A
    rotate over nbuf packed weights (more than the MALL) so HBM is measured."""
    a_h = dg.normal(405, (M, K)).astype("float16")
    b_h = dg.q4_1_blocks(406, K, N)
    a = torch.from_numpy(a_h).cuda()
    base = torch.from_numpy(b_h).cuda()
    op = na.MatMul(transpose_b=False)
    nb = nbuf if M <= 48 else 1
    packed = []
    for i in range(nb):
        raw = base if i == 0 else torch.roll(base, shifts=20 * i, dims=1).contiguous()
        # prepacked on torch's current stream, which also owns raw's memory
        packed.append(op.prepack(na.tensor(raw, dtype=na.DT_Q4_1, shape=[K, N]))[1])
        torch.cuda.synchronize()
    c = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    at, ct = na.tensor(a), na.tensor(c)
    wsn = op.workspace_size([at, packed[0]], [ct])
    ws = torch.empty(max(wsn, 1), dtype=torch.uint8, device="cuda")
    s = stream.cuda_stream
    it = [0]

    def step():
        w = packed[it[0] % nb]
        it[0] += 1
        op.compute([ct], [at, w], stream=s, workspace=ws)

    t = Timer(stream).time(step, steps, warmup)
    out = {"us": t["mean_ms"] * 1e3, "M": M, "K": K, "N": N, "weight_layout": "[K][N/32 blocks], prepacked planes"}
    if M <= 16:
        nbytes = N * (K // 32) * 20 + K * M * 2 + N * M * 4
        out.update(gbs=nbytes / (t["mean_ms"] * 1e-3) / 1e9, bytes=nbytes)
        out["frac_hbm"] = out["gbs"] / PEAK_HBM_GBS
    else:
        out["tflops"] = 2.0 * M * N * K / (t["mean_ms"] * 1e-3) / 1e12
        out["frac_f16_mfma"] = out["tflops"] / PEAK_F16_TFLOPS
    if cpu_seconds > 0:
        # nnops packs no q4_1 form (matmul_helper.cpp:695-723): its route for
        # this weight reads the raw [K][N/32] blocks
        by = N * (K // 32) * 20 + K * M * 2 + N * M * 2
        out["cpu_baseline"] = cpu_q4_1(a_h, b_h, N, False, by, cpu_seconds,
                                       f"config 4 M={M} over the raw [K][N/32] weight (nnops has no packed "
                                       f"q4_1 form)")
    return out


def cfg1_case(torch, dg, na, stream, steps, warmup, cpu_seconds=0.0):
    """Config 1: s8 x s8 -> s32, A [128,1024], B [1024,1024] ([K,N], the
    MatMul form), no bias, no epilogue, dense; launch/latency bound."""
    M, K, N = 128, 1024, 1024
    a_h = dg.ints(101, (M, K), -127, 127)
    b_h = dg.ints(102, (K, N), -127, 127)
    a, b = torch.from_numpy(a_h).cuda(), torch.from_numpy(b_h).cuda()
    c = torch.zeros((M, N), dtype=torch.int32, device="cuda")
    s = stream.cuda_stream
    probe = na.GemmI8Args()
    probe.m, probe.n, probe.k = M, N, K
    wsp = torch.empty(max(na.lib().nnops_hip_gemm_i8_workspace_size(C.byref(probe)), 1), dtype=torch.uint8,
                      device="cuda")
    t = Timer(stream).time(lambda: na.gemm_i8(a, b, c, workspace=wsp, stream=s), steps, warmup)
    ops = 2.0 * M * N * K
    out = {"tops": ops / (t["mean_ms"] * 1e-3) / 1e12, "us": t["mean_ms"] * 1e3, "M": M, "K": K, "N": N,
           "weight_layout": "[K,N]", "out": "s32", "timing": t["timing"]}
    out["frac_int8_mfma"] = out["tops"] / PEAK_INT8_TOPS
    if cpu_seconds > 0:
        out["cpu_baseline"] = cpu_i8(a_h, b_h, False, False, None, 0, cpu_seconds, "TOPS", "config 1")
    return out


def vendor_reference(torch, steps=50, warmup=10):
    """The vendor libraries on the same shapes, as a yardstick for the
    hand-written kernels: hipBLASLt's int8 GEMM (torch._int_mm, int32 out)
    at config 2's 4096^3 with B row- and column-major, and its f16 GEMM at
    config 4's 512 x 4096 x 14336 (no dequantization) and at 4096^3. Eager
    launches on the current stream, HIP events around `steps` calls."""
    def t(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps * 1e3
    out = {}
    a = torch.randint(-127, 127, (4096, 4096), dtype=torch.int8, device="cuda")
    b = torch.randint(-127, 127, (4096, 4096), dtype=torch.int8, device="cuda")
    bt = b.t().contiguous().t()
    for name, bb in (("int8_4096_b_row_major", b), ("int8_4096_b_col_major", bt)):
        us = t(lambda: torch._int_mm(a, bb))
        out[name] = {"us": us, "tops": 2 * 4096 ** 3 / us / 1e6}
    for name, (m, k, n) in (("f16_512x4096x14336", (512, 4096, 14336)), ("f16_4096", (4096, 4096, 4096))):
        x = torch.randn(m, k, dtype=torch.float16, device="cuda")
        w = torch.randn(k, n, dtype=torch.float16, device="cuda")
        us = t(lambda: x @ w)
        out[name] = {"us": us, "tflops": 2 * m * k * n / us / 1e6}
    return out


def cfg5_case(torch, dg, na, stream, steps, warmup):
    import numpy as np
    M, K, N = 333, 14336, 4096
    xa = torch.from_numpy(dg.act_s8(501, (M, 14400))).cuda()
    x = xa[:, :K]
    w = torch.from_numpy(dg.ints(502, (K, N), -127, 127)).cuda()
    sb = torch.from_numpy(dg.uniform(503, (N,), 0.001, 0.01)).cuda()
    bias = torch.from_numpy(dg.ints(504, (N,), -5000, 5000, np.int32)).cuda()
    ya = torch.from_numpy(dg.ints(505, (M, 4160), -128, 127)).cuda()
    y = ya[:, :N]
    op = na.MatMul(output_dtype=na.DT_S8, act=na.EP_GELU, residual_pre_activation=False,
                   float_epilogue=True)
    # add_to on MatMul is expressed with Linear semantics through the facade's Linear;
    # here the [K,N] weight goes through MatMul + float epilogue, residual after GELU.
    lin = na.Linear(output_dtype=na.DT_S8, act=na.EP_GELU, add_to=True)
    wt = w.t().contiguous()  # Linear's [N,K] weight
    ins = [na.tensor(x, scale=0.02), na.tensor(wt, scale_data=sb, granularity=2), na.tensor(bias)]
    outs = [na.tensor(y, scale=2.0)]
    wsn = lin.workspace_size(ins, outs)
    ws = torch.empty(max(wsn, 1), dtype=torch.uint8, device="cuda")
    s = stream.cuda_stream
    del op
    t = Timer(stream).time(lambda: lin.compute(outs, ins, stream=s, workspace=ws), steps, warmup)
    ops = 2.0 * M * N * K
    tops = ops / (t["mean_ms"] * 1e-3) / 1e12
    return {"tops": tops, "frac_int8_mfma": tops / PEAK_INT8_TOPS, "us": t["mean_ms"] * 1e3,
            "M": M, "K": K, "N": N, "a_pitch": 14400, "c_pitch": 4160, "weight_layout": "[N,K]",
            "timing": t["timing"],
            "cpu_baseline": {"value": None, "unit": "TOPS", "cores": 0, "kind": "reference",
                             "sample": "n/a: nnops has no route for an s8 add_to destination "
                                       "(src/backend/cpu/matmul/linear.cpp:226) nor a GELU on an integer one"}}


def dense_fp_case(torch, dg, na, stream, steps, warmup, M, N=4096, K=4096, f16=True, nbuf=1, cpu_seconds=0.0):
    """nnops' dense float route (MatMul f16 x f16 or f32 x f32, B [N, K]):
    C = A B with f32 accumulation. M <= 16 rotates over nbuf weights (more
    than the MALL) so HBM is measured."""
    dt = torch.float16 if f16 else torch.float32
    npdt = "float16" if f16 else "float32"
    import numpy as np
    a_h = dg.normal(440 + M, (M, K)).astype(npdt)
    b_h = dg.normal(441, (N, K)).astype(npdt)
    a = torch.from_numpy(a_h).cuda()
    base = torch.from_numpy(b_h).cuda()
    bs = [base] + [torch.roll(base, shifts=i, dims=1).contiguous() for i in range(1, nbuf)]
    c = torch.empty((M, N), dtype=dt, device="cuda")
    s = stream.cuda_stream
    # room for any plan's partials (split K, or an unaligned destination)
    ws = torch.empty(4 * M * N + (1 << 20), dtype=torch.uint8, device="cuda")
    it = [0]

    def step():
        na.gemm_fp(a, bs[it[0] % nbuf], c, trans_b=True, workspace=ws, stream=s)
        it[0] += 1
    t = Timer(stream).time(step, steps, warmup)
    es = 2 if f16 else 4
    by = N * K * es + M * K * es + M * N * es
    fl = 2.0 * M * N * K
    out = {"us": t["mean_ms"] * 1e3, "M": M, "K": K, "N": N, "dtype": npdt, "weight_layout": "[N,K]",
           "timing": t["timing"], "tflops": fl / (t["mean_ms"] * 1e-3) / 1e12,
           "gbs": by / (t["mean_ms"] * 1e-3) / 1e9}
    if M <= 16:
        out["frac_hbm"] = out["gbs"] / PEAK_HBM_GBS
        out["bytes"] = by
    else:
        out["frac_mfma"] = out["tflops"] / (PEAK_F16_TFLOPS if f16 else PEAK_F32_TFLOPS)
    if cpu_seconds > 0:
        cc = np.zeros((M, N), npdt)
        out["cpu_baseline"] = cpu_call(
            lambda cpu, cores: cpu.ref_cpu_matmul_fp(a_h.ctypes.data, b_h.ctypes.data, cc.ctypes.data, M, N, K, 1,
                                                     int(f16), cores),
            cpu_seconds, by if M <= 16 else fl, "GB/s" if M <= 16 else "TFLOPS",
            f"dense {npdt} {M}x{K}x{N} (nnops' CPU MatMul)")
    return out


def qdq_case(torch, dg, na, stream, steps, warmup, R=4096, C=4096, dequant=False, cpu_seconds=0.0):
    """QuantizeLinear f16 [R,C] -> s8 (per-token scales and zero points), or
    DequantizeLinear s8 -> f16, through the operator API. HBM-bound."""
    import numpy as np
    sc_h = dg.uniform(601, (R,), 0.01, 0.05)
    zp_h = dg.ints(602, (R,), -8, 8, np.int8)
    x_h = dg.ints(603, (R, C), -128, 127) if dequant else dg.normal(603, (R, C), 1.0).astype("float16")
    scale = torch.from_numpy(sc_h).cuda()
    zp = torch.from_numpy(zp_h).cuda()
    if dequant:
        x = torch.from_numpy(x_h).cuda()
        y = torch.empty((R, C), dtype=torch.float16, device="cuda")
        op = na.DequantizeLinear(axis=-1, output_dtype=na.DT_F16)
    else:
        x = torch.from_numpy(x_h).cuda()
        y = torch.empty((R, C), dtype=torch.int8, device="cuda")
        op = na.QuantizeLinear(axis=-1, output_dtype=na.DT_S8)
    ins = [na.tensor(x), na.tensor(scale), na.tensor(zp)]
    outs = [na.tensor(y)]
    s = stream.cuda_stream
    t = Timer(stream).time(lambda: op.compute(outs, ins, stream=s), steps, warmup)
    nbytes = R * C * 3 + R * 5
    gbs = nbytes / (t["mean_ms"] * 1e-3) / 1e9
    out = {"gbs": gbs, "frac_hbm": gbs / PEAK_HBM_GBS, "us": t["mean_ms"] * 1e3, "bytes": nbytes,
           "shape": [R, C], "op": "DequantizeLinear s8->f16" if dequant else "QuantizeLinear f16->s8",
           "granularity": "per token"}
    if cpu_seconds > 0:
        yc = np.zeros((R, C), np.float16 if dequant else np.int8)
        out["cpu_baseline"] = cpu_call(
            lambda cpu, cores: cpu.ref_cpu_qdq_f16(x_h.ctypes.data, sc_h.ctypes.data, zp_h.ctypes.data,
                                                   yc.ctypes.data, R, C, int(dequant), cores),
            cpu_seconds, nbytes, "GB/s", f"{out['op']} {R}x{C} per token (nnops' CPU operator)")
    return out


def fp_act_case(torch, dg, na, stream, steps, warmup, M=4096, N=4096, K=4096, dq_only=False, cpu_seconds=0.0):
    """The fp-activation int8 MatMul at config 2's shape: f16 A with per-token
    scales, s8 [N,K] weights with per-channel scales, f16 out (quantize A into
    the workspace, int8 GEMM, dequantize). dq_only: the int8 pair with an f16
    destination (the dequantizing output pass alone)."""
    import numpy as np
    w_h = dg.ints(702, (N, K), -127, 127)
    sb_h = dg.uniform(703, (N,), 0.001, 0.01)
    bias_h = dg.normal(704, (N,)).astype("float16")
    sa_h = dg.uniform(705, (M,), 0.01, 0.03)
    a_h = dg.act_s8(701, (M, K)) if dq_only else dg.normal(701, (M, K), 1.0).astype("float16")
    w = torch.from_numpy(w_h).cuda()
    sb = torch.from_numpy(sb_h).cuda()
    bias = torch.from_numpy(bias_h).cuda()
    c = torch.empty((M, N), dtype=torch.float16, device="cuda")
    sa = torch.from_numpy(sa_h).cuda()
    if dq_only:
        a = torch.from_numpy(a_h).cuda()
        op = na.Linear(output_dtype=na.DT_F16, act=na.EP_RELU)
        ins = [na.tensor(a, scale_data=sa, granularity=1), na.tensor(w, scale_data=sb, granularity=2),
               na.tensor(bias)]
    else:
        a = torch.from_numpy(a_h).cuda()
        op = na.MatMul(transpose_b=True, act=na.EP_RELU)
        ins = [na.tensor(a, scale_data=sa, granularity=1), na.tensor(w, scale_data=sb, granularity=2),
               na.tensor(bias)]
    outs = [na.tensor(c)]
    ws = torch.empty(max(op.workspace_size(ins, outs), 1), dtype=torch.uint8, device="cuda")
    s = stream.cuda_stream
    t = Timer(stream).time(lambda: op.compute(outs, ins, stream=s, workspace=ws), steps, warmup)
    ops = 2.0 * M * N * K
    tops = ops / (t["mean_ms"] * 1e-3) / 1e12
    out = {"tops": tops, "frac_int8_mfma": tops / PEAK_INT8_TOPS, "us": t["mean_ms"] * 1e3, "M": M, "N": N,
           "K": K, "route": "int8 pair -> f16 (dequantizing destination)" if dq_only
           else "f16 A (per-token QuantParams) x s8 -> f16"}
    if cpu_seconds > 0:
        import numpy as np
        cc = np.zeros((M, N), np.float16)
        out["cpu_baseline"] = cpu_call(
            lambda cpu, cores: cpu.ref_cpu_matmul_dq_f16(a_h.ctypes.data, int(not dq_only), sa_h.ctypes.data,
                                                         w_h.ctypes.data, sb_h.ctypes.data, bias_h.ctypes.data,
                                                         cc.ctypes.data, M, N, K, 1, cores),
            cpu_seconds, ops, "TOPS", f"{out['route']} {M}x{K}x{N} (nnops' CPU MatMul: "
                                      f"{'DqRoute' if dq_only else 'matmul_dq_from_fp'})")
    return out


def ceilings(torch, na, stream):
    """What this MI355X sustains outside our kernels: dense int8 MFMA fed
    from registers (random and constant operands: the power budget lowers the
    clock with the operands' switching), non-temporal streaming reads of 45 MiB
    and 180 MiB rotated over 8 buffers (the cfg3/cfg4 GEMV sizes; the fixed
    per-launch cost is the difference of the two), and an empty launch, each
    timed as a HIP graph of back-to-back launches like the workloads."""
    from nnops_amd import _lib as L
    lib = L.diag_lib()
    s = stream.cuda_stream
    out = torch.zeros(2048 * 256, dtype=torch.int32, device="cuda")
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (2048 * 256 * 24,), dtype=torch.int32, device="cuda")
    res = {}
    for constant in (0, 1):
        blocks, iters = 2048, 2000
        t = Timer(stream).time(lambda: lib.nnops_hip_diag_mfma_i8(src.data_ptr(), out.data_ptr(), blocks, iters,
                                                                  constant, s), 10, 3)
        ops = blocks * 4 * iters * 8 * 65536.0
        res["mfma_i8_tops_" + ("constant" if constant else "random")] = ops / (t["mean_ms"] * 1e-3) / 1e12
    for mib in (45, 180):
        nbuf = 8
        bufs = [torch.randint(0, 100, (mib * 2 ** 20,), dtype=torch.uint8, device="cuda") for _ in range(nbuf)]
        it = [0]

        def rd():
            b = bufs[it[0] % nbuf]
            it[0] += 1
            lib.nnops_hip_diag_stream_read(b.data_ptr(), b.numel(), out.data_ptr(), 1024, s)

        t = Timer(stream).time(rd, 40, 8)
        res[f"stream_read_{mib}MiB_us"] = t["mean_ms"] * 1e3
        res[f"stream_read_{mib}MiB_gbs"] = mib * 2 ** 20 / (t["mean_ms"] * 1e-3) / 1e9
        del bufs
    t = Timer(stream).time(lambda: lib.nnops_hip_diag_empty(out.data_ptr(), s), 100, 10)
    res["empty_launch_us"] = t["mean_ms"] * 1e3
    # two-point fit: t(bytes) = fixed + bytes / rate
    t45, t180 = res["stream_read_45MiB_us"], res["stream_read_180MiB_us"]
    rate = (180 - 45) * 2 ** 20 / ((t180 - t45) * 1e-6)
    res["stream_asymptotic_gbs"] = rate / 1e9
    res["stream_fixed_us"] = t45 - 45 * 2 ** 20 / rate * 1e6
    return res


def measured_traffic(kernel_key):
    """HBM bytes per launch of a kernel from the committed counter summary
    (two rocprofv3 --pmc passes, FETCH_SIZE and WRITE_SIZE, scaled by the same
    counters' reading of a plain copy of known size); None if absent."""
    path = os.path.join(ROOT, "profiles", "traffic_counters.txt")
    if not os.path.exists(path):
        return None
    vals = {}
    for line in open(path):
        line = line.strip()
        if line.startswith("#") or "=" not in line:
            continue
        k, v = line.split("=", 1)
        vals[k.strip()] = v.strip()
    try:
        fs, ws = float(vals["fetch_scale"]), float(vals["write_scale"])
        f = float(vals[f"{kernel_key}.fetch_kib"]) * fs
        w = float(vals[f"{kernel_key}.write_kib"]) * ws
    except (KeyError, ValueError):
        return None
    return (f + w) * 1024.0


def cpu_baseline(seconds):
    """nnops' own CPU path on a bounded sample of config 2: its MatMul int8
    route (AVX-512-VNNI panels, compiled from the reference sources into
    oracle/_ref/libnnops_cpu.so) on row blocks of the same 4096^3 problem, one
    call per block over a std::thread pool of this host's cores. Falls back to
    the reference's naive oracle (tests/reference/matmul_int8_ref) and then to
    the oracle port when those are what this host has."""
    import concurrent.futures as cf
    import numpy as np
    import oracle
    import datagen as dg
    M = N = K = 4096
    a = dg.act_s8(201, (M, K))
    w = dg.ints(202, (N, K), -127, 127)
    sb = dg.uniform(203, (N,), 0.001, 0.01)
    bias = dg.ints(204, (N,), -5000, 5000, np.int32)
    cores = max(1, min(16, len(os.sched_getaffinity(0))))
    out = np.zeros((M, N), np.int8)
    cpu = oracle.cpu_lib()
    if cpu is not None:
        # the whole problem per call; repeated until `seconds` have passed
        reps = 0
        t0 = time.perf_counter()
        while reps == 0 or time.perf_counter() - t0 < seconds:
            rc = cpu.ref_cpu_matmul_s8(a.ctypes.data, w.ctypes.data, bias.ctypes.data, out.ctypes.data, M, N, K,
                                       0.02, sb.ctypes.data, 0.05, 0, 1, cores)
            if rc != 0:
                raise RuntimeError(f"nnops CPU MatMul failed: status {rc}")
            reps += 1
        dt = time.perf_counter() - t0
        return {"value": 2.0 * reps * M * N * K / dt / 1e12, "unit": "TOPS", "cores": cores, "kind": "reference",
                "sample": f"config 2 in full (4096^3, s8 out, per-channel scales, bias, relu), {reps} calls in "
                          f"{dt:.1f}s; nnops' CPU MatMul (src/backend/cpu/matmul, AVX-512-VNNI) compiled from "
                          f"source, {cores} threads"}
    ref = oracle.ref_lib()
    rows_per = 8

    def block(r0):
        if ref is not None:
            ref.ref_matmul_int8(a[r0:].ctypes.data, w.ctypes.data, bias.ctypes.data, out[r0:].ctypes.data,
                                rows_per, N, K, K, K, N, 1, 0, None, 0.02, None, 0, sb.ctypes.data, 1.0,
                                None, 0, 0.05, 0, 1, 1)
        else:
            oracle.gemm_i8(a, w, trans_b=True, bias=bias, out_kind=oracle.OUT_S8, s_a=0.02, s_b=sb,
                           s_out=0.05, act=oracle.ACT_RELU, rows=(r0, r0 + rows_per), c=out)
        return rows_per

    done = 0
    t0 = time.perf_counter()
    with cf.ThreadPoolExecutor(cores) as ex:
        r = 0
        while time.perf_counter() - t0 < seconds and r < M:
            batch = list(range(r, min(M, r + rows_per * cores), rows_per))
            done += sum(ex.map(block, batch))
            r += rows_per * cores
    dt = time.perf_counter() - t0
    tops = 2.0 * done * N * K / dt / 1e12
    return {"value": tops, "unit": "TOPS", "cores": cores,
            "kind": "reference" if ref is not None else "port",
            "sample": f"config 2 rows [0,{done}) of 4096 (s8 out, per-channel scales, bias, relu) in "
                      f"{dt:.1f}s; " + ("nnops tests/reference/matmul_int8_ref (naive loops) compiled from source"
                                        if ref is not None else "oracle/oracle.c restatement")
                      + f", {cores} threads"}


# the kernels of each bench line whose HBM traffic per call the committed
# counter summary holds (profiles/traffic_counters.txt)
LINE_TRAFFIC = {
    "cfg1_s32_128x1024x1024": ["gemm_i8_ring_cfg1"],
    "cfg3_int8_gemv_m1_kn_s32": ["gemv_i8_kn_cfg3_m1", "gemm_i8_reduce_cfg3_m1"],
    "cfg3_int8_gemv_m1_kn_s8": ["gemv_i8_kn_cfg3_m1", "gemm_i8_reduce_cfg3_m1"],
    "cfg3_int8_gemv_m4_kn_s32": ["gemv_i8_kn_tr_cfg3_m4_m16"],
    "cfg3_int8_gemv_m4_kn_s8": ["gemv_i8_kn_tr_cfg3_m4_m16"],
    "cfg3_int8_gemv_m16_kn_s32": ["gemv_i8_kn_tr_cfg3_m4_m16"],
    "cfg3_int8_gemv_m16_kn_s8": ["gemv_i8_kn_tr_cfg3_m4_m16"],
    "cfg3_int8_gemv_m1_nk_s32": ["gemv_i8_rows_cfg3_m1"],
    "cfg3_int8_gemv_m4_nk_s32": ["gemv_i8_rows_cfg3_m4"],
    "cfg3_int8_gemv_m16_nk_s32": ["gemv_i8_lds_cfg3_m16"],
    "cfg3_int8_gemv_m1_kn_prepacked": ["gemv_i8_rows_cfg3_m1"],
    "cfg3_int8_gemv_m16_kn_prepacked": ["gemv_i8_lds_cfg3_m16"],
    "cfg4_q4_1_gemv_m1": ["gemv_q4_1_pipe_cfg4_m1"],
    "cfg4_q4_1_gemm_m512": ["gemm_q4_1_ring_cfg4_m512"],
    "cfg4_q4_1_gemv_m1_kn": ["gemv_q4_1_kn_dma_cfg4_m1"],
    "cfg4_q4_1_gemm_m512_kn": ["gemm_q4_1_kn_ring_cfg4_m512"],
    "cfg4_q4_1_m8_decode_batch": ["gemv_q4_1_skinny_cfg4_m8"],
    "cfg4_q4_1_gemm_m512_f32a": ["split_a_f32_cfg4_m512", "gemm_q4_1_ring_split_cfg4_m512"],
    "cfg4_q4_1_gemv_m1_kn_prepacked": ["gemv_q4_1_bcm_cfg4_m1_packed"],
    "cfg4_q4_1_gemm_m512_kn_prepacked": ["gemm_q4_1_kn_ring_cfg4_m512_packed"],
    "cfg4_q4_1_m8_decode_batch_kn_prepacked": ["gemv_q4_1_bcm_mfma_cfg4_m8_packed"],
    "gated_ffn_swiglu_m1": ["gemv_q4_1_pipe_gated_m1"],
    "gated_ffn_swiglu_m512": ["gemm_q4_1_ring_gated_m512"],
    "cfg5_s8_addto_gelu": ["gemm_i8_ring_cfg5", "gemm_i8_reduce_cfg5"],
    "dq_gemm_4096_f16_out": ["gemm_i8_ring_dq_f16"],
    "fp_act_matmul_4096_f16": ["quantize_linear_4096", "gemm_i8_ring_dq_f16"],
    "dense_f16_gemm_4096": ["gemm_f16_ring_4096"],
    "dense_f16_gemv_m1_14336x4096": ["gemv_fp_nk_f16_m1"],
    "quantize_linear_4096x4096_f16": ["quantize_linear_4096"],
    "dequantize_linear_4096x4096_f16": ["dequantize_linear_4096"],
}


def line_traffic(key):
    """HBM megabytes per call of a bench line's kernels from the counter
    summary, or None where it holds no figure for them."""
    keys = LINE_TRAFFIC.get(key)
    if not keys:
        return None
    vals = [measured_traffic(k) for k in keys]
    return None if any(v is None for v in vals) else round(sum(vals) / 1e6, 2)


def summarize(secondary):
    """One compact entry per secondary line: step time, fraction of the
    bounding roofline, the HBM megabytes per call its kernels moved (counter
    summary; null where none) and the CPU baseline (value, unit, threads) or
    the reason it is absent."""
    out = {}
    for key, r in secondary.items():
        frac = next((r[k] for k in ("frac_hbm", "frac_int8_mfma", "frac_f16_mfma", "frac_f32_mfma", "frac_mfma")
                     if k in r), None)
        bound = next((b for k, b in (("frac_hbm", "hbm"), ("frac_int8_mfma", "int8"), ("frac_f16_mfma", "f16"),
                                     ("frac_f32_mfma", "f32"), ("frac_mfma", "mfma")) if k in r), None)
        e = {"us": round(r["us"], 2), "frac": None if frac is None else round(frac, 3), "of": bound,
             "traffic_mb": line_traffic(key)}
        cb = r.get("cpu_baseline")
        if cb is None:
            e["cpu"] = None
        elif cb.get("value") is None:
            e["cpu"] = cb.get("sample", "n/a")[:90]
        else:
            e["cpu"] = [round(cb["value"], 2), cb["unit"], cb["cores"]]
        out[key] = e
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is designed, not implemented)"}))
        sys.exit(2)
    import torch
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import datagen as dg
    import nnops_amd as na
    na.load()
    stream = torch.cuda.Stream()

    if args.workload == "copy":
        # plain device copy of 256 MiB, the reference for scaling FETCH_SIZE /
        # WRITE_SIZE readings (profiles/traffic_counters.txt)
        x = torch.empty(2 ** 28, dtype=torch.uint8, device="cuda")
        x.fill_(1)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"workload": "copy", "bytes_per_copy": 2 ** 28, "copies": 3}))
        return
    if args.workload == "vendor":
        ours = {"cfg2_s8_ring": run_cfg2(args, torch, dg, na, stream)["ms"] * 1e3,
                "cfg4_q4_1_gemm_m512": q41_gemm_case(torch, dg, na, stream, max(5, args.steps // 5),
                                                     args.warmup)["us"]}
        print(json.dumps({"workload": "vendor", "vendor": vendor_reference(torch), "ours_us": ours}))
        return
    if args.workload == "ceilings":
        print(json.dumps({"workload": "ceilings", **ceilings(torch, na, stream)}))
        return
    cs = 0.0 if args.no_cpu_baseline else args.cpu_seconds_each
    if args.workload != "cfg2":
        res = {"cfg1": lambda: cfg1_case(torch, dg, na, stream, args.steps, args.warmup, cs),
               "cfg3": lambda: gemv_i8_case(torch, dg, na, stream, args.steps, args.warmup, cpu_seconds=cs),
               "cfg4": lambda: gemv_q41_case(torch, dg, na, stream, args.steps, args.warmup, cpu_seconds=cs),
               "cfg4_gemm": lambda: {"blocks_along_k": q41_gemm_case(torch, dg, na, stream, args.steps, args.warmup),
                                     "blocks_along_n": q41_gemm_case(torch, dg, na, stream, args.steps, args.warmup,
                                                                     trans_b=False)},
               "dense": lambda: {"f16_gemm_4096": dense_fp_case(torch, dg, na, stream, args.steps, args.warmup,
                                                                 M=4096),
                                 "f16_gemv_m1": dense_fp_case(torch, dg, na, stream, args.steps, args.warmup, M=1,
                                                              N=14336, nbuf=4)},
               "gated_ffn": lambda: {"m1": gated_ffn_case(torch, dg, na, stream, args.steps, args.warmup),
                                     "m512": gated_ffn_case(torch, dg, na, stream, args.steps, args.warmup,
                                                            M=512)},
               "cfg5": lambda: cfg5_case(torch, dg, na, stream, args.steps, args.warmup)}[args.workload]()
        print(json.dumps({"workload": args.workload, **res}))
        return

    main_res = run_cfg2(args, torch, dg, na, stream)
    secondary = {}
    if not args.no_secondary:
        st, wu = args.steps, args.warmup
        few = max(5, st // 5)
        secondary["cfg1_s32_128x1024x1024"] = cfg1_case(torch, dg, na, stream, st, wu, cs)
        for M in (1, 4, 16):
            for s8 in (False, True):
                secondary[f"cfg3_int8_gemv_m{M}_kn_{'s8' if s8 else 's32'}"] = gemv_i8_case(
                    torch, dg, na, stream, st, wu, M=M, trans_b=False, out_s8=s8, cpu_seconds=cs)
            secondary[f"cfg3_int8_gemv_m{M}_nk_s32"] = gemv_i8_case(torch, dg, na, stream, st, wu, M=M, trans_b=True,
                                                                   cpu_seconds=cs)
        for M in (1, 16):
            secondary[f"cfg3_int8_gemv_m{M}_kn_prepacked"] = gemv_i8_case(torch, dg, na, stream, st, wu, M=M,
                                                                         prepacked=True, cpu_seconds=cs)
        secondary["cfg4_q4_1_gemv_m1"] = gemv_q41_case(torch, dg, na, stream, st, wu, cpu_seconds=cs)
        secondary["cfg4_q4_1_gemm_m512"] = q41_gemm_case(torch, dg, na, stream, few, wu, cpu_seconds=cs)
        secondary["cfg4_q4_1_gemv_m1_kn"] = gemv_q41_case(torch, dg, na, stream, st, wu, trans_b=False,
                                                          cpu_seconds=cs)
        secondary["cfg4_q4_1_gemm_m512_kn"] = q41_gemm_case(torch, dg, na, stream, few, wu, trans_b=False,
                                                            cpu_seconds=cs)
        secondary["cfg4_q4_1_m8_decode_batch"] = q41_gemm_case(torch, dg, na, stream, st, wu, M=8, cpu_seconds=cs)
        secondary["cfg4_q4_1_gemm_m512_f32a"] = q41_gemm_case(torch, dg, na, stream, few, wu, a_f32=True,
                                                              cpu_seconds=cs)
        secondary["cfg4_q4_1_gemv_m1_kn_prepacked"] = q41_packed_case(torch, dg, na, stream, st, wu, M=1,
                                                                      cpu_seconds=cs)
        secondary["cfg4_q4_1_gemm_m512_kn_prepacked"] = q41_packed_case(torch, dg, na, stream, few, wu, M=512,
                                                                        cpu_seconds=cs)
        secondary["cfg4_q4_1_m8_decode_batch_kn_prepacked"] = q41_packed_case(torch, dg, na, stream, st, wu, M=8,
                                                                              cpu_seconds=cs)
        secondary["gated_ffn_swiglu_m1"] = gated_ffn_case(torch, dg, na, stream, st, wu, cpu_seconds=cs)
        secondary["gated_ffn_swiglu_m512"] = gated_ffn_case(torch, dg, na, stream, few, wu, M=512, cpu_seconds=cs)
        secondary["cfg5_s8_addto_gelu"] = cfg5_case(torch, dg, na, stream, few, wu)
        secondary["dq_gemm_4096_f16_out"] = fp_act_case(torch, dg, na, stream, few, wu, dq_only=True,
                                                        cpu_seconds=cs)
        secondary["fp_act_matmul_4096_f16"] = fp_act_case(torch, dg, na, stream, few, wu, cpu_seconds=cs)
        secondary["dense_f16_gemm_4096"] = dense_fp_case(torch, dg, na, stream, few, wu, M=4096, cpu_seconds=cs)
        secondary["dense_f16_gemv_m1_14336x4096"] = dense_fp_case(torch, dg, na, stream, st, wu, M=1, N=14336,
                                                                   nbuf=4, cpu_seconds=cs)
        secondary["quantize_linear_4096x4096_f16"] = qdq_case(torch, dg, na, stream, st, wu, cpu_seconds=cs)
        secondary["dequantize_linear_4096x4096_f16"] = qdq_case(torch, dg, na, stream, st, wu, dequant=True,
                                                                cpu_seconds=cs)
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds)
    line = {
        "metric": METRIC, "value": main_res["value"], "unit": main_res["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": main_res["ms"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": main_res["dtype"], "data": "synthetic (seeded xorshift128+, BASELINE config 2 distributions)",
        "config": main_res["config"], "roofline": main_res["roofline"], "cpu_baseline": cpu,
        "timing": main_res["timing"], "eager_ms_per_step": main_res["eager_ms_per_step"],
        "graph_ms_per_step": main_res["t"].get("graph_ms"),
        "summary": summarize(secondary),
    }
    # the full per-line records first, then the headline line (the last one,
    # kept short enough for a log tail to hold it whole)
    if secondary:
        print(json.dumps({"secondary_detail": secondary}))
    print(json.dumps(line))


if __name__ == "__main__":
    main()
