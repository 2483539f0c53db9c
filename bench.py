#!/usr/bin/env python3
"""bench.py — throughput of the MI355X dense-contraction hot path.

One JSON line on stdout. The headline workload (`--workload dit`, default)
is BASELINE configs[4]: the DiT/QwenImage transformer GEMMs in bf16 with f32
accumulation at M=4096 (QKV 3072→9216, MLP-up 3072→12288 + GELU, MLP-down
12288→3072). A "step" is one pass of the three Gemm calls (f32 activations
in HBM, rounded to bf16 on their way in, bf16 weights packed once). `value`
is step FLOPs / step wall time (TFLOPS).

The other BASELINE configs are measured in the same run and reported under
"workloads" (skip with --no-extra): the reference's Gemm+ReLU case,
BERT-base f32 projections,
int8 MatMulInteger + DequantizeLinear and decode GEMV M=1/4/16
(configs[3], weights rotated over 3 copies so HBM, not the 256 MB Infinity
Cache, serves them).

roofline: the dominant kernel's algorithmic FLOPs (or bytes) per launch over
its average launch duration in steady state (after ROOFLINE_WARM untimed
passes), timed with HIP events on the session stream (the stream the kernels
run on). roofline.traffic is the kernel's HBM bytes
per launch as counted by rocprofv3 (FETCH_SIZE + WRITE_SIZE, each scaled by
what the counter reads for a plain copy of known size) over `bench.py
--probe`; the summary, with its commands, is profiles/dit_gemm_traffic.md,
and bench.py reads the figure from there. cpu_baseline: the reference's amd64 CPU
algorithm restated in C++ (oracle/baseline.cpp, kind "port"), timed on a
bounded row sample of the same workload on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GEMM TFLOPS (bf16/fp32), int8 TOPS, GEMV HBM GB/s; % of MI355X roofline"
PEAK = {"bf16": 2516.6, "f32": 157.3, "i8": 5033.2, "hbm": 8000.0}  # TFLOP/s, TOP/s, GB/s
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "dit_gemm_traffic.md")
PROBE_COPY_BYTES = 256 << 20
# Untimed passes of the three DiT GEMMs before `roofline` times ten: about 30 ms of sustained load,
# over which the MI355X clock settles (it is still rising during the headline's warm-up when that
# is the driver's 5 steps), so `roofline` describes the kernel in steady state, as the profiles do.
ROOFLINE_WARM = 40


def measured_traffic():
    """HBM bytes per DiT GEMM launch from the committed rocprofv3 summary, or None."""
    try:
        with open(TRAFFIC_SUMMARY) as f:
            for line in f:
                if line.startswith("bytes_per_launch ="):
                    return int(line.split("=")[1])
    except OSError:
        pass
    return None


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def normal32(rng, shape, scale):
    return rng.normal(0, scale, shape).astype(np.float32)


def time_steps(sess, step, steps: int, warmup: int):
    for _ in range(warmup):
        step()
    sess.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    sess.sync()
    return (time.perf_counter() - t0) * 1e3 / steps


def cpu_info() -> dict:
    """The host CPU the baseline runs on: model, CPUs in this process's affinity mask, the threads used, and
    the micro-kernels the baseline's start-up probe picked (AVX-512 only when >5% faster than AVX2, VNNI int8
    when present: kernels/gemm/ukernel_amd64.go:65-93, kernels/gemm/qkernel_pick_amd64.go:18)."""
    import oracle

    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    affinity = len(os.sched_getaffinity(0))
    # all CPUs this process may run on (GOMAXPROCS = every core: the reference's INGOT_WORKERS=nproc), unless
    # the host declares a smaller CPU share for this job through OMP_NUM_THREADS
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(affinity, share) if share > 0 else affinity
    rule = (f"OMP_NUM_THREADS={share} (this job's CPU share) of {affinity} CPUs in the affinity mask"
            if 0 < share < affinity else f"every CPU in the affinity mask ({affinity})")
    kernel, vnni = oracle.base_active_kernel()
    return {"model": model, "affinity_cpus": affinity, "threads": threads, "threads_rule": rule,
            "f32_kernel": kernel, "int8_kernel": "avx512-vnni" if vnni else "avx2-madd"}


def cpu_time(fn, seconds: float):
    """Median wall time of fn() over repeated calls after one warm-up call, for about `seconds`."""
    fn()
    times, t_end = [], time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() >= t_end or len(times) >= 100000:
            break
    return float(np.median(times)), len(times)


def cpu_entry(value, unit, info, kind_sample, **extra):
    out = {"value": value, "unit": unit, "cores": info["threads"], "model": info["model"],
           "affinity_cpus": info["affinity_cpus"], "threads_rule": info["threads_rule"], "kernels": f"{info['f32_kernel']} f32, {info['int8_kernel']} int8",
           "kind": "port", "sample": kind_sample}
    out.update(extra)
    return out


def event_ms(sess, fn, reps: int, warm: int = 1) -> float:
    """Average GPU time of fn() (HIP events on the session stream) after `warm` untimed calls."""
    for _ in range(warm):
        fn()
    sess.sync()
    sess.timer_start()
    for _ in range(reps):
        fn()
    return sess.timer_stop() / reps


# ---------------- workloads ----------------

class Dit:
    name = "dit"
    seed = 20260405  # numpy PCG64 (np.random.default_rng), recorded in the JSON line
    shapes = [(3072, 9216, "qkv"), (3072, 12288, "mlp_up_gelu"), (12288, 3072, "mlp_down")]

    def __init__(self, sess, L):
        self.sess, self.L = sess, L
        rng = np.random.default_rng(self.seed)
        self.M = 4096
        self.a = {k: sess.to_device(rng.normal(0, 1, (self.M, k)).astype(np.float32)) for k in (3072, 12288)}
        self.w, self.y, self.acts = [], [], []
        for k, n, tag in self.shapes:
            # f32 N(0, 0.02) weights, packed once as bf16 (RNE) by the library
            self.w.append(sess.upload_weight(normal32(rng, (n, k), 0.02), trans=True, pack_dtype=L.DT_BF16))
            self.y.append(sess.empty(L.DT_F32, (self.M, n)))
            self.acts.append(L.ACT_GELU_ERF if tag.endswith("gelu") else L.ACT_NONE)
        self.flops = sum(2.0 * self.M * n * k for k, n, _ in self.shapes)
        self.calls = [sess.prepare_gemm(self.a[k], w, y, self.M, act=act, math=L.MATH_BF16)
                      for (k, n, _), w, y, act in zip(self.shapes, self.w, self.y, self.acts)]

    def step(self):
        for call in self.calls:
            call()

    def default_math_report(self, steps: int, warmup: int):
        """The same step under the library's default math for f32 A with bf16 weights: the f32-class hi/lo split
        (A = hi + lo, both bf16, two MFMA products per tile), standing in for the reference's f32 math over
        exactly widened bf16 weights (ops/matmul.go:77-137, kernels/gemm/gemm.go:920-962). It is what a caller
        gets without GPUBF16."""
        calls = [self.sess.prepare_gemm(self.a[k], w, y, self.M, act=act)
                 for (k, n, _), w, y, act in zip(self.shapes, self.w, self.y, self.acts)]

        def step():
            for call in calls:
                call()

        ms = time_steps(self.sess, step, steps, warmup)
        return {"TFLOPS": round(self.flops / (ms * 1e-3) / 1e12, 2), "ms_per_step": round(ms, 4),
                "math": "default (bf16 hi/lo split of f32 A, f32 accumulate)",
                "mfma_flops_per_step": 2 * self.flops,
                "note": "value counts the step's algorithmic FLOPs; the hi/lo kind issues twice as many MFMA FLOPs"}

    def kernel_roofline(self):
        """The bf16 MFMA GEMM kernel alone: activations already bf16 (one launch per Gemm)."""
        L, s = self.L, self.sess
        a16 = {}
        for k, t in self.a.items():
            a16[k] = s.empty(L.DT_BF16, (self.M, k))
            s.cast_bf16(t, a16[k])

        calls = [s.prepare_gemm(a16[k], w, y, self.M, act=act, a_dtype=L.DT_BF16)
                 for (k, n, _), w, y, act in zip(self.shapes, self.w, self.y, self.acts)]

        def launches():
            for call in calls:
                call()

        ms = event_ms(s, launches, 10, warm=ROOFLINE_WARM) / len(self.shapes)
        flops = self.flops / len(self.shapes)
        for t in a16.values():
            t.free()
        achieved = flops / (ms * 1e-3) / 1e12
        return {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK["bf16"], "unit": "TFLOP/s",
                "frac": round(achieved / PEAK["bf16"], 4), "traffic": measured_traffic(),
                "kernel": "gemm_kernel<bf16> (256x192 for QKV, 256x256 for MLP-up, 256x192 with register-staged weights for MLP-down)",
                "avg_launch_us": round(ms * 1e3, 2),
                "flops_per_launch": flops,
                "zero_operands": self.zero_operand_rate()}

    def zero_operand_rate(self):
        """The same kernels, shapes and launch order on all-zero A and weights. The schedule, the data movement
        and the instruction stream are identical; only the operand bits differ, so the gap to the random-data
        rate is what the operand values cost through the MFMA arrays' power draw (the clock drops under the
        power limit). Time bound by operand traffic (MLP-down in this order) is the same for both."""
        L, s = self.L, self.sess
        a16 = {k: s.empty(L.DT_BF16, (self.M, k)) for k in (3072, 12288)}
        for t in a16.values():
            s.memset(t, 0)
        ws = [s.upload_weight(np.zeros((n, k), np.float32), trans=True, pack_dtype=L.DT_BF16)
              for k, n, _ in self.shapes]
        calls = [s.prepare_gemm(a16[k], w, y, self.M, act=act, a_dtype=L.DT_BF16)
                 for (k, n, _), w, y, act in zip(self.shapes, ws, self.y, self.acts)]

        def launches():
            for call in calls:
                call()

        ms = event_ms(s, launches, 10, warm=ROOFLINE_WARM) / len(self.shapes)
        for t in a16.values():
            t.free()
        for w in ws:
            w.free()
        achieved = self.flops / len(self.shapes) / (ms * 1e-3) / 1e12
        return {"achieved": round(achieved, 1), "frac": round(achieved / PEAK["bf16"], 4),
                "avg_launch_us": round(ms * 1e3, 2)}

    def compare_hipblaslt(self, reps: int = 20):
        """The bf16 GEMM kernel against hipBLASLt (torch.mm with bf16 operands and f32 output, the same output
        type as the Gemm op) on the same operand values, per DiT GEMM: each side timed with HIP events over
        `reps` back-to-back launches on its own stream, four times, alternating (the first rounds run while
        the clock settles, so the minimum is compared). Neither includes the activation pack. Prints one
        JSON line per GEMM."""
        import torch

        L, s = self.L, self.sess
        rng = np.random.default_rng(self.seed)
        for (k, n, tag), act in zip(self.shapes, self.acts):
            a = rng.normal(0, 1, (self.M, k)).astype(np.float32)
            w = normal32(rng, (n, k), 0.02)
            da = s.to_device(a)
            a16 = s.empty(L.DT_BF16, (self.M, k))
            s.cast_bf16(da, a16)
            wt = s.upload_weight(w, trans=True, pack_dtype=L.DT_BF16)
            y = s.empty(L.DT_F32, (self.M, n))
            call = s.prepare_gemm(a16, wt, y, self.M, a_dtype=L.DT_BF16)
            ta = torch.from_numpy(a).to("cuda").to(torch.bfloat16)
            tw = torch.from_numpy(w).to("cuda").to(torch.bfloat16)

            def blas():
                return torch.mm(ta, tw.t(), out_dtype=torch.float32)

            def blas_ms():
                for _ in range(3):
                    blas()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(reps):
                    blas()
                e1.record()
                torch.cuda.synchronize()
                return e0.elapsed_time(e1) / reps

            ours, theirs = [], []
            for _ in range(4):
                ours.append(event_ms(s, call, reps) * 1e3)
                theirs.append(blas_ms() * 1e3)
            flops = 2.0 * self.M * n * k
            print(json.dumps({"gemm": f"{tag} {self.M}x{k}x{n}", "ours_us": [round(v, 1) for v in ours],
                              "hipblaslt_us": [round(v, 1) for v in theirs],
                              "ours_tflops": round(flops / (min(ours) * 1e-6) / 1e12, 1),
                              "hipblaslt_tflops": round(flops / (min(theirs) * 1e-6) / 1e12, 1),
                              "epilogue": "none on either side"}),
                  flush=True)
            for t in (da, a16, y):
                t.free()
            wt.free()
            del ta, tw
        self.compare_hipblaslt_sequence()

    def compare_hipblaslt_sequence(self, reps: int = 10, rounds: int = 4):
        """The same comparison in the bench's order (QKV, MLP-up, MLP-down, repeated; no epilogue on either
        side), after about a second of both sequences: per-launch HIP events, medians per round, the two sides
        alternating round by round. One JSON line."""
        import ctypes as C

        import torch

        L, s = self.L, self.sess
        rng = np.random.default_rng(self.seed)
        ours, theirs = {}, {}
        keep = []
        for k, n, tag in self.shapes:
            a = rng.normal(0, 1, (self.M, k)).astype(np.float32)
            w = normal32(rng, (n, k), 0.02)
            da = s.to_device(a)
            a16 = s.empty(L.DT_BF16, (self.M, k))
            s.cast_bf16(da, a16)
            wt = s.upload_weight(w, trans=True, pack_dtype=L.DT_BF16)
            y = s.empty(L.DT_F32, (self.M, n))
            ours[tag] = s.prepare_gemm(a16, wt, y, self.M, a_dtype=L.DT_BF16)
            ta = torch.from_numpy(a).to("cuda").to(torch.bfloat16)
            tw = torch.from_numpy(w).to("cuda").to(torch.bfloat16)
            theirs[tag] = (lambda ta=ta, tw=tw: torch.mm(ta, tw.t(), out_dtype=torch.float32))
            keep += [da, a16, y, wt, ta, tw]
        st = C.c_void_p()
        L.check(s.lib.ingot_rocm_stream(s.h, C.byref(st)))
        ext = torch.cuda.ExternalStream(st.value)
        cur = torch.cuda.current_stream()
        tags = [t for _, _, t in self.shapes]

        def timed(fns, stream, n):
            evs = []
            for _ in range(n):
                for t in tags:
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    fns[t]()
                    e1.record(stream)
                    evs.append((t, e0, e1))
            s.sync()
            torch.cuda.synchronize()
            out = {}
            for t, e0, e1 in evs:
                out.setdefault(t, []).append(e0.elapsed_time(e1) * 1e3)
            return {t: round(float(np.median(v)), 1) for t, v in out.items()}

        t_end = time.perf_counter() + 1.0
        while time.perf_counter() < t_end:
            timed(ours, ext, 2)
            timed(theirs, cur, 2)
        r_ours, r_theirs = [], []
        for _ in range(rounds):
            r_ours.append(timed(ours, ext, reps))
            r_theirs.append(timed(theirs, cur, reps))
        avg = lambda r: round(sum(r.values()) / len(r), 1)
        print(json.dumps({"sequence": "qkv, mlp_up (no epilogue), mlp_down, repeated", "ours_us": r_ours,
                          "hipblaslt_us": r_theirs, "ours_avg_per_round": [avg(r) for r in r_ours],
                          "hipblaslt_avg_per_round": [avg(r) for r in r_theirs]}), flush=True)
        for t in keep:
            if hasattr(t, "free"):
                t.free()

    def sequence_probe(self, reps: int = 10):
        """Per-launch GPU time of each DiT GEMM kernel (bf16 activations, as `roofline` launches them) in four
        orders: the bench's sequence (QKV, MLP-up, MLP-down, repeated), one GEMM repeated alone (its operands stay
        in the Infinity Cache), and each GEMM after filling 1 GiB (a write pass: the cache full of dirty lines)
        or after reading 1 GiB (a 1 GiB f32 → bf16 cast: mostly clean lines). HIP events on the session stream
        around each launch, no synchronisation between launches; medians over `reps`. INGOT_GEMM_CFG selects a
        tile for all three GEMMs. The sequence runs for about a second first, and is measured again at the end.
        One JSON line."""
        import ctypes as C

        import torch

        L, s = self.L, self.sess
        a16 = {}
        for k, t in self.a.items():
            a16[k] = s.empty(L.DT_BF16, (self.M, k))
            s.cast_bf16(t, a16[k])
        calls = {tag: s.prepare_gemm(a16[k], w, y, self.M, act=act, a_dtype=L.DT_BF16)
                 for (k, n, tag), w, y, act in zip(self.shapes, self.w, self.y, self.acts)}
        fill = s.empty(L.DT_U8, (1 << 30,))
        src, dst = s.empty(L.DT_F32, (1 << 28,)), s.empty(L.DT_BF16, (1 << 28,))
        st = C.c_void_p()
        L.check(s.lib.ingot_rocm_stream(s.h, C.byref(st)))
        ext = torch.cuda.ExternalStream(st.value)

        def timed(order, n):
            evs = []
            for _ in range(n):
                for item in order:
                    if isinstance(item, str):
                        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                        e0.record(ext)
                        calls[item]()
                        e1.record(ext)
                        evs.append((item, e0, e1))
                    else:
                        item()
            s.sync()
            torch.cuda.synchronize()
            out = {}
            for tag, e0, e1 in evs:
                out.setdefault(tag, []).append(e0.elapsed_time(e1) * 1e3)
            return {t: round(float(np.median(v)), 1) for t, v in out.items()}

        tags = [t for _, _, t in self.shapes]
        wflush, rflush = (lambda: s.memset(fill, 0)), (lambda: s.cast_bf16(src, dst))
        t_end = time.perf_counter() + 1.0  # about a second of the sequence first: the clock leaves its idle state
        while time.perf_counter() < t_end:
            timed(tags, 4)
        res = {"gemm_cfg": os.environ.get("INGOT_GEMM_CFG", "default"), "sequence": timed(tags, reps)}
        res["alone"] = {t: timed([t], reps)[t] for t in tags}
        res["after_1GiB_fill"] = timed([x for t in tags for x in (wflush, t)], reps // 2)
        res["after_1GiB_read"] = timed([x for t in tags for x in (rflush, t)], reps // 2)
        res["sequence_again"] = timed(tags, reps)
        print(json.dumps(res), flush=True)
        for t in list(a16.values()) + [fill, src, dst]:
            t.free()

    def probe(self):
        """One plain copy of PROBE_COPY_BYTES (counter calibration), then one launch of each GEMM."""
        L, s = self.L, self.sess
        src, dst = s.empty(L.DT_U8, (PROBE_COPY_BYTES,)), s.empty(L.DT_U8, (PROBE_COPY_BYTES,))
        s.memset(src, 1)
        s.copy_d2d(dst, src)
        a16 = {}
        for k, t in self.a.items():
            a16[k] = s.empty(L.DT_BF16, (self.M, k))
            s.cast_bf16(t, a16[k])
        for (k, n, _), w, y, act in zip(self.shapes, self.w, self.y, self.acts):
            s.gemm(a16[k], w, y, self.M, act=act, a_dtype=L.DT_BF16)
        s.sync()

    def cpu_baseline(self, info, seconds: float):
        import oracle

        rng = np.random.default_rng(self.seed)
        rows = 288  # two MC blocks of the reference's blocking, per GEMM
        packs = [oracle.PackedB(oracle.f32_to_bf16(normal32(rng, (n, k), 0.02)), trans_b=True, bf16=True)
                 for k, n, _ in self.shapes]
        a = {k: rng.normal(0, 1, (rows, k)).astype(np.float32) for k in (3072, 12288)}
        outs = [np.empty((rows, n), np.float32) for _, n, _ in self.shapes]

        def once():
            for (k, n, tag), pb, o in zip(self.shapes, packs, outs):
                oracle.base_sgemm(a[k], pb, gelu=tag.endswith("gelu"), threads=info["threads"], out=o)

        t, reps = cpu_time(once, seconds)
        flops = sum(2.0 * rows * n * k for k, n, _ in self.shapes)
        return cpu_entry(round(flops / t / 1e12, 4), "TFLOPS", info,
                         f"the 3 DiT GEMMs on {rows} of 4096 rows (bf16 weights widened per panel, f32 A); "
                         f"median of {reps} passes", ms_per_step_full=round(t * 4096 / rows * 1e3, 2))


class GemmRelu:
    """BASELINE configs[0], the reference's own CPU-runnable case: one ONNX Gemm, Y = ReLU(A·Bᵀ + bias), f32,
    A [128,256] ~U(-1,1), B [512,256] ~U(-1,1) (transB = 1), bias [512] ~N(0,0.1), ReLU fused into the store.
    33.6 MFLOP per call: launch-bound, so also reported as µs per call (HIP events, back-to-back calls)."""
    name = "gemm_relu"
    seed = 7  # numpy PCG64 (np.random.default_rng), recorded in the JSON line

    def __init__(self, sess, L):
        rng = np.random.default_rng(self.seed)
        self.sess = sess
        self.M, self.K, self.N = 128, 256, 512
        a = sess.to_device(rng.uniform(-1, 1, (self.M, self.K)).astype(np.float32))
        self.w = sess.upload_weight(rng.uniform(-1, 1, (self.N, self.K)).astype(np.float32), trans=True,
                                    pack_dtype=L.DT_F32)
        b = sess.to_device(rng.normal(0, 0.1, self.N).astype(np.float32))
        self.y = sess.empty(L.DT_F32, (self.M, self.N))
        self.keep = (a, b)
        self.call = sess.prepare_gemm(a, self.w, self.y, self.M, beta=1.0, c=b, c_mode=L.C_ROW, act=L.ACT_RELU)
        self.flops = 2.0 * self.M * self.N * self.K

    def step(self):
        self.call()

    def report(self, ms):
        us = event_ms(self.sess, self.call, 200) * 1e3
        return {"value": round(self.flops / (us * 1e-6) / 1e12, 3), "unit": "TFLOPS", "us_per_call": round(us, 2),
                "ms_per_step": round(ms, 4), "dtype": "f32"}

    def cpu_baseline(self, info, seconds: float):
        """The whole op on the host: packed-B f32 GEMM with the bias at the store, then the separate Relu node."""
        import oracle

        rng = np.random.default_rng(self.seed)
        a = rng.uniform(-1, 1, (self.M, self.K)).astype(np.float32)
        pb = oracle.PackedB(rng.uniform(-1, 1, (self.N, self.K)).astype(np.float32), trans_b=True, bf16=False)
        bias = rng.normal(0, 0.1, self.N).astype(np.float32)
        y = np.empty((self.M, self.N), np.float32)

        def once():
            oracle.base_sgemm(a, pb, bias=bias, threads=info["threads"], out=y)
            np.maximum(y, 0, out=y)

        t, reps = cpu_time(once, seconds)
        return cpu_entry(round(self.flops / t / 1e12, 4), "TFLOPS", info,
                         f"the full Gemm+ReLU (128x256 . 512); median of {reps} calls", us_per_call=round(t * 1e6, 2))


class Bert:
    name = "bert"
    seed = 1  # numpy PCG64 (np.random.default_rng), recorded in the JSON line
    shapes = [(768, 2304, 0), (768, 768, 0), (768, 3072, 1), (3072, 768, 0)]

    def __init__(self, sess, L):
        self.sess, self.L = sess, L
        rng = np.random.default_rng(self.seed)
        self.M = 1024
        self.a = {k: sess.to_device(rng.normal(0, 1, (self.M, k)).astype(np.float32)) for k in (768, 3072)}
        self.w, self.b, self.y = [], [], []
        for k, n, _ in self.shapes:
            self.w.append(sess.upload_weight(rng.normal(0, 0.02, (k, n)).astype(np.float32), trans=False,
                                             pack_dtype=L.DT_F32))
            self.b.append(sess.to_device(rng.normal(0, 0.02, n).astype(np.float32)))
            self.y.append(sess.empty(L.DT_F32, (self.M, n)))
        self.flops = sum(2.0 * self.M * n * k for k, n, _ in self.shapes)
        self.calls = [sess.prepare_gemm(self.a[k], w, y, self.M, beta=1.0, c=b, c_mode=L.C_ROW,
                                        act=L.ACT_GELU_ERF if gelu else L.ACT_NONE)
                      for (k, n, gelu), w, b, y in zip(self.shapes, self.w, self.b, self.y)]

    def step(self):
        for call in self.calls:
            call()

    def probe(self):
        """One launch of each BERT projection (for rocprofv3 --pmc)."""
        self.step()
        self.sess.sync()

    def report(self, ms):
        v = self.flops / (ms * 1e-3) / 1e12
        return {"value": round(v, 2), "unit": "TFLOPS", "ms_per_step": round(ms, 4), "dtype": "f32",
                "roofline_frac": round(v / PEAK["f32"], 4), "peak": PEAK["f32"]}

    def cpu_baseline(self, info, seconds: float):
        """The four projections at full size: packed-B f32 GEMMs with the bias at the store, GELU per finished
        strip on FFN-up (SgemmPackedBEpi)."""
        import oracle

        rng = np.random.default_rng(self.seed)
        a = {k: rng.normal(0, 1, (self.M, k)).astype(np.float32) for k in (768, 3072)}
        packs = [oracle.PackedB(rng.normal(0, 0.02, (k, n)).astype(np.float32), trans_b=False, bf16=False)
                 for k, n, _ in self.shapes]
        biases = [rng.normal(0, 0.02, n).astype(np.float32) for _, n, _ in self.shapes]
        outs = [np.empty((self.M, n), np.float32) for _, n, _ in self.shapes]

        def once():
            for (k, n, gelu), pb, b, o in zip(self.shapes, packs, biases, outs):
                oracle.base_sgemm(a[k], pb, bias=b, gelu=bool(gelu), threads=info["threads"], out=o)

        t, reps = cpu_time(once, seconds)
        return cpu_entry(round(self.flops / t / 1e12, 4), "TFLOPS", info,
                         f"the 4 BERT projections at M = 1024; median of {reps} passes", ms_per_step=round(t * 1e3, 3))


class Int8:
    name = "int8"
    seed = 3  # numpy PCG64 (np.random.default_rng), recorded in the JSON line

    def __init__(self, sess, L):
        self.sess, self.L = sess, L
        rng = np.random.default_rng(self.seed)
        self.M, self.K, self.N = 1024, 768, 3072
        self.a = sess.to_device(rng.integers(0, 256, (self.M, self.K)).astype(np.uint8), L.DT_U8)
        self.w = sess.upload_weight(rng.integers(-127, 128, (self.K, self.N)).astype(np.int8), trans=False,
                                    pack_dtype=L.DT_I8)
        sc = (rng.uniform(0.001, 0.01, self.N).astype(np.float32) * np.float32(0.02)).astype(np.float32)
        self.scale = sess.to_device(sc)
        self.y = sess.empty(L.DT_F32, (self.M, self.N))
        self.ops = 2.0 * self.M * self.N * self.K
        self.bytes = self.M * self.K + self.K * self.N + 4 * self.M * self.N
        self.call = sess.prepare_matmul_integer(self.a, self.w, self.M, 128, scale=self.scale, y_f32=self.y)

    def step(self):
        self.call()

    def probe(self):
        """One plain copy of PROBE_COPY_BYTES (counter calibration), then one MatMulInteger + dequant call."""
        L, s = self.L, self.sess
        src, dst = s.empty(L.DT_U8, (PROBE_COPY_BYTES,)), s.empty(L.DT_U8, (PROBE_COPY_BYTES,))
        s.memset(src, 1)
        s.copy_d2d(dst, src)
        self.call()
        s.sync()

    def report(self, ms):
        tops = self.ops / (ms * 1e-3) / 1e12
        gbs = self.bytes / (ms * 1e-3) / 1e9
        return {"value": round(tops, 2), "unit": "TOPS", "ms_per_step": round(ms, 4), "dtype": "i8",
                "us_per_call": round(ms * 1e3, 2), "GB_per_s": round(gbs, 1), "hbm_frac": round(gbs / PEAK["hbm"], 4),
                "mfma_frac": round(tops / PEAK["i8"], 4)}

    def cpu_baseline(self, info, seconds: float):
        """The full MatMulInteger (exact int32, VNNI when the host has it) then the per-column dequantisation
        pass (the reference's separate DequantizeLinear node)."""
        import oracle

        rng = np.random.default_rng(self.seed)
        a = rng.integers(0, 256, (self.M, self.K)).astype(np.uint8)
        bt = np.ascontiguousarray(rng.integers(-127, 128, (self.K, self.N)).astype(np.int8).T)
        sc = (rng.uniform(0.001, 0.01, self.N).astype(np.float32) * np.float32(0.02)).astype(np.float32)
        y = np.empty((self.M, self.N), np.float32)

        def once():
            yi = oracle.base_qgemm(a, bt, 128, threads=info["threads"])
            np.multiply(yi.astype(np.float32), sc, out=y)

        t, reps = cpu_time(once, seconds)
        return cpu_entry(round(self.ops / t / 1e12, 4), "TOPS", info,
                         f"the full MatMulInteger + DequantizeLinear; median of {reps} calls",
                         us_per_call=round(t * 1e6, 1))


class Decode:
    name = "decode"
    seed = 4  # numpy PCG64 (np.random.default_rng), recorded in the JSON line
    shapes = [(2048, 6144), (2048, 2048), (2048, 11264), (5632, 2048)]
    copies = 3  # > 256 MB of weights in rotation: HBM, not the Infinity Cache

    def __init__(self, sess, L, M=1):
        self.sess, self.L, self.M = sess, L, M
        rng = np.random.default_rng(self.seed)
        self.x = {k: sess.to_device(rng.normal(0, 1, (16, k)).astype(np.float32)) for k in (2048, 5632)}
        self.w = [[sess.upload_weight(normal32(rng, (n, k), 0.02), trans=True, pack_dtype=L.DT_BF16)
                   for k, n in self.shapes] for _ in range(self.copies)]
        self.y = [sess.empty(L.DT_F32, (16, n)) for _, n in self.shapes]
        self.i = 0
        self.wbytes = sum(2.0 * n * k for k, n in self.shapes)
        # prepared calls per (M, weight copy): argument blocks built once
        self.calls = {M: [[sess.prepare_gemm(self.x[k], w, y, M) for (k, n), w, y in zip(self.shapes, ws, self.y)]
                          for ws in self.w] for M in (1, 4, 16)}

    def compare_stream_read(self, reps: int = 20):
        """The M = 1 GEMV of each decode shape against reading the same weight bytes with vendor code: a
        torch.sum over a bf16 tensor of the weight's shape (torch's reduction kernel, f32 accumulation), and a
        device-to-device torch copy of the same bytes (which also writes them). Each side rotates over as many
        distinct buffers as exceed 320 MB together (beyond the 256 MB Infinity Cache, so HBM serves them), timed
        with HIP events over `reps` passes, four alternating rounds; the minimum of each is compared. One JSON
        line per shape."""
        import torch

        s = self.sess
        rng = np.random.default_rng(self.seed)
        for j, (k, n) in enumerate(self.shapes):
            copies = int(np.ceil(320e6 / (2.0 * n * k)))
            wh = normal32(rng, (n, k), 0.02)
            tw = [torch.from_numpy(wh).to("cuda").to(torch.bfloat16) for _ in range(copies)]
            dst = torch.empty_like(tw[0])
            ws = [s.upload_weight(wh, trans=True, pack_dtype=self.L.DT_BF16) for _ in range(copies)]
            calls = [s.prepare_gemm(self.x[k], w, self.y[j], 1) for w in ws]

            def ours():
                for call in calls:
                    call()

            def torch_ms(fn):
                fn()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(reps):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                return e0.elapsed_time(e1) / reps

            def tsum():
                for t in tw:
                    torch.sum(t, dtype=torch.float32)

            def copy():
                for t in tw:
                    dst.copy_(t)

            g, r, cp = [], [], []
            for _ in range(4):
                g.append(event_ms(s, ours, reps) / copies * 1e3)
                r.append(torch_ms(tsum) / copies * 1e3)
                cp.append(torch_ms(copy) / copies * 1e3)
            wb = 2.0 * n * k
            print(json.dumps({"shape": f"{k}x{n}", "weight_MB": round(wb / 1e6, 2), "copies": copies,
                              "gemv_m1_us": round(min(g), 2), "gemv_m1_GB_per_s": round(wb / min(g) / 1e3, 1),
                              "torch_sum_us": round(min(r), 2), "torch_sum_GB_per_s": round(wb / min(r) / 1e3, 1),
                              "d2d_copy_us": round(min(cp), 2), "d2d_copy_read_GB_per_s": round(wb / min(cp) / 1e3, 1)}),
                  flush=True)
            del tw, dst
            for w in ws:
                w.free()

    def bytes_step(self, M):
        return self.wbytes + sum(4.0 * M * (k + n) for k, n in self.shapes)

    def probe(self):
        """One plain copy of PROBE_COPY_BYTES (counter calibration), then one step at M = 1, 4 and 16, each on
        its own weight copy."""
        L, s = self.L, self.sess
        src, dst = s.empty(L.DT_U8, (PROBE_COPY_BYTES,)), s.empty(L.DT_U8, (PROBE_COPY_BYTES,))
        s.memset(src, 1)
        s.copy_d2d(dst, src)
        for c, M in enumerate((1, 4, 16)):
            for call in self.calls[M][c]:
                call()
        s.sync()

    def step(self, M=None):
        M = M or self.M
        calls = self.calls[M][self.i % self.copies]
        self.i += 1
        for call in calls:
            call()

    def kernels(self, M):
        """Which kernel each shape runs at this M (the routing of gemm_core: the decode GEMV for M <= 4, and
        for M = 5..16 when N < 4096; the tiled GEMM otherwise)."""
        return {f"{k}x{n}": "gemv" if M <= 4 or (M <= 16 and n < 4096) else "gemm" for k, n in self.shapes}

    def report(self):
        out = {}
        for M in (1, 4, 16):
            ms = time_steps(self.sess, lambda: self.step(M), 60, 10)
            gbs = self.bytes_step(M) / (ms * 1e-3) / 1e9
            kern = self.kernels(M)
            leg = {"GB_per_s": round(gbs, 1), "us_per_step": round(ms * 1e3, 2), "kernels": kern}
            if all(v == "gemv" for v in kern.values()):
                leg["hbm_frac"] = round(gbs / PEAK["hbm"], 4)
            else:
                # a decode-step rate (weight + activation bytes over the step), not one kernel's HBM roofline
                leg["step_bytes_frac_of_hbm"] = round(gbs / PEAK["hbm"], 4)
            out[f"m{M}"] = leg
        # per-shape time at M = 1: back-to-back launches of one shape (HIP events) rotating over as many copies
        # of its weight as exceed 320 MB together, so HBM serves them and not the 256 MB Infinity Cache
        # (three copies of one shape would fit in it)
        per = {}
        rng = np.random.default_rng(self.seed + 7)
        for j, (k, n) in enumerate(self.shapes):
            wb = 2.0 * n * k
            wh = normal32(rng, (n, k), 0.02)
            ws = [self.sess.upload_weight(wh, trans=True, pack_dtype=self.L.DT_BF16)
                  for _ in range(int(np.ceil(320e6 / wb)))]
            calls = [self.sess.prepare_gemm(self.x[k], w, self.y[j], 1) for w in ws]

            def launches():
                for call in calls:
                    call()
            ms = event_ms(self.sess, launches, 10) / len(calls)
            b = wb + 4.0 * (k + n)
            per[f"{k}x{n}"] = {"us": round(ms * 1e3, 2), "GB_per_s": round(b / (ms * 1e-3) / 1e9, 1),
                               "copies": len(calls)}
            for w in ws:
                w.free()
        out["m1_per_shape"] = per
        # the same step on grouped-int8 weights (ingot_weight_quant="int8"): bytes = int8 weights + f32 scales
        L = self.L
        wq = [[self.sess.upload_weight(normal32(np.random.default_rng(self.seed + 1 + c), (n, k), 0.02), trans=True,
                                       pack_dtype=L.PACK_I8G) for k, n in self.shapes] for c in range(self.copies)]
        i = [0]

        qcalls = [[self.sess.prepare_gemm(self.x[k], w, y, 1) for (k, n), w, y in zip(self.shapes, ws, self.y)]
                  for ws in wq]

        def step_i8g():
            calls = qcalls[i[0] % self.copies]
            i[0] += 1
            for call in calls:
                call()
        ms = time_steps(self.sess, step_i8g, 60, 10)
        qbytes = sum(n * k + 4.0 * n * k / 64 + 4.0 * (k + n) for k, n in self.shapes)
        out["m1_i8g"] = {"GB_per_s": round(qbytes / (ms * 1e-3) / 1e9, 1), "us_per_step": round(ms * 1e3, 2),
                         "bytes_per_step": qbytes}
        for cp in wq:
            for w in cp:
                w.free()
        return out

    def cpu_baseline(self, info, seconds: float):
        """The M = 1 decode step on the host: the four bf16-weight GEMVs with a widening dot (GemvBF16),
        successive steps rotating over four copies of the weights (412 MB), so that the host's caches cannot
        hold the weights of the step they serve, as the GPU side rotates its copies beyond the Infinity Cache."""
        import oracle

        rng = np.random.default_rng(self.seed)
        xs = {k: rng.normal(0, 1, (1, k)).astype(np.float32) for k in (2048, 5632)}
        ws = [oracle.f32_to_bf16(normal32(rng, (n, k), 0.02)) for k, n in self.shapes]
        copies = 4
        sets = [ws] + [[w.copy() for w in ws] for _ in range(copies - 1)]
        turn = [0]

        def once():
            cur = sets[turn[0] % copies]
            turn[0] += 1
            for (k, n), w in zip(self.shapes, cur):
                oracle.base_gemv_bf16(xs[k], w, threads=info["threads"])

        t, reps = cpu_time(once, seconds)
        return cpu_entry(round(self.bytes_step(1) / t / 1e9, 2), "GB/s", info,
                         f"the M = 1 decode step (4 GEMVs, 103 MB of bf16 weights), steps rotating over {copies} "
                         f"weight copies ({copies * self.wbytes / 1e6:.0f} MB); median of {reps} steps",
                         us_per_step=round(t * 1e6, 1))


class FfnGraph:
    """BERT FFN block (configs[1] shapes) as a graph session: MatMul+Add → GELU → MatMul+Add, planned with
    fuseMatMulBias + epilogue activations in f32, and under GPUBF16 (bf16 products, bf16-resident hidden)."""
    name = "ffn_graph"
    seed = 6  # numpy PCG64 (np.random.default_rng), recorded in the JSON line
    TEXT = """
input x f32 1024,768
const W1 f32 768,3072
const b1 f32 3072
const W2 f32 3072,768
const b2 f32 768
node MatMul x,W1 -> h1
node Add h1,b1 -> h2
node ingot.Gelu h2 -> h3
node MatMul h3,W2 -> h4
node Add h4,b2 -> y
output y
"""

    def __init__(self, sess, L):
        from ingot_amd import Graph
        self.sess, self.L = sess, L
        rng = np.random.default_rng(self.seed)
        self.x = sess.to_device(rng.normal(0, 1, (1024, 768)).astype(np.float32))
        self.c = {"W1": normal32(rng, (768, 3072), 0.02), "b1": normal32(rng, (3072,), 0.02),
                  "W2": normal32(rng, (3072, 768), 0.02), "b2": normal32(rng, (768,), 0.02)}
        self.c = {k: sess.to_device(v) for k, v in self.c.items()}
        self.graphs = {}
        base = L.GRAPH_FUSE_BIAS | L.GRAPH_FUSE_ACT
        for mode, flags in (("f32", base), ("gpubf16", base | L.GRAPH_HALF)):
            g = Graph(sess, self.TEXT)
            for k, v in self.c.items():
                g.bind(k, v)
            g.compile(flags)
            self.graphs[mode] = g
        self.flops = 2 * 2.0 * 1024 * 768 * 3072

    def report(self):
        out = {}
        for mode, g in self.graphs.items():
            def step(g=g):
                (y,) = g.run({"x": self.x})
                y.free()
            ms = time_steps(self.sess, step, 50, 10)
            out[mode] = {"TFLOPS": round(self.flops / (ms * 1e-3) / 1e12, 2), "us_per_step": round(ms * 1e3, 2),
                         "plan": g.stats()}
        return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=20)
    # The clock settles over the first ~40 DiT steps (~35 ms) of sustained load: per block of 10
    # steps on MI355X 1.37 (first launches), 0.86, 0.84, 0.83, 0.82 ms, then 0.81-0.82 ms for the
    # next 350 steps. 50 untimed steps put the timed ones in that steady state.
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="dit", choices=["dit", "bert", "int8", "decode"])
    ap.add_argument("--no-extra", action="store_true", help="measure only the headline workload")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=8.0, help="CPU-baseline time budget of the DiT leg")
    ap.add_argument("--cpu-seconds-extra", type=float, default=3.0,
                    help="CPU-baseline time budget of each other workload")
    ap.add_argument("--probe", nargs="?", const="dit",
                    choices=["dit", "decode", "bert", "int8", "hipblaslt", "streamread", "sequence"],
                    help="counter probe for rocprofv3 --pmc: one calibration copy, then one launch of each DiT GEMM "
                         "(dit, the default) or one decode GEMV step at M = 1, 4, 16 (decode); bert: one launch of "
                         "each BERT f32 projection; int8: one calibration copy, then one MatMulInteger + dequant call; "
                         "hipblaslt: the DiT GEMM kernel against hipBLASLt on the same operands (one JSON line each); "
                         "streamread: the M = 1 decode GEMVs against a vendor read (torch.sum) and a device copy of the "
                         "same weight bytes (one JSON line each); sequence: per-launch times of the DiT GEMM kernels "
                         "in the bench's order, alone, and after a 1 GiB write or read pass (one JSON line)")
    args = ap.parse_args()
    if args.gpus != 1:
        log("bench.py: this build measures one GPU (the path has no multi-GPU component); run with --gpus 1")
        return 2

    if args.probe in ("hipblaslt", "streamread", "sequence"):
        # torch's HIP runtime is loaded and initialised before the library's (started the other way round,
        # torch finds no GPU)
        import torch

        torch.cuda.init()
    from ingot_amd import Session
    from ingot_amd import _lib as L

    sess = Session(0)
    if args.probe == "hipblaslt":
        Dit(sess, L).compare_hipblaslt()
        sess.close()
        return 0
    if args.probe == "sequence":
        Dit(sess, L).sequence_probe()
        sess.close()
        return 0
    if args.probe == "streamread":
        Decode(sess, L).compare_stream_read()
        sess.close()
        return 0
    if args.probe:
        {"dit": Dit, "decode": Decode, "bert": Bert, "int8": Int8}[args.probe](sess, L).probe()
        sess.close()
        return 0
    res = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "data": "synthetic"}
    if args.workload == "dit":
        log("dit: set-up")
        wl = Dit(sess, L)
        ms = time_steps(sess, wl.step, args.steps, args.warmup)
        res.update({"value": round(wl.flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOPS", "ms_per_step": round(ms, 4),
                    "dtype": "bf16",
                    "config": {"workload": "DiT/QwenImage transformer GEMMs (BASELINE configs[4])", "M": 4096,
                               "gemms": ["3072x9216", "3072x12288+gelu", "12288x3072"],
                               "activations": "f32, bf16 RNE on load", "weights": "bf16", "accumulate": "f32",
                               "global_batch": 4096, "parallelism": "none (1 GPU)", "seed": Dit.seed,
                               "prng": "numpy PCG64 (np.random.default_rng)"}})
        log(f"dit: {res['value']} TFLOPS, {ms:.3f} ms/step; kernel roofline")
        res["roofline"] = wl.kernel_roofline()
        log("dit: default-math (hi/lo) step")
        res["dit_default_math"] = wl.default_math_report(args.steps, args.warmup)
        info = cpu_info() if not args.no_cpu_baseline else None
        if info:
            log(f"dit: cpu baseline on {info['threads']} threads ({info['model']})")
            res["cpu_baseline"] = wl.cpu_baseline(info, args.cpu_seconds)
    else:
        wl = {"bert": Bert, "int8": Int8, "decode": Decode}[args.workload](sess, L)
        if args.workload == "decode":
            rep = wl.report()
            res.update({"value": rep["m1"]["GB_per_s"], "unit": "GB/s", "ms_per_step": rep["m1"]["us_per_step"] / 1e3,
                        "dtype": "bf16", "config": {"workload": "decode GEMV M=1 (BASELINE configs[3])", "seed": wl.seed},
                        "detail": rep})
        else:
            ms = time_steps(sess, wl.step, args.steps, args.warmup)
            rep = wl.report(ms)
            res.update({"value": rep["value"], "unit": rep["unit"], "ms_per_step": rep["ms_per_step"],
                        "dtype": rep["dtype"], "config": {"workload": args.workload, "seed": wl.seed}, "detail": rep})
    if args.workload == "dit" and not args.no_extra:
        extra = {}
        for cls in (GemmRelu, Bert, Int8):
            log(f"{cls.name}: measuring")
            w = cls(sess, L)
            extra[cls.name] = w.report(time_steps(sess, w.step, 50, 10))
            extra[cls.name]["seed"] = cls.seed
            if info:
                extra[cls.name]["cpu_baseline"] = w.cpu_baseline(info, args.cpu_seconds_extra)
        log("decode: measuring")
        dec = Decode(sess, L)
        extra["decode"] = dec.report()
        extra["decode"]["seed"] = Decode.seed
        if info:
            extra["decode"]["cpu_baseline"] = dec.cpu_baseline(info, args.cpu_seconds_extra)
        log("ffn graph: measuring")
        extra["ffn_graph"] = FfnGraph(sess, L).report()
        extra["ffn_graph"]["seed"] = FfnGraph.seed
        res["workloads"] = extra
    sess.close()
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
