"""Benchmark of the gfx950 quantized GGML products on one MI355X.

Step = one Q4_K decode GEMV at M = 1, 4 and 8 (K = 3840, N = 15360, bf16 activations, f32
out), each on a different copy of the weights: the copies rotate through more than 512 MiB so the
256 MiB last-level cache cannot serve them. `value` is the weight bytes of the timed steps over
their wall time (HIP graph replay, inputs resident in HBM). The Q4_K prefill GEMM (M = 512, 1%
outlier columns) is timed the same way and reported under "gemm"; the Q8_0 GEMV, the six layer
GEMMs at M = 256 and the Q6_K vocabulary projection with its argmax under "configs".

Roofline entries use each kernel's average launch duration: one HIP graph of R back-to-back
launches per kernel, replayed between two events recorded on the stream the graph runs on,
divided by R (the device runs the launches back to back, so this tracks the kernel-trace
durations of rocprofv3).

CPU baseline: the oracle's port of the reference CPU path (quant.rs decode + f32-accumulate
matmul, OpenMP) on the same Q4_K matrix at M = 1, timed on this host.

HBM traffic: two rocprofv3 --pmc passes over a short run of the same launches (FETCH_SIZE, then
WRITE_SIZE, KiB per dispatch), each scaled by what the counter reads in the same pass for a
device-to-device copy of the same byte count, whose traffic is known.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-traffic] [--no-configs]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import shutil
import signal
import sqlite3
import statistics
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "jevons-rs_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16/bf16 MFMA
ROTATION_BYTES = 512 << 20

METRIC = "Q4_K GEMV weight GB/s (% HBM peak); Q4_K GEMM TFLOPS (% MFMA peak)"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_time_ms(fn, reps):
    """Average duration of one launch of `fn(i)`: a graph of `reps` launches replayed between
    two events on the replay stream."""
    import torch

    g = graph_of(fn, reps)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        g.replay()  # warm
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(s)
        g.replay()
        t1.record(s)
    t1.synchronize()
    torch.cuda.current_stream().wait_stream(s)
    return t0.elapsed_time(t1) / reps


def graph_of(fn, count):
    import torch

    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(count):
                fn(i)
    torch.cuda.current_stream().wait_stream(s)
    return g


GEMV_N, GEMV_K, GEMV_MS = 15360, 3840, (1, 4, 8)


class StreamProbe:
    """The code object's memory floor probe (jv_probe_stream_read), launched through the HIP
    module API: one launch reads `nbytes` with 16-byte loads, `per` bytes per workgroup."""

    def __init__(self):
        import ctypes as C

        import jevons_qmm as jq

        self.C = C
        self.hip = C.CDLL("libamdhip64.so")
        self.mod, self.fn = C.c_void_p(), C.c_void_p()
        self._ok(self.hip.hipModuleLoad(C.byref(self.mod), jq.HSACO_PATH.encode()))
        self._ok(self.hip.hipModuleGetFunction(C.byref(self.fn), self.mod, b"jv_probe_stream_read"))

    @staticmethod
    def _ok(e):
        if e != 0:
            raise RuntimeError(f"HIP error {e}")

    def launch(self, src, nbytes, per, sink):
        import torch

        C = self.C
        units = nbytes // 16
        per_u = per // 16
        grid = (units + per_u - 1) // per_u
        a_src, a_units, a_per, a_sink = (C.c_void_p(src.data_ptr()), C.c_int64(units), C.c_int32(per_u),
                                         C.c_void_p(sink.data_ptr()))
        args = (C.c_void_p * 4)(*[C.cast(C.pointer(a), C.c_void_p) for a in (a_src, a_units, a_per, a_sink)])
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        self._ok(self.hip.hipModuleLaunchKernel(self.fn, grid, 1, 1, 512, 1, 1, 0, stream, args, None))


def stream_floor(nbytes, copies, reps, pers=None):
    """Average duration (us) of one streaming read of `nbytes`, each launch on the next of
    `copies` buffers (the products' weight rotation), for several bytes per workgroup (`pers`,
    by default the four below)."""
    import torch

    probe = StreamProbe()
    bufs = [torch.full((nbytes,), i, dtype=torch.uint8, device="cuda") for i in range(copies)]
    sink = torch.zeros(nbytes // 16, dtype=torch.int32, device="cuda")
    res = {}
    # one Q4_K tile (16 rows x 15 blocks, the M=1 kernel's workgroup), half and twice that, and
    # one range per compute unit
    for per in pers or (17280, 34560, 69120, (nbytes + 255) // 256 // 16 * 16 + 16):
        probe.launch(bufs[0], nbytes, per, sink)
        torch.cuda.synchronize()
        t = kernel_time_ms(lambda r, per=per: probe.launch(bufs[r % copies], nbytes, per, sink), reps)
        res[str(per)] = round(t * 1e3, 3)
    del bufs
    return res


def pmc_child():
    """Launch workload of the traffic passes: each GEMV launch 20 times on rotating weight copies,
    then a device copy of the weight byte count 20 times."""
    import numpy as np
    import torch

    import jevons_qmm as jq
    from jevons_qmm import synth

    n, k = GEMV_N, GEMV_K
    gpu = jq.Gpu(0)
    raw = synth.weights(jq.Q4K, 2, n, k)
    raw_dev = torch.from_numpy(raw).cuda()
    copies = max(2, math.ceil(ROTATION_BYTES / raw.size))
    mats = [jq.QMatrix.upload_device(gpu, jq.Q4K, n, k, 1, raw_dev) for _ in range(copies)]
    x8 = synth.normal_rows(21, 8, k)
    xb = torch.from_numpy(synth.to_bf16(x8).view(np.int16).copy()).view(torch.bfloat16).cuda()
    scratch = jq.SplitScratch(gpu)
    for m in GEMV_MS:
        xm = xb[:m].contiguous()
        out = torch.empty((m, n), dtype=torch.float32, device="cuda")
        for r in range(20):
            jq.matmul(gpu, xm, m, mats[r % copies], out, scratch)
        torch.cuda.synchronize()
    srcs = [torch.empty(raw.size, dtype=torch.uint8, device="cuda") for _ in range(copies)]
    dst = torch.empty(raw.size, dtype=torch.uint8, device="cuda")
    for r in range(20):
        dst.copy_(srcs[r % copies])
    torch.cuda.synchronize()
    print("pmc child done", flush=True)


def pmc_gemm_child():
    """Launch workload of the tiled products' counter passes (run by hand under rocprofv3 --pmc):
    the Q4_K GEMM M=512 K=3840 N=15360 (256 x 128 tiles), the Q6_K down projection M=256
    K=15360 N=3840 (64 x 64 tiles) and the Q6_K vocabulary projection M=32 K=3840 N=262144
    (32 x 64 tiles), ten launches each on two alternating weight copies."""
    import numpy as np
    import torch

    import jevons_qmm as jq
    from jevons_qmm import synth

    gpu = jq.Gpu(0)
    for fmt, m, n, k, plan in ((jq.Q4K, 512, 15360, 3840, jq.Plan(256, 128, 1)),
                               (jq.Q6K, 256, 3840, 15360, jq.Plan(64, 64, 1)),
                               (jq.Q6K, 32, 262144, 3840, jq.Plan(32, 64, 1))):
        raw_dev = torch.from_numpy(synth.weights(fmt, 2, n, k)).cuda()
        mats = [jq.QMatrix.upload_device(gpu, fmt, n, k, 1, raw_dev) for _ in range(2)]
        del raw_dev
        xb = torch.from_numpy(synth.to_bf16(synth.normal_rows(1, m, k)).view(np.int16).copy())
        x = xb.view(torch.bfloat16).cuda()
        out = torch.empty((m, n), dtype=torch.float32, device="cuda")
        for r in range(10):
            jq.matmul_plan(gpu, x, m, mats[r % 2], out, None, plan)
        torch.cuda.synchronize()
        del mats
    print("pmc child done", flush=True)


def _pmc_pass(counter, workdir):
    """One rocprofv3 pass of `counter` over the child workload -> {kernel name: [values]}."""
    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    out = os.path.join(workdir, counter)
    cmd = [prof, "--pmc", counter, "-d", out, "-o", "run", "--", sys.executable,
           os.path.abspath(__file__), "--pmc-child"]
    proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                            start_new_session=True, env=dict(os.environ, TMPDIR=workdir))
    try:
        text = proc.communicate(timeout=150)[0].decode(errors="replace")
    except subprocess.TimeoutExpired:
        os.killpg(proc.pid, signal.SIGKILL)
        proc.communicate()
        raise RuntimeError(f"rocprofv3 --pmc {counter} timed out")
    if "pmc child done" not in text:
        raise RuntimeError(f"rocprofv3 --pmc {counter} failed: {text[-400:]}")
    dbs = [os.path.join(r, f) for r, _, fs in os.walk(out) for f in fs if f.endswith("_results.db")]
    if not dbs:
        raise RuntimeError(f"rocprofv3 --pmc {counter} wrote no database")
    vals = {}
    for db in dbs:
        con = sqlite3.connect(db)
        for name, lds, v in con.execute(
                "select kernel_name, lds_block_size, value from counters_collection "
                "where counter_name = ?", (counter,)):
            # the LDS size tells launches of one kernel at different m apart
            vals.setdefault(f"{name}@lds{lds}" if name.startswith("jv_") else name, []).append(v)
        con.close()
    return vals


def measure_traffic(wbytes):
    """HBM bytes per launch of each GEMV kernel, from FETCH_SIZE and WRITE_SIZE scaled by the
    same counters' reading for a device copy of `wbytes` bytes."""
    workdir = tempfile.mkdtemp(prefix="jv_pmc_")
    try:
        res = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            vals = _pmc_pass(counter, workdir)
            copy = [v for name, vs in vals.items() if "copyBuffer" in name for v in vs]
            kern = {name: statistics.median(vs) for name, vs in vals.items() if name.startswith("jv_")}
            if not copy or not kern:
                raise RuntimeError(f"{counter}: no copy or product dispatches recorded")
            kib_copy = statistics.median(copy)
            factor = wbytes / (kib_copy * 1024.0)
            res[counter] = {"copy_kib": kib_copy, "factor": factor,
                            "kernels_kib": kern,
                            "kernels_bytes": {nm: v * 1024.0 * factor for nm, v in kern.items()}}
        names = sorted(res["FETCH_SIZE"]["kernels_bytes"])
        per_kernel = {nm: round(res["FETCH_SIZE"]["kernels_bytes"][nm] +
                                res["WRITE_SIZE"]["kernels_bytes"].get(nm, 0.0))
                      for nm in names}
        return {
            "per_kernel_bytes": per_kernel,
            "fetch_factor": round(res["FETCH_SIZE"]["factor"], 4),
            "write_factor": round(res["WRITE_SIZE"]["factor"], 4),
            "copy_fetch_kib": res["FETCH_SIZE"]["copy_kib"],
            "copy_write_kib": res["WRITE_SIZE"]["copy_kib"],
        }
    finally:
        shutil.rmtree(workdir, ignore_errors=True)


def measure_configs(gpu, steps):
    """Kernel durations of the other product configurations, each against its roofline:
    Q8_0 GEMV (M=1, K=N=4096; weights rotated), the six layer GEMMs of one transformer block at
    M=256 (Q4_K q/k/v/o/gate_up, Q6_K down), the Q6_K vocabulary projection (K=3840,
    N=262144, M = 1, 8, 32) with the per-row argmax of its logits, and the expert-grouped
    Q4_K products of the routing step's gate/up shape at prefill (512 tokens) and at decode
    (8 tokens)."""
    import numpy as np
    import torch

    import jevons_qmm as jq
    from jevons_qmm import synth

    def mats(kind, n, k, copies, seed):
        raw = synth.weights(kind, seed, n, k)
        dev = torch.from_numpy(raw).cuda()
        ms = [jq.QMatrix.upload_device(gpu, kind, n, k, 1, dev) for _ in range(copies)]
        del dev
        return ms, raw.size

    def xrows(m, k, seed):
        xb = synth.to_bf16(synth.normal_rows(seed, m, k)).view(np.int16).copy()
        return torch.from_numpy(xb).view(torch.bfloat16).cuda()

    scratch = jq.SplitScratch(gpu)
    res = {}
    # Q8_0 GEMV
    n, k = 4096, 4096
    ms, wbytes = mats(jq.Q8_0, n, k, max(2, math.ceil(ROTATION_BYTES / (n * k // 32 * 34))), 3)
    x = torch.from_numpy(synth.normal_rows(1, 1, k)).cuda()  # f32 activations, as the config states
    out = torch.empty((1, n), dtype=torch.float32, device="cuda")
    jq.matmul(gpu, x, 1, ms[0], out, scratch)  # buffers grow outside graph capture
    t = kernel_time_ms(lambda r: jq.matmul(gpu, x, 1, ms[r % len(ms)], out, scratch), steps)
    gbs = wbytes / (t * 1e-3) / 1e9
    res["q8_0_gemv"] = {"workload": f"Q8_0 GEMV M=1 K={k} N={n}, f32 activations, f32 out",
                        "kernel_us": round(t * 1e3, 3), "weight_bytes": wbytes,
                        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    del ms
    log("q8_0 gemv:", res["q8_0_gemv"])
    # layer GEMMs at M = 256: a denoising block's canvas products, whose plans come from the
    # plan tuner without the row-invariance requirement (Tuner::dense(w, m, false),
    # tune.rs:162-174; split-K allowed); the prefill-style whole-K auto plans are timed beside
    # them. The q, k and v projections also run as one product [8192, 3840] on their shared input.
    layers = [("q", jq.Q4K, 4096, 3840), ("k", jq.Q4K, 2048, 3840), ("v", jq.Q4K, 2048, 3840),
              ("o", jq.Q4K, 3840, 4096), ("gate_up", jq.Q4K, 30720, 3840), ("down", jq.Q6K, 3840, 15360),
              ("qkv", jq.Q4K, 4096 + 2 * 2048, 3840)]
    m = 256
    tuner = jq.Tuner.new(gpu, None)
    per = {}
    for name, kind, n, k in layers:
        ms, _ = mats(kind, n, k, 2, 5)
        x = xrows(m, k, 2)
        out = torch.empty((m, n), dtype=torch.float32, device="cuda")
        tuner.tune_dense(ms, m, False, x, out, scratch)
        row = {"n": n, "k": k, "format": "Q6_K" if kind == jq.Q6K else "Q4_K", "gflop": round(2e-9 * m * n * k, 3)}
        for mode, plan in (("canvas", tuner.dense(ms[0], m, False)), ("prefill", jq.Plan.auto(ms[0], m, row_invariant=True))):
            jq.matmul_plan(gpu, x, m, ms[0], out, scratch, plan)
            t = kernel_time_ms(lambda r: jq.matmul_plan(gpu, x, m, ms[r % 2], out, scratch, plan), max(4, steps // 4))
            row[mode] = {"plan": [plan.bm, plan.bn, plan.splits], "us": round(t * 1e3, 2),
                         "tflops": round(2.0 * m * n * k / (t * 1e-3) / 1e12, 1)}
        per[name] = row
        del ms
    six = ("q", "k", "v", "o", "gate_up", "down")
    fused = ("qkv", "o", "gate_up", "down")
    flops = sum(2.0 * m * per[nm]["n"] * per[nm]["k"] for nm in six)

    def total(names, mode):
        return sum(per[nm][mode]["us"] for nm in names)

    tf = flops / (total(fused, "canvas") * 1e-6) / 1e12
    res["layer_gemms_m256"] = {
        "workload": "one transformer block's six GEMMs at M=256 (a denoising block), bf16 activations, "
                    "f32 out; canvas plans from the tuner (split-K allowed), q/k/v fused into one product",
        "gemms": per,
        "total_us": round(total(fused, "canvas"), 2),
        "total_us_separate_qkv": round(total(six, "canvas"), 2),
        "total_us_prefill_plans": round(total(six, "prefill"), 2),
        "total_us_prefill_plans_fused_qkv": round(total(fused, "prefill"), 2),
        "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}}
    log("layer gemms:", res["layer_gemms_m256"])
    # Q6_K vocabulary projection and argmax
    n, k = 262144, 3840
    ms, wbytes = mats(jq.Q6K, n, k, 1, 4)
    lm = {}
    for m in (1, 8, 32):
        x = xrows(m, k, 3)
        out = torch.empty((m, n), dtype=torch.float32, device="cuda")
        jq.matmul(gpu, x, m, ms[0], out, scratch)
        jq.argmax_rows(gpu, out, scratch)
        jq.matmul_argmax(gpu, x, m, ms[0], out, 30.0, scratch)  # its buffers grow before capture

        def three_steps(r):  # the reference's order: product, soft cap, greedy per row
            jq.matmul(gpu, x, m, ms[0], out, scratch)
            jq.softcap_logits(gpu, out, 30.0)
            jq.argmax_rows(gpu, out, scratch)

        # the product alone, the argmax alone, the three steps, and the product with the soft
        # cap and greedy fused (cap 30, and cap 0: greedy only); five interleaved rounds,
        # medians, so that the differences are not the drift between separate timings
        fns = [lambda r: jq.matmul(gpu, x, m, ms[0], out, scratch),
               lambda r: jq.argmax_rows(gpu, out, scratch),
               three_steps,
               lambda r: jq.matmul_argmax(gpu, x, m, ms[0], out, 30.0, scratch),
               lambda r: jq.matmul_argmax(gpu, x, m, ms[0], out, 0.0, scratch)]
        runs = [[] for _ in fns]
        for _ in range(5):
            for fn, rr in zip(fns, runs):
                rr.append(kernel_time_ms(fn, max(4, steps // 10)))
        t, ta, t3, tf, tf0 = (statistics.median(rr) for rr in runs)
        gbs = wbytes / (t * 1e-3) / 1e9
        lm[str(m)] = {"kernel_us": round(t * 1e3, 2), "weight_GBps": round(gbs, 1),
                      "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                      "tflops": round(2.0 * m * n * k / (t * 1e-3) / 1e12, 1),
                      "argmax_us": round(ta * 1e3, 2),
                      # greedy fused into the product (jv_matmul_argmax, no soft cap), less the
                      # product alone
                      "fused_argmax_us": round((tf0 - t) * 1e3, 2),
                      # soft cap 30 and greedy after the product: as three launches, and fused
                      # into the product (jv_matmul_argmax), each less the product alone
                      "softcap_argmax_us": round((t3 - t) * 1e3, 2),
                      "fused_softcap_argmax_us": round((tf - t) * 1e3, 2),
                      "fused_total_us": round(tf * 1e3, 2)}
    del ms
    # the floor of one plain streaming read of the same bytes (one copy exceeds the last-level
    # cache): 16-byte loads, 17,280 and 69,120 bytes per workgroup
    floor_lm = min(stream_floor(wbytes, 1, max(4, steps // 20), pers=(17280, 69120)).values())
    res["q6k_lm_head"] = {"workload": f"Q6_K vocabulary projection K={k} N={n} + per-row argmax, bf16 activations, f32 logits",
                          "weight_bytes": wbytes, "per_m": lm, "stream_floor_us": floor_lm,
                          "stream_floor_GBps": round(wbytes / (floor_lm * 1e-6) / 1e9, 1)}
    log("q6k lm_head:", res["q6k_lm_head"])
    # expert-grouped product (MoE gate/up): 128 Q4_K experts [1408, 2816], 512 tokens routed to
    # 8 experts each (seeded uniform routing), grouped into jobs on the device
    experts, n, k, tokens, top_k = 128, 1408, 2816, 512, 8
    raw = synth.weights(jq.Q4K, 6, experts * n, k)
    w = jq.QMatrix.upload_device(gpu, jq.Q4K, n, k, experts, torch.from_numpy(raw).cuda())
    rng = np.random.default_rng(7)
    route = np.stack([rng.choice(experts, top_k, replace=False) for _ in range(tokens)]).reshape(-1)
    ids = torch.from_numpy(route.astype(np.int32)).cuda()
    x = xrows(tokens, k, 8)
    out = torch.empty((tokens * top_k, n), dtype=torch.float32, device="cuda")
    # the job plan as the reference picks it (Tuner::grouped, tune.rs:177-189, model.rs:803-805):
    # the tuner's measured pick among rows {32, 64} x columns {64, 128} on its balanced routing;
    # every candidate is also timed on this routing
    a = tokens * top_k
    route_cap = a
    jobs_len = 1 + 2 * ((a + 31) // 32 + experts)
    tbuf = {nm: torch.empty(sz, dtype=torch.int32, device="cuda")
            for nm, sz in (("ids", route_cap), ("sorted", route_cap), ("offsets", experts + 1), ("jobs", jobs_len))}
    tuner = jq.Tuner.new(gpu, None)
    xt = xrows(a, k, 10)  # the tuner's input: one row per assignment (tune.rs:191-193)
    tuner.tune_grouped([w], tokens, top_k, xt, out, tbuf["ids"], tbuf["sorted"], tbuf["offsets"], tbuf["jobs"], scratch)
    del xt
    pick = tuner.grouped(w, tokens)
    flops = 2.0 * tokens * top_k * n * k
    cands = {}
    for bm, bn in ((32, 64), (32, 128), (64, 64), (64, 128)):
        g = jq.group_routes(gpu, ids, experts, bm, in_div=top_k)
        jq.matmul_grouped(gpu, x, w, g, out, bm, bn, 1, scratch)
        tc = kernel_time_ms(lambda r: jq.matmul_grouped(gpu, x, w, g, out, bm, bn, 1, scratch), max(4, steps // 10))
        cands[f"{bm}x{bn}"] = round(tc * 1e3, 2)
    t = cands[f"{pick[0]}x{pick[1]}"] * 1e-3
    tf = flops / (t * 1e-3) / 1e12
    # the grouping of the same routes into the picked plan's jobs (jv_group_routes), written
    # into the buffers of a first call
    g = jq.group_routes(gpu, ids, experts, pick[0], in_div=top_k)
    tg = kernel_time_ms(lambda r: jq.group_routes(gpu, ids, experts, pick[0], in_div=top_k, into=g),
                        max(4, steps // 10))
    res["moe_grouped"] = {"workload": f"Q4_K expert-grouped product, {experts} experts N={n} K={k}, {tokens} tokens x top-{top_k}, "
                                      "jobs on the tuner's plan, bf16 activations, f32 out",
                          "group_routes_us": round(tg * 1e3, 2),
                          "plan": {"bm": pick[0], "bn": pick[1]}, "kernel_us_by_plan": cands,
                          "kernel_us": round(t * 1e3, 2), "weight_bytes": raw.size,
                          "weight_GBps": round(raw.size / (t * 1e-3) / 1e9, 1),
                          "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                                       "unit": "TFLOP/s", "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}}
    # decode-time expert product: 8 tokens routed to 8 of the 128 experts each (64 assignments)
    # on the small-row grouped path in jobs of up to 4 rows (SMALL_GROUP_ROWS, model.rs:265),
    # timed over weight copies that together exceed the last-level cache
    tokens_d = 8
    route_d = np.stack([rng.choice(experts, top_k, replace=False) for _ in range(tokens_d)]).reshape(-1)
    touched = len(set(route_d.tolist()))
    tbytes = touched * (raw.size // experts)
    copies = max(2, math.ceil(ROTATION_BYTES / tbytes))
    raw_dev = torch.from_numpy(raw).cuda()
    wd = [w] + [jq.QMatrix.upload_device(gpu, jq.Q4K, n, k, experts, raw_dev) for _ in range(copies - 1)]
    del raw_dev
    ids_d = torch.from_numpy(route_d.astype(np.int32)).cuda()
    xd = xrows(tokens_d, k, 9)
    outd = torch.empty((tokens_d * top_k, n), dtype=torch.float32, device="cuda")
    gd = jq.group_routes(gpu, ids_d, experts, 4, in_div=top_k)
    jq.matvec_grouped(gpu, xd, w, gd, outd, 4)
    t = kernel_time_ms(lambda r: jq.matvec_grouped(gpu, xd, wd[r % copies], gd, outd, 4), max(4, steps // 10))
    gbs = tbytes / (t * 1e-3) / 1e9
    res["moe_grouped_decode"] = {"workload": f"Q4_K expert-grouped small-row product, {experts} experts N={n} K={k}, "
                                             f"{tokens_d} tokens x top-{top_k} ({touched} experts touched), "
                                             "jobs of up to 4 rows, bf16 activations, f32 out",
                                 "kernel_us": round(t * 1e3, 2), "weight_bytes_touched": tbytes,
                                 "rotation_copies": copies,
                                 "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                                              "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    del w, wd
    log("moe grouped:", res["moe_grouped"])
    log("moe grouped decode:", res["moe_grouped_decode"])
    return res


def cpu_baseline(raw, n, k, x32):
    """The oracle's port of the reference CPU path on this host's cores: GGML block decode
    (quant.rs:83-101) then an f32-accumulate matmul (OpenMP over all cores). Main figure: the
    Q4_K matrix at M = 1, decode + matmul, about 10 s of repetitions; beside it the matmul alone
    on pre-decoded f32 weights, one thread on 1024 rows, and the Q8_0 GEMV (M = 1, K = N = 4096,
    f32 activations) decode + matmul, about 3 s each."""
    import numpy as np

    import oracle as O
    from jevons_qmm import synth

    threads = O.omp_max_threads()
    wdec = np.empty(n * k, np.float32)
    nbytes = n * k // 256 * 144

    def timed(fn, seconds):
        fn()  # warm
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            fn()
            reps += 1
        return (time.perf_counter() - t0) / reps, reps

    dt, reps = timed(lambda: O.cpu_dequant_matmul(O.Q4K, raw, n, k, x32[:1], threads=threads, wdec=wdec), 10.0)
    # the matmul alone: wdec holds the decoded weights from the runs above
    dm, reps_m = timed(lambda: O.cpu_dequant_matmul(O.Q4K, raw, n, k, x32[:1], threads=threads, wdec=wdec,
                                                    decode=False), 3.0)
    # single thread on a 1024-row slice of the same matrix
    rows1 = 1024
    raw1 = raw[: rows1 * k // 256 * 144]
    d1, _ = timed(lambda: O.cpu_dequant_matmul(O.Q4K, raw1, rows1, k, x32[:1], threads=1, wdec=wdec), 3.0)
    # Q8_0 GEMV M = 1, K = N = 4096, f32 activations
    n8 = k8 = 4096
    raw8 = synth.weights(O.Q8_0, 3, n8, k8)
    x8 = synth.normal_rows(1, 1, k8)
    w8 = np.empty(n8 * k8, np.float32)
    d8, reps8 = timed(lambda: O.cpu_dequant_matmul(O.Q8_0, raw8, n8, k8, x8, threads=threads, wdec=w8), 3.0)
    return {
        "value": round(nbytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"Q4_K decode + f32 matmul, M=1, K={k}, N={n} (full matrix), {reps} reps in ~10 s",
        "ms_per_call": round(dt * 1e3, 3),
        "matmul_only_predecoded": {"ms_per_call": round(dm * 1e3, 3), "q4k_weight_GBps": round(nbytes / dm / 1e9, 3),
                                   "f32_weight_GBps": round(n * k * 4 / dm / 1e9, 3), "reps": reps_m},
        "one_thread_1024_rows": {"q4k_weight_GBps": round(rows1 * k // 256 * 144 / d1 / 1e9, 3)},
        "q8_0_gemv_4096": {"ms_per_call": round(d8 * 1e3, 3), "weight_GBps": round(raw8.size / d8 / 1e9, 3),
                           "reps": reps8, "cores": threads},
        "cpu_model": _cpu_model(),
    }


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--gemm-steps", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-traffic", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the Q8_0, layer and lm_head lines")
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--pmc-gemm", action="store_true",
                    help="only launch the tiled products (a workload for rocprofv3 --pmc runs)")
    args = ap.parse_args()
    if args.pmc_gemm:
        pmc_gemm_child()
        return
    if args.pmc_child:
        pmc_child()
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import jevons_qmm as jq
    from jevons_qmm import synth

    n, k = GEMV_N, GEMV_K
    ms = GEMV_MS
    gpu = jq.Gpu(0)
    log("device", gpu.info.arch.decode(), "CUs", gpu.info.compute_units)
    raw = synth.weights(jq.Q4K, 2, n, k)
    wbytes = raw.size
    raw_dev = torch.from_numpy(raw).cuda()
    copies = max(2, math.ceil(ROTATION_BYTES / wbytes))
    mats = [jq.QMatrix.upload_device(gpu, jq.Q4K, n, k, 1, raw_dev) for _ in range(copies)]
    del raw_dev
    log(f"weights {wbytes} B x {copies} copies = {wbytes * copies / 2**20:.0f} MiB")

    x8 = synth.normal_rows(21, 8, k)
    xb = torch.from_numpy(synth.to_bf16(x8).view(np.int16).copy()).view(torch.bfloat16).cuda()
    xs = {m: xb[:m].contiguous() for m in ms}
    outs = {m: torch.empty((m, n), dtype=torch.float32, device="cuda") for m in ms}
    scratch = jq.SplitScratch(gpu)  # split-K partials (SplitScratch, gemm.rs:1041-1065)

    def gemv_step(i):
        for j, m in enumerate(ms):
            jq.matmul(gpu, xs[m], m, mats[(3 * i + j) % copies], outs[m], scratch)

    gemv_step(0)
    torch.cuda.synchronize()
    g_warm = graph_of(gemv_step, args.warmup)
    g_timed = graph_of(gemv_step, args.steps)
    g_warm.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g_timed.replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    value = 3 * wbytes / (ms_per_step * 1e-3) / 1e9

    # per-kernel durations (M = 1, 4, 8)
    reps = 100
    kt = [kernel_time_ms(lambda r, m=m: jq.matmul(gpu, xs[m], m, mats[r % copies], outs[m], scratch), reps)
          for m in ms]
    per_m = {m: {"kernel_us": round(t * 1e3, 3), "weight_GBps": round(wbytes / (t * 1e-3) / 1e9, 1)}
             for m, t in zip(ms, kt)}
    avg_kernel_ms = sum(kt) / len(kt)
    achieved = wbytes / (avg_kernel_ms * 1e-3) / 1e9
    log("gemv per M:", per_m)
    floor = stream_floor(wbytes, copies, reps)
    log("stream floor (us by bytes per workgroup):", floor)

    # prefill GEMM, M = 512
    mg = 512
    xg32 = synth.normal_rows(31, mg, k, outlier_frac=0.01)
    xg = torch.from_numpy(synth.to_bf16(xg32).view(np.int16).copy()).view(torch.bfloat16).cuda()
    og = torch.empty((mg, n), dtype=torch.float32, device="cuda")
    plan = jq.Plan.auto(mats[0], mg, row_invariant=True)

    def gemm_step(i):
        jq.matmul_plan(gpu, xg, mg, mats[i % copies], og, None, plan)

    gemm_step(0)
    torch.cuda.synchronize()
    gg = graph_of(gemm_step, args.gemm_steps)
    gg.replay()
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    gg.replay()
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    gemm_ms = (t3 - t2) * 1e3 / args.gemm_steps
    flops = 2.0 * mg * n * k
    gk = kernel_time_ms(gemm_step, 30)
    gemm = {
        "workload": f"Q4_K prefill GEMM M={mg} K={k} N={n}, bf16 activations (1% outlier columns x20), f32 out",
        "plan": {"bm": plan.bm, "bn": plan.bn, "splits": plan.splits},
        "ms_per_step": round(gemm_ms, 4),
        "value": round(flops / (gemm_ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "roofline": {"bound": "mfma", "achieved": round(flops / (gk * 1e-3) / 1e12, 2),
                     "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(flops / (gk * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                     "traffic": None,
                     # the duration is the activation packing and the product together (one
                     # call); the product kernel alone is in the kernel-trace summary
                     "duration_includes": "jv_pack_x + product"},
    }
    log("gemm:", gemm)

    configs = None if args.no_configs else measure_configs(gpu, 100)

    cpu = None if args.no_cpu else cpu_baseline(raw, n, k, x8)
    if cpu:
        log("cpu:", cpu)

    traffic, traffic_detail = None, None
    if not args.no_traffic:
        try:
            traffic_detail = measure_traffic(wbytes)
            gemv_bytes = [b for nm, b in traffic_detail["per_kernel_bytes"].items() if "qmv" in nm]
            if gemv_bytes:
                traffic = round(statistics.mean(gemv_bytes))
            log("traffic:", traffic_detail)
        except Exception as e:  # the counters are a report, not the measurement
            traffic_detail = {"error": str(e)[:300]}
            log("traffic measurement failed:", e)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": f"Q4_K decode GEMV K={k} N={n}, M in {{1,4,8}} per step, bf16 activations, f32 out",
            "weight_bytes_per_launch": wbytes,
            "rotation_copies": copies,
            "per_m": per_m,
            # plain 16-byte streaming read of the same bytes and rotation, by bytes per workgroup
            "stream_floor_us": min(floor.values()),
            "stream_floor_by_workgroup_bytes": floor,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "traffic_detail": traffic_detail,
        "gemm": gemm,
        "configs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
