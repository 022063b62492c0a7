#!/usr/bin/env python3
"""Benchmark of the quantized linear path on one MI355X.

Headline workload (`value`): the Q5_K GEMM at the Z-Image DiT FFN shape,
X fp32 [M=4096, K=3840] ~ N(0,1) with 1% of the K channels x20, W [N=10240,
K=3840] ~ N(0,0.02) packed to Q5_K, output fp32 [4096, 10240].  One step is
one full pixhip_matmul call: quantize X to Q8_K, then the int8-MFMA GEMM.
Inputs are resident in HBM before timing starts.

Also reported in the same JSON line: the GEMM kernel alone (the roofline
object, against the int8 MFMA peak), the quantize pass alone, the M=1 decode
matvec (Q5_K, Q8_0 and Q6_K, W [18944, 3584], 100 repeats rotating >= 1 GiB of
weight copies so the 256 MB Infinity Cache cannot serve them), the other
specified workloads (`workloads`: a single Q8_0 linear [256, 3840] x [3840,
3840], every linear of a Z-Image DiT block at M = 4608 and of a Qwen-Image edit
block at M = 8448, each linear and the block back to back, and the DiT
FFN-down with Q6_K weights), the same step with host
(pinned) operands staged over PCIe, self-attention at the DiT block's shape
(30 heads of 128 over 4608 tokens) and the VAE mid-block's (one head of 512
over 16384 tokens), one whole Z-Image DiT block through the C ABI (`block`:
4608 tokens, per-op times and shares), the rest of the op surface (`surface`:
norms, layouts and row moves at the models' shapes, against the HBM peak), VAE
convolutions (`conv`, against the bf16 MFMA peak), and the reference CPU path
(cpu_quant_matmul, tensor_attention) timed on this host on the same inputs.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-blocks]

Progress goes to stderr; stdout carries exactly one JSON line.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q5_K/Q8_0 GEMM TOPS (% i8 MFMA peak); M=1 matvec GB/s (% HBM peak)"
PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, 2.5 PFLOP/s
MALL_DEFEAT_BYTES = 1 << 30  # rotate >= 1 GiB of weights per matvec series
COPY_BYTES = 1 << 29  # the plain copy that calibrates the HBM byte counters

GEMM_M, GEMM_K, GEMM_N = 4096, 3840, 10240
MV_K, MV_N = 3584, 18944
WARMUP_FLOOR_MS = 50.0  # device time before the headline series
SERIES_FLOOR_MS = 20.0  # device time per timed series of the other workloads

# The other workloads: (name, tokens, activation row scales, [(linear, type, K, N)]).
WORKLOADS = [
    ("q8_0_linear", 256, None, [("linear", "Q8_0", 3840, 3840)]),
    ("dit_block", 4096 + 512, None, [("qkv", "Q5_K", 3840, 11520), ("out", "Q5_K", 3840, 3840), ("w1", "Q5_K", 3840, 10240),
                                     ("w3", "Q5_K", 3840, 10240), ("w2", "Q8_0", 10240, 3840)]),
    ("qwen_edit_block", 4096 + 4096 + 256, (0.1, 10.0),
     [("qkv", "Q5_K", 3072, 9216), ("out", "Q5_K", 3072, 3072), ("ff_up", "Q5_K", 3072, 12288), ("ff_down", "Q5_K", 12288, 3072)]),
    ("q6_K_ffn_down", 4096 + 512, None, [("w2", "Q6_K", 10240, 3840)]),
]
# HBM bytes per launch measured for these linears' GEMM kernels (profiles/hbm_traffic.json)
TRAFFIC_KEYS = {("q8_0_linear", "linear"): "gemm_q8_0_linear", ("dit_block", "w2"): "gemm_q8_0_w2"}
WORKLOAD_TEXT = {
    "q8_0_linear": "single Q8_0 linear, X[256,3840] W[3840,3840]",
    "dit_block": "Z-Image DiT block linears, M=4608 (4096 image + 512 text), Q5_K except FFN-down Q8_0",
    "qwen_edit_block": "Qwen-Image edit block linears, M=8448 (2x4096 image + 256 text), Q5_K, per-token scales log-uniform [0.1,10]",
    "q6_K_ffn_down": "Z-Image DiT FFN-down with Q6_K weights (the type Q5_K_M files give ffn_down), M=4608",
}


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def affinity_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_threads():
    """Threads for the CPU reference: every core this process may run on
    (the reference's -t default is hardware_concurrency, src/tensor.cpp:97-101)."""
    return max(1, affinity_cores())


def cpu_info():
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    # The reference's quantized kernels take their AVX2 path (target("avx2,fma,f16c"))
    # when the CPU has these.
    return {"cpu": model, "nproc": affinity_cores(), "os_cpu_count": os.cpu_count(),
            "avx2": "avx2" in flags, "fma": "fma" in flags, "f16c": "f16c" in flags, "avx512f": "avx512f" in flags}


def row_rel(y, r):
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    return float((np.abs(y - r).max(axis=-1) / np.maximum(np.abs(r).max(axis=-1), 1e-30)).max())


class CpuBaseline:
    """The reference CPU path: oracle/_ref (the reference's own kernels_quant.cpp,
    built from its sources) when present, else the oracle's C restatement."""

    def __init__(self, threads):
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle_lib

        self.ol = oracle_lib
        self.threads = threads
        ref = oracle_lib.reference()
        if ref is not None:
            self.kind, self.lib, self.prefix = "reference", ref, "ref"
            ref.ref_set_threads(threads)
        else:
            self.kind, self.lib, self.prefix = "port", oracle_lib.oracle(), "orc"

    def matmul(self, wb, wtype, x, rows):
        return self.ol.quant_matmul(self.lib, self.prefix, wb, wtype, x, rows, threads=self.threads)


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (profiles/hbm_traffic.json: FETCH_SIZE + WRITE_SIZE per dispatch, scaled by
    a plain copy of known size), or None when it has not been measured."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)["kernels"][kernel]["bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def gemm_workload(synth):
    log("generating Q5_K GEMM inputs (M=4096 K=3840 N=10240)")
    x = synth.normal(synth.SEED_ACTIVATIONS, (GEMM_M, GEMM_K))
    ch = synth.outlier_channels(GEMM_K)
    x[:, ch] *= 20.0
    w = synth.normal(synth.SEED_WEIGHTS, (GEMM_N, GEMM_K), std=0.02)
    wb = synth.pack_q5_K(w)
    del w
    return x, wb, ch


def timed_series(sess, run_once, min_reps, floor_ms=SERIES_FLOOR_MS):
    """Average device ms of run_once() (which enqueues one step) over a series of
    at least min_reps steps and floor_ms of device time, after a warm-up of the
    same length."""
    sess.synchronize()
    sess.timer_start()
    run_once()
    once = max(sess.timer_stop(), 1e-3)
    reps = max(min_reps, int(np.ceil(floor_ms / once)))
    for _ in range(reps):
        run_once()
    sess.timer_start()
    for _ in range(reps):
        run_once()
    return sess.timer_stop() / reps, reps


def workload_inputs(synth, name, m, row_scale, linears):
    """Seeded inputs of one workload, all SplitMix64 + Box-Muller streams with
    the headline's seeds: one activation matrix per distinct K (ascending K),
    drawn as consecutive pieces of stream 1337 (~N(0,1)); the per-token scales
    (log-uniform, where given) from stream 1339, one piece per activation
    matrix; the weights of the linears, in their listed order, as consecutive
    pieces of stream 1338 (~N(0, 0.02)).  Q5_K and Q6_K weights are packed
    here; Q8_0 weights are returned as float32 and quantized by the HIP
    quantizer (bit-exact quantize_row_q8_0_ref)."""
    xs, at, st = {}, 0, 0
    for k in sorted({k for _, _, k, _ in linears}):
        x = synth.normal(synth.SEED_ACTIVATIONS, (m, k), start=at)
        at += m * k + (m * k) % 2
        if row_scale:
            x *= synth.log_uniform(synth.SEED_OUTLIERS, m, *row_scale, start=st)[:, None]
            st += m
        xs[k] = x
    ws, wt = {}, 0
    for lin, wtype, k, n in linears:
        wf = synth.normal(synth.SEED_WEIGHTS, (n, k), std=0.02, start=wt)
        wt += n * k + (n * k) % 2
        ws[lin] = synth.pack_q5_K(wf) if wtype == "Q5_K" else synth.pack_q6_K(wf) if wtype == "Q6_K" else wf
    return xs, ws


def bench_workloads(sess, synth, _lib, types, steps):
    """Every linear of each workload timed alone (quantize + GEMM per step, and
    the GEMM alone), then the workload's linears back to back as one series.
    Returns the JSON records and, per workload, what the CPU leg needs."""
    out, keep = {}, {}
    both = _lib.STAGE_QUANTIZE | _lib.STAGE_MULTIPLY
    for name, m, row_scale, linears in WORKLOADS:
        log(f"workload {name}: generating inputs")
        xs, ws = workload_inputs(synth, name, m, row_scale, linears)
        xbs = {k: sess.to_device(x) for k, x in xs.items()}
        handles, ybs, recs, wbytes = [], [], {}, {}
        for lin, wtype, k, n in linears:
            if wtype == "Q8_0":  # quantize the float weights with the HIP quantizer
                wdev, qdev = sess.to_device(ws[lin]), sess.alloc(n * k // 32 * 34)
                _lib.check(sess.quantize_q8_0(wdev.ptr, qdev.ptr, n, k), "quantize weights")
                ws[lin] = qdev.download(np.uint8, n * k // 32 * 34).reshape(n, -1)
                wdev.free()
                qdev.free()
            wbytes[lin] = ws[lin]
            h = sess.weight(f"bench:{name}:{lin}", ws[lin], types[wtype], k, n)
            yb = sess.alloc(m * n * 4)
            handles.append((h, xbs[k].ptr, yb.ptr))
            ybs.append(yb)
            ops = 2.0 * m * n * k
            step_ms, reps = timed_series(sess, lambda: _lib.check(sess.matmul_stage(h, xbs[k].ptr, m, yb.ptr, both), lin), steps)
            gemm_ms, _ = timed_series(sess, lambda: _lib.check(sess.matmul_stage(h, None, m, yb.ptr, _lib.STAGE_MULTIPLY), lin),
                                      steps)
            recs[lin] = {"M": m, "K": k, "N": n, "type": wtype, "us": round(step_ms * 1e3, 2),
                         "tops": round(ops / (step_ms * 1e-3) / 1e12, 2),
                         "frac": round(ops / (step_ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4),
                         "gemm_us": round(gemm_ms * 1e3, 2), "gemm_tops": round(ops / (gemm_ms * 1e-3) / 1e12, 2),
                         "gemm_frac": round(ops / (gemm_ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4), "reps": reps}
            if (name, lin) in TRAFFIC_KEYS:
                recs[lin]["traffic"] = measured_traffic(TRAFFIC_KEYS[(name, lin)])
            log(f"  {lin} [{m},{k}]x[{n}] {wtype}: {step_ms * 1e3:.1f} us ({recs[lin]['frac'] * 100:.1f}%), "
                f"GEMM {gemm_ms * 1e3:.1f} us ({recs[lin]['gemm_frac'] * 100:.1f}%)")

        def block():
            for h, xp, yp in handles:
                _lib.check(sess.matmul(h, xp, m, yp), name)

        block_ms, block_reps = timed_series(sess, block, max(3, steps // len(linears)))
        ops = sum(2.0 * m * n * k for _, _, k, n in linears)
        ys = {}
        for (lin, _, _, n), yb in zip(linears, ybs):
            ys[lin] = yb.download(np.float32, m * n).reshape(m, n)
            yb.free()
        for xb in xbs.values():
            xb.free()
        rec = {"workload": WORKLOAD_TEXT[name], "linears": recs}
        if len(linears) > 1:
            rec["total"] = {"us": round(block_ms * 1e3, 2), "tops": round(ops / (block_ms * 1e-3) / 1e12, 2),
                            "frac": round(ops / (block_ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4),
                            "sum_of_linears_us": round(sum(r["us"] for r in recs.values()), 2), "reps": block_reps,
                            "ops": ops}
            log(f"  {name} back to back: {block_ms * 1e3:.1f} us ({rec['total']['frac'] * 100:.1f}%)")
        out[name] = rec
        keep[name] = (xs, wbytes, ys, linears)
    return out, keep


def cpu_workloads(cpu, types, out, keep):
    """The reference CPU path on the same inputs: every linear in full (a few
    seconds on 16 threads); with the oracle restatement instead, 64 token rows
    per linear and the time scaled to the full M."""
    for name, (xs, wbytes, ys, linears) in keep.items():
        total = 0.0
        for lin, wtype, k, n in linears:
            x = xs[k]
            rows = x.shape[0] if cpu.kind == "reference" else min(64, x.shape[0])
            cpu.matmul(wbytes[lin][:8], types[wtype], x[:4], 8)  # pool warm-up
            t = time.perf_counter()
            yc = cpu.matmul(wbytes[lin], types[wtype], x[:rows], n)
            sec = (time.perf_counter() - t) * x.shape[0] / rows
            err = row_rel(ys[lin][:rows], yc)
            r = out[name]["linears"][lin]
            r["cpu_us"] = round(sec * 1e6, 1)
            r["cpu_tops"] = round(2.0 * x.shape[0] * n * k / sec / 1e12, 4)
            r["cpu_rows_timed"] = rows
            r["parity_max_row_rel_err_vs_cpu"] = err
            total += sec
            log(f"  CPU {name}.{lin}: {sec * 1e3:.1f} ms; GPU vs CPU rel err {err:.2e}")
        if "total" in out[name]:
            out[name]["total"]["cpu_us"] = round(total * 1e6, 1)
            out[name]["total"]["cpu_tops"] = round(out[name]["total"]["ops"] / total / 1e12, 4)


def bench_pcie(sess, _lib, w, x, reps=10):
    """The headline step through pixhip_matmul with host operands in pinned
    memory (what hip_matmul receives from HipAllocator vectors): X copied to
    HBM, quantize + GEMM, Y copied back, synchronously, timed on the host clock."""
    hip = sess.lib  # libpixhip.so resolves the HIP runtime it links
    hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
    hip.hipHostFree.argtypes = [ctypes.c_void_p]
    xp, yp = ctypes.c_void_p(), ctypes.c_void_p()
    nx, ny = GEMM_M * GEMM_K * 4, GEMM_M * GEMM_N * 4
    if hip.hipHostMalloc(ctypes.byref(xp), nx, 0) or hip.hipHostMalloc(ctypes.byref(yp), ny, 0):
        raise RuntimeError("hipHostMalloc failed")
    try:
        ctypes.memmove(xp, x.ctypes.data, nx)
        for _ in range(3):
            _lib.check(sess.matmul(w, xp.value, GEMM_M, yp.value), "pixhip_matmul (host operands)")
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            _lib.check(sess.matmul(w, xp.value, GEMM_M, yp.value), "pixhip_matmul (host operands)")
            ts.append(time.perf_counter() - t)
    finally:
        hip.hipHostFree(xp)
        hip.hipHostFree(yp)
    sec = float(np.median(ts))
    return {"workload": "the headline step with X and Y in pinned host memory (pixhip_matmul stages them through HBM)",
            "us": round(sec * 1e6, 1), "tops": round(2.0 * GEMM_M * GEMM_N * GEMM_K / sec / 1e12, 2),
            "h2d_bytes": nx, "d2h_bytes": ny, "clock": f"host perf_counter, median of {reps} synchronous calls"}


def bench_pcie_ops(sess, synth, _lib, reps=5):
    """One VAE convolution (3x3, 256 x 256 pixels, 512 -> 512 channels) and the
    DiT attention (30 heads of 128, 4608 tokens) with every tensor in pinned
    host memory, as HipAllocator hands PixTensorVals to the backend, against
    the same call on device-resident tensors; both timed on the host clock
    around the call and a synchronisation (median of `reps`)."""
    hip = sess.lib
    hip.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
    hip.hipHostFree.argtypes = [ctypes.c_void_p]
    pinned = []

    def host(a):
        p = ctypes.c_void_p()
        if hip.hipHostMalloc(ctypes.byref(p), a.nbytes, 0):
            raise RuntimeError("hipHostMalloc failed")
        pinned.append(p)
        ctypes.memmove(p, a.ctypes.data, a.nbytes)
        return p.value

    def clock(fn):
        fn()
        sess.synchronize()
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            fn()
            sess.synchronize()
            ts.append(time.perf_counter() - t)
        return float(np.median(ts))

    out = {}
    try:
        wd, ht, cin, cout, k = CONV_CASES[0]
        w = (synth.normal(synth.SEED_WEIGHTS, (cout, cin * k * k)) / np.float32(np.sqrt(cin * k * k))).astype(np.float16)
        h = sess.conv_weight(f"bench:conv:{wd}:{cin}:{cout}", w.view(np.uint8), 1, k, k, cin, cout)
        x = np.resize(synth.normal(synth.SEED_ACTIVATIONS, (1 << 20,)), (wd * ht, cin))
        b = synth.normal(synth.SEED_OUTLIERS, (cout,))
        y = np.zeros((wd * ht, cout), np.float32)
        hx, hb, hy = host(x), host(b), host(y)
        xb, bb, yb = sess.to_device(x), sess.to_device(b), sess.alloc(y.nbytes)
        t_host = clock(lambda: _lib.check(sess.conv2d(h, hx, wd, ht, hy, None, hb), "conv2d (pinned)"))
        t_dev = clock(lambda: _lib.check(sess.conv2d(h, xb.ptr, wd, ht, yb.ptr, None, bb.ptr), "conv2d"))
        for bf in (xb, bb, yb):
            bf.free()
        moved = x.nbytes + y.nbytes + b.nbytes
        out["conv"] = {"workload": f"VAE conv {k}x{k}, {wd}x{ht} pixels, {cin} -> {cout} channels, input, bias and output "
                                   "in pinned host memory",
                       "us": round(t_host * 1e6, 1), "device_resident_us": round(t_dev * 1e6, 1), "pcie_bytes": moved,
                       "gbs_over_pcie": round(moved / (t_host - t_dev) / 1e9, 1) if t_host > t_dev else None}
        log(f"pinned-host conv: {t_host * 1e6:.0f} us (device-resident {t_dev * 1e6:.0f} us)")

        rows, heads, dim = 4608, 30, 128
        ch = heads * dim
        q = synth.normal(synth.SEED_ACTIVATIONS, (rows, ch))
        kk = synth.normal(synth.SEED_WEIGHTS, (rows, ch))
        v = synth.normal(synth.SEED_OUTLIERS, (rows, ch))
        hq, hk, hv, ho = host(q), host(kk), host(v), host(np.zeros_like(q))
        qb, kb, vb, ob = sess.to_device(q), sess.to_device(kk), sess.to_device(v), sess.alloc(q.nbytes)
        t_host = clock(lambda: _lib.check(sess.attention(hq, rows, hk, hv, rows, heads, heads, ch, ho), "attention (pinned)"))
        t_dev = clock(lambda: _lib.check(sess.attention(qb.ptr, rows, kb.ptr, vb.ptr, rows, heads, heads, ch, ob.ptr), "attention"))
        for bf in (qb, kb, vb, ob):
            bf.free()
        moved = 4 * q.nbytes
        out["attention"] = {"workload": f"self-attention, {heads} heads of {dim}, {rows} tokens, q, k, v and the output in "
                                        "pinned host memory",
                            "us": round(t_host * 1e6, 1), "device_resident_us": round(t_dev * 1e6, 1), "pcie_bytes": moved,
                            "gbs_over_pcie": round(moved / (t_host - t_dev) / 1e9, 1) if t_host > t_dev else None}
        log(f"pinned-host attention: {t_host * 1e6:.0f} us (device-resident {t_dev * 1e6:.0f} us)")
    finally:
        for p in pinned:
            hip.hipHostFree(p)
    for v in out.values():
        v["clock"] = f"host perf_counter around the call and a synchronisation, median of {reps}"
    return out


def bench_fused(sess, synth, _lib, Q5_K, Q8_0, reps):
    """The producers of a linear layer's input fused with its quantizer, at the
    DiT block's shapes, each against the same work done unfused (the producer
    writing fp32, then the quantize pass reading it back):
      norm    RMS norm + weight + modulation of X[4608, 3840] -> Q8_K (QKV / FFN-in)
      gate    SiLU(G) * U of [4608, 10240] -> Q8_0 (FFN-down input)
    Algorithmic bytes: fp32 inputs read once, planar activations written once
    (Q8_K 1 + 1/64 + 1/8 B per value, Q8_0 1 + 1/8).  Also two of the
    elementwise ops around the linears, in place: RoPE and the residual add."""
    m = 4608
    out = {}

    def timed(fn):
        # Warm up for >= 40 ms of device time: after the host-side set-up the
        # device's first milliseconds run up to 30% slower.
        fn()
        sess.synchronize()
        sess.timer_start()
        fn()
        once = sess.timer_stop()
        for _ in range(int(40.0 / max(once, 1e-3)) + 1):
            fn()
        sess.synchronize()
        sess.timer_start()
        for _ in range(reps):
            fn()
        return sess.timer_stop() / reps

    k = 3840
    x = synth.normal(synth.SEED_ACTIVATIONS, (m, k))
    nw = (1.0 + 0.1 * synth.normal(synth.SEED_WEIGHTS, (1, k))[0]).astype(np.float32)
    mod = (0.1 * synth.normal(synth.SEED_OUTLIERS, (1, k))[0]).astype(np.float32)
    xb, wb, mb, yb = sess.to_device(x), sess.to_device(nw), sess.to_device(mod), sess.alloc(m * k * 4)
    wq = sess.weight("bench:fused:q5k", synth.pack_q5_K(synth.normal(synth.SEED_WEIGHTS, (256, k), std=0.02)), Q5_K, k, 256)
    fused_ms = timed(lambda: _lib.check(sess.norm_quantize(Q5_K, xb.ptr, m, k, wb.ptr, 1e-5, 0, mb.ptr), "norm_quantize"))
    sep_ms = timed(lambda: (_lib.check(sess.norm_quantize(0, xb.ptr, m, k, wb.ptr, 1e-5, 0, mb.ptr, yb.ptr), "norm"),
                            _lib.check(sess.matmul_stage(wq, yb.ptr, m, None, _lib.STAGE_QUANTIZE), "quantize")))
    alg = m * k * 4 + m * k * (1 + 1 / 64 + 1 / 8) + 2 * k * 4
    out["norm_q8_K"] = {"workload": f"RMS norm + weight + modulation, X[{m},{k}] -> Q8_K", "us": round(fused_ms * 1e3, 2),
                        "gbs": round(alg / (fused_ms * 1e-3) / 1e9, 1), "frac": round(alg / (fused_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                        "unfused_us": round(sep_ms * 1e3, 2), "bytes": int(alg)}
    for b in (xb, wb, mb, yb):
        b.free()

    k = 10240
    g = synth.normal(synth.SEED_ACTIVATIONS, (m, k), std=3.0)
    u = synth.normal(synth.SEED_WEIGHTS, (m, k))
    gb, ub, yb = sess.to_device(g), sess.to_device(u), sess.alloc(m * k * 4)
    del g, u
    wq = sess.weight("bench:fused:q80", np.zeros((256, k // 32 * 34), np.uint8), Q8_0, k, 256)
    fused_ms = timed(lambda: _lib.check(sess.silu_gate_quantize(Q8_0, gb.ptr, ub.ptr, m, k), "silu_gate_quantize"))
    sep_ms = timed(lambda: (_lib.check(sess.silu_gate_quantize(0, gb.ptr, ub.ptr, m, k, yb.ptr), "silu_gate"),
                            _lib.check(sess.matmul_stage(wq, yb.ptr, m, None, _lib.STAGE_QUANTIZE), "quantize")))
    alg = m * k * 8 + m * k * (1 + 1 / 8)
    out["silu_gate_q8_0"] = {"workload": f"SiLU(G) * U, [{m},{k}] -> Q8_0", "us": round(fused_ms * 1e3, 2),
                             "gbs": round(alg / (fused_ms * 1e-3) / 1e9, 1),
                             "frac": round(alg / (fused_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                             "unfused_us": round(sep_ms * 1e3, 2), "bytes": int(alg)}
    for b in (gb, ub, yb):
        b.free()

    # Elementwise ops at the DiT block's attention shapes: RoPE on Q [4608, 3840]
    # (30 heads of 128) and the residual add [4608, 3840]; bytes = read + write.
    k = 3840
    qb = sess.to_device(synth.normal(synth.SEED_ACTIVATIONS, (m, k)))
    rb = sess.to_device(synth.normal(synth.SEED_WEIGHTS, (m, k)))
    th = (synth.normal(synth.SEED_OUTLIERS, (m, 64)) * 3.0).astype(np.float64)
    cb, sb = sess.to_device(np.cos(th).astype(np.float32)), sess.to_device(np.sin(th).astype(np.float32))
    rope_ms = timed(lambda: _lib.check(sess.rope(qb.ptr, m, k, 30, cb.ptr, sb.ptr, 0), "rope"))
    add_ms = timed(lambda: _lib.check(sess.pointwise(4, qb.ptr, rb.ptr, m, k), "add"))
    for name, ms, nbytes, what in (("rope", rope_ms, m * k * 8 + m * 64 * 8, f"RoPE, Q[{m},{k}], 30 heads of 128"),
                                   ("add", add_ms, m * k * 12, f"residual add [{m},{k}]")):
        out[name] = {"workload": what, "us": round(ms * 1e3, 2), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "bytes": int(nbytes)}
    for b in (qb, rb, cb, sb):
        b.free()
    for name, v in out.items():
        log(f"{name}: {v['us']} us ({v['gbs']} GB/s)" + (f"; unfused {v['unfused_us']} us" if "unfused_us" in v else ""))
    return out


# (key, tokens, heads, head size, kernel, workload text)
ATTN_SHAPES = [
    ("attention", 4608, 30, 128, "attn_kernel<128>",
     "self-attention, 30 heads of 128, 4608 tokens, not causal (Z-Image DiT: 4096 image + 512 text tokens)"),
    ("attention_vae", 16384, 1, 512, "attn_wide_kernel<128>",
     "self-attention, one head of 512, 16384 tokens, not causal (Z-Image VAE mid-block at a 128 x 128 latent)"),
]
ATTN_CPU_ROWS = 32  # query rows the CPU reference is timed on


def bench_attention(sess, synth, _lib, reps, shape):
    """tensor_attention at one model shape (not causal).  Algorithmic work 4 *
    heads * rows^2 * dim flops (the two products); the kernel runs each fp32
    product as three bf16 MFMA terms, so its matrix-core work is 3x that,
    priced against the dense bf16 peak."""
    key, rows, heads, dim, kernel, text = shape
    ch = heads * dim
    q = synth.normal(synth.SEED_ACTIVATIONS, (rows, ch))
    k = synth.normal(synth.SEED_WEIGHTS, (rows, ch))
    v = synth.normal(synth.SEED_OUTLIERS, (rows, ch))
    qb, kb, vb, ob = sess.to_device(q), sess.to_device(k), sess.to_device(v), sess.alloc(q.nbytes)

    def run():
        _lib.check(sess.attention(qb.ptr, rows, kb.ptr, vb.ptr, rows, heads, heads, ch, ob.ptr), "attention")

    ms, n = timed_series(sess, run, max(5, reps // 5))
    y = ob.download(np.float32, rows * ch).reshape(rows, ch)
    for b in (qb, kb, vb, ob):
        b.free()
    flops = 4.0 * heads * rows * rows * dim
    tf = flops / (ms * 1e-3) / 1e12
    log(f"{key} {heads}x{dim} over {rows} tokens: {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s "
        f"({3 * tf:.1f} TFLOP/s of bf16 MFMA work)")
    rec = {"workload": text, "us": round(ms * 1e3, 2), "tflops": round(tf, 2), "reps": n,
           "roofline": {"kernel": kernel, "bound": "mfma", "achieved": round(3 * tf, 2), "peak": PEAK_BF16_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(3 * tf / PEAK_BF16_TFLOPS, 4), "traffic": measured_traffic(key),
                        "work_per_launch": f"3 x 4*heads*rows^2*dim = {3 * flops:.4e} bf16 MFMA flops (fp32 products as three bf16 terms)"}}
    return rec, (shape, q, k, v, y)


def cpu_attention(cpu, rec, data):
    """The reference's tensor_attention (oracle/_ref, or the oracle) on the
    first ATTN_CPU_ROWS query rows against every key, the time scaled to all
    rows (each row's work is the same), and the GPU rows checked against it."""
    (key, tokens, heads, dim, _, _), q, k, v, y = data
    rows = ATTN_CPU_ROWS
    cpu.ol.attention(cpu.lib, cpu.prefix, q[:4], k[:64], v[:64], heads, heads)  # pool warm-up
    t = time.perf_counter()
    yc = cpu.ol.attention(cpu.lib, cpu.prefix, q[:rows], k, v, heads, heads)
    sec = (time.perf_counter() - t) * tokens / rows
    err = row_rel(y[:rows], yc)
    flops = 4.0 * heads * tokens * tokens * dim
    rec["cpu_baseline"] = {"value": round(flops / sec / 1e12, 5), "unit": "TFLOP/s", "cores": cpu.threads, "kind": cpu.kind,
                           "sample": f"first {rows} of {tokens} query rows, all keys, scaled to all rows",
                           "us": round(sec * 1e6, 1)}
    rec["parity_max_row_rel_err_vs_cpu"] = err
    log(f"CPU {key}: {sec * 1e3:.0f} ms (scaled); GPU vs CPU rel err {err:.2e}")


BLOCK_CAPTION, BLOCK_IMAGE, BLOCK_PATCH_WIDTH = 512, 4096, 64  # the DiT's joint sequence: caption rows, then a 64 x 64 grid


def bench_block(sess, synth, _lib, reps):
    """One Z-Image DiT block (z_block, src/inference.cpp:293-345) through the C
    ABI (pixelina_amd/zimage.py) at 4608 tokens with its timestep modulation:
    the whole block back to back, then each of its ops alone (in block order,
    so every op finds the state its predecessor leaves) for per-op shares.
    Linears Q5_K except FFN-down and the modulation Q8_0 (HIP quantizer),
    weights from stream 1338 in the order qkv, out, w1, w3, w2, modulation;
    x and the timestep from stream 1337; norm weights 1 + N(0, 0.1) and the
    modulation bias N(0, 0.1) from stream 1339."""
    from pixelina_amd import Q5_K, Q8_0, zimage

    rows = BLOCK_CAPTION + BLOCK_IMAGE
    lin, at = {}, 0
    for key in ("qkv", "out", "w1", "w3", "w2", "modulation"):
        inner, n = zimage.ZBlockWeights.SHAPES[key]
        wf = synth.normal(synth.SEED_WEIGHTS, (n, inner), std=0.02, start=at)
        at += n * inner + (n * inner) % 2
        if key in ("w2", "modulation"):
            wdev, qdev = sess.to_device(wf), sess.alloc(n * inner // 32 * 34)
            _lib.check(sess.quantize_q8_0(wdev.ptr, qdev.ptr, n, inner), "quantize weights")
            lin[key] = (qdev.download(np.uint8, n * inner // 32 * 34).reshape(n, -1), Q8_0)
            wdev.free()
            qdev.free()
        else:
            lin[key] = (synth.pack_q5_K(wf), Q5_K)
        del wf
    vec, vt = {}, 0
    for key, n in (("attention_norm1", zimage.HIDDEN), ("attention_norm2", zimage.HIDDEN), ("ffn_norm1", zimage.HIDDEN),
                   ("ffn_norm2", zimage.HIDDEN), ("q_norm", zimage.HEAD_DIM), ("k_norm", zimage.HEAD_DIM),
                   ("modulation_bias", 4 * zimage.HIDDEN)):
        g = synth.normal(synth.SEED_OUTLIERS, (n,), std=0.1, start=vt)
        vt += n + n % 2
        vec[key] = g if key == "modulation_bias" else 1.0 + g
    x = synth.normal(synth.SEED_ACTIVATIONS, (rows, zimage.HIDDEN))
    t = synth.normal(synth.SEED_ACTIVATIONS, (1, zimage.TIME_DIM), start=x.size)
    cc, cs = zimage.rotary(BLOCK_CAPTION, 0, 0, False)
    ic, iS = zimage.rotary(BLOCK_IMAGE, BLOCK_CAPTION, BLOCK_PATCH_WIDTH, True)
    wts = zimage.ZBlockWeights(sess, "bench:zblock", lin, vec)
    blk = zimage.ZBlock(sess, wts, rows)
    xb, tb = sess.to_device(x), sess.to_device(t)
    cb, sb = sess.to_device(np.concatenate([cc, ic])), sess.to_device(np.concatenate([cs, iS]))
    ops = blk.ops(xb.ptr, cb.ptr, sb.ptr, tb.ptr)

    def run():
        for _, fn in ops:
            fn()

    block_ms, n = timed_series(sess, run, max(3, reps // 10))
    per = {}
    for name, fn in ops:
        ms, k = timed_series(sess, fn, max(5, reps // 5), floor_ms=5.0)
        per[name] = ms
    total = sum(per.values())
    gemm_ops = {"modulation": 2.0 * zimage.TIME_DIM * 4 * zimage.HIDDEN,
                "qkv": 2.0 * rows * zimage.HIDDEN * 3 * zimage.HIDDEN, "out": 2.0 * rows * zimage.HIDDEN ** 2,
                "w1": 2.0 * rows * zimage.HIDDEN * zimage.INTERMEDIATE, "w3": 2.0 * rows * zimage.HIDDEN * zimage.INTERMEDIATE,
                "w2": 2.0 * rows * zimage.INTERMEDIATE * zimage.HIDDEN}
    attn_flops = 4.0 * zimage.HEADS * rows * rows * zimage.HEAD_DIM
    for b in (xb, tb, cb, sb):
        b.free()
    blk.free()
    wts.free()
    rec = {"workload": f"Z-Image DiT block (z_block) at {rows} tokens ({BLOCK_CAPTION} caption + {BLOCK_IMAGE} image), "
                       f"hidden {zimage.HIDDEN}, {zimage.HEADS} heads of {zimage.HEAD_DIM}, timestep-modulated; "
                       "Q5_K linears, Q8_0 FFN-down and modulation",
           "us": round(block_ms * 1e3, 2), "reps": n, "sum_of_ops_us": round(total * 1e3, 2),
           "linear_int8_tops": round(sum(gemm_ops.values()) / (block_ms * 1e-3) / 1e12, 2),
           "attention_tflops": round(attn_flops / (per["attention"] * 1e-3) / 1e12, 2),
           "ops": {k: {"us": round(v * 1e3, 2), "share": round(v / total, 4)} for k, v in per.items()},
           "note": "each op timed alone in block order; shares of the sum of the ops; ops that enqueue several launches "
                   "(split: 3 row copies, head_norm and rope: q and k) are one entry"}
    log(f"block {rows} tokens: {block_ms * 1e3:.1f} us (sum of ops {total * 1e3:.1f} us); "
        + ", ".join(f"{k} {v * 1e3:.0f}" for k, v in per.items()))
    return rec


# The rest of the op surface at the models' shapes: (name, workload text).
# Every case rotates over enough buffer copies (>= 1 GiB) that the 256 MB
# Infinity Cache cannot serve a repeat, and is priced by its algorithmic HBM
# bytes (each input read once, each output written once) against 8 TB/s.
SURFACE_ROTATE_BYTES = 1 << 30


def bench_surface(sess, synth, _lib):
    out = {}

    def case(name, text, nbytes, make, min_reps=20):
        copies = max(1, int(np.ceil(SURFACE_ROTATE_BYTES / nbytes)))
        sets = [make() for _ in range(copies)]
        state = {"i": 0}

        def run():
            bufs, fn = sets[state["i"] % copies]
            state["i"] += 1
            fn(bufs)

        ms, n = timed_series(sess, run, min_reps)
        for bufs, _ in sets:
            for b in bufs:
                b.free()
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"workload": text, "us": round(ms * 1e3, 2), "value": round(gbs, 1), "unit": "GB/s", "reps": n,
                     "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                  "frac": round(gbs / PEAK_HBM_GBS, 4), "work_per_launch": f"{nbytes} bytes"}}
        log(f"{name}: {ms * 1e3:.1f} us, {gbs:.0f} GB/s ({gbs / PEAK_HBM_GBS:.1%} of HBM peak)")

    # one SplitMix64 block (seed 1337) of 2^20 values, tiled over every operand
    block = synth.normal(synth.SEED_ACTIVATIONS, (1 << 20,))

    def dev(shape, scale=1.0):
        return sess.to_device(np.resize(block * np.float32(scale), shape))

    # z_residual with the gate, DiT activations [4608, 3840]
    r, c = 4608, 3840
    case("residual_gated", f"z_residual x[{r},{c}] += o * tanh(gate part 2)", 3 * r * c * 4 + c * 4,
         lambda: ((dev((r, c)), dev((r, c)), dev((6 * c,), 0.3)),
                  lambda b: _lib.check(sess.pointwise_ex(9, b[0].ptr, b[1].ptr, b[2].ptr, r, c, 2), "residual")))
    # qwen_image_modulate, scale form, Qwen-Image edit stream [8448, 3072]
    r, c = 8448, 3072
    case("qwen_modulate", f"qwen_image_modulate x[{r},{c}] *= 1 + p (256 text rows on parameter row 1)", 2 * r * c * 4 + 2 * c * 4,
         lambda: ((dev((r, c)), dev((2, 6 * c), 0.3)),
                  lambda b: _lib.check(sess.qwen_modulate(b[0].ptr, r, c, b[1].ptr, 6 * c, 256, 1), "qwen modulate")))
    # tensor_l2norm over the Qwen VAE decoder's full-resolution pixels
    r, c = 1024 * 1024, 96
    case("l2norm", f"tensor_l2norm [{r},{c}] (Qwen VAE, 1024x1024 pixels)", 2 * r * c * 4 + c * 4,
         lambda: ((dev((r, c)), dev((c,)), sess.alloc(r * c * 4)),
                  lambda b: _lib.check(sess.l2norm(b[0].ptr, r, c, b[1].ptr, 1e-12, b[2].ptr), "l2norm")), min_reps=10)
    # tensor_groupnorm over the Flux VAE decoder's full-resolution pixels
    r, c = 1024 * 1024, 128
    case("groupnorm", f"tensor_groupnorm(32) [{r},{c}] (VAE, 1024x1024 pixels; 3 passes: 2 reads + 1 write)", 2 * r * c * 4 + 2 * c * 4,
         lambda: ((dev((r, c)), dev((c,)), dev((c,)), sess.alloc(r * c * 4)),
                  lambda b: _lib.check(sess.groupnorm(b[0].ptr, r, c, b[1].ptr, b[2].ptr, b[3].ptr), "groupnorm")), min_reps=10)
    # tensor_upsample of the VAE's 512x512 x 128 stage to 1024x1024
    w, c = 512, 128
    case("upsample", f"tensor_upsample [{w}x{w},{c}] -> [{2 * w}x{2 * w},{c}]", 5 * w * w * c * 4,
         lambda: ((dev((w * w, c)), sess.alloc(4 * w * w * c * 4)),
                  lambda b: _lib.check(sess.layout(17, b[0].ptr, w * w, c, b[1].ptr, 4 * w * w, c, w), "upsample")), min_reps=10)
    # the DiT's q / k / v split of the fused projection
    r, c = 4608, 3840
    case("copy_rows", f"vulkan_copy_rows: k = qkv[{r},{3 * c}][:, {c}:{2 * c}]", 2 * r * c * 4,
         lambda: ((dev((r, 3 * c)), sess.alloc(r * c * 4)),
                  lambda b: _lib.check(sess.copy_rows(b[0].ptr, r, 3 * c, b[1].ptr, r, c, r, 0, c, 0), "copy rows")))
    return out


# VAE convolutions (implicit GEMM on split-bf16 MFMA): (width, height, cin, cout, kernel)
CONV_CASES = [(256, 256, 512, 512, 3), (1024, 1024, 128, 128, 3), (128, 128, 16, 512, 3)]


def bench_conv(sess, synth, _lib):
    """tensor_conv at VAE decoder shapes with F16 weights.  Algorithmic work
    2 * pixels * cout * cin * k^2; the kernel runs each product as three bf16
    MFMA terms, so its matrix-core work is 3x that, priced against the dense
    bf16 peak.  Inputs: SplitMix64 normals, weights from seed 1338 scaled by
    1/sqrt(fan-in), the image a 2^20-value block of seed 1337 tiled over the
    pixels, the bias from seed 1339."""
    out = {}
    block = synth.normal(synth.SEED_ACTIVATIONS, (1 << 20,))
    for wd, ht, cin, cout, k in CONV_CASES:
        w = (synth.normal(synth.SEED_WEIGHTS, (cout, cin * k * k)) / np.float32(np.sqrt(cin * k * k))).astype(np.float16)
        h = sess.conv_weight(f"bench:conv:{wd}:{cin}:{cout}", w.view(np.uint8), 1, k, k, cin, cout)
        xb = sess.to_device(np.resize(block, (wd * ht, cin)))
        bb = sess.to_device(synth.normal(synth.SEED_OUTLIERS, (cout,)))
        yb = sess.alloc(wd * ht * cout * 4)

        def run():
            _lib.check(sess.conv2d(h, xb.ptr, wd, ht, yb.ptr, None, bb.ptr), "conv2d")

        ms, n = timed_series(sess, run, 5)
        for b in (xb, bb, yb):
            b.free()
        flops = 2.0 * wd * ht * cout * cin * k * k
        tf = flops / (ms * 1e-3) / 1e12
        name = f"conv{k}x{k}_{wd}x{ht}_{cin}to{cout}"
        out[name] = {"workload": f"VAE conv {k}x{k}, {wd}x{ht} pixels, {cin} -> {cout} channels, F16 weights, bias",
                     "us": round(ms * 1e3, 1), "tflops": round(tf, 1), "reps": n,
                     "roofline": {"kernel": "conv_image_kernel" if cin % 32 == 0 else "conv_gather_kernel", "bound": "mfma",
                                  "achieved": round(3 * tf, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                  "frac": round(3 * tf / PEAK_BF16_TFLOPS, 4),
                                  "work_per_launch": f"3 x 2*pixels*cout*cin*k^2 = {3 * flops:.4e} bf16 MFMA flops"}}
        log(f"{name}: {ms * 1e3:.0f} us, {tf:.1f} TFLOP/s ({3 * tf:.0f} TFLOP/s of bf16 MFMA work, "
            f"{3 * tf / PEAK_BF16_TFLOPS:.1%} of peak)")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # untimed steps, continued until >= 50 ms of device time: the first 5-50 ms
    # of work on an idle device run up to 30% slower (clock / power ramp)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--matvec-reps", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-matvec", action="store_true")
    ap.add_argument("--no-fused", action="store_true", help="skip the fused norm / SiLU-gate producers")
    ap.add_argument("--no-blocks", action="store_true", help="skip the single Q8_0 linear and the block workloads")
    ap.add_argument("--no-pcie", action="store_true", help="skip the host-operand (PCIe-inclusive) step")
    ap.add_argument("--no-attention", action="store_true", help="skip the DiT- and VAE-shape attention")
    ap.add_argument("--no-surface", action="store_true", help="skip the norms, layouts and row moves")
    ap.add_argument("--no-conv", action="store_true", help="skip the VAE convolutions")
    ap.add_argument("--no-block", action="store_true", help="skip the whole DiT block")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one plain 512 MiB device copy (the calibration kernel for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    from pixelina_amd import Q5_K, Q6_K, Q8_0, Session, _lib, synth

    x, wb, ch = gemm_workload(synth)
    ops = 2.0 * GEMM_M * GEMM_N * GEMM_K
    out = {}
    with Session(0) as sess:
        device = sess.device_name()
        log(f"device {device}")
        w = sess.weight("bench:gemm:q5k", wb, Q5_K, GEMM_K, GEMM_N)
        xb = sess.to_device(x)
        yb = sess.alloc(GEMM_M * GEMM_N * 4)
        both = _lib.STAGE_QUANTIZE | _lib.STAGE_MULTIPLY
        warm_steps = max(1, args.warmup)
        warm_ms = sess.bench_matmul([w], xb.ptr, GEMM_M, yb.ptr, both, warm_steps)
        while warm_ms < WARMUP_FLOOR_MS:
            more = int((WARMUP_FLOOR_MS - warm_ms) / (warm_ms / warm_steps)) + 1
            warm_ms += sess.bench_matmul([w], xb.ptr, GEMM_M, yb.ptr, both, more)
            warm_steps += more
        log(f"warmup {warm_steps} steps, {warm_ms:.1f} ms of device time")
        log(f"timing {args.steps} steps (quantize + GEMM)")
        ms_step = sess.bench_matmul([w], xb.ptr, GEMM_M, yb.ptr, both, args.steps) / args.steps
        ms_gemm = sess.bench_matmul([w], xb.ptr, GEMM_M, yb.ptr, _lib.STAGE_MULTIPLY, args.steps) / args.steps
        ms_quant = sess.bench_matmul([w], xb.ptr, GEMM_M, yb.ptr, _lib.STAGE_QUANTIZE, args.steps) / args.steps
        _lib.check(sess.matmul(w, xb.ptr, GEMM_M, yb.ptr), "pixhip_matmul")
        y_gpu = yb.download(np.float32, GEMM_M * GEMM_N).reshape(GEMM_M, GEMM_N)
        log(f"step {ms_step * 1e3:.1f} us, GEMM {ms_gemm * 1e3:.1f} us, quantize {ms_quant * 1e3:.1f} us")
        xb.free()
        yb.free()
        pcie = None if args.no_pcie else bench_pcie(sess, _lib, w, x)
        if pcie:
            log(f"host operands (PCIe-inclusive): {pcie['us']:.0f} us per step")
            pcie = {"headline": pcie, **bench_pcie_ops(sess, synth, _lib)}
        types = {"Q5_K": Q5_K, "Q6_K": Q6_K, "Q8_0": Q8_0}
        workloads, keep = ({}, {}) if args.no_blocks else bench_workloads(sess, synth, _lib, types, args.steps)
        gguf_bytes, resident_bytes = sess.residency()

        matvec = {}
        if not args.no_matvec:
            xv = synth.normal(synth.SEED_ACTIVATIONS, (1, MV_K))
            wv = synth.normal(synth.SEED_WEIGHTS, (MV_N, MV_K), std=0.02)
            # Q8_0 weights from the HIP quantizer (bit-exact quantize_row_q8_0_ref)
            wdev = sess.to_device(wv)
            qdev = sess.alloc(MV_N * MV_K // 32 * 34)
            _lib.check(sess.quantize_q8_0(wdev.ptr, qdev.ptr, MV_N, MV_K), "quantize weights")
            wq8 = qdev.download(np.uint8, MV_N * MV_K // 32 * 34).reshape(MV_N, -1)
            wdev.free()
            qdev.free()
            wq5 = synth.pack_q5_K(wv)
            wq6 = synth.pack_q6_K(wv)
            del wv
            xvb = sess.to_device(xv)
            yvb = sess.alloc(MV_N * 4)
            for name, wtype, wbytes in (("q5_K", Q5_K, wq5), ("q8_0", Q8_0, wq8), ("q6_K", Q6_K, wq6)):
                copies = int(np.ceil(MALL_DEFEAT_BYTES / wbytes.nbytes))
                handles = [sess.weight(f"bench:mv:{name}:{i}", wbytes, wtype, MV_K, MV_N) for i in range(copies)]
                sess.bench_matmul(handles, xvb.ptr, 1, yvb.ptr, both, copies)
                ms = sess.bench_matmul(handles, xvb.ptr, 1, yvb.ptr, both, args.matvec_reps) / args.matvec_reps
                _lib.check(sess.matmul(handles[0], xvb.ptr, 1, yvb.ptr), "matvec")
                yv = yvb.download(np.float32, MV_N)
                alg = wbytes.nbytes + 4 * MV_K + 4 * MV_N
                gbs = alg / (ms * 1e-3) / 1e9
                log(f"matvec {name}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s over {copies} weight copies")
                matvec[name] = {"us": ms * 1e3, "gbs": gbs, "bytes": alg, "copies": copies, "rotated_bytes": copies * wbytes.nbytes,
                                "y": yv, "w": wbytes, "type": wtype}
            xvb.free()
            yvb.free()
        fused = {} if args.no_fused else bench_fused(sess, synth, _lib, Q5_K, Q8_0, args.steps)
        attention = {} if args.no_attention else {sh[0]: bench_attention(sess, synth, _lib, args.steps, sh) for sh in ATTN_SHAPES}
        surface = None if args.no_surface else bench_surface(sess, synth, _lib)
        conv = None if args.no_conv else bench_conv(sess, synth, _lib)
        block = None if args.no_block else bench_block(sess, synth, _lib, args.steps)
        if args.calibrate_copy:
            src, dst = sess.alloc(COPY_BYTES), sess.alloc(COPY_BYTES)
            sess.copy_device(dst.ptr, src.ptr, COPY_BYTES)
            sess.synchronize()
            log(f"calibration copy: {COPY_BYTES >> 20} MiB read + {COPY_BYTES >> 20} MiB written (copy16_kernel)")
            src.free()
            dst.free()
        n_cached, cached_bytes = sess.cache_info()
        log(f"weight cache: {n_cached} entries, {cached_bytes / 2**30:.2f} GiB")

    tops_step = ops / (ms_step * 1e-3) / 1e12
    tops_gemm = ops / (ms_gemm * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(tops_step, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm_steps,
        "warmup_ms": round(warm_ms, 2),
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": ("synthetic: SplitMix64 + Box-Muller for every workload, seeds 1337 (X), 1338 (W), 1339 (outlier "
                 "channels, per-token scales); the block workloads draw consecutive pieces of the same streams"),
        "config": {"workload": "Q5_K GEMM M=4096 K=3840 N=10240 (Z-Image DiT FFN), quantize + GEMM per step",
                   "M": GEMM_M, "K": GEMM_K, "N": GEMM_N, "weight_type": "Q5_K", "activation_type": "Q8_K",
                   "outlier_channels": int(len(ch)), "device": device},
        "roofline": {"kernel": "gemm_kq_kernel<Q5_K>", "bound": "mfma", "achieved": round(tops_gemm, 2), "peak": PEAK_INT8_TOPS,
                     "unit": "TOP/s", "frac": round(tops_gemm / PEAK_INT8_TOPS, 4), "traffic": measured_traffic("gemm_q5_K"),
                     "work_per_launch": f"2*M*N*K = {ops:.4e} int8 ops", "avg_launch_us": round(ms_gemm * 1e3, 2)},
        "gemm_only": {"us": round(ms_gemm * 1e3, 2), "tops": round(tops_gemm, 2)},
        "quantize": {"us": round(ms_quant * 1e3, 2), "gbs": round((GEMM_M * GEMM_K * 4 + GEMM_M * GEMM_K * 1.14) / (ms_quant * 1e-3) / 1e9, 1)},
    }
    if matvec:
        line["matvec"] = {
            k: {"workload": f"{k} matvec x[1,{MV_K}] W[{MV_N},{MV_K}], {args.matvec_reps} reps over {v['copies']} copies "
                            f"({v['rotated_bytes'] / 2**30:.2f} GiB)",
                "us": round(v["us"], 3), "value": round(v["gbs"], 1), "unit": "GB/s",
                "roofline": {"bound": "hbm", "achieved": round(v["gbs"], 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                             "frac": round(v["gbs"] / PEAK_HBM_GBS, 4), "traffic": measured_traffic(f"matvec_{k}"),
                             "work_per_launch": f"W + 4K + 4N = {v['bytes']} bytes"}}
            for k, v in matvec.items()}

    if fused:
        line["fused"] = fused
    for key, (rec, _) in attention.items():
        line[key] = rec
    if surface:
        line["surface"] = surface
    if conv:
        line["conv"] = conv
    if block:
        line["block"] = block
    if workloads:
        line["workloads"] = workloads
    if pcie:
        line["pcie_inclusive"] = pcie
    line["residency"] = {"gguf_bytes": gguf_bytes, "resident_bytes": resident_bytes,
                         "ratio": round(resident_bytes / max(gguf_bytes, 1), 3),
                         "note": "device bytes per GGUF byte of the headline and workload weights (GEMM layouts)"}

    if not args.no_cpu:
        threads = cpu_threads()
        cpu = CpuBaseline(threads)
        host = cpu_info()
        log(f"CPU baseline ({cpu.kind}, {threads} threads of {host['nproc']}, {host['cpu']})")
        if cpu.kind == "reference":
            xs, sample = x, f"full workload M={GEMM_M} N={GEMM_N} K={GEMM_K}, median of 3 after a pool warm-up"
            cpu.matmul(wb[:64], Q5_K, x[:16], 64)
            times = []
            for _ in range(3):
                t = time.perf_counter()
                y_cpu = cpu.matmul(wb, Q5_K, xs, GEMM_N)
                times.append(time.perf_counter() - t)
            t_cpu = float(np.median(times))
        else:
            rows = 256
            xs, sample = x[:rows], f"first {rows} tokens of the workload (N={GEMM_N} K={GEMM_K}), one run"
            t = time.perf_counter()
            y_cpu = cpu.matmul(wb, Q5_K, xs, GEMM_N)
            t_cpu = time.perf_counter() - t
        cpu_tops = 2.0 * xs.shape[0] * GEMM_N * GEMM_K / t_cpu / 1e12
        parity = row_rel(y_gpu[: xs.shape[0]], y_cpu)
        log(f"CPU {t_cpu:.2f} s -> {cpu_tops * 1e3:.1f} GOPS; GPU vs CPU max row rel err {parity:.2e}")
        line["cpu_baseline"] = {"value": round(cpu_tops, 5), "unit": "TOPS", "cores": threads, "kind": cpu.kind,
                                "sample": sample, "seconds": round(t_cpu, 3), **host,
                                "threads_rule": "every core in the process's affinity mask (the reference's -t default)"}
        line["parity"] = {"max_row_rel_err_vs_cpu": parity, "tolerance": 1e-4, "rows_checked": int(xs.shape[0])}
        for k, v in matvec.items():
            reps = args.matvec_reps
            cpu.matmul(v["w"], v["type"], xv, MV_N)
            ts = []
            for _ in range(reps):
                t = time.perf_counter()
                yc = cpu.matmul(v["w"], v["type"], xv, MV_N)
                ts.append(time.perf_counter() - t)
            tc = float(np.median(ts))
            err = row_rel(v["y"][None, :], yc)
            line["matvec"][k]["cpu_baseline"] = {"value": round(v["bytes"] / tc / 1e9, 2), "unit": "GB/s", "cores": threads,
                                                 "kind": cpu.kind, "sample": f"full matvec, median of {reps}",
                                                 "us": round(tc * 1e6, 1)}
            line["matvec"][k]["parity_max_row_rel_err"] = err
            log(f"CPU matvec {k}: {tc * 1e6:.0f} us; GPU vs CPU rel err {err:.2e}")
        if keep:
            cpu_workloads(cpu, types, workloads, keep)
        for rec, data in attention.values():
            cpu_attention(cpu, rec, data)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
