#!/usr/bin/env python3
"""Benchmark of the conv/GEMM hot path on one MI355X.

Headline (the `value`): the fused MatMul + bias + GELU of A[16,512,768] x W[768,3072] + b[3072]
on fp16 MFMA with fp32 accumulation, in TFLOP/s, with inputs resident in HBM. One step = one
launch of the fused Gemm dispatch over the whole batch (M = 8192 rows). Timing uses HIP events on
the session's stream around exactly `--steps` launches, after `--warmup` untimed ones and, whatever
`--warmup` asks, at least MIN_WARM_MS of untimed launches in all: after a cold start the GPU runs
launches ~20 to ~500 of this load up to ~17% slower (55 against 47 us per launch; the first ~20 run
at full speed) until its clocks settle after ~30 ms. The warmup actually run is reported as
`warmup_run`.

Also reported on the same line:
  roofline      the Gemm kernel's achieved TFLOP/s vs the dense fp16 MFMA peak (2.5 PFLOP/s), and
                its HBM traffic per launch from the committed rocprofv3 counter summary
  cpu_baseline  the CPU oracle (a C++ restatement of the reference's AVX-512/AVX2 Gemm micro-kernel
                + GELU epilogue) on the same workload, all host cores
  gemm_bf16     the same Gemm with bf16 storage (bf16 matrix cores, fp32 accumulation)
  detector / detector_fp32 / recognizer / recognizer_bf16 / mobilenetv3
                ms per image of the whole networks (HIP-graph replay), per-kernel-class roofline
  conv3x3       the fp32 Conv3x3 + bias + ReLU 1x64x64x64 kernel (us, TFLOP/s)
  conv_large_f16 / conv_large_bf16
                the Conv3x3 + bias + ReLU over 8x128x128, 256 -> 256 channels (154.6 GFLOP) on the halo
                tile (input halos in LDS, weights through an LDS-DMA ring) in fp16 / bf16 storage, against
                the dense MFMA peak
  ops           the kernels of the rest of the ExecOp surface (resize, pad, transpose, slice, unary,
                depth-space, pools, MatMul) at detector / recognizer sizes, GB/s vs the HBM peak
  hbm_kernels   the convnets' bandwidth-bound kernels (depthwise 5x5 s1 / 3x3 s2, the SE passes, nearest,
                elementwise) past the L2: GB/s from algorithmic bytes and from the committed
                rocprofv3 FETCH_SIZE / WRITE_SIZE counts (profiles/traffic_hbm_kernels.json)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import struct
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_FP32_TFLOPS = 157.3    # MI355X fp32 (matrix)
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def traffic_from_profiles(workload: str, kernel: str):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 PMC summary; None when
    the summary was taken on another kernel (a tiling that the backend no longer selects)."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        d = json.load(f)
    if d.get("kernel") != kernel:
        log(f"traffic summary is for {d.get('kernel')}, the bench runs {kernel}: traffic not reported")
        return None
    return d.get("bytes_per_launch")


MIN_WARM_MS = 150.0  # untimed launches before the headline's timed region, at least (see the docstring)


def bench_gemm(steps: int, warmup: int, storage="f16"):
    from simdonnx_amd import graphs
    from simdonnx_amd.backend import HipBackend, HipInferenceSession
    from simdonnx_amd import native as N

    hip = HipBackend.default()
    plan, ins = graphs.matmul_bias_gelu()
    flops = graphs.matmul_flops()
    g = hip.graph(plan, storage)
    names = [d[0] for d in g.dispatches]
    kernels = g.kernels
    with HipInferenceSession(g) as s:
        s.set_input(ins[0])
        s.run()  # stage the input into the arena once: the timed region reads it resident in HBM
        warm_ms, warm_n = 0.0, 0
        if warmup > 0:
            warm_ms, warm_n = s.time(warmup), warmup
        while warm_ms < MIN_WARM_MS:  # past the clock transient of a cold start, whatever `warmup` was
            warm_ms += s.time(200)
            warm_n += 200
        N.thin().sox_device_sync()
        t0 = time.perf_counter()
        ms = s.time(steps)  # HIP events on the session stream around exactly `steps` launches
        N.thin().sox_device_sync()
        wall = time.perf_counter() - t0
        per_launch_ms = ms / steps
        prof = s.profile(5)
    g.release()
    return dict(flops=flops, ms_total=ms, per_launch_ms=per_launch_ms, wall_s=wall, dispatches=names,
                kernels=kernels, kernel_ms=[p[2] for p in prof],
                warmup_run={"launches": warm_n, "ms": round(warm_ms, 1)})


def bench_mfma_peak(iters: int = 4000, reps: int = 20):
    """The matrix-core rate this GPU sustains on random fp16 operands with no memory traffic: the probe
    kernel of the Gemm code object (sox_probe_mfma_f16), launched through the thin C ABI with two
    waves per SIMD, timed with HIP events (median of `reps` launches after warm-up)."""
    import ctypes
    from simdonnx_amd import build as B
    from simdonnx_amd import native as N
    from simdonnx_amd.backend import HipBackend
    hip = HipBackend.default()
    T = N.thin()
    with open(os.path.join(B.BUILD, "gemm.hsaco"), "rb") as f:
        mod = hip.load_module(f.read())
    fn = N.c_void_p()
    N.check(T.sox_module_function(ctypes.byref(fn), mod, b"sox_probe_mfma_f16"), "probe kernel")
    cus = hip.device.compute_units
    threads = 512  # 8 waves per workgroup, one workgroup per CU: 2 waves per SIMD
    out = N.c_void_p()
    N.check(T.sox_malloc(ctypes.byref(out), cus * threads * 4), "probe output")
    stream = N.c_void_p()
    N.check(T.sox_stream_create(ctypes.byref(stream)), "stream")
    ev = [N.c_void_p(), N.c_void_p()]
    for e in ev:
        N.check(T.sox_event_create(ctypes.byref(e)), "event")
    grid = (N.c_uint32 * 3)(cus, 1, 1)
    block = (N.c_uint32 * 3)(threads, 1, 1)

    def launch(n):
        args = struct.pack("<QiI", out.value, n, 12345)
        buf = ctypes.create_string_buffer(args, len(args))
        N.check(T.sox_launch(fn, grid, block, 0, stream, buf, len(args)), "probe launch")

    for _ in range(200):  # warm-up: the clock settles under sustained matrix load
        launch(iters)
    times = []
    for _ in range(reps):
        N.check(T.sox_event_record(ev[0], stream), "event")
        launch(iters)
        N.check(T.sox_event_record(ev[1], stream), "event")
        N.check(T.sox_event_sync(ev[1]), "event")
        ms = N.c_float()
        N.check(T.sox_event_elapsed_ms(ctypes.byref(ms), ev[0], ev[1]), "event")
        times.append(ms.value)
    for e in ev:
        T.sox_event_destroy(e)
    T.sox_stream_destroy(stream)
    T.sox_free(out)
    ms = statistics.median(times)
    flops = cus * (threads // 64) * iters * 4 * 32 * 32 * 16 * 2
    tf = flops / (ms * 1e-3) / 1e12
    return dict(workload=f"{cus} CUs x 8 waves x {iters} x 4 v_mfma_f32_32x32x16_f16, random operands, no memory",
                ms=round(ms, 4), tflop_s=round(tf, 1), frac_of_peak=round(tf / PEAK_FP16_TFLOPS, 4))


def bench_vendor_gemm(reps: int = 500):
    """The vendor BLAS (hipBLASLt through torch) on the headline shape, for scale beside the fused kernel:
    A[8192,768] x W[768,3072] as a plain product, with the bias (linear), and with the bias and a separate
    GELU (the unfused form of what the fused kernel computes). fp16 and bf16, HIP events over `reps`
    launches after warm-up on torch's current stream. A reported reference point, never `value`."""
    import torch
    M, K, N = 8192, 768, 3072
    g = torch.Generator(device="cuda").manual_seed(0)
    res = {"workload": "A[8192,768] x W[768,3072] (+ b[3072]) (-> GELU), torch.matmul / F.linear / F.gelu"}
    for name, dt in (("f16", torch.float16), ("bf16", torch.bfloat16)):
        a = torch.randn(M, K, device="cuda", dtype=dt, generator=g)
        w = (torch.randn(N, K, device="cuda", dtype=dt, generator=g) * 0.02).contiguous()
        wt = w.t().contiguous()
        b = torch.rand(N, device="cuda", dtype=dt, generator=g) * 0.2 - 0.1
        legs = {"matmul": lambda: a @ wt, "linear_bias": lambda: torch.nn.functional.linear(a, w, b),
                "linear_bias_gelu": lambda: torch.nn.functional.gelu(torch.nn.functional.linear(a, w, b))}
        r = {}
        for leg, f in legs.items():
            for _ in range(100):
                f()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                f()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / reps * 1e3
            r[leg] = {"us": round(us, 2), "tflop_s": round(2 * M * N * K / us / 1e6, 1)}
        res[name] = r
    return res


def bench_lds_peak(iters: int = 2000, reps: int = 10):
    """Per-CU throughput of the two LDS paths the Gemm ring lives on (probe.hip, one 16-wave workgroup
    per CU): ds_read_b128 with 16 KiB in flight per wave, and global_load_lds_dwordx4 from L2-resident
    data. HIP events, median of `reps` launches after warm-up; bytes per cycle at the device's
    reported peak clock (a lower bound on bytes per actual cycle)."""
    import ctypes
    from simdonnx_amd import build as B
    from simdonnx_amd import native as N
    from simdonnx_amd.backend import HipBackend
    hip = HipBackend.default()
    T = N.thin()
    with open(os.path.join(B.BUILD, "probe.hsaco"), "rb") as f:
        mod = hip.load_module(f.read())
    cus, threads = hip.device.compute_units, 1024
    clock_ghz = hip.device.clock_khz / 1e6
    out, src = N.c_void_p(), N.c_void_p()
    N.check(T.sox_malloc(ctypes.byref(out), cus * threads * 4), "probe output")
    N.check(T.sox_malloc(ctypes.byref(src), 64 * 65536), "probe source")
    stream = N.c_void_p()
    N.check(T.sox_stream_create(ctypes.byref(stream)), "stream")
    ev = [N.c_void_p(), N.c_void_p()]
    for e in ev:
        N.check(T.sox_event_create(ctypes.byref(e)), "event")
    grid = (N.c_uint32 * 3)(cus, 1, 1)
    block = (N.c_uint32 * 3)(threads, 1, 1)
    res = {}
    for name, per_round in (("sox_probe_lds_read", 16 * 16 * 1024), ("sox_probe_lds_dma", 16 * 8 * 1024)):
        fn = N.c_void_p()
        N.check(T.sox_module_function(ctypes.byref(fn), mod, name.encode()), "probe kernel")
        args = struct.pack("<QQii", out.value, src.value, iters, 0)
        buf = ctypes.create_string_buffer(args, len(args))
        for _ in range(20):
            N.check(T.sox_launch(fn, grid, block, 0, stream, buf, len(args)), "probe launch")
        times = []
        for _ in range(reps):
            N.check(T.sox_event_record(ev[0], stream), "event")
            N.check(T.sox_launch(fn, grid, block, 0, stream, buf, len(args)), "probe launch")
            N.check(T.sox_event_record(ev[1], stream), "event")
            N.check(T.sox_event_sync(ev[1]), "event")
            ms = N.c_float()
            N.check(T.sox_event_elapsed_ms(ctypes.byref(ms), ev[0], ev[1]), "event")
            times.append(ms.value)
        ms = statistics.median(times)
        per_cu = per_round * iters / (ms * 1e-3)  # bytes / s per CU
        res[name.replace("sox_probe_", "")] = dict(us=round(ms * 1e3, 1), tb_s=round(per_cu * cus / 1e12, 2),
                                                    gb_s_per_cu=round(per_cu / 1e9, 1),
                                                    bytes_per_clk_at_peak_clock=round(per_cu / (clock_ghz * 1e9), 1))
    for e in ev:
        T.sox_event_destroy(e)
    T.sox_stream_destroy(stream)
    T.sox_free(out)
    T.sox_free(src)
    return dict(workload=f"{cus} CUs x 16 waves: ds_read_b128 (16 KiB in flight per wave) and "
                         f"global_load_lds_dwordx4 from L2, {iters} rounds", peak_clock_ghz=clock_ghz, **res)


def bench_conv_large(steps: int, storage="f16"):
    """A large conv: Conv3x3 s1 p1 + bias + ReLU, NHWC, 8x128x128, 256 -> 256 channels (154.6 GFLOP),
    16-bit storage, against the dense MFMA peak (the backend's choice, reported in `kernels`: the halo
    tile, or the implicit-GEMM ring under SIMDONNX_HIP_NO_H256)."""
    from simdonnx_amd import synth
    from simdonnx_amd.backend import HipBackend, HipInferenceSession
    from simdonnx_amd.plan import NHWC, PlanBuilder
    n, h, w, c = 8, 128, 128, 256
    pb = PlanBuilder()
    x = pb.input((n, c, h, w), NHWC, "x")
    y = pb.conv(x, synth.he_normal(64, 1, (c, c, 3, 3)), synth.uniform(64, 2, (c,), -0.1, 0.1), pad=1, act="relu",
                name="conv")
    hip = HipBackend.default()
    g = hip.graph(pb.build(y), storage)
    kern = g.kernels  # the code object functions (the ring tiling), not the op labels
    with HipInferenceSession(g) as s:
        s.set_input(synth.normal(64, 3, (n, h, w, c), 1.0))
        s.run()
        warm_ms = s.time(100)
        while warm_ms < MIN_WARM_MS:  # past the clock transient of a cold start (as the headline leg)
            warm_ms += s.time(100)
        ms = s.time(steps) / steps
    g.release()
    flops = 2 * n * h * w * c * c * 9
    tf = flops / (ms * 1e-3) / 1e12
    return dict(workload=f"conv3x3 s1 p1 + bias + ReLU, NHWC {n}x{h}x{w}, {c}->{c}, {storage} storage",
                kernels=kern, us=round(ms * 1e3, 2), tflop_s=round(tf, 1), frac_of_peak=round(tf / PEAK_FP16_TFLOPS, 4))


def bench_conv(steps: int):
    from simdonnx_amd import graphs
    from simdonnx_amd.backend import HipBackend, HipInferenceSession
    hip = HipBackend.default()
    plan, ins = graphs.conv3x3_bias_relu()
    g = hip.graph(plan, False)
    with HipInferenceSession(g) as s:
        s.set_input(ins[0])
        s.run()
        s.time(20)
        ms = s.time(steps)
    g.release()
    us = ms / steps * 1e3
    fl = graphs.conv3x3_flops()
    return dict(us=us, tflops=fl / (us * 1e-6) / 1e12, frac_fp32_peak=fl / (us * 1e-6) / 1e12 / PEAK_FP32_TFLOPS)


NETWORKS = {
    "mobilenetv3": ("mobilenetv3_small", "MobileNetV3-small block stack, 1x3x640x640, fp16 storage", 1, True),
    "detector": ("dbnet", "DBNet-style detector (MobileNetV3-small + FPN + ConvT head), 1x3x960x960, fp16 storage",
                 1, True),
    "detector_fp32": ("dbnet", "DBNet-style detector (MobileNetV3-small + FPN + ConvT head), 1x3x960x960, fp32 "
                      "storage", 1, False),
    "recognizer": ("svtr", "SVTR-style recognizer, 32x3x48x320, fp16 storage", 32, True),
    "recognizer_bf16": ("svtr", "SVTR-style recognizer, 32x3x48x320, bf16 storage", 32, "bf16"),
}


def bench_network(key: str, steps: int, replay: bool = True):
    """ms per image of a whole network plan, HIP-graph replay (or node-by-node launches with
    replay=False), inputs resident (and with staging), plus the per-kernel-class roofline from a
    per-dispatch event profile."""
    from simdonnx_amd import graphs
    from simdonnx_amd.backend import HipBackend, HipInferenceSession
    fn, desc, images, half = NETWORKS[key]
    hip = HipBackend.default()
    plan, ins = getattr(graphs, fn)()
    g = hip.graph(plan, half)
    with HipInferenceSession(g) as s:
        s.set_input(ins[0])
        s.set_replay(replay)
        replayed = s.replaying
        s.run()
        s.time(200)  # ~0.1 s: the clock ramps up under sustained load
        ms = s.time(steps) / steps
        ms_e2e = s.time(max(steps // 2, 1), staging=True) / max(steps // 2, 1)
        prof = s.profile(5)
    ndisp = len(g.dispatches)
    g.release()
    per_node = {}
    for name, node, t in prof:
        per_node.setdefault(node, [name, 0.0])[1] += t
    classes = {}
    tot_fl = tot_by = 0
    peak = PEAK_FP16_TFLOPS if half else PEAK_FP32_TFLOPS  # the bf16 dense peak equals fp16's
    for node, (name, t) in per_node.items():
        fl, by = graphs.node_cost(plan, plan.nodes[node], 2 if half else 4)
        tot_fl += fl
        tot_by += by
        c = classes.setdefault(name, dict(ms=0.0, n=0, flops=0, bytes=0))
        c["ms"] += t
        c["n"] += 1
        c["flops"] += fl
        c["bytes"] += by
    out = []
    for name, c in sorted(classes.items(), key=lambda kv: -kv[1]["ms"]):
        gbs = c["bytes"] / (c["ms"] * 1e-3) / 1e9
        tfl = c["flops"] / (c["ms"] * 1e-3) / 1e12
        bound = "mfma" if name in ("conv", "gemm", "gemm_ln") and c["flops"] / max(c["bytes"], 1) > peak / 8 else "hbm"
        frac = tfl / peak if bound == "mfma" else gbs / PEAK_HBM_GBS
        out.append(dict(kernel=name, nodes=c["n"], ms=round(c["ms"], 4), gb_s=round(gbs, 1), tflop_s=round(tfl, 2),
                        bound=bound, frac=round(frac, 4)))
    return dict(workload=desc, ms_per_image=round(ms / images, 4), images_per_s=round(images / (ms * 1e-3), 1),
                ms_per_batch=round(ms, 4), ms_per_image_with_staging=round(ms_e2e / images, 4), dispatches=ndisp,
                replay=replayed,
                gflop=round(tot_fl / 1e9, 3), algorithmic_mb=round(tot_by / 1e6, 1),
                kernel_sum_ms=round(sum(t for _, _, t in prof), 4), kernels=out[:8])


def bench_copy(steps: int):
    """Plain copy of 128 Mi fp16 elements through the backend (the traffic-counter calibration kernel)."""
    from simdonnx_amd.backend import HipBackend, HipInferenceSession
    from simdonnx_amd.plan import PlanBuilder
    import numpy as np
    pb = PlanBuilder()
    n = 128 << 20
    x = pb.input((n,), None, "x")
    y = pb.unary("Copy", x, name="copy")
    plan = pb.build(y)
    hip = HipBackend.default()
    g = hip.graph(plan, True)
    with HipInferenceSession(g) as s:
        s.set_input(np.zeros(n, np.float32))
        s.run()
        ms = s.time(steps) / steps
    g.release()
    return dict(bytes_per_launch=2 * n * 2, ms=ms, gb_s=2 * n * 2 / (ms * 1e-3) / 1e9)


def bench_recognizer_ctc(steps: int, replay: bool = True):
    """The recognizer with the fused CTC head (HipCtcProjection) in place of head Gemm + softmax:
    the features plan replayed (HIP events), then the head on the device features, host-timed per
    call including its launch, the copy home of the indices and probabilities and the wait."""
    from simdonnx_amd import graphs
    from simdonnx_amd.backend import HipBackend, HipCtcProjection, HipInferenceSession
    hip = HipBackend.default()
    plan, ins, (hw, hb) = graphs.svtr(head="features")
    ctc = HipCtcProjection(hip, hw, hb, hw.shape[0], hw.shape[1])
    g = hip.graph(plan, True)
    rows = plan.values[plan.output].count // hw.shape[0]
    with HipInferenceSession(g) as s:
        s.set_input(ins[0])
        s.set_replay(replay)
        s.run()
        s.time(200)
        ms_feat = s.time(steps) / steps
        for _ in range(20):
            ctc.argmax(s, plan.output, 32, rows // 32)
        t0 = time.perf_counter()
        for _ in range(steps):
            ctc.argmax(s, plan.output, 32, rows // 32)
        ms_head = (time.perf_counter() - t0) * 1e3 / steps
    g.release()
    ctc.close()
    return dict(workload="SVTR-style recognizer, 32x3x48x320, fused CTC head (argmax + probability per row)",
                ms_features=round(ms_feat, 4), ms_ctc_head_host=round(ms_head, 4),
                ms_per_batch=round(ms_feat + ms_head, 4), rows=rows, classes=int(hw.shape[1]))


def bench_image_session(steps: int):
    """HipImageSession on a 1920x1080 Bgr24 frame through a small image-to-image model (3x3 conv 3->8
    + relu, 3x3 conv 8->3 + sigmoid, fp16): host-timed frames (upload, pixels -> NHWC, the model,
    NHWC -> pixels, download, wait), and the device time of the two pixel kernels from a profile of
    the same dispatches against the HBM roofline (bytes: the image once + the 3-channel fp16 tensor)."""
    import numpy as np
    from simdonnx_amd import synth
    from simdonnx_amd.backend import HipBackend, HipImageSession
    from simdonnx_amd.plan import NHWC, PlanBuilder
    hip = HipBackend.default()
    unit = np.tile(np.arange(256, dtype=np.float32) / np.float32(255), 3)
    width, height = 1920, 1080
    s = HipImageSession(hip, unit, pad_multiple=32)
    th, tw = s.tensor_size(width, height)
    pb = PlanBuilder()
    x = pb.input((1, 3, th, tw), NHWC, "image")
    y = pb.conv(x, synth.normal(61, 1, (8, 3, 3, 3), 0.3), synth.uniform(61, 2, (8,), -0.1, 0.1), act="relu", name="c1")
    y = pb.conv(y, synth.normal(61, 3, (3, 8, 3, 3), 0.2), synth.uniform(61, 4, (3,), 0.2, 0.4), act="sigmoid", name="c2")
    g = hip.graph(pb.build(y), True)
    src = np.random.default_rng(3).integers(0, 256, (height, width * 3), dtype=np.uint8)
    dst = np.empty_like(src)
    for _ in range(5):
        s.run(g, src, width, height, "Bgr24", dst)
    t0 = time.perf_counter()
    for _ in range(steps):
        s.run(g, src, width, height, "Bgr24", dst)
    ms = (time.perf_counter() - t0) * 1e3 / steps
    s.close()
    g.release()
    return dict(workload=f"image session {width}x{height} Bgr24 -> {th}x{tw} tensor, 2-conv fp16 model, pixels in/out",
                ms_per_frame=round(ms, 4), frames_per_s=round(1e3 / ms, 1), image_mb=round(width * height * 3 / 1e6, 2))


def bench_unit_runner(steps: int):
    """16 OCR-line units of 8 widths (a text line [1, 3, 32, w] -> conv 3x3 s2 + GELU -> 1x1 conv), fp16:
    one HipUnitRunner run (one wave over 4 streams: upload, dispatches, download per unit, then one
    wait) against the same units as 16 sessions run one after another. Host-timed per batch."""
    import numpy as np
    from simdonnx_amd import synth
    from simdonnx_amd.backend import HipBackend, HipInferenceSession, HipUnitRunner
    from simdonnx_amd.plan import NHWC, PlanBuilder
    hip = HipBackend.default()
    widths = [64, 96, 128, 160, 192, 256, 320, 480] * 2
    graphs, xs = [], []
    for i, w in enumerate(widths):
        pb = PlanBuilder()
        x = pb.input((1, 3, 32, w), NHWC, "line")
        y = pb.conv(x, synth.he_normal(81, 1, (32, 3, 3, 3)), synth.uniform(81, 2, (32,), -0.1, 0.1), stride=2, pad=1,
                    act="gelu", name="c1")
        y = pb.conv(y, synth.he_normal(81, 3, (16, 32, 1, 1)), None, name="c2")
        graphs.append(hip.graph(pb.build(y), True))
        xs.append(synth.normal(82, i, (1, 32, w, 3), 1.0))
    r = HipUnitRunner(hip, streams=4)
    for g in graphs:
        r.add(g)
    for k, x in enumerate(xs):
        r.input(k)[:] = x.reshape(-1)

    def run_runner():
        r.submit()
        r.wait()

    sessions = [HipInferenceSession(g) for g in graphs]
    for s, x in zip(sessions, xs):
        s.set_input(x)

    def run_sessions():
        for s in sessions:
            s.run()

    out = {}
    for name, fn in (("runner_4_streams", run_runner), ("sequential_sessions", run_sessions)):
        for _ in range(5):
            fn()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        out[f"ms_{name}"] = round((time.perf_counter() - t0) * 1e3 / steps, 4)
    for s in sessions:
        s.close()
    r.close()
    for g in graphs:
        g.release()
    return dict(workload="16 OCR-line units (8 widths 64..480), conv3x3 s2 + GELU -> 1x1, fp16, host-timed per batch",
                **out)


def _ops_cases():
    """One-node plans of the rest of the ExecOp surface at the sizes the detector / recognizer shapes
    give them (fp16 storage): (label, plan, inputs, algorithmic bytes, flops). Bytes count each
    tensor read or written once at 2 bytes per element."""
    import numpy as np
    from simdonnx_amd import synth
    from simdonnx_amd.plan import NHWC, PlanBuilder
    cases = []

    def img(shape):
        return synth.normal(77, 1, shape, 1.0)

    def add_case(label, build, shapes, out_elems, flops=0):
        pb = PlanBuilder()
        y = build(pb)
        ins = [img(sh) for sh in shapes]
        cases.append((label, pb.build(y), ins, 2 * (sum(int(np.prod(sh)) for sh in shapes) + out_elems), flops))

    add_case("bilinear x2 + addend, 1x240x240x24 -> 480x480",
             lambda pb: pb.resize_bilinear(pb.input((1, 24, 240, 240), NHWC, "x"), 2, pb.input((1, 24, 480, 480), NHWC, "a"),
                                           relu=True, name="bil"),
             [(1, 240, 240, 24), (1, 480, 480, 24)], 480 * 480 * 24)
    add_case("pad reflect 3, 1x480x480x32",
             lambda pb: pb.pad(pb.input((1, 32, 480, 480), NHWC, "x"), (0, 0, 3, 3, 0, 0, 3, 3), 1, name="pad"),
             [(1, 480, 480, 32)], 486 * 486 * 32)
    add_case("transpose NHWC->NCHW, 1x480x480x24",
             lambda pb: pb.transpose(pb.input((1, 480, 480, 24), None, "x"), (0, 3, 1, 2), name="tr"),
             [(1, 480, 480, 24)], 480 * 480 * 24)
    add_case("slice k of packed qkv, 32x80x576 -> 32x80x192",
             lambda pb: pb.slice(pb.input((32, 80, 576), None, "x"), (192,), (384,), (2,), (1,), name="sl"),
             [(32, 80, 576)], 32 * 80 * 192)
    add_case("tanh, 8M elements",
             lambda pb: pb.scalar_act("Tanh", pb.input((8 << 20,), None, "x"), 1.0, 1.0, name="tanh"),
             [(8 << 20,)], 8 << 20)
    add_case("depth-to-space b2 DCR, 1x240x240x96 -> 480x480x24",
             lambda pb: pb.depth_to_space(pb.input((1, 96, 240, 240), NHWC, "x"), 2, False, name="d2s"),
             [(1, 240, 240, 96)], 480 * 480 * 24)
    add_case("avgpool 3x3 s2, 1x240x240x64",
             lambda pb: pb.avg_pool(pb.input((1, 64, 240, 240), NHWC, "x"), (3, 3), (2, 2), (1, 1, 1, 1), name="avg"),
             [(1, 240, 240, 64)], 120 * 120 * 64)
    add_case("global avgpool, 1x240x240x96",
             lambda pb: pb.global_avg_pool(pb.input((1, 96, 240, 240), NHWC, "x"), name="gap"),
             [(1, 240, 240, 96)], 96)
    add_case("safediv, 1x480x480x24",
             lambda pb: pb.safe_div(pb.input((1, 480, 480, 24), None, "a"), pb.input((1, 480, 480, 24), None, "b"),
                                    1e-3, -4.0, 4.0, name="sd"),
             [(1, 480, 480, 24), (1, 480, 480, 24)], 480 * 480 * 24)
    add_case("channel shift 5 groups along W, 1x120x120x96",
             lambda pb: pb.channel_shift(pb.input((1, 96, 120, 120), NHWC, "x"), 3, (16, 32, 48, 64, 80),
                                         (-2, -1, 0, 1, 2), name="sh"),
             [(1, 120, 120, 96)], 120 * 120 * 96)
    wh = synth.normal(78, 3, (1, 24), 0.2)
    add_case("uphead x2 + skip -> 1 ch sigmoid, 1x240x240x24 -> 480x480",
             lambda pb: pb.up_head(pb.input((1, 24, 240, 240), NHWC, "x"), pb.input((1, 24, 480, 480), NHWC, "s"), wh,
                                   np.zeros(1, np.float32), 2, resize_relu=True, skip_relu=True, act="sigmoid",
                                   name="uh"),
             [(1, 240, 240, 24), (1, 480, 480, 24)], 480 * 480)
    add_case("matmul 192 x [80,32]x[32,80]",
             lambda pb: pb.matmul(pb.input((192, 80, 32), None, "a"), pb.input((192, 32, 80), None, "b"), name="mm"),
             [(192, 80, 32), (192, 32, 80)], 192 * 80 * 80, 2 * 192 * 80 * 32 * 80)
    return cases


def bench_ops(steps: int):
    """Per-launch time of each kernel of the rest of the ExecOp surface, against the HBM roofline."""
    from simdonnx_amd.backend import HipBackend, HipInferenceSession
    hip = HipBackend.default()
    out = []
    for label, plan, ins, nbytes, flops in _ops_cases():
        g = hip.graph(plan, True)
        kern = [d[0] for d in g.dispatches]
        with HipInferenceSession(g) as s:
            for i, x in enumerate(ins):
                s.set_input(x, i)
            s.run()
            s.time(20)
            ms = s.time(steps) / steps
        g.release()
        gbs = nbytes / (ms * 1e-3) / 1e9
        rec = dict(op=label, kernels=kern, us=round(ms * 1e3, 2), algorithmic_mb=round(nbytes / 1e6, 2),
                   gb_s=round(gbs, 1), bound="hbm", frac=round(gbs / PEAK_HBM_GBS, 4))
        if flops:
            rec["tflop_s"] = round(flops / (ms * 1e-3) / 1e12, 2)
        out.append(rec)
    return out


def _hbm_cases():
    """The convnets' bandwidth-bound kernels at sizes past the L2 (fp16 storage): (label, plan, inputs,
    {kernel: algorithmic bytes per launch}). Bytes count each tensor read or written once."""
    from simdonnx_amd import synth
    from simdonnx_amd.plan import NHWC, PlanBuilder
    cases = []

    def img(seed, shape):
        return synth.normal(79, seed, shape, 1.0)

    def f16b(*shape):
        n = 1
        for d in shape:
            n *= d
        return 2 * n

    pb = PlanBuilder()
    x = pb.input((4, 240, 80, 80), NHWC, "x")
    y = pb.conv(x, synth.uniform(79, 1, (240, 1, 5, 5), -0.3, 0.3), synth.uniform(79, 2, (240,), -0.1, 0.1), pad=2,
                group=240, act="hardswish", name="dw")
    cases.append(("depthwise 5x5 s1 + hardswish, 4x80x80x240", pb.build(y), [img(1, (4, 80, 80, 240))],
                  {"sox_dwt_f16_k5s1": 2 * f16b(4, 80, 80, 240) + f16b(25, 240) + 4 * 240}))
    pb = PlanBuilder()
    x = pb.input((4, 64, 320, 320), NHWC, "x")
    y = pb.conv(x, synth.uniform(79, 3, (64, 1, 3, 3), -0.3, 0.3), synth.uniform(79, 4, (64,), -0.1, 0.1), stride=2,
                pad=1, group=64, act="relu", name="dw")
    cases.append(("depthwise 3x3 s2 + relu, 4x320x320x64 -> 160x160", pb.build(y), [img(2, (4, 320, 320, 64))],
                  {"sox_dwt_f16_k3s2": f16b(4, 320, 320, 64) + f16b(4, 160, 160, 64) + f16b(9, 64) + 4 * 64}))
    # the largest MobileNetV3-small SE block: 20x20x576, r = 144, projection to 96 channels (folded)
    c, r, wn, tiles = 576, 144, 96, 9
    pb = PlanBuilder()
    x = pb.input((1, c, 20, 20), NHWC, "x")
    d = pb.conv(x, synth.uniform(79, 5, (c, 1, 5, 5), -0.3, 0.3), synth.uniform(79, 6, (c,), -0.1, 0.1), pad=2,
                group=c, act="hardswish", name="dw")
    gate = pb.channel_gate(d, synth.uniform(79, 7, (r, c, 1, 1), -0.1, 0.1), synth.uniform(79, 8, (r,), -0.1, 0.1),
                           synth.uniform(79, 9, (c, r, 1, 1), -0.1, 0.1), synth.uniform(79, 10, (c,), -0.1, 0.1),
                           act1="relu", hard=True, alpha=1.0 / 6.0, beta=0.5, name="se")
    y = pb.conv(pb.mul(d, gate, name="scale"), synth.uniform(79, 11, (wn, c, 1, 1), -0.1, 0.1), None, name="proj")
    groups = (c + 63) // 64
    cases.append(("SE gate 1x20x20x576, r 144, folded into a 576 -> 96 projection", pb.build(y),
                  [img(3, (1, 20, 20, c))],
                  {"sox_se_fc1": 4 * (tiles * c + r * c + groups * r),
                   "sox_se_fc2_f16": 4 * (groups * r + c * r + r + c) + 2 * f16b(wn, c)}))
    pb = PlanBuilder()
    y = pb.resize_nearest(pb.input((4, 96, 160, 160), NHWC, "x"), 2, name="up")
    cases.append(("nearest x2, 4x160x160x96 -> 320x320", pb.build(y), [img(4, (4, 160, 160, 96))],
                  {"sox_nearest_f16_v": f16b(4, 160, 160, 96) + f16b(4, 320, 320, 96)}))
    pb = PlanBuilder()
    y = pb.add(pb.input((4, 96, 160, 160), NHWC, "a"), pb.input((4, 96, 160, 160), NHWC, "b"), act="relu", name="add")
    cases.append(("add + relu, 4x160x160x96", pb.build(y), [img(5, (4, 160, 160, 96)), img(6, (4, 160, 160, 96))],
                  {"sox_ew_f16": 3 * f16b(4, 160, 160, 96)}))
    return cases


def bench_hbm_kernels(steps: int):
    """Per-launch time of the convnets' bandwidth-bound kernels (HIP events around each dispatch, the
    minimum over `steps` runs), with achieved GB/s from the algorithmic bytes and, where the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary covers the kernel, from the counted HBM bytes."""
    from simdonnx_amd.backend import HipBackend, HipInferenceSession
    hip = HipBackend.default()
    path = os.path.join(ROOT, "profiles", "traffic_hbm_kernels.json")
    counted = json.load(open(path))["kernels"] if os.path.exists(path) else {}
    out = []
    for label, plan, ins, alg in _hbm_cases():
        g = hip.graph(plan, True)
        kernels = g.kernels
        wgs = [grid[0] * grid[1] * grid[2] for _, grid, _ in g.dispatches]
        with HipInferenceSession(g) as s:
            for i, x in enumerate(ins):
                s.set_input(x, i)
            s.run()
            prof = s.profile(steps)
        g.release()
        for (name, node, ms), k, nwg in zip(prof, kernels, wgs):
            if k not in alg:
                continue
            rec = dict(op=label, kernel=k, us=round(ms * 1e3, 2), algorithmic_mb=round(alg[k] / 1e6, 3),
                       gb_s=round(alg[k] / (ms * 1e-3) / 1e9, 1))
            rec["frac"] = round(rec["gb_s"] / PEAK_HBM_GBS, 4)
            c = counted.get(k)
            if c and c.get("workgroups") == nwg:  # counted on this kernel at this launch shape
                rec["traffic_mb"] = round(c["bytes_per_launch"] / 1e6, 3)
                rec["traffic_gb_s"] = round(c["bytes_per_launch"] / (ms * 1e-3) / 1e9, 1)
                rec["traffic_frac"] = round(rec["traffic_gb_s"] / PEAK_HBM_GBS, 4)
            out.append(rec)
        if not any(k in alg for k in kernels):
            raise RuntimeError(f"{label}: none of {sorted(alg)} in the dispatches {kernels}")
    return out


def cpu_info():
    """The host the CPU baseline ran on: model, logical CPUs used, physical cores, oracle ISA tier."""
    import oracle as O
    model, cores = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            phys = core = None
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model == "unknown":
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
            if phys is not None:
                cores.add((phys, core))
    except OSError:
        pass
    tier = "avx512" if O.tier_available(O.TIER_AVX512) else "avx2" if O.tier_available(O.TIER_AVX2) else "scalar"
    return dict(model=model, logical_cpus_used=cpu_threads(), physical_cores=len(cores) or None, isa_tier=tier)


def _median_ms(fn, runs=20, warmups=3):
    """Median wall time of `runs` calls after `warmups` untimed ones (page-in, thread pool, caches)."""
    for _ in range(warmups):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return round(statistics.median(ts) * 1e3, 3)


def cpu_configs():
    """The oracle (the reference's CPU kernels restated) on the other benchmark configurations, all host
    threads, median ms of 20 runs after 3 warm-ups: config 1 at full size, configs 3 and 4 per image at
    full size, config 5 on its full batch of 32 images (ms per image)."""
    import oracle as O
    from oracle.interp import run_plan
    from simdonnx_amd import graphs
    O.set_threads(cpu_threads())
    out = {"method": "median of 20 runs after 3 warm-ups, all host threads"}
    plan, ins = graphs.conv3x3_bias_relu()
    out["conv3x3_bias_relu_fp32_ms"] = _median_ms(lambda: run_plan(plan, ins))
    plan, ins = graphs.mobilenetv3_small()
    out["mobilenetv3_ms_per_image"] = _median_ms(lambda: run_plan(plan, ins))
    plan, ins = graphs.dbnet()
    out["detector_ms_per_image"] = _median_ms(lambda: run_plan(plan, ins))
    plan, ins = graphs.svtr()
    batch = plan.values[plan.inputs[0]].shape[0]
    out["recognizer_ms_per_image"] = round(_median_ms(lambda: run_plan(plan, ins)) / batch, 3)
    out["recognizer_batch"] = batch
    return out


def cpu_baseline():
    """The oracle Gemm + GELU on the full workload (M = 8192), all host threads; and on one thread over
    the first 1024 rows (the reference bench's micro mode, Program.cs:12). Each: median of 20 runs
    after 3 warm-ups."""
    import oracle as O
    from simdonnx_amd import graphs
    plan, ins = graphs.matmul_bias_gelu()
    node = plan.nodes[0]
    a = ins[0].reshape(-1, ins[0].shape[-1])
    w = plan.values[node.ins[1]].data
    b = plan.values[node.p.bias].data
    threads = cpu_threads()
    O.set_threads(threads)
    med = _median_ms(lambda: O.gemm(a, w, b, act="gelu")) * 1e-3
    info = cpu_info()
    O.set_threads(1)
    rows = 1024
    ms1 = _median_ms(lambda: O.gemm(a[:rows], w, b, act="gelu"))
    O.set_threads(threads)
    flops1 = 2 * rows * a.shape[1] * w.shape[1]
    return dict(value=graphs.matmul_flops() / med / 1e12, unit="TFLOP/s", cores=threads, kind="port",
                sample=f"full workload M=8192 K=768 N=3072 + GELU, median of 20 runs after 3 warm-ups, "
                       f"{med*1e3:.1f} ms, {info['isa_tier']} tier (C++ restatement of Nhwc.Gemm512 / Epilogue512)",
                one_thread={"value": round(flops1 / (ms1 * 1e-3) / 1e12, 4), "unit": "TFLOP/s", "cores": 1,
                            "sample": f"first {rows} rows (M={rows}, K=768, N=3072) + GELU, median of 20 runs "
                                      f"after 3 warm-ups, {ms1:.1f} ms"},
                cpu=info)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=2000)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-vendor", action="store_true",
                    help="skip the vendor BLAS leg (its child process; for profiler runs, whose preloaded library "
                         "may hold the GPU before the child would start)")
    ap.add_argument("--no-replay", action="store_true",
                    help="launch network dispatches one by one instead of replaying a HIP graph (profiler runs)")
    ap.add_argument("--only", choices=["gemm", "gemm_bf16", "mfma_peak", "lds_peak", "vendor_gemm", "conv_large", "conv_large_bf16", "conv", "detector", "detector_fp32", "recognizer",
                                       "recognizer_bf16", "mobilenetv3", "copy", "ops", "hbm_kernels",
                                       "recognizer_ctc", "image", "runner"],
                    help="run one workload only (profiling runs); prints its own JSON line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this backend is single-device (the reference's GPU backends are; "
              "VkDevice.cs:128). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.only:
        fn = {"gemm": lambda: bench_gemm(args.steps, args.warmup), "conv": lambda: bench_conv(args.steps),
              "gemm_bf16": lambda: bench_gemm(args.steps, args.warmup, "bf16"),
              "mfma_peak": lambda: bench_mfma_peak(), "lds_peak": lambda: bench_lds_peak(),
              "vendor_gemm": lambda: bench_vendor_gemm(),
              "conv_large": lambda: bench_conv_large(args.steps),
              "conv_large_bf16": lambda: bench_conv_large(args.steps, "bf16"),
              "copy": lambda: bench_copy(args.steps),
              "ops": lambda: {"ops": bench_ops(args.steps)},
              "hbm_kernels": lambda: {"hbm_kernels": bench_hbm_kernels(args.steps)},
              "recognizer_ctc": lambda: bench_recognizer_ctc(args.steps, not args.no_replay),
              "image": lambda: bench_image_session(args.steps),
              "runner": lambda: bench_unit_runner(args.steps)}.get(args.only) or (lambda: bench_network(args.only, args.steps, not args.no_replay))
        r = fn()
        print(json.dumps({"only": args.only, **{k: v for k, v in r.items() if k != "kernel_ms"}}), flush=True)
        return
    # the vendor BLAS leg first, in a child process started before this process touches the GPU: torch
    # carries its own HIP runtime, which does not see the device in a process where this backend's runtime
    # is already initialised
    try:
        if args.no_vendor:
            raise RuntimeError("skipped (--no-vendor)")
        import subprocess
        cr = subprocess.run([sys.executable, os.path.abspath(__file__), "--only", "vendor_gemm"], capture_output=True,
                            text=True, timeout=300)
        lines = [ln for ln in cr.stdout.splitlines() if ln.startswith("{")]
        if cr.returncode != 0 or not lines:
            raise RuntimeError(f"vendor_gemm leg exited {cr.returncode}: {cr.stderr[-400:]}")
        vendor = {k: v for k, v in json.loads(lines[-1]).items() if k != "only"}
        log(f"vendor gemm (fp16 linear+bias+gelu): {vendor['f16']['linear_bias_gelu']['tflop_s']} TFLOP/s")
    except Exception as e:
        vendor = {"error": repr(e)}
    r = bench_gemm(args.steps, args.warmup)
    per_s = r["per_launch_ms"] * 1e-3
    tflops = r["flops"] / per_s / 1e12
    log(f"gemm: {r['per_launch_ms']*1e3:.1f} us/launch, {tflops:.1f} TFLOP/s, dispatches {r['dispatches']}")
    out = {
        "metric": "fused MatMul+bias+GELU TFLOP/s (fp16 MFMA, fp32 accum); detector ms/image",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_run": r["warmup_run"],
        "ms_per_step": round(r["per_launch_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (SplitMix64 counter generator, seeded)",
        "config": {"workload": "matmul_bias_gelu: A[16,512,768] x W[768,3072] + b[3072] -> GELU, fp16 storage",
                   "global_batch": 16, "seq_len": 512, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_FP16_TFLOPS, 4),
                     "kernel": r["kernels"][0],
                     "traffic": traffic_from_profiles("matmul_bias_gelu", r["kernels"][0])},
    }
    try:
        rb = bench_gemm(max(args.steps // 4, 1), min(args.warmup, 500), "bf16")
        tb = rb["flops"] / (rb["per_launch_ms"] * 1e-3) / 1e12
        out["gemm_bf16"] = {"workload": "matmul_bias_gelu with bf16 storage (v_mfma_f32_32x32x16_bf16, fp32 accum)",
                            "us_per_launch": round(rb["per_launch_ms"] * 1e3, 2), "tflop_s": round(tb, 2),
                            "frac_of_peak": round(tb / PEAK_FP16_TFLOPS, 4), "dispatches": rb["dispatches"]}
        log(f"gemm bf16: {rb['per_launch_ms']*1e3:.1f} us/launch, {tb:.1f} TFLOP/s")
    except Exception as e:
        out["gemm_bf16"] = {"error": repr(e)}
    for key in ("detector", "detector_fp32", "recognizer", "recognizer_bf16", "mobilenetv3"):
        try:
            out[key] = bench_network(key, 200, not args.no_replay)
            log(f"{key}: {out[key]['ms_per_image']} ms/image")
        except Exception as e:  # reported, never hidden
            out[key] = {"error": repr(e)}
    try:
        out["mfma_peak_probe"] = bench_mfma_peak()
        log(f"mfma probe: {out['mfma_peak_probe']['tflop_s']} TFLOP/s")
    except Exception as e:
        out["mfma_peak_probe"] = {"error": repr(e)}
    try:
        out["lds_peak_probe"] = bench_lds_peak()
    except Exception as e:
        out["lds_peak_probe"] = {"error": repr(e)}
    out["vendor_gemm"] = vendor
    try:
        out["conv_large_f16"] = bench_conv_large(50)
        log(f"large conv: {out['conv_large_f16']['tflop_s']} TFLOP/s")
    except Exception as e:
        out["conv_large_f16"] = {"error": repr(e)}
    try:
        out["conv_large_bf16"] = bench_conv_large(50, "bf16")
        log(f"large conv bf16: {out['conv_large_bf16']['tflop_s']} TFLOP/s")
    except Exception as e:
        out["conv_large_bf16"] = {"error": repr(e)}
    try:
        out["conv3x3_bias_relu_fp32"] = bench_conv(200)
    except Exception as e:
        out["conv3x3_bias_relu_fp32"] = {"error": repr(e)}
    try:
        out["recognizer_ctc"] = bench_recognizer_ctc(200, not args.no_replay)
    except Exception as e:
        out["recognizer_ctc"] = {"error": repr(e)}
    try:
        out["image_session"] = bench_image_session(100)
    except Exception as e:
        out["image_session"] = {"error": repr(e)}
    try:
        out["unit_runner"] = bench_unit_runner(100)
    except Exception as e:
        out["unit_runner"] = {"error": repr(e)}
    try:
        out["ops"] = bench_ops(200)
    except Exception as e:
        out["ops"] = {"error": repr(e)}
    try:
        out["hbm_kernels"] = bench_hbm_kernels(50)
    except Exception as e:
        out["hbm_kernels"] = {"error": repr(e)}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
        try:
            out["cpu_baseline"]["configs"] = cpu_configs()
        except Exception as e:
            out["cpu_baseline"]["configs"] = {"error": repr(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
