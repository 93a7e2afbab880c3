"""Benchmark of the MI355X quantized linear layer on BASELINE.json's headline configs.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20]

One step = one decode GEMV y[1, 11008] = x[1, 4096] . W^T over a Q4_0 weight
W[11008, 4096] (the Llama-7B gate/up projection; BASELINE's "4096x11008 b=1").
The weight is uploaded as >= 1 GiB of distinct copies and the steps rotate over
them, so every step streams its 25.4 MB from HBM rather than from the 256 MB
Infinity Cache.  Inputs are resident in HBM before timing starts.

`value` = algorithmic bytes per step (W bytes + x + y) x steps / wall time of the
timed region (HIP events on the launch stream, device synchronised on both sides).
The timed launches are captured once in a HIP graph and replayed, so host launch
cost is excluded; `roofline.achieved` divides the same bytes by the average launch
duration over the timed region (region time / launches, which includes the
graph's back-to-back dispatch gap).  The Q8_0 prefill GEMM
(W[11008, 4096], M = 512, bf16 X) is measured the same way and reported under
"gemm".  `cpu_baseline` times the reference's per-token CPU path (f32 GEMV over
weights dequantized at load, one thread, restated in oracle/) on the host cores.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "openmini-v1_amd"))

METRIC = "Q4_0 GEMV HBM GB/s (% of peak) at 4096x11008 b=1; Q8_0 GEMM TFLOP/s M=512"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
Q4_0, Q4_1, Q8_0, Q4_K, Q5_K, Q6_K = 2, 3, 7, 12, 13, 14
TYPE_NAME = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k", Q4_1: "q4_1", Q5_K: "q5_k"}
MALL_DEFEAT_BYTES = 1 << 30
SUSTAINED_LAUNCHES = 500  # back-to-back launches of the sustained-load figures
# the Llama-70B-style q / gate / down projections (N, K, seed),
# weights N(0, 0.015)
SHAPES_70B = ((8192, 8192, 0x5EED0064), (28672, 8192, 0x5EED0065), (8192, 28672, 0x5EED0066))
SIGMA_70B = 0.015


def sha256(a: np.ndarray) -> str:
    """SHA-256 of a synthetic input buffer's bytes, recorded so runs can be compared
    input for input."""
    import hashlib
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


EAGER = False  # --eager: launch directly instead of from a graph (counter-collection runs)


def time_steps(launch, steps: int, stream, hipr) -> float:
    """Wall time (ms) of `steps` back-to-back launches replayed from one HIP graph
    (captured once, so host launch cost is not what is measured), between events
    on `stream`, with the device synchronised on both sides."""
    if EAGER:
        hipr.hip().hipDeviceSynchronize()
        e0, e1 = hipr.Event(), hipr.Event()
        e0.record(stream)
        for i in range(steps):
            launch(i)
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_ms(e1)
    graph = hipr.Graph(stream, lambda s: [launch(i) for i in range(steps)])
    graph.launch(stream)  # untimed replay
    hipr.hip().hipDeviceSynchronize()
    e0, e1 = hipr.Event(), hipr.Event()
    e0.record(stream)
    graph.launch(stream)
    e1.record(stream)
    e1.synchronize()
    hipr.hip().hipDeviceSynchronize()
    return e0.elapsed_ms(e1)


_BLOCKS = {}


def weight_blocks(qtype, N, K, seed, sigma=0.02):
    """Synthetic GGUF blocks of W[N, K] ~ N(0, sigma), generated once per process for
    the legs that share a weight (the 70B shapes at several batch sizes)."""
    from openmini_qmm import synth
    key = (qtype, N, K, seed, sigma)
    if key not in _BLOCKS:
        _BLOCKS[key] = (synth.kquant_blocks(qtype, N, K, seed=seed) if qtype in (Q4_K, Q5_K, Q6_K)
                        else synth.weight_blocks(qtype, N, K, seed=seed, sigma=sigma))
    return _BLOCKS[key]


def bench_gemv(qmm, hipr, stream, steps, warmup, N, K, qtype=Q4_0, batch=1, seed=0x5EED0001, sigma=0.02,
               sustained_steps=0):
    from openmini_qmm import synth
    blocks = weight_blocks(qtype, N, K, seed, sigma)
    wbytes = blocks.size  # GGUF bytes: the algorithmic weight bytes
    copies = max(2, -(-MALL_DEFEAT_BYTES // wbytes))
    log(f"gemv type={qtype} N={N} K={K} B={batch}: {copies} weight copies x {wbytes} B")
    ws = [qmm.QuantizedWeight(qtype, blocks, N, K) for _ in range(copies)]
    x = synth.normal(seed + 0x8000, (batch, K), 1.0)
    dx = qmm.DeviceBuffer.from_numpy(x)
    dy = qmm.DeviceBuffer(batch * N * 4)
    dy_check = qmm.DeviceBuffer(batch * N * 4)
    sh = stream.handle

    def launch(i):
        ws[i % copies].gemv(dx, dy, batch, sh)

    for i in range(warmup):
        launch(i)
    stream.synchronize()
    # every copy computes the same y (bitwise: fixed reduction order)
    ws[0].gemv(dx, dy_check, batch, sh)
    ws[-1].gemv(dx, dy, batch, sh)
    stream.synchronize()
    if not np.array_equal(dy.download(np.float32, (batch, N)), dy_check.download(np.float32, (batch, N))):
        raise RuntimeError("GEMV copies disagree")
    total_ms = time_steps(launch, steps, sh, hipr)
    per_launch_ms = total_ms / steps
    alg_bytes = wbytes + batch * K * 4 + batch * N * 4
    sustained = None
    if sustained_steps:
        # the same launches over a longer run: the part's power management settles
        # within milliseconds of full-rate streaming, which a short run does not reach
        ms_s = time_steps(launch, sustained_steps, sh, hipr) / sustained_steps
        sustained = {"launches": sustained_steps, "kernel_us": round(ms_s * 1e3, 3),
                     "gbs": round(alg_bytes / (ms_s * 1e-3) / 1e9, 2),
                     "frac": round(alg_bytes / (ms_s * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "run_ms": round(ms_s * sustained_steps, 3)}
    res = {
        "N": N, "K": K, "batch": batch, "weight_bytes": wbytes, "alg_bytes_per_step": alg_bytes,
        # the timed region's launches use copies 0 .. min(steps, copies) - 1
        "weight_copies": copies, "rotated_bytes": min(steps, copies) * wbytes,
        "ms_per_step": total_ms / steps, "kernel_ms": per_launch_ms,
        "gbs_wall": alg_bytes * steps / (total_ms * 1e-3) / 1e9,
        "gbs_kernel": alg_bytes / (per_launch_ms * 1e-3) / 1e9,
        "blocks": blocks, "x": x, "sha256": {"weight": sha256(blocks), "x": sha256(x)},
        "sustained": sustained,
    }
    for w in ws:
        w.close()
    return res


def bench_gemm(qmm, hipr, stream, steps, warmup, N=11008, K=4096, M=512, qtype=Q8_0, seed=0x5EED0003,
               sigma=0.02, f32_x=False):
    """The prefill GEMM on bf16 activations, or (f32_x) on fp32 activations through
    openmini_qmm_gemm_f32 (split pre-pass + GEMM, both timed, workspace preallocated)."""
    from openmini_qmm import _native, synth
    blocks = weight_blocks(qtype, N, K, seed, sigma)
    copies = max(2, -(-(MALL_DEFEAT_BYTES // 2) // blocks.size))
    log(f"gemm type={qtype} N={N} K={K} M={M}{' f32 x' if f32_x else ''}: {copies} weight copies")
    ws = [qmm.QuantizedWeight(qtype, blocks, N, K) for _ in range(copies)]
    x32 = synth.normal(seed + 0x8000, (M, K), 1.0)
    xb = synth.to_bf16_bits(x32)
    dx = qmm.DeviceBuffer.from_numpy(x32 if f32_x else xb)
    dy = qmm.DeviceBuffer(M * N * 4)
    work = qmm.gemm_f32_workspace(M, K) if f32_x else None
    sh = stream.handle
    shape = _native.lib().openmini_qmm_gemm_launch_shape(ws[0].handle, M, int(f32_x))
    min_rows = int(_native.lib().openmini_qmm_gemm_min_rows(ws[0].handle))

    def launch(i):
        if f32_x:
            ws[i % copies].gemm_f32(dx, dy, M, work, sh)
        else:
            ws[i % copies].gemm_bf16(dx, dy, M, sh)

    for i in range(warmup):
        launch(i)
    stream.synchronize()
    total_ms = time_steps(launch, steps, sh, hipr)
    per_launch_ms = total_ms / steps
    flops = 2.0 * M * N * K
    for w in ws:
        w.close()
    return {
        "N": N, "K": K, "M": M, "weight_copies": copies, "launch_shape": shape, "gemm_min_rows": min_rows,
        "sha256": {"weight": sha256(blocks), ("x_f32" if f32_x else "x_bf16"): sha256(x32 if f32_x else xb)},
        "ms_per_step": total_ms / steps, "kernel_ms": per_launch_ms,
        "tflops_wall": flops * steps / (total_ms * 1e-3) / 1e12,
        "tflops_kernel": flops / (per_launch_ms * 1e-3) / 1e12,
        "flops": flops,
    }


def bench_floor(qmm, hipr, stream, steps, warmup, nbytes: int) -> dict:
    """The single-launch floor at the headline size: the read-only streaming kernel
    (openmini_qmm_stream_read) over `nbytes`, rotated over >= 1 GiB of distinct
    buffers and timed exactly like the GEMV (graph replay, events on the stream)."""
    nbytes = nbytes // 16 * 16
    copies = max(2, -(-MALL_DEFEAT_BYTES // nbytes))
    bufs = [qmm.DeviceBuffer(nbytes) for _ in range(copies)]
    for b in bufs:
        b.fill(0x5A)
    sink = qmm.DeviceBuffer(256)
    sh = stream.handle

    def launch(i):
        qmm.stream_read(bufs[i % copies], nbytes, sink, sh)

    for i in range(warmup):
        launch(i)
    stream.synchronize()
    ms = time_steps(launch, steps, sh, hipr) / steps
    for b in bufs:
        b.free()
    return {"bytes": nbytes, "copies": copies, "us": ms * 1e3, "gbs": nbytes / (ms * 1e-3) / 1e9}


def bench_ceiling(qmm, hipr, stream, steps, warmup, M, N=11008, K=4096, qtype=Q8_0) -> dict:
    """The prefill GEMM's compute-only ceiling (openmini_qmm_gemm_ceiling): the GEMM's
    grid and per-block register work for the same M x N x K, without memory traffic,
    timed like the GEMM (graph replay, events on the stream)."""
    sink = qmm.DeviceBuffer(256)
    sh = stream.handle

    def launch(i):
        qmm.gemm_ceiling(qtype, M, N, K, sink, sh)

    for i in range(warmup):
        launch(i)
    stream.synchronize()
    ms = time_steps(launch, steps, sh, hipr) / steps
    sink.free()
    return {"us": ms * 1e3, "tflops": 2.0 * M * N * K / (ms * 1e-3) / 1e12}


def bench_dense_bf16(steps, warmup, M, N=11008, K=4096) -> dict:
    """Yardstick: a dense bf16 GEMM of the same shape through torch.mm (hipBLASLt),
    y_bf16[M, N] = x_bf16[M, K] . W_bf16[N, K]^T with fp32 accumulation: the weight
    row-major [N, K] as the quantized kernels hold it (hipBLASLt's fastest layout for
    this shape on MI355X, ahead of a [K, N] weight), dense bf16 (2 bytes per weight
    against the quantized 0.56-1.06), rotated over >= 512 MB of copies, timed with
    torch events over `steps` launches."""
    import torch
    dev = torch.device("cuda", 0)
    gen = torch.Generator().manual_seed(0x5EED00B1)
    x = torch.randn(M, K, generator=gen).to(torch.bfloat16).to(dev)
    w = (torch.randn(N, K, generator=gen) * 0.02).to(torch.bfloat16)
    copies = max(2, -(-(MALL_DEFEAT_BYTES // 2) // (w.numel() * 2)))
    ws = [w.to(dev) for _ in range(copies)]
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    for i in range(warmup):
        torch.mm(x, ws[i % copies].t(), out=y)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        torch.mm(x, ws[i % copies].t(), out=y)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    del ws
    return {"M": M, "us": ms * 1e3, "tflops": 2.0 * M * N * K / (ms * 1e-3) / 1e12, "weight_copies": copies}


def copy_calibration(qmm, hipr, stream, reps: int = 5, nbytes: int = 256 << 20) -> dict:
    """A plain streaming copy of `nbytes` (openmini_qmm_stream_copy), the yardstick the
    FETCH_SIZE / WRITE_SIZE counters are scaled by: it reads and writes exactly
    `nbytes` each per launch."""
    src, dst = qmm.DeviceBuffer(nbytes), qmm.DeviceBuffer(nbytes)
    src.fill(1)
    ms = time_steps(lambda i: qmm.stream_copy(dst, src, nbytes, stream.handle), reps, stream.handle, hipr)
    src.free()
    dst.free()
    return {"bytes": nbytes, "launches": reps, "gbs_read_plus_write": 2 * nbytes * reps / (ms * 1e-3) / 1e9}


def committed_traffic(workload: str):
    """HBM bytes per launch of the GEMV kernel from the committed rocprofv3 counter
    summary profiles/<workload>_traffic.md (FETCH_SIZE + WRITE_SIZE, each scaled by
    the same counter's reading for the calibration copy kernel), or None."""
    path = os.path.join(ROOT, "profiles", f"{workload}_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip()), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


def cpu_baseline(gemv: dict, seconds: float) -> dict:
    """The reference's per-token CPU path, restated in oracle/ (kind "port"): f32 GEMV
    over weights dequantized once at load (quant_loader.rs:76-92, model.rs:1050-1064,
    matrixmultiply single-threaded), timed on this host for ~`seconds`."""
    from oracle import oracle
    N, K = gemv["N"], gemv["K"]
    w = oracle.dequantize(Q4_0, gemv["blocks"], N * K).reshape(N, K)
    x = gemv["x"]
    y_ref = oracle.cpu_asrun_linear(w, x, None, False)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.cpu_asrun_linear(w, x, None, False)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per_call = el / reps
    # all host cores (up to the box's 16-core share) on the quant_simd-style fused path
    threads = max(1, min(16, os.cpu_count() or 1))
    y = np.empty((1, N), dtype=np.float32)
    rows = np.linspace(0, N, threads + 1).astype(int)

    def part(i):
        oracle.cpu_fused_linear(Q4_0, gemv["blocks"], N, K, x, y, int(rows[i]), int(rows[i + 1]))

    with cf.ThreadPoolExecutor(threads) as ex:
        list(ex.map(part, range(threads)))
        reps_f, t0 = 0, time.perf_counter()
        while True:
            list(ex.map(part, range(threads)))
            reps_f += 1
            el_f = time.perf_counter() - t0
            if el_f >= seconds / 2:
                break

        # the same f32 GEMV on all cores, rows split evenly (OpenMP-style)
        ya = np.empty((1, N), dtype=np.float32)

        def part_asrun(i):
            ya[:, rows[i]:rows[i + 1]] = oracle.cpu_asrun_linear(w[rows[i]:rows[i + 1]], x, None, False)

        list(ex.map(part_asrun, range(threads)))
        reps_a, t0 = 0, time.perf_counter()
        while True:
            list(ex.map(part_asrun, range(threads)))
            reps_a += 1
            el_a = time.perf_counter() - t0
            if el_a >= seconds / 4:
                break
    assert np.max(np.abs(y - y_ref)) <= 1e-3 * np.max(np.abs(y_ref))
    per_call_f = el_f / reps_f
    assert np.array_equal(ya.view(np.uint32), y_ref.view(np.uint32))  # same per-row order
    per_call_a = el_a / reps_a
    # as written: every linear() call also materialises W^T (model.rs:1052), one thread
    wt = np.empty(N * K, dtype=np.float32)
    reps_t, t0 = 0, time.perf_counter()
    while True:
        yt = oracle.cpu_asrun_linear(w, x, wt, True)
        reps_t += 1
        el_t = time.perf_counter() - t0
        if el_t >= seconds / 4:
            break
    assert np.max(np.abs(yt - y_ref)) <= 1e-3 * np.max(np.abs(y_ref))
    per_call_t = el_t / reps_t
    del wt
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    b = gemv["alg_bytes_per_step"]
    return {
        "value": round(b / per_call / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"{reps} calls of the f32 GEMV over the dequantized {N}x{K} weight "
                  f"({el:.1f} s); GB/s counts the same Q4_0 algorithmic bytes as the GPU",
        "ms_per_call": round(per_call * 1e3, 3),
        "host": {"cpu_model": model, "nproc": os.cpu_count()},
        "all_cores_fused": {"value": round(b / per_call_f / 1e9, 3), "unit": "GB/s",
                            "cores": threads, "ms_per_call": round(per_call_f * 1e3, 3),
                            "sample": f"{reps_f} calls, quant_simd-style dequant+dot from the "
                                      f"Q4_0 blocks, {threads} threads"},
        "all_cores_asrun": {"value": round(b / per_call_a / 1e9, 3), "unit": "GB/s",
                            "cores": threads, "ms_per_call": round(per_call_a * 1e3, 3),
                            "sample": f"{reps_a} calls, the f32 GEMV above with rows split over "
                                      f"{threads} threads"},
        "as_written": {"value": round(b / per_call_t / 1e9, 3), "unit": "GB/s", "cores": 1,
                       "ms_per_call": round(per_call_t * 1e3, 3),
                       "sample": f"{reps_t} calls, each also materialising W^T (model.rs:1052 "
                                 f"weight.t().to_owned()) before the f32 product"},
    }


def bench_weight_path(qmm, hipr, stream, steps, warmup, N=11008, K=4096):
    """The load-side rows on the GPU, on one 11008 x 4096 projection:
    * dequantization of raw GGUF blocks to f32 (quant::dequantize, GpuQuantOps;
      openmini_qmm_dequantize_any_device) for Q4_0, Q8_0, Q4_K and F16, graph-replayed over
      rotated inputs like the GEMV;
    * the upload of raw Q4_0 blocks already in device memory (openmini_qmm_upload_device:
      the weight's allocation plus the repack into chunks), timed as whole calls.
    Bytes counted: GGUF bytes read + bytes written (f32 outputs / chunks)."""
    from openmini_qmm import _native, synth
    L = _native.lib()
    sh = stream.handle
    n = N * K
    res = {"dequantize": []}
    for qtype, name in ((Q4_0, "q4_0"), (Q8_0, "q8_0"), (12, "q4_k"), (1, "f16")):
        if qtype == 1:
            raw = np.random.default_rng(0x5EED0053).integers(0, 256, n * 2, dtype=np.uint8)
            raw[1::2] &= 0x7B  # finite halves
        elif qtype == 12:
            raw = np.random.default_rng(0x5EED0050).integers(0, 256, n // 256 * 144, dtype=np.uint8)
            raw[1::144] &= 0x7B  # finite fp16 d and dmin
            raw[3::144] &= 0x7B
        else:
            raw = synth.weight_blocks(qtype, N, K, seed=0x5EED0051 + qtype)
        copies = max(2, -(-(MALL_DEFEAT_BYTES // 2) // raw.size))
        ins = [qmm.DeviceBuffer.from_numpy(raw) for _ in range(copies)]
        outs = [qmm.DeviceBuffer(n * 4) for _ in range(2)]

        def launch(i):
            rc = L.openmini_qmm_dequantize_any_device(qtype, ins[i % copies].ptr, raw.size, n, outs[i % 2].ptr, sh)
            if rc:
                raise RuntimeError(L.openmini_qmm_last_error().decode())

        for i in range(warmup):
            launch(i)
        stream.synchronize()
        ms = time_steps(launch, steps, sh, hipr) / steps
        alg = raw.size + n * 4
        res["dequantize"].append({"workload": f"{name}_dequant_n{N}_k{K}", "unit": "GB/s",
                                  "value": round(alg / (ms * 1e-3) / 1e9, 2), "kernel_us": round(ms * 1e3, 3),
                                  "frac": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                  "alg_bytes_per_step": alg, "sha256": {"gguf": sha256(raw)}})
        for b in ins + outs:
            b.free()
    raw = synth.weight_blocks(Q4_0, N, K, seed=0x5EED0052)
    d_raw = qmm.DeviceBuffer.from_numpy(raw)
    for w in [qmm.QuantizedWeight.from_device(Q4_0, d_raw, raw.size, N, K, sh) for _ in range(3)]:
        stream.synchronize()
        w.close()
    reps = 20
    hipr.hip().hipDeviceSynchronize()
    e0, e1 = hipr.Event(), hipr.Event()
    e0.record(sh)
    ws = [qmm.QuantizedWeight.from_device(Q4_0, d_raw, raw.size, N, K, sh) for _ in range(reps)]
    e1.record(sh)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / reps
    chunk_bytes = ws[0].info().device_bytes
    for w in ws:
        w.close()
    alg = raw.size + chunk_bytes
    res["upload"] = {"workload": f"q4_0_upload_device_n{N}_k{K}", "unit": "GB/s",
                     "value": round(alg / (ms * 1e-3) / 1e9, 2), "us_per_call": round(ms * 1e3, 3),
                     "frac": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes_per_call": alg,
                     "includes": "the weight's hipMalloc and the repack kernel",
                     "sha256": {"gguf": sha256(raw)}}
    # the same upload into caller memory (openmini_qmm_upload_device_into): one arena,
    # no allocation per call, the repack alone; sources and destinations rotated past
    # the MALL
    per = (chunk_bytes + 255) // 256 * 256
    srcs = [d_raw] + [qmm.DeviceBuffer.from_numpy(raw) for _ in range(3)]
    arena = qmm.DeviceBuffer(per * reps)

    def upload_into(i):
        return qmm.QuantizedWeight.from_device_into(Q4_0, srcs[i % len(srcs)], raw.size, N, K, arena,
                                                    (i % reps) * per, sh)

    for i in range(3):
        upload_into(i).close()  # a handle closes without touching the arena or the stream
    stream.synchronize()
    e0.record(sh)
    ws = [upload_into(i) for i in range(reps)]
    e1.record(sh)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / reps
    for w in ws:
        w.close()
    for b in srcs + [arena]:
        b.free()
    res["upload_into"] = {"workload": f"q4_0_upload_device_into_n{N}_k{K}", "unit": "GB/s",
                          "value": round(alg / (ms * 1e-3) / 1e9, 2), "us_per_call": round(ms * 1e3, 3),
                          "frac": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes_per_call": alg,
                          "includes": "the repack kernel (caller-provided weight memory)",
                          "sha256": {"gguf": sha256(raw)}}
    return res


def bench_layer(qmm, hipr, stream, steps, warmup, qtype=Q4_0, H=4096, I=11008, seed=0x5EED0010):
    """One Llama-7B decode layer's seven projections at batch 1 (q, k, v, o [H, H];
    gate, up [I, H]; down [H, I]) over distinct layers' weights (>= 1 GiB rotated):
    grouped as 4 launches (q/k/v together, o, gate/up with the silu * up epilogue,
    down) and, for comparison, as 7 single-weight launches plus nothing else (the
    grouped path also does the SwiGLU product the separate path leaves out)."""
    from openmini_qmm import synth
    shapes = [(H, H)] * 4 + [(I, H), (I, H), (H, I)]
    blocks = [synth.weight_blocks(qtype, n, k, seed=seed + i) for i, (n, k) in enumerate(shapes)]
    layer_bytes = sum(b.size for b in blocks)
    copies = max(2, -(-MALL_DEFEAT_BYTES // layer_bytes))
    log(f"layer type={qtype}: {copies} layers x {layer_bytes} B")
    layers = [[qmm.QuantizedWeight(qtype, b, n, k) for b, (n, k) in zip(blocks, shapes)]
              for _ in range(copies)]
    x = synth.normal(seed + 0x8000, (1, H), 1.0)
    dx = qmm.DeviceBuffer.from_numpy(x)
    dq, dk, dv, do, dd = (qmm.DeviceBuffer(H * 4) for _ in range(5))
    dg, du, dh = (qmm.DeviceBuffer(I * 4) for _ in range(3))
    sh = stream.handle

    def grouped(i):
        q, k, v, o, g, u, d = layers[i % copies]
        qmm.gemv_multi((q, k, v), dx, (dq, dk, dv), 1, sh)
        o.gemv(dx, do, 1, sh)
        qmm.ffn_gate_up(g, u, dx, dh, 1, sh)
        d.gemv(dh, dd, 1, sh)

    def separate(i):
        q, k, v, o, g, u, d = layers[i % copies]
        q.gemv(dx, dq, 1, sh)
        k.gemv(dx, dk, 1, sh)
        v.gemv(dx, dv, 1, sh)
        o.gemv(dx, do, 1, sh)
        g.gemv(dx, dg, 1, sh)
        u.gemv(dx, du, 1, sh)
        d.gemv(dh, dd, 1, sh)

    res = {"H": H, "I": I, "layer_bytes": layer_bytes, "layers": copies,
           "sha256": {"weights": sha256(np.concatenate(blocks)), "x": sha256(x)}}
    for name, fn in (("grouped", grouped), ("separate", separate)):
        for i in range(warmup):
            fn(i)
        stream.synchronize()
        ms = time_steps(fn, steps, sh, hipr)
        res[name + "_us"] = ms / steps * 1e3
        res[name + "_gbs"] = layer_bytes * steps / (ms * 1e-3) / 1e9
    for ws in layers:
        for w in ws:
            w.close()
    return res


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM leg")
    ap.add_argument("--no-layer", action="store_true", help="skip the decode-layer leg")
    ap.add_argument("--no-batch", action="store_true", help="skip the batched-decode legs")
    ap.add_argument("--no-weight-path", action="store_true", help="skip the dequantize / upload legs")
    ap.add_argument("--no-shapes", action="store_true", help="skip the other batch-1 decode shapes")
    ap.add_argument("--eager", action="store_true",
                    help="launch directly instead of replaying a HIP graph (for counter runs)")
    ap.add_argument("--dense-bf16", action="store_true",
                    help="also time a dense bf16 GEMM of the prefill shapes through torch (hipBLASLt)")
    ap.add_argument("--dense-only", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run the streaming-copy yardstick kernel (for counter runs)")
    args = ap.parse_args(argv)
    global EAGER
    EAGER = args.eager
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build targets a single MI355X and runs no "
              f"collectives (asked for --gpus {args.gpus})", file=sys.stderr)
        return 2

    if args.dense_only:  # the child process of --dense-bf16: torch only, one JSON line
        print(json.dumps([bench_dense_bf16(max(10, args.steps // 4), max(3, args.warmup // 4), m)
                          for m in (128, 512, 2048)]), flush=True)
        return 0
    dense = []
    if args.dense_bf16 and not args.no_gemm:
        # torch carries its own HIP runtime: it runs in a child process started before
        # this one touches the GPU, so the two runtimes never share a process
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--dense-only", "--steps", str(args.steps),
                            "--warmup", str(args.warmup)], capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            print(r.stderr[-2000:], file=sys.stderr)
            return r.returncode
        dense = json.loads(r.stdout.strip().splitlines()[-1])
        for d in dense:
            log(f"dense bf16 torch.mm M={d['M']}: {d['us']:.2f} us, {d['tflops']:.1f} TFLOP/s")

    import openmini_qmm as qmm
    from openmini_qmm import hip_runtime as hipr
    qmm.init(0)
    stream = qmm.Stream()
    info = qmm.HipQuantOps().device_info()
    log(info)

    sustained_steps = max(SUSTAINED_LAUNCHES, args.steps)
    g = bench_gemv(qmm, hipr, stream, args.steps, args.warmup, N=11008, K=4096, sustained_steps=sustained_steps)
    log(f"q4_0 gemv 11008x4096: wall {g['gbs_wall']:.1f} GB/s, kernel {g['gbs_kernel']:.1f} GB/s "
        f"({g['kernel_ms'] * 1e3:.2f} us)")
    down = bench_gemv(qmm, hipr, stream, args.steps, args.warmup, N=4096, K=11008, seed=0x5EED0002)
    log(f"q4_0 gemv 4096x11008: wall {down['gbs_wall']:.1f} GB/s, kernel {down['gbs_kernel']:.1f} GB/s")
    gemm = None
    prefill = []
    if not args.no_gemm:
        gemm = bench_gemm(qmm, hipr, stream, max(10, args.steps // 4), max(3, args.warmup // 4))
        gemm["ceiling"] = bench_ceiling(qmm, hipr, stream, max(10, args.steps // 4), max(3, args.warmup // 4), M=512)
        log(f"q8_0 gemm M=512: wall {gemm['tflops_wall']:.1f} TFLOP/s, kernel "
            f"{gemm['tflops_kernel']:.1f} TFLOP/s; compute-only ceiling {gemm['ceiling']['us']:.2f} us "
            f"({gemm['ceiling']['tflops']:.1f} TFLOP/s)")
        # the other prefill sizes of BASELINE configs[3]
        for m in (128, 2048):
            r = bench_gemm(qmm, hipr, stream, max(10, args.steps // 8), max(3, args.warmup // 4), M=m)
            c = bench_ceiling(qmm, hipr, stream, max(10, args.steps // 8), max(3, args.warmup // 4), M=m)
            prefill.append({"workload": f"q8_0_gemm_n11008_k4096_m{m}_bf16x", "unit": "TFLOP/s",
                            "value": round(r["tflops_kernel"], 2), "kernel_us": round(r["kernel_ms"] * 1e3, 3),
                            "frac": round(r["tflops_kernel"] / BF16_PEAK_TFLOPS, 4),
                            "ceiling_us": round(c["us"], 3), "frac_of_ceiling": round(c["us"] / (r["kernel_ms"] * 1e3), 4),
                            "launch_shape": r["launch_shape"], "sha256": r["sha256"]})
            log(f"q8_0 gemm M={m}: {r['kernel_ms'] * 1e3:.2f} us, {r['tflops_kernel']:.1f} TFLOP/s")
        # prefill on K-quant weights (Llama-7B up projection, M = 512)
        for qtype in (Q4_K, Q6_K):
            r = bench_gemm(qmm, hipr, stream, max(10, args.steps // 8), max(3, args.warmup // 4), qtype=qtype,
                           seed=0x5EED0081 + qtype)
            prefill.append({"workload": f"{TYPE_NAME[qtype]}_gemm_n11008_k4096_m512_bf16x", "unit": "TFLOP/s",
                            "value": round(r["tflops_kernel"], 2), "kernel_us": round(r["kernel_ms"] * 1e3, 3),
                            "frac": round(r["tflops_kernel"] / BF16_PEAK_TFLOPS, 4),
                            "launch_shape": r["launch_shape"], "sha256": r["sha256"]})
            log(f"{TYPE_NAME[qtype]} gemm M=512: {r['kernel_ms'] * 1e3:.2f} us, {r['tflops_kernel']:.1f} TFLOP/s")
        # the 70B q / gate / down projections at prefill M = 1024
        for n, k, seed in SHAPES_70B:
            r = bench_gemm(qmm, hipr, stream, max(10, args.steps // 10), max(3, args.warmup // 4), N=n, K=k,
                           M=1024, qtype=Q4_0, seed=seed, sigma=SIGMA_70B)
            prefill.append({"workload": f"q4_0_gemm_n{n}_k{k}_m1024_bf16x", "unit": "TFLOP/s",
                            "value": round(r["tflops_kernel"], 2), "kernel_us": round(r["kernel_ms"] * 1e3, 3),
                            "frac": round(r["tflops_kernel"] / BF16_PEAK_TFLOPS, 4),
                            "launch_shape": r["launch_shape"], "sha256": r["sha256"]})
            log(f"q4_0 gemm {n}x{k} M=1024: {r['kernel_ms'] * 1e3:.2f} us, {r['tflops_kernel']:.1f} TFLOP/s")
        # the fp32-activation prefill (linear_gemm's own input type, the operator's route
        # from 128 rows on) at configs[3]'s M = 512, against the bf16 leg above
        r = bench_gemm(qmm, hipr, stream, max(10, args.steps // 4), max(3, args.warmup // 4), f32_x=True)
        prefill.append({"workload": "q8_0_gemm_n11008_k4096_m512_f32x", "unit": "TFLOP/s",
                        "value": round(r["tflops_kernel"], 2), "kernel_us": round(r["kernel_ms"] * 1e3, 3),
                        "frac": round(r["tflops_kernel"] / BF16_PEAK_TFLOPS, 4),
                        "time_vs_bf16x": round(r["kernel_ms"] / gemm["kernel_ms"], 3),
                        "includes": "the split pre-pass (fp32 x -> fp16 hi / lo) and the GEMM",
                        "launch_shape": r["launch_shape"], "sha256": r["sha256"]})
        log(f"q8_0 gemm M=512 f32 x: {r['kernel_ms'] * 1e3:.2f} us, {r['tflops_kernel']:.1f} TFLOP/s "
            f"({r['kernel_ms'] / gemm['kernel_ms']:.2f}x the bf16 leg)")
        # a short prompt on the FFN up shape: linear() on 96 fp32 rows takes the fp32 GEMM
        # here (from openmini_qmm_gemm_min_rows rows on), timed beside the batched-GEMV
        # passes of 16 rows it ran before
        m_short = 96
        rl = bench_gemm(qmm, hipr, stream, max(10, args.steps // 4), max(3, args.warmup // 4), M=m_short, f32_x=True)
        gl = bench_gemv(qmm, hipr, stream, max(10, args.steps // 4), max(3, args.warmup // 4), N=11008, K=4096,
                       qtype=Q8_0, batch=m_short, seed=0x5EED0003)
        prefill.append({"workload": f"q8_0_linear_n11008_k4096_m{m_short}_f32x", "unit": "TFLOP/s",
                        "value": round(rl["tflops_kernel"], 2), "kernel_us": round(rl["kernel_ms"] * 1e3, 3),
                        "frac": round(rl["tflops_kernel"] / BF16_PEAK_TFLOPS, 4),
                        "route": ("fp32 GEMM" if m_short >= rl["gemm_min_rows"] else "decode GEMVs"),
                        "gemm_min_rows": rl["gemm_min_rows"],
                        "gemv_passes_us": round(gl["kernel_ms"] * 1e3, 3),
                        "launch_shape": rl["launch_shape"], "sha256": rl["sha256"]})
        log(f"q8_0 linear M={m_short} f32 x: GEMM {rl['kernel_ms'] * 1e3:.2f} us vs GEMV passes "
            f"{gl['kernel_ms'] * 1e3:.2f} us")
    layer = None
    if not args.no_layer:
        layer = bench_layer(qmm, hipr, stream, max(10, args.steps // 4), max(3, args.warmup // 4))
        log(f"decode layer: grouped {layer['grouped_us']:.2f} us ({layer['grouped_gbs']:.1f} GB/s), "
            f"separate {layer['separate_us']:.2f} us ({layer['separate_gbs']:.1f} GB/s)")
    batched = []
    if not args.no_batch:
        # BASELINE configs[1] (Q8_0 up / down, batch 8) and configs[4] (70B q / gate / down,
        # batch 4 and 16); the 70B legs share their weights with the batch-1 legs below
        legs = [(Q8_0, 11008, 4096, 8, 0x5EED0011, 0.02), (Q8_0, 4096, 11008, 8, 0x5EED0012, 0.02)]
        legs += [(Q4_0, n, k, b, seed, SIGMA_70B) for n, k, seed in SHAPES_70B for b in (4, 16)]
        for qtype, n, k, b, seed, sigma in legs:
            r = bench_gemv(qmm, hipr, stream, max(20, args.steps // 2), max(5, args.warmup // 2), N=n, K=k,
                           qtype=qtype, batch=b, seed=seed, sigma=sigma)
            name = "q4_0" if qtype == Q4_0 else "q8_0"
            batched.append({"workload": f"{name}_gemv_n{n}_k{k}_b{b}", "unit": "GB/s",
                            "value": round(r["gbs_kernel"], 2), "kernel_us": round(r["kernel_ms"] * 1e3, 3),
                            "frac": round(r["gbs_kernel"] / HBM_PEAK_GBS, 4),
                            "alg_bytes_per_step": r["alg_bytes_per_step"], "sha256": r["sha256"]})
            log(f"batched {batched[-1]['workload']}: {r['kernel_ms'] * 1e3:.2f} us, {r['gbs_kernel']:.1f} GB/s")
    shapes = []
    sustained = [{"workload": "q4_0_gemv_n11008_k4096_b1", "steps_value": round(g["kernel_ms"] * 1e3, 3),
                  **g["sustained"]}]
    if not args.no_shapes:
        # the remaining decode configs of the measurement table (batch 1)
        legs = [(Q4_0, 4096, 4096, 0x5EED0061, 0.02), (Q8_0, 11008, 4096, 0x5EED0062, 0.02),
                (Q8_0, 4096, 11008, 0x5EED0063, 0.02)]
        legs += [(Q4_0, n, k, seed, SIGMA_70B) for n, k, seed in SHAPES_70B]
        for qtype, n, k, seed, sigma in legs:
            r = bench_gemv(qmm, hipr, stream, max(20, args.steps // 2), max(5, args.warmup // 2), N=n, K=k,
                           qtype=qtype, batch=1, seed=seed, sigma=sigma,
                           sustained_steps=sustained_steps if (n, k) == (28672, 8192) else 0)
            name = "q4_0" if qtype == Q4_0 else "q8_0"
            shapes.append({"workload": f"{name}_gemv_n{n}_k{k}_b1", "unit": "GB/s",
                           "value": round(r["gbs_kernel"], 2), "kernel_us": round(r["kernel_ms"] * 1e3, 3),
                           "frac": round(r["gbs_kernel"] / HBM_PEAK_GBS, 4),
                           "alg_bytes_per_step": r["alg_bytes_per_step"], "sha256": r["sha256"]})
            if r["sustained"]:
                sustained.append({"workload": shapes[-1]["workload"], "steps_value": shapes[-1]["kernel_us"],
                                  **r["sustained"]})
            log(f"decode {shapes[-1]['workload']}: {r['kernel_ms'] * 1e3:.2f} us, {r['gbs_kernel']:.1f} GB/s")
    kquant = []
    if not args.no_shapes:
        # decode GEMV on K-quant weights (Llama-7B up / down shapes at batch 1; the up
        # shape at batch 8 through the batched kernel)
        # and on the block-minimum types Q4_1 and Q5_K (GGUF bytes counted: Q5_K's chunks
        # hold its 5-bit codes in the 6-bit Q6_K form, 27% above them)
        for qtype, n, k, b, seed in ((Q4_K, 11008, 4096, 1, 0x5EED0071), (Q4_K, 4096, 11008, 1, 0x5EED0072),
                                     (Q6_K, 11008, 4096, 1, 0x5EED0073), (Q6_K, 4096, 11008, 1, 0x5EED0074),
                                     (Q4_K, 11008, 4096, 8, 0x5EED0075), (Q6_K, 11008, 4096, 8, 0x5EED0076),
                                     (Q4_1, 11008, 4096, 1, 0x5EED0077), (Q4_1, 4096, 11008, 1, 0x5EED0078),
                                     (Q5_K, 11008, 4096, 1, 0x5EED0079), (Q4_1, 11008, 4096, 8, 0x5EED007A),
                                     (Q5_K, 11008, 4096, 8, 0x5EED007B)):
            r = bench_gemv(qmm, hipr, stream, max(20, args.steps // 2), max(5, args.warmup // 2), N=n, K=k,
                           qtype=qtype, batch=b, seed=seed)
            kquant.append({"workload": f"{TYPE_NAME[qtype]}_gemv_n{n}_k{k}_b{b}", "unit": "GB/s",
                           "value": round(r["gbs_kernel"], 2), "kernel_us": round(r["kernel_ms"] * 1e3, 3),
                           "frac": round(r["gbs_kernel"] / HBM_PEAK_GBS, 4),
                           "alg_bytes_per_step": r["alg_bytes_per_step"], "sha256": r["sha256"]})
            log(f"decode {kquant[-1]['workload']}: {r['kernel_ms'] * 1e3:.2f} us, {r['gbs_kernel']:.1f} GB/s")
    wpath = None
    if not args.no_weight_path:
        wpath = bench_weight_path(qmm, hipr, stream, max(20, args.steps // 4), max(3, args.warmup // 4))
        for r in wpath["dequantize"]:
            log(f"dequantize {r['workload']}: {r['kernel_us']:.2f} us, {r['value']:.1f} GB/s")
        log(f"upload {wpath['upload']['workload']}: {wpath['upload']['us_per_call']:.2f} us per call, "
            f"{wpath['upload']['value']:.1f} GB/s")
        log(f"upload {wpath['upload_into']['workload']}: {wpath['upload_into']['us_per_call']:.2f} us per call, "
            f"{wpath['upload_into']['value']:.1f} GB/s")
    copy = None
    if args.calibrate_copy:
        copy = copy_calibration(qmm, hipr, stream)
        log(f"stream copy {copy['bytes']} B: {copy['gbs_read_plus_write']:.1f} GB/s read+write")
    floor = bench_floor(qmm, hipr, stream, args.steps, args.warmup, g["alg_bytes_per_step"])
    log(f"read-only floor {floor['bytes']} B: {floor['us']:.2f} us ({floor['gbs']:.1f} GB/s)")
    # the same floor for every other GEMV leg, over that leg's algorithmic bytes
    floors = {g["alg_bytes_per_step"]: floor}
    for rec in batched + shapes + kquant + [{"alg_bytes_per_step": down["alg_bytes_per_step"]}]:
        nb = rec["alg_bytes_per_step"]
        if nb not in floors:
            floors[nb] = bench_floor(qmm, hipr, stream, max(20, args.steps // 2), max(5, args.warmup // 2), nb)
            log(f"read-only floor {floors[nb]['bytes']} B: {floors[nb]['us']:.2f} us")
        if "kernel_us" in rec:
            rec["floor_us"] = round(floors[nb]["us"], 3)
            rec["frac_of_floor"] = round(floors[nb]["us"] / rec["kernel_us"], 4)
    down_floor = floors[down["alg_bytes_per_step"]]["us"]
    cpu = None if args.no_cpu else cpu_baseline(g, args.cpu_seconds)

    achieved = g["gbs_kernel"]
    workload = "q4_0_gemv_n11008_k4096_b1"
    traffic, traffic_src = committed_traffic(workload)
    out = {
        "metric": METRIC,
        "value": round(g["gbs_wall"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "arith": "int8 MFMA on 4-digit (30-bit) block-floating activations (int32-exact per block), fp32 accumulation",
        "data": "synthetic",
        "config": {"workload": workload, "N": g["N"], "K": g["K"], "batch": 1,
                   "weight": "Q4_0 from N(0, 0.02)", "x": "f32 N(0, 1)",
                   "weight_copies": g["weight_copies"], "rotated_bytes": g["rotated_bytes"],
                   "alg_bytes_per_step": g["alg_bytes_per_step"], "sha256": g["sha256"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src, "kernel_us": round(g["kernel_ms"] * 1e3, 3),
                     "floor_us": round(floor["us"], 3), "frac_of_floor": round(floor["us"] / (g["kernel_ms"] * 1e3), 4),
                     "floor": "openmini_qmm_stream_read over the same bytes, same protocol"},
        "pct_of_hbm_peak_wall": round(100.0 * g["gbs_wall"] / HBM_PEAK_GBS, 2),
        "down_proj": {"workload": "q4_0_gemv_n4096_k11008_b1", "value": round(down["gbs_wall"], 2),
                      "unit": "GB/s", "kernel_gbs": round(down["gbs_kernel"], 2),
                      "kernel_us": round(down["kernel_ms"] * 1e3, 3), "floor_us": round(down_floor, 3),
                      "frac_of_floor": round(down_floor / (down["kernel_ms"] * 1e3), 4), "sha256": down["sha256"]},
        "cpu_baseline": cpu,
    }
    if copy:
        out["copy_calibration"] = copy
    if gemm:
        out["gemm"] = {
            "metric": "Q8_0 GEMM TFLOP/s M=512", "workload": "q8_0_gemm_n11008_k4096_m512_bf16x",
            "sha256": gemm["sha256"],
            "value": round(gemm["tflops_wall"], 2), "unit": "TFLOP/s", "dtype": "bf16",
            "ms_per_step": round(gemm["ms_per_step"], 6),
            "launch_shape": gemm["launch_shape"],
            "roofline": {"bound": "mfma", "achieved": round(gemm["tflops_kernel"], 2),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(gemm["tflops_kernel"] / BF16_PEAK_TFLOPS, 4), "traffic": None,
                         "kernel_us": round(gemm["kernel_ms"] * 1e3, 3),
                         "ceiling_us": round(gemm["ceiling"]["us"], 3),
                         "ceiling_tflops": round(gemm["ceiling"]["tflops"], 2),
                         "frac_of_ceiling": round(gemm["ceiling"]["us"] / (gemm["kernel_ms"] * 1e3), 4),
                         "ceiling": "openmini_qmm_gemm_ceiling: the same grid and per-block register work, "
                                    "no memory traffic"},
        }
    if prefill:
        out["prefill_sizes"] = prefill
    if dense:
        out["gemm"]["yardstick_dense_bf16"] = {
            "what": "torch.mm(x_bf16, W_bf16[N, K].t()) -> bf16 (hipBLASLt), dense bf16 weights of the same "
                    "shape, rotated over >= 512 MB",
            "legs": [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in d.items()} for d in dense]}
    if batched:
        out["batched_decode"] = batched
    if shapes:
        out["decode_shapes"] = shapes
    out["sustained"] = {
        "what": f"the same graph-replayed launches as the leg, {sustained_steps} back to back (the leg itself "
                f"runs {args.steps} or half that); steps_value is the leg's own us per launch",
        "legs": sustained}
    if kquant:
        out["kquant_decode"] = kquant
    if wpath:
        out["weight_path"] = wpath
    if layer:
        out["decode_layer"] = {
            "workload": "q4_0_llama7b_layer_7proj_b1", "unit": "GB/s",
            "value": round(layer["grouped_gbs"], 2), "us_per_layer": round(layer["grouped_us"], 3),
            "launches": 4, "separate_gbs": round(layer["separate_gbs"], 2),
            "separate_us_per_layer": round(layer["separate_us"], 3), "separate_launches": 7,
            "layer_bytes": layer["layer_bytes"], "layers_rotated": layer["layers"], "sha256": layer["sha256"],
        }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
