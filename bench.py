"""Benchmark: ResNet-101 fp32 224x224 on one MI355X through the SPINNV2 C API.

A step is one spkv2_run of the whole network over one batch whose input is
already resident in HBM (a device buffer bound with spkv2_bind_input).
Workload: ResNet-101-style bottleneck CNN, batch
64, He-normal weights with BN folded, N(0,1) input, seed 42 (synthetic data,
random-init weights of the real architecture).

Reported:
  value          images/sec at batch 64 over the timed K steps (the node
                 loop captured into a HIP graph during warmup and replayed;
                 --eager times the plain node loop instead);
  roofline       conv implicit-GEMM throughput: conv FLOP per step / the
                 summed kernel-trace durations of the conv nodes' launches
                 per step (the committed rocprofv3 summary of this workload),
                 against the fp32 MFMA peak; beside it the live figures of
                 this run: HIP events around every node on the run stream in
                 a separate eager pass of W + K steps, and the timed step;
  graph_matches_eager  the timed graph replay's output is bit-identical to
                 the eager pass's output of the same input;
  b1_*           batch-1 latency and images/sec (HIP-graph replay);
  cpu_baseline   the reference runtime (cpu_generic package: naive conv on
                 x86) on one batch-1 image, timed on the host;
  int8, elementwise, yolo   INT8 ResNet-50, the memory-bound ops against
                 the HBM peak, YOLOv10n 640 images/s (sections of their own);
  int8_config_mode  INT8 ResNet-50 in BASELINE configs[4]'s own semantics
                 (asymmetric activations, int8 tensors between nodes,
                 fixed-point requantization), against the int8 MFMA peak.

    python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--batch 64] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP32_MFMA_PEAK_TFLOPS = 157.3
INT8_MFMA_PEAK_TOPS = 5000.0
HBM_PEAK_GBPS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _ref_leg(args: list[str], threads: int, timeout_s: float) -> dict | None:
    env = dict(os.environ)
    env["OMP_NUM_THREADS"] = str(threads)
    cmd = [sys.executable, "-m", "oracle.cpu_baseline", "--model", "resnet101", "--batch", "1", *args]
    try:
        out = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=timeout_s)
    except subprocess.TimeoutExpired:
        log("cpu baseline leg timed out")
        return None
    if out.returncode != 0:
        log(f"cpu baseline leg failed: {out.stderr[-400:]}")
        return None
    return json.loads(out.stdout.strip().splitlines()[-1])


def cpu_baseline(timeout_s: float = 300.0) -> tuple[dict | None, dict | None]:
    """The reference runtime on the host: (1) its cpu_generic package, whose
    bnns conv kind falls back to the naive single-threaded reference conv on
    x86 (what the reference's own x86 build runs), one image; (2) the labelled
    second row, cpu_generic without the bnns token: its AVX2 im2col+SGEMM conv
    with OpenMP over the host cores (at most the 16 of one GPU's share), one
    warmup then up to 20 runs or 15 s.  Statistics as spkv2_bench.c:136-159."""
    from oracle.cpu_baseline import host_cpu
    from oracle.ref_runtime import available

    if not available():
        log("cpu baseline skipped: oracle/_ref/libspkv2_ref.so not built")
        return None, None
    host = host_cpu()
    log("cpu baseline: reference cpu_generic runtime, ResNet-101 b=1, one image (naive conv, 1 thread)")
    r = _ref_leg(["--profile", "cpu_generic", "--runs", "1"], 1, timeout_s)
    base = None
    if r:
        base = {"value": r["images_per_sec"], "unit": "images/sec", "cores": 1, "kind": "reference",
                "sample": "ResNet-101 fp32 b=1, one 224x224 image, reference cpu_generic package "
                          "(bnns kind -> naive single-threaded reference conv on x86)",
                "seconds": r["avg_s"], "host": host,
                "stats_ms": {k: r[k] for k in ("min_ms", "avg_ms", "p50_ms", "p90_ms", "max_ms")}}
    threads = max(1, min(host["nproc"] or 1, 16))
    log(f"cpu baseline second row: cpu_generic without simd_bnns_fp32 (AVX2 im2col+SGEMM), {threads} threads")
    r2 = _ref_leg(["--profile", "cpu_generic_nobnns", "--runs", "20", "--warmup", "1", "--max-seconds", "15"],
                  threads, timeout_s)
    simd = None
    if r2:
        simd = {"label": "cpu_generic without simd_bnns_fp32", "value": r2["images_per_sec"], "unit": "images/sec",
                "cores": threads, "kind": "reference",
                "sample": f"ResNet-101 fp32 b=1, {r2['runs']} runs after 1 warmup, reference cpu_generic package "
                          "without the bnns token (AVX2 im2col + SGEMM conv, OpenMP)",
                "runs": r2["runs"], "host": host,
                "stats_ms": {k: r2[k] for k in ("min_ms", "avg_ms", "p50_ms", "p90_ms", "max_ms")}}
    return base, simd


def copy_calibration(mib: int, reps: int) -> None:
    """Runs the runtime's plain copy kernel (a Flatten node whose output the
    planner cannot alias to the graph input) over `mib` MiB, `reps` times:
    the known-size reference for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE."""
    from spinnv2_amd.runtime import DeviceBuffer, Model, load_library
    from spinnv2_amd.spk.graph import Graph
    from spinnv2_amd.spk import write_spk

    lib = load_library()
    n = mib * (1 << 20) // 4
    g = Graph("copy")
    x = g.input("x", [1, n])
    g.mark_output(g.flatten(x))
    m = Model(write_spk(g, "mi355x"), lib=lib)
    buf = DeviceBuffer(n * 4, lib)
    buf.upload(np.zeros(n, np.float32))
    m.bind_input(0, buf)
    for _ in range(reps):
        m.run()
    lib.spkv2_device_synchronize()
    assert m.kernel_name(0) == "copy", m.kernel_name(0)
    print(json.dumps({"copy_kernel_bytes_read": n * 4, "copy_kernel_bytes_written": n * 4, "dispatches": reps}))
    m.close()
    buf.free()


# GEMM views (M = output features, K, N = columns) of ResNet-101 b=64 layers
# and one large square problem, for the vendor-library calibration
VENDOR_GEMM_SHAPES = [
    ("s3_3x3_as_gemm", 256, 2304, 12544),
    ("s3_1x1_reduce", 256, 1024, 12544),
    ("s3_1x1_expand", 1024, 256, 12544),
    ("s4_3x3_as_gemm", 512, 4608, 3136),
    ("square_4096", 4096, 4096, 4096),
]


def vendor_gemm(reps: int) -> dict:
    """Calibration, not the product: fp32 GEMM TFLOP/s of the vendor library
    (torch.matmul on ROCm, TF32-style reduced precision off) beside this
    runtime's Gemm node on the same problem (Y[N, M] = X[N, K] W[K, M]; the
    node's HIP-graph replay, wall-clocked), on the GEMM shapes of ResNet-101's
    stage-3/4 layers (what its convs compute, without the gather) and a square
    problem."""
    import torch

    from spinnv2_amd.runtime import DeviceBuffer, Model, load_library
    from spinnv2_amd.spk import models, write_spk

    torch.backends.cuda.matmul.allow_tf32 = False
    lib = load_library()
    out = []
    for name, M, K, N in VENDOR_GEMM_SHAPES:
        flop = 2.0 * M * K * N
        a = torch.randn(M, K, device="cuda:0")
        b = torch.randn(K, N, device="cuda:0")
        for _ in range(3):
            c = a @ b
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            c = a @ b
        e1.record()
        torch.cuda.synchronize()
        t_vendor = e0.elapsed_time(e1) / reps * 1e-3
        del a, b, c
        g = models.single_gemm(N, K, M, bias=False)
        m = Model(write_spk(g, "mi355x"), lib=lib)
        x = models.make_input(g.tensors[g.inputs[0]].shape)
        xb = DeviceBuffer(x.nbytes, lib)
        xb.upload(x)
        m.bind_input(0, xb)
        m.set_graph_mode(True)
        for _ in range(3):
            m.run()
        lib.spkv2_device_synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            m.run()
        lib.spkv2_device_synchronize()
        t_ours = (time.perf_counter() - t0) / reps
        out.append({"shape": name, "M": M, "K": K, "N": N, "vendor_tflops": round(flop / t_vendor / 1e12, 1),
                    "spkv2_gemm_tflops": round(flop / t_ours / 1e12, 1), "spkv2_kernel": m.kernel_name(0)})
        m.close()
        xb.free()
    return {"vendor_gemm": out, "peak_tflops": 157.3}


def pmc_traffic(name: str = "conv_igemm_f32_resnet101_b64_traffic.txt") -> dict | None:
    """HBM bytes of the conv kernels per step, from a committed rocprofv3
    --pmc summary (FETCH_SIZE and WRITE_SIZE passes scaled by the copy
    kernel's reading).  None when no summary is committed."""
    p = ROOT / "profiles" / name
    if not p.exists():
        return None
    vals = {}
    for line in p.read_text().splitlines():
        if line.startswith("result "):
            k, v = line[len("result "):].split("=", 1)
            vals[k.strip()] = float(v)
    return vals or None


def bit_identical(a: np.ndarray, b: np.ndarray) -> bool:
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))


def batch1_latency(depth: int, steps: int, lib, eager: bool = False) -> tuple[float, bool]:
    """Batch-1 latency: ms per spkv2_run of a HIP-graph-captured node loop
    (the plain node loop with eager), input already resident on the device;
    and whether the last timed run's output is bit-identical to an eager
    run's before it."""
    from spinnv2_amd.runtime import DeviceBuffer, Model
    from spinnv2_amd.spk import models, write_spk

    g1 = models.resnet(depth, 1)
    m1 = Model(write_spk(g1, "mi355x"), lib=lib)
    x1 = models.make_input(g1.tensors[g1.inputs[0]].shape)
    x1buf = DeviceBuffer(x1.nbytes, lib)
    x1buf.upload(x1)
    m1.bind_input(0, x1buf)
    m1.run()
    eager_out = m1.get_output(0)
    m1.set_graph_mode(not eager)
    for _ in range(5):
        m1.run()
    lib.spkv2_device_synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        m1.run()
    lib.spkv2_device_synchronize()
    b1_ms = (time.perf_counter() - t0) * 1e3 / steps
    same = bit_identical(m1.get_output(0), eager_out)
    m1.close()
    x1buf.free()
    return b1_ms, same


def int8_resnet50(lib, steps: int, warmup: int, b1_steps: int, batch: int = 64, node_report: bool = False,
                  eager: bool = False) -> dict:
    """INT8 ResNet-50: per-channel symmetric int8
    weights, per-tensor activation scales calibrated on 16 seeded single-image
    batches with the repo's fp32 forward, int32 accumulation, reference
    dequantization.  Returns images/s at `batch`, batch-1 latency, and the
    int8 conv throughput (conv node device time: quantize pass + int8 GEMM +
    epilogue) against the int8 MFMA peak."""
    from spinnv2_amd.runtime import DeviceBuffer, Model
    from spinnv2_amd.spk import models, write_spk
    from spinnv2_amd.spk.quantize import calibrate_activation_scales, quantize_conv_weights

    t0 = time.time()
    g1 = models.resnet(50, 1)
    samples = [models.make_input(g1.tensors[g1.inputs[0]].shape, 1000 + i) for i in range(16)]
    act = calibrate_activation_scales(g1, samples)
    log(f"int8: calibrated {len(act)} activation scales on 16 batches in {time.time() - t0:.1f}s")

    def build(b):
        g = models.resnet(50, b)
        wq = quantize_conv_weights(g)
        return g, write_spk(g, "mi355x", quant_params=wq + act)

    g, blob = build(batch)
    ops = {}
    hbm = 0  # algorithmic bytes of the INT8 convs under the reference's fp32-in / fp32-out semantics
    node_bytes = {}
    for n in g.nodes:
        if n.op_type == "Conv":
            xsh = g.shape(n.inputs[0])
            y = g.shape(n.outputs[0])
            w = g.tensors[n.inputs[1]].shape
            ops[n.id] = 2 * y[0] * y[1] * y[2] * y[3] * w[1] * w[2] * w[3]
            y_bytes = 4 * y[0] * y[1] * y[2] * y[3]
            nb = 4 * xsh[0] * xsh[1] * xsh[2] * xsh[3] + w[0] * w[1] * w[2] * w[3] + y_bytes
            nb += y_bytes if len(n.inputs) > 3 else 0      # fused residual
            nb += 4 * y[1] if len(n.inputs) > 2 else 0     # bias
            node_bytes[n.id] = nb
            hbm += nb
    x = models.make_input(g.tensors[g.inputs[0]].shape)
    m = Model(blob, lib=lib)
    xin = DeviceBuffer(x.nbytes, lib)
    xin.upload(x)
    m.bind_input(0, xin)
    # per-node device times in an eager pass of their own; images/s from
    # HIP-graph replays of the node loop
    m.set_profiling(True)
    for _ in range(warmup):
        m.run()
    m.reset_node_times()
    lib.spkv2_device_synchronize()
    for _ in range(steps):
        m.run()
    lib.spkv2_device_synchronize()
    m.set_profiling(False)
    eager_out = m.get_output(0)
    m.set_graph_mode(not eager)
    for _ in range(warmup):
        m.run()
    lib.spkv2_device_synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        m.run()
    lib.spkv2_device_synchronize()
    elapsed = time.perf_counter() - t0
    graph_same = bit_identical(m.get_output(0), eager_out)
    m.set_graph_mode(False)
    conv_ms = 0.0
    for nid in ops:
        ms, cnt = m.node_time(nid)
        conv_ms += ms / max(cnt, 1)
        if node_report:
            n = g.nodes[nid]
            xs_, ws_ = g.shape(n.inputs[0]), g.tensors[n.inputs[1]].shape
            log(f"int8 node {nid:3d} {xs_[1]}x{xs_[2]}->{ws_[0]} k{ws_[2]} s{n.attrs['strides'][0]} "
                f"{m.kernel_name(nid):52s} {ms / max(cnt, 1) * 1e3:8.1f} us {ops[nid] / (ms / max(cnt, 1)) / 1e9:7.1f} TOP/s "
                f"{node_bytes[nid] / (ms / max(cnt, 1)) / 1e6:7.1f} GB/s")
    names = sorted({m.kernel_name(nid).split("<")[0] for nid in ops})
    m.close()
    xin.free()
    total_ops = sum(ops.values())
    # Roofline of the int8 conv kernels on what they measurably do: their
    # HBM bytes per step (FETCH_SIZE + WRITE_SIZE counters) and their summed
    # kernel-trace duration per step, both from the committed rocprofv3
    # summaries of this workload (at batch 64 only), so the fractions
    # reproduce from profiles/; the bound is the roof they are nearer to.
    # The live per-node HIP-event time (eager loop, launch gaps and event
    # overhead inside each node) is reported beside it as an upper bound.
    roof = None
    t8 = pmc_traffic("conv_igemm_i8_resnet50_b64_traffic.txt") if batch == 64 else None
    k8 = pmc_traffic("conv_igemm_i8_resnet50_b64_kernel_stats.txt") if batch == 64 else None
    if t8 and k8 and "conv_igemm_i8_ms_per_run" in k8:
        kms = k8["conv_igemm_i8_ms_per_run"]
        traffic_b = t8["conv_hbm_bytes_per_step"]
        gbps = traffic_b / (kms * 1e-3) / 1e9
        tops_k = total_ops / (kms * 1e-3) / 1e12
        f_hbm, f_mfma = gbps / HBM_PEAK_GBPS, tops_k / INT8_MFMA_PEAK_TOPS
        roof = {"bound": "hbm" if f_hbm >= f_mfma else "mfma",
                "achieved": gbps if f_hbm >= f_mfma else tops_k,
                "peak": HBM_PEAK_GBPS if f_hbm >= f_mfma else INT8_MFMA_PEAK_TOPS,
                "unit": "GB/s" if f_hbm >= f_mfma else "TOP/s", "frac": max(f_hbm, f_mfma),
                "traffic": traffic_b, "kernel_ms_per_step": kms,
                "basis": "HBM bytes (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-kernel scaled) and summed kernel-trace "
                         "durations of the conv_igemm_i8 launches of one step (profiles/)",
                "hbm_frac": f_hbm, "mfma_frac": f_mfma, "mfma_tops": tops_k}
    tops = total_ops / (conv_ms * 1e-3) / 1e12
    out = {"workload": "resnet50_int8_224", "batch": batch, "images_per_sec": batch * steps / elapsed,
           "ms_per_step": elapsed * 1e3 / steps, "timed_mode": "eager" if eager else "hip_graph",
           "graph_matches_eager": graph_same,
           "semantics": "reference kernel_conv_int8 (conv_int8.c:121-210): per-channel symmetric int8 weights, "
                        "per-tensor symmetric activations (zero point 0), int32 accumulate, float dequantize + "
                        "bias + fp32 residual + Relu; fp32 tensors between nodes",
           "conv_event_ms_per_step": conv_ms,
           "conv_gop_per_image": total_ops / batch / 1e9, "conv_kernels": names,
           "roofline": roof,
           "mfma_by_events": {"achieved": tops, "peak": INT8_MFMA_PEAK_TOPS, "unit": "TOP/s",
                              "frac": tops / INT8_MFMA_PEAK_TOPS},
           "fp32_io_bytes_per_step": hbm,
           "floor_ms": {"hbm_fp32_io": hbm / HBM_PEAK_GBPS / 1e6, "mfma": total_ops / INT8_MFMA_PEAK_TOPS / 1e9}}
    if b1_steps > 0:
        g1q, blob1 = build(1)
        m1 = Model(blob1, lib=lib)
        x1 = models.make_input(g1q.tensors[g1q.inputs[0]].shape)
        b1 = DeviceBuffer(x1.nbytes, lib)
        b1.upload(x1)
        m1.bind_input(0, b1)
        m1.run()
        eager1 = m1.get_output(0)
        m1.set_graph_mode(not eager)
        for _ in range(5):
            m1.run()
        lib.spkv2_device_synchronize()
        t0 = time.perf_counter()
        for _ in range(b1_steps):
            m1.run()
        lib.spkv2_device_synchronize()
        out["b1_ms_per_image"] = (time.perf_counter() - t0) * 1e3 / b1_steps
        out["b1_graph_matches_eager"] = bit_identical(m1.get_output(0), eager1)
        m1.close()
        b1.free()
    return out


def int8_config_mode(lib, steps: int, warmup: int, b1_steps: int, batch: int = 64, node_report: bool = False,
                     eager: bool = False) -> dict:
    """INT8 ResNet-50 224x224 in BASELINE configs[4]'s own semantics (no
    reference counterpart): per-channel symmetric int8 weights, per-tensor
    asymmetric activation scales and zero points from min/max over 16
    seeded calibration batches, int8 tensors between nodes, int32
    accumulation, fixed-point requantization with round-half-away and a
    fused Relu clamp.  images/s at `batch` (graph replay), batch-1 latency,
    and the int8 conv launches against the int8 MFMA peak."""
    from spinnv2_amd.runtime import DeviceBuffer, Model
    from spinnv2_amd.spk import models, write_spk
    from spinnv2_amd.spk.quantize import quantize_int8_activations

    t0 = time.time()
    cal = models.resnet(50, 1)
    samples = [models.make_input(cal.tensors[cal.inputs[0]].shape, 1000 + i) for i in range(16)]

    def build(b):
        g = models.resnet(50, b)
        qp = quantize_int8_activations(g, samples, calibrate_on=cal)
        return g, write_spk(g, "mi355x", quant_params=qp)

    g, blob = build(batch)
    log(f"int8 config mode: calibrated and quantized in {time.time() - t0:.1f}s")
    ops, in_bytes = {}, 0
    for n in g.nodes:
        if n.op_type == "Conv":
            y = g.shape(n.outputs[0])
            w = g.tensors[n.inputs[1]].shape
            ops[n.id] = 2 * y[0] * y[1] * y[2] * y[3] * w[1] * w[2] * w[3]
    total_ops = sum(ops.values())
    x = models.make_input(g.tensors[g.inputs[0]].shape)
    m = Model(blob, lib=lib)
    xin = DeviceBuffer(x.nbytes, lib)
    xin.upload(x)
    m.bind_input(0, xin)
    m.set_profiling(True)
    for _ in range(warmup):
        m.run()
    m.reset_node_times()
    lib.spkv2_device_synchronize()
    for _ in range(steps):
        m.run()
    lib.spkv2_device_synchronize()
    m.set_profiling(False)
    eager_out = m.get_output(0)
    m.set_graph_mode(not eager)
    for _ in range(warmup):
        m.run()
    lib.spkv2_device_synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        m.run()
    lib.spkv2_device_synchronize()
    elapsed = time.perf_counter() - t0
    graph_same = bit_identical(m.get_output(0), eager_out)
    m.set_graph_mode(False)
    conv_ms = 0.0
    for nid in ops:
        ms, cnt = m.node_time(nid)
        conv_ms += ms / max(cnt, 1)
        if node_report:
            n = g.nodes[nid]
            xs_, ws_ = g.shape(n.inputs[0]), g.tensors[n.inputs[1]].shape
            t_ms = ms / max(cnt, 1)
            log(f"q8 node {nid:3d} {xs_[1]}x{xs_[2]}->{ws_[0]} k{ws_[2]} s{n.attrs['strides'][0]} "
                f"{m.kernel_name(nid):52s} {t_ms * 1e3:8.1f} us {ops[nid] / t_ms / 1e9:7.1f} TOP/s")
    m.close()
    xin.free()
    # roofline time basis as the fp32 headline's: the summed kernel-trace
    # durations of the conv launches per step from the committed summary
    k8 = pmc_traffic("conv_igemm_q8_resnet50_b64_kernel_stats.txt") if batch == 64 else None
    kms = k8.get("q8_conv_kernels_ms_per_run") if k8 else None
    t8 = pmc_traffic("conv_igemm_q8_resnet50_b64_traffic.txt") if batch == 64 else None
    traffic_b = t8.get("conv_hbm_bytes_per_step") if t8 else None
    basis_ms = kms if kms else conv_ms
    tops = total_ops / (basis_ms * 1e-3) / 1e12
    out = {"workload": "resnet50_int8_config_224", "batch": batch, "images_per_sec": batch * steps / elapsed,
           "ms_per_step": elapsed * 1e3 / steps, "timed_mode": "eager" if eager else "hip_graph",
           "graph_matches_eager": graph_same,
           "semantics": "BASELINE configs[4]: per-channel symmetric int8 weights, per-tensor asymmetric int8 "
                        "activations (min/max over 16 calibration batches), int8 tensors between nodes, int32 "
                        "accumulate, fixed-point requantize (round half away), fused Relu clamp; no reference "
                        "counterpart (checked against the oracle's restatement)",
           "conv_gop_per_image": total_ops / batch / 1e9,
           "roofline": {"bound": "mfma", "achieved": tops, "peak": INT8_MFMA_PEAK_TOPS, "unit": "TOP/s",
                        "frac": tops / INT8_MFMA_PEAK_TOPS, "traffic": traffic_b,
                        "kernel_ms_per_step": kms,
                        "basis": ("summed kernel-trace durations of the conv launches per step "
                                  "(profiles/conv_igemm_q8_resnet50_b64_kernel_stats.txt)" if kms
                                  else "HIP events around every conv node, eager pass (upper bound of the time)"),
                        "event_basis": {"conv_ms_per_step": conv_ms,
                                        "tops": total_ops / (conv_ms * 1e-3) / 1e12,
                                        "frac": total_ops / (conv_ms * 1e-3) / 1e12 / INT8_MFMA_PEAK_TOPS}},
           "hbm_frac_of_traffic": (traffic_b / (kms * 1e-3) / 1e9 / HBM_PEAK_GBPS) if traffic_b and kms else None}
    if b1_steps > 0:
        g1, blob1 = build(1)
        m1 = Model(blob1, lib=lib)
        x1 = models.make_input(g1.tensors[g1.inputs[0]].shape)
        b1 = DeviceBuffer(x1.nbytes, lib)
        b1.upload(x1)
        m1.bind_input(0, b1)
        m1.run()
        eager1 = m1.get_output(0)
        m1.set_graph_mode(not eager)
        for _ in range(5):
            m1.run()
        lib.spkv2_device_synchronize()
        t0 = time.perf_counter()
        for _ in range(b1_steps):
            m1.run()
        lib.spkv2_device_synchronize()
        out["b1_ms_per_image"] = (time.perf_counter() - t0) * 1e3 / b1_steps
        out["b1_graph_matches_eager"] = bit_identical(m1.get_output(0), eager1)
        m1.close()
        b1.free()
    return out


def yolo_v10n(lib, steps: int, node_report: bool = False, eager: bool = False, batches=(1, 16)) -> dict:
    """YOLOv10n-style detector at 640x640, batch 1 and
    16: images/s from HIP-graph replays of the node loop (the whole YOLO op
    set on the device: C2f Split/Concat, SPPF, PSA MatMul + Softmax, Resize,
    DFL Softmax, TopK, GatherElements), plus the node time by op type from an
    eager pass with per-node events."""
    from collections import defaultdict

    from spinnv2_amd.runtime import DeviceBuffer, Model
    from spinnv2_amd.spk import models, write_spk

    out = {"workload": "yolov10n_640"}
    for batch in batches:
        g = models.yolo_v10n(batch)
        m = Model(write_spk(g, "mi355x"), lib=lib)
        x = models.make_input(g.tensors[g.inputs[0]].shape)
        xb = DeviceBuffer(x.nbytes, lib)
        xb.upload(x)
        m.bind_input(0, xb)
        m.set_profiling(True)
        m.run()
        m.reset_node_times()
        for _ in range(3):
            m.run()
        lib.spkv2_device_synchronize()
        by_op = defaultdict(float)
        for n in g.nodes:
            ms, cnt = m.node_time(n.id)
            by_op[n.op_type] += ms / max(cnt, 1)
        m.set_profiling(False)
        m.set_graph_mode(not eager)
        for _ in range(3):
            m.run()
        lib.spkv2_device_synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            m.run()
        lib.spkv2_device_synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        m.set_graph_mode(False)
        out[f"b{batch}_ms_per_step"] = ms
        out[f"b{batch}_images_per_sec"] = batch * 1e3 / ms
        if batch == 16:
            out["node_ms_by_op_b16"] = {k: round(v, 4) for k, v in sorted(by_op.items(), key=lambda kv: -kv[1])}
        if node_report:
            for k, v in sorted(by_op.items(), key=lambda kv: -kv[1]):
                log(f"yolo b={batch} {k:20s} {v:8.3f} ms")
        m.close()
        xb.free()
    return out


# Memory-bound ops at ResNet / YOLO shapes: (label, single_op args, algorithmic bytes)
ELEMENTWISE = [
    ("maxpool_3x3s2_b64_64x112", ("MaxPool", [64, 64, 112, 112]), 4 * (64 * 64 * 112 * 112 + 64 * 64 * 56 * 56)),
    ("add_b64_256x56", ("Add", [64, 256, 56, 56]), 12 * 64 * 256 * 56 * 56),
    ("resize2x_b16_128x80", ("Resize", [16, 128, 80, 80]), 20 * 16 * 128 * 80 * 80),
    ("softmax_4096x1000", ("Softmax", [4096, 1000]), 8 * 4096 * 1000),
]


def elementwise(lib, reps: int = 20) -> dict:
    """Achieved HBM GB/s of the memory-bound kernels (device time from HIP
    events around the node), against the 8 TB/s peak; algorithmic bytes are
    each op's reads + writes, every element once."""
    from spinnv2_amd.runtime import Model
    from spinnv2_amd.spk import models, write_spk

    out = {}
    for label, (op, shape), nbytes in ELEMENTWISE:
        g = models.single_op(op, shape)
        m = Model(write_spk(g, "mi355x"), lib=lib)
        for i, t in enumerate(g.inputs):
            m.set_input(i, models.make_input(g.tensors[t].shape, 7 + i))
        m.run()
        m.set_profiling(True)
        m.reset_node_times()
        for _ in range(reps):
            m.run()
        lib.spkv2_device_synchronize()
        ms, cnt = m.node_time(g.nodes[0].id)
        us = ms / max(cnt, 1) * 1e3
        gbps = nbytes / (us * 1e-6) / 1e9
        out[label] = {"kernel": m.kernel_name(g.nodes[0].id), "us": us, "gbps": gbps,
                      "frac": gbps / HBM_PEAK_GBPS, "bytes": nbytes}
        m.close()
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--depth", type=int, default=101)
    ap.add_argument("--b1-steps", type=int, default=50)
    ap.add_argument("--eager", action="store_true",
                    help="time every section without HIP-graph replay (for kernel tracing)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--node-report", action="store_true", help="print per-node device times to stderr")
    ap.add_argument("--no-host-io", action="store_true", help="skip the host-buffer (PCIe) pass")
    ap.add_argument("--no-int8", action="store_true", help="skip the INT8 ResNet-50 section")
    ap.add_argument("--int8-only", action="store_true", help="run only the INT8 ResNet-50 section")
    ap.add_argument("--int8-config-only", action="store_true",
                    help="run only the INT8 ResNet-50 section in BASELINE configs[4]'s own semantics")
    ap.add_argument("--no-int8-config", action="store_true", help="skip the INT8 configuration-semantics section")
    ap.add_argument("--no-elementwise", action="store_true", help="skip the memory-bound op section")
    ap.add_argument("--no-yolo", action="store_true", help="skip the YOLOv10n section")
    ap.add_argument("--yolo-only", action="store_true", help="run only the YOLOv10n section")
    ap.add_argument("--yolo-batch", type=int, choices=(1, 16), default=None,
                    help="with --yolo-only: only this batch (a profile of one shape)")
    ap.add_argument("--elementwise-only", action="store_true", help="run only the memory-bound op section")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="only compare fp32 GEMM rates with the vendor library (torch.matmul) on ResNet shapes")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="only run the plain copy kernel over this many MiB (PMC counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build targets a single MI355X); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration_mib:
        copy_calibration(args.copy_calibration_mib, args.steps)
        return
    if args.vendor_gemm:
        print(json.dumps(vendor_gemm(max(args.steps, 20))), flush=True)
        return

    from spinnv2_amd.runtime import DeviceBuffer, Model, load_library
    from spinnv2_amd.spk import models, write_spk

    lib = load_library()
    if args.elementwise_only:
        print(json.dumps(elementwise(lib)), flush=True)
        return
    if args.yolo_only:
        batches = (args.yolo_batch,) if args.yolo_batch else (1, 16)
        print(json.dumps(yolo_v10n(lib, max(args.steps, 10), args.node_report, args.eager, batches)), flush=True)
        return
    if args.int8_config_only:
        print(json.dumps(int8_config_mode(lib, args.steps, args.warmup, args.b1_steps, args.batch, args.node_report,
                                          args.eager)), flush=True)
        return
    if args.int8_only:
        print(json.dumps(int8_resnet50(lib, args.steps, args.warmup, args.b1_steps, args.batch, args.node_report,
                                       args.eager)), flush=True)
        return
    base, base_simd = (None, None) if args.no_cpu_baseline else cpu_baseline()

    # ---------------------------------------------------------- batch B
    t0 = time.time()
    g = models.resnet(args.depth, args.batch)
    blob = write_spk(g, "mi355x")
    conv_nodes = [n.id for n in g.nodes if n.op_type == "Conv"]
    flops_per_node = {}
    for n in g.nodes:
        if n.op_type == "Conv":
            y = g.shape(n.outputs[0])
            w = g.tensors[n.inputs[1]].shape
            flops_per_node[n.id] = 2 * y[0] * y[1] * y[2] * y[3] * w[1] * w[2] * w[3]
    conv_flops = sum(flops_per_node.values())
    # minimum HBM bytes of the conv nodes: weights + input + output (+ residual) read/written once
    conv_alg_bytes = 0
    for n in g.nodes:
        if n.op_type == "Conv":
            conv_alg_bytes += 4 * sum(int(np.prod(g.tensors[t].shape)) for t in n.inputs)
            conv_alg_bytes += 4 * int(np.prod(g.shape(n.outputs[0])))
    traffic = pmc_traffic()
    x = models.make_input(g.tensors[g.inputs[0]].shape)
    log(f"resnet{args.depth} b={args.batch}: package {len(blob) / 1e6:.1f} MB built in {time.time() - t0:.1f}s")

    t0 = time.time()
    m = Model(blob, lib=lib)
    log(f"load + prepare (weights upload, tile tuning) {time.time() - t0:.2f}s")
    xin = DeviceBuffer(x.nbytes, lib)
    xin.upload(x)
    m.bind_input(0, xin)
    # per-node device times (HIP events around every node on the run stream)
    # for the roofline: an eager pass of its own, so the events stay out of
    # the timed region below
    m.set_profiling(True)
    for _ in range(args.warmup):
        m.run()
    m.reset_node_times()
    lib.spkv2_device_synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        m.run()
    lib.spkv2_device_synchronize()
    profiled_elapsed = time.perf_counter() - t0
    m.set_profiling(False)
    eager_logits = m.get_output(0)
    # the timed region: the node loop captured once into a HIP graph (during
    # warmup) and replayed, input resident in HBM
    if not args.eager:
        m.set_graph_mode(True)
    for _ in range(args.warmup):
        m.run()
    lib.spkv2_device_synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        m.run()
    lib.spkv2_device_synchronize()
    elapsed = time.perf_counter() - t0
    logits = m.get_output(0)
    graph_same = bit_identical(logits, eager_logits)
    m.set_graph_mode(False)
    logits = logits.reshape(args.batch, -1)
    # host-buffer interface (spkv2_set_input / spkv2_get_output copy over PCIe
    # each step): reported beside, never as, the value
    pcie_ips = None
    if not args.no_host_io:
        pcie_steps = max(1, min(args.steps, 5))
        t0 = time.perf_counter()
        for _ in range(pcie_steps):
            m.set_input(0, x)
            m.run()
            m.get_output(0)
        pcie_ips = args.batch * pcie_steps / (time.perf_counter() - t0)
        m.bind_input(0, xin)
    conv_ms = 0.0
    node_ms = {}
    for nid in range(len(g.nodes)):
        ms, cnt = m.node_time(nid)
        node_ms[nid] = ms / max(cnt, 1)
        if nid in flops_per_node:
            conv_ms += node_ms[nid]
    total_node_ms = sum(node_ms.values())
    if args.node_report:
        for nid, ms in node_ms.items():
            n = g.nodes[nid]
            extra = ""
            if nid in flops_per_node:
                extra = f" {flops_per_node[nid] / ms / 1e9:.1f} TFLOP/s"
            log(f"node {nid:3d} {n.op_type:18s} {m.kernel_name(nid):44s} {ms:8.3f} ms{extra}")
    m.close()
    xin.free()
    ms_per_step = elapsed * 1e3 / args.steps
    conv_tflops = conv_flops / (conv_ms * 1e-3) / 1e12
    # Roofline time basis: the summed kernel-trace durations of every launch
    # of the conv nodes (GEMM, split-K epilogue, padding) per step, from the
    # committed rocprofv3 summary of this workload, so the fraction
    # reproduces from profiles/.  Beside it, two live figures of this run:
    # per-node HIP events (event overhead and launch gaps inside the node:
    # an upper bound of the conv time) and the whole timed graph step (every
    # kernel of the network: a looser upper bound).
    kstats = (pmc_traffic("conv_igemm_f32_resnet101_b64_kernel_stats.txt")
              if (args.depth, args.batch) == (101, 64) else None)
    trace_ms = kstats.get("conv_kernels_ms_per_run") if kstats else None
    roof_tflops = conv_flops / (trace_ms * 1e-3) / 1e12 if trace_ms else conv_tflops

    # ---------------------------------------------------------- batch 1
    b1_ms, b1_same = batch1_latency(args.depth, args.b1_steps, lib, args.eager) if args.b1_steps > 0 else (None, None)

    int8 = None if args.no_int8 else int8_resnet50(lib, args.steps, args.warmup, args.b1_steps, eager=args.eager)
    int8_cfg = (None if args.no_int8_config
                else int8_config_mode(lib, args.steps, args.warmup, args.b1_steps, eager=args.eager))
    ew = None if args.no_elementwise else elementwise(lib)
    yolo = None if args.no_yolo else yolo_v10n(lib, max(args.steps, 10), eager=args.eager)

    result = {
        "metric": "ResNet-101 224^2 images/sec (b=64); conv TFLOP/s as % of fp32 MFMA peak",
        "value": args.batch * args.steps / elapsed,
        "unit": "images/sec",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) input, random-init He-normal weights, BN folded (seed 42)",
        "config": {"workload": f"resnet{args.depth}_fp32_224", "batch": args.batch, "image": 224,
                   "conv_gflop_per_image": conv_flops / args.batch / 1e9, "conv_nodes": len(conv_nodes),
                   "parallelism": "single GPU"},
        "timed_mode": "eager" if args.eager else "hip_graph",
        "profiled_eager_images_per_sec": args.batch * args.steps / profiled_elapsed,
        "host_io_images_per_sec": pcie_ips,
        "b1_ms_per_image": b1_ms,
        "b1_images_per_sec": 1e3 / b1_ms if b1_ms else None,
        "conv_ms_per_step": conv_ms,
        "node_ms_per_step": total_node_ms,
        "graph_matches_eager": graph_same,
        "b1_graph_matches_eager": b1_same,
        "roofline": {"bound": "mfma", "achieved": roof_tflops, "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": roof_tflops / FP32_MFMA_PEAK_TFLOPS,
                     "basis": ("summed kernel-trace durations of the conv nodes' launches per step "
                               "(profiles/conv_igemm_f32_resnet101_b64_kernel_stats.txt, result conv_kernels_ms_per_run)"
                               if trace_ms else "HIP events around every conv node (no committed trace for this shape)"),
                     "kernel_ms_per_step": trace_ms,
                     "event_basis": {"conv_ms_per_step": conv_ms, "tflops": conv_tflops,
                                     "frac": conv_tflops / FP32_MFMA_PEAK_TFLOPS,
                                     "note": "HIP events per node, eager pass of this run: an upper bound of the time"},
                     "step_basis": {"ms_per_step": ms_per_step,
                                    "tflops": conv_flops / (ms_per_step * 1e-3) / 1e12,
                                    "frac": conv_flops / (ms_per_step * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS,
                                    "note": "conv FLOP over the whole timed graph step (all kernels)"},
                     "traffic": traffic.get("conv_hbm_bytes_per_step") if traffic else None,
                     "traffic_basis": "HBM bytes of all conv launches of one step (rocprofv3 FETCH_SIZE + "
                                      "WRITE_SIZE, copy-kernel scaled; profiles/)" if traffic else None,
                     "algorithmic_bytes": conv_alg_bytes,
                     "kernel": "conv_igemm_f32 (all conv nodes)"},
        "cpu_baseline": base,
        "cpu_baseline_simd": base_simd,
        "int8": int8,
        "int8_config_mode": int8_cfg,
        "elementwise": ew,
        "yolo": yolo,
        "top1_image0": int(logits[0].argmax()),
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
