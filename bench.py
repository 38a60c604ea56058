#!/usr/bin/env python3
"""Talker decode-step benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu-baseline]

A "step" is one Talker decode step of the resident greedy loop (28 layers + final norm
+ codec head + greedy code0 + next-embedding gather), all inputs resident in HBM.
Default workload = the north-star target: 1.7B-shape Talker, int8 per-row weights,
batch 1, KV cache holding 2048 positions (seeded synthetic bf16 K/V uploaded through
the library's upload_kv, as the reference does after its CPU prefill), then W warmup
and K timed greedy steps, each run as ONE launch of the fused step kernel.  Weights
are seeded random-init N(0, 0.02) (no checkpoints offline), quantized on the device
by the library's bit-exact int8 quantizer.

Prints ONE JSON line (metric/unit from BASELINE.json).  The timed region is bracketed
by hipDeviceSynchronize and measured with HIP events recorded on the library's stream.
The roofline object is for the dominant (only) kernel of the timed region, the fused
decode step: algorithmic bytes of the K steps of one launch / that launch's duration.
With W == K the two launches rocprof sees have the same length, so its average kernel
duration is comparable with the HIP-event figure.  kernels_us times the unfused
per-kernel path (diagnostic).  cpu_baseline times the reference engine's own
qwen_talker_step (built from its sources into oracle/_ref) on the host cores.
"""
from __future__ import annotations

import argparse
import ctypes as C
import hashlib
import importlib.util
import json
import os
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0


def _pkg():
    pdir = os.path.join(ROOT, "qwen3-tts_amd")
    spec = importlib.util.spec_from_file_location("qwen3_tts_amd", os.path.join(pdir, "__init__.py"),
                                                  submodule_search_locations=[pdir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["qwen3_tts_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class HipEvents:
    """hipEvent timing on an arbitrary stream (the library's, not torch's)."""

    def __init__(self):
        self.rt = C.CDLL("libamdhip64.so")
        self.rt.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.rt.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.rt.hipEventSynchronize.argtypes = [C.c_void_p]
        self.rt.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.rt.hipDeviceSynchronize.argtypes = []

    def event(self):
        e = C.c_void_p()
        assert self.rt.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.rt.hipEventRecord(e, stream) == 0

    def elapsed_ms(self, a, b):
        assert self.rt.hipEventSynchronize(b) == 0
        ms = C.c_float()
        assert self.rt.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return ms.value

    def device_sync(self):
        assert self.rt.hipDeviceSynchronize() == 0


DEFAULT_WORKLOAD = "talker-1.7B-int8-b1-L2048"
# fused kernel kinds (qwen_hip_talker_fused_kernel): label, the sources that define it
FUSED_KERNELS = {
    2: ("ps::{ns}::k_rstep role-specialised fused decode step ({prec})",
        ("qt_rstep.hip", "qt_step_common.h", "qt_attn_mf.h", "qt_device.h")),
    1: ("ps::k_pstep<{prec}> fused decode step", ("qt_pstep.hip", "qt_step_common.h", "qt_attn_mf.h", "qt_device.h")),
}


def fused_label(L, g, prec, hidden):
    """Name of the kernel that runs the state's fused step (qt_rstep.hip is built per geometry
    and weight type: ps::rs for hidden 2048 int8, ps::rs4 for hidden 2048 q4_0, ps::rs06 for
    hidden 1024 int8, ps::rs06b for hidden 1024 bf16)."""
    kind = L.qwen_hip_talker_fused_kernel(g.h)
    ns = ("rs4" if prec == "int4" else "rs") if hidden == 2048 else ("rs06b" if prec == "bf16" else "rs06")
    return kind, FUSED_KERNELS.get(kind, ("unfused per-kernel path",))[0].format(prec=prec, ns=ns)


def kernel_source_sha256(kind):
    h = hashlib.sha256()
    for f in FUSED_KERNELS[kind][1]:
        with open(os.path.join(ROOT, "qwen3-tts_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


def refuse_if_device_error(L, g, workload):
    """The fused kernels' waits are bounded: one that gives up sets the device error flag
    and the remaining steps end early, so a launch with the flag set must not be timed."""
    if L.qwen_hip_talker_sync(g.h) != 0:
        msg = L.qwen_hip_last_error().decode(errors="replace")
        print(json.dumps({"error": f"{workload}: the timed launch failed: {msg}", "value": None}), flush=True)
        sys.exit(1)


# BASELINE configs 1-5 as short runs of their workloads (each in a child process, before the
# headline's own measurement): (key, workload, extra arguments); config 4 also in int8 (the
# one-launch CP frame)
CONFIG_RUNS = [
    ("1_0.6B_bf16_L256", "talker-0.6B-bf16-b1-L256", ["--steps", "256", "--warmup", "16"]),
    ("2_0.6B_int8_grow0-2048", "talker-0.6B-int8-grow2048", []),
    ("3_1.7B_q4_0_L512", "talker-1.7B-int4-b1-L512", ["--steps", "32", "--warmup", "8"]),
    ("3_1.7B_q4_0_L2048", "talker-1.7B-int4-b1-L2048", ["--steps", "32", "--warmup", "8"]),
    ("3_1.7B_q4_0_L4096", "talker-1.7B-int4-b1-L4096", ["--steps", "32", "--warmup", "8"]),
    ("4_cp_0.6B_bf16_frame", "cp-0.6B-bf16-frame", ["--steps", "100", "--warmup", "10"]),
    ("4_cp_0.6B_int8_frame", "cp-0.6B-int8-frame", ["--steps", "100", "--warmup", "10"]),
    ("5_1.7B_int8_b32_ragged", "talker-1.7B-int8-b32-ragged", ["--steps", "16", "--warmup", "4"]),
]


def run_configs():
    res = {}
    for key, wl, extra in CONFIG_RUNS:
        cmd = [sys.executable, os.path.abspath(__file__), "--workload", wl, "--no-cpu-baseline", "--no-configs",
               "--kernel-launches", "0", *extra]
        t0 = time.time()
        try:
            p = subprocess.run(cmd, capture_output=True, text=True, timeout=240)
            lines = [x for x in p.stdout.splitlines() if x.startswith("{")]
            if not lines:
                raise RuntimeError(f"exit {p.returncode}: " + " | ".join(p.stderr.strip().splitlines()[-3:]))
            r = json.loads(lines[-1])
            res[key] = {"workload": wl, "value": r.get("value"), "unit": r.get("unit"),
                        "roofline_frac": (r.get("roofline") or {}).get("frac"), "steps": r.get("steps"),
                        "wall_s": round(time.time() - t0, 1)}
            if "error" in r:
                res[key]["error"] = r["error"]
        except Exception as ex:  # one config's failure is reported, not fatal to the line
            res[key] = {"workload": wl, "value": None, "error": str(ex)[:200], "wall_s": round(time.time() - t0, 1)}
        log(f"[bench] config {key}: {res[key]}")
    return res


WORKLOADS = {
    # name: (shape, precision, prefill L, default timed steps)
    "talker-1.7B-int8-b1-L2048": ("1.7B", "int8", 2048, 64),
    "talker-0.6B-int8-b1-L2048": ("0.6B", "int8", 2048, 64),
    "talker-0.6B-bf16-b1-L256": ("0.6B", "bf16", 256, 256),
    "talker-1.7B-int4-b1-L512": ("1.7B", "int4", 512, 64),
    "talker-1.7B-int4-b1-L2048": ("1.7B", "int4", 2048, 64),
    "talker-1.7B-int4-b1-L4096": ("1.7B", "int4", 4096, 64),
}
# KV grown from 0 over the timed steps (config 2): (shape, precision, total steps, steps per launch)
GROW_WORKLOADS = {
    "talker-0.6B-int8-grow2048": ("0.6B", "int8", 2048, 256),
}
# Code Predictor frames: (shape, precision, default timed frames, two-position prefill)
CP_WORKLOADS = {
    "cp-0.6B-bf16-frame": ("0.6B", "bf16", 500, False),
    "cp-0.6B-int8-frame": ("0.6B", "int8", 500, False),
    "cp-0.6B-int8-frame-prefill2": ("0.6B", "int8", 500, True),
}
# the Code Predictor's batched pass (qwen_hip_cp_batch_step): (shape, precision, streams)
CP_BATCH_WORKLOADS = {
    "cp-0.6B-int8-b32": ("0.6B", "int8", 32),
    "cp-0.6B-bf16-b32": ("0.6B", "bf16", 32),
}
# Talker prefill of S positions (qwen_talker_prefill): (shape, decode precision, S, default timed prefills)
PREFILL_WORKLOADS = {
    "talker-1.7B-prefill-S128": ("1.7B", "int8", 128, 20),
    "talker-1.7B-prefill-S512": ("1.7B", "int8", 512, 8),
}
BF16_MFMA_PEAK_TFS = 2500.0
# the device frame loop with the reference's default sampling (temperature 0.9, top-k 50,
# repetition penalty 1.05): (shape, precision, prefill L, default timed steps)
SAMPLED_WORKLOADS = {
    "talker-1.7B-int8-b1-L2048-sampled": ("1.7B", "int8", 2048, 64),
}
# the whole frame loop on the device (qwen_hip_generate: code0 sampling, CP frame, next
# input, Talker step) at the reference's defaults: (shape, precision, prefill L, frames)
FRAME_WORKLOADS = {
    "frame-0.6B-bf16-sampled": ("0.6B", "bf16", 256, 64),
    "frame-0.6B-int8-sampled": ("0.6B", "int8", 256, 64),
    "frame-1.7B-int8-sampled": ("1.7B", "int8", 2048, 64),
}
# the speech decoder (codes -> 24 kHz audio, one-shot): (frames per decode, default timed decodes)
SD_WORKLOADS = {
    "sd-decode-125frames": (125, 10),
}
# the speech decoder's exact streaming decode: (frames per stream, frames per chunk, timed streams)
SD_STREAM_WORKLOADS = {
    "sd-stream-125frames-chunk10": (125, 10, 5),
}
F32_MFMA_PEAK_TFS = 157.3
# batched workloads: (shape, precision, streams, KV length range, default timed steps)
BATCH_WORKLOADS = {
    "talker-1.7B-int8-b32-ragged": ("1.7B", "int8", 32, (128, 4096), 16),
    "talker-1.7B-int4-b32-ragged": ("1.7B", "int4", 32, (128, 4096), 16),
    "talker-1.7B-bf16-b32-ragged": ("1.7B", "bf16", 32, (128, 4096), 16),
}


def weight_bytes(shape, prec):
    """Algorithmic weight bytes per step: every layer matrix once (+ int8 row scales,
    q4 f16 block scales), norms, final norm."""
    s = shape
    mats = [(s.q_dim + 2 * s.kv_dim, s.hidden), (s.hidden, s.q_dim), (2 * s.inter, s.hidden), (s.hidden, s.inter)]
    per = 0
    for r, c in mats:
        if prec == "bf16":
            per += r * c * 2
        elif prec == "int8":
            per += r * c + 4 * r
        else:
            per += r * c // 2 + 2 * r * (c // 32)
    norms = (2 * s.hidden + 2 * s.head_dim) * 4
    return s.layers * (per + norms) + s.hidden * 4


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS) + sorted(BATCH_WORKLOADS) + sorted(CP_WORKLOADS)
                    + sorted(PREFILL_WORKLOADS) + sorted(GROW_WORKLOADS) + sorted(SAMPLED_WORKLOADS)
                    + sorted(FRAME_WORKLOADS) + sorted(SD_WORKLOADS) + sorted(SD_STREAM_WORKLOADS)
                    + sorted(CP_BATCH_WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the short runs of BASELINE configs 1-5 that the default workload's line carries")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--kernel-launches", type=int, default=200)
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="before the timed region, one device-to-device copy of this many MiB (a kernel of "
                         "known HBM traffic, to scale rocprofv3 FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the decode path shards as independent "
                                   "data-parallel streams with no exchange between GPUs; run --gpus 1"}))
        sys.exit(2)

    # the config runs go first, each in a child process, while this process has not touched
    # the GPU: a cooperative launch holds the device's global wave-sync resource until its
    # process ends, so a child could not launch its own persistent kernel after ours
    configs = run_configs() if (not args.no_configs and args.workload == DEFAULT_WORKLOAD) else None
    _pkg()
    if args.workload in BATCH_WORKLOADS:
        return bench_batch(args)
    if args.workload in CP_WORKLOADS:
        return bench_cp(args)
    if args.workload in CP_BATCH_WORKLOADS:
        return bench_cp_batch(args)
    if args.workload in PREFILL_WORKLOADS:
        return bench_prefill(args)
    if args.workload in GROW_WORKLOADS:
        return bench_grow(args)
    if args.workload in SAMPLED_WORKLOADS:
        return bench_sampled(args)
    if args.workload in FRAME_WORKLOADS:
        return bench_frames(args)
    if args.workload in SD_WORKLOADS:
        return bench_sd(args)
    if args.workload in SD_STREAM_WORKLOADS:
        return bench_sd_stream(args)
    from qwen3_tts_amd import hip, synth
    shape_name, prec, Lpre, dsteps = WORKLOADS[args.workload]
    K = args.steps or dsteps
    W = K if args.warmup is None else args.warmup
    s = synth.SHAPES[shape_name]
    kv_max = max(4096, Lpre + K + W + 8)
    seed = 0x5EED0001

    t0 = time.time()
    only = lambda n: not n.startswith("talker.code_predictor.")  # noqa: E731
    tens = synth.generate(s, seed, 0.0, threads=int(os.environ.get("OMP_NUM_THREADS", "16")), only=only)
    log(f"[bench] generated {shape_name} weights in {time.time() - t0:.1f}s")
    layers = hip.layers_from_tensors(tens, s)
    cos, sin = synth.rope_tables(s.head_dim, s.rope_theta, kv_max)
    fnorm = synth.bf16_to_f32(tens["talker.model.norm.weight"])
    t0 = time.time()
    g = hip.Talker(s, layers, fnorm, cos, sin, hip.BF16, kv_max, quantize_to=hip.PREC[prec])
    log(f"[bench] device init + quantize ({prec}) {time.time() - t0:.1f}s")
    head = np.ascontiguousarray(tens["talker.codec_head.weight"])
    emb = np.ascontiguousarray(tens["talker.model.codec_embedding.weight"])
    L = hip.lib()
    ev = HipEvents()
    stream = L.qwen_hip_talker_stream(g.h)

    # KV cache: Lpre positions of seeded synthetic bf16 K/V (values do not change timing),
    # handed over with upload_kv from pageable host memory (the reference's hand-off after
    # its CPU prefill); the upload alone is timed
    rng = np.random.default_rng(0x5EED0002)
    kv_upload = None
    if Lpre > 0:
        kvk = synth.f32_to_bf16_rne(rng.normal(0, 1.0, (s.layers, Lpre, s.kv_dim)).astype(np.float32))
        kvv = synth.f32_to_bf16_rne(rng.normal(0, 0.1, (s.layers, Lpre, s.kv_dim)).astype(np.float32))
        # the first hand-off after init, then a second one of the same bytes (a state
        # serving its next utterance)
        dts = []
        for _ in range(2):
            t0 = time.perf_counter()
            hip.check(L.qwen_hip_talker_upload_kv(g.h, kvk.ctypes.data, kvv.ctypes.data, Lpre, Lpre), "upload_kv")
            dts.append(time.perf_counter() - t0)
        nb = kvk.nbytes + kvv.nbytes
        kv_upload = {"positions": Lpre, "bytes": int(nb), "ms": round(dts[0] * 1e3, 2), "gbs": round(nb / dts[0] / 1e9, 2),
                     "ms_next": round(dts[1] * 1e3, 2), "gbs_next": round(nb / dts[1] / 1e9, 2),
                     "source": "pageable host memory"}
        log(f"[bench] upload_kv of {Lpre} positions ({nb / 1e6:.0f} MB): {dts[0] * 1e3:.1f} ms, "
            f"{kv_upload['gbs']:.1f} GB/s (next call {dts[1] * 1e3:.1f} ms, {kv_upload['gbs_next']:.1f} GB/s)")
        del kvk, kvv
    e0 = synth.bf16_to_f32(emb[1234])
    g.greedy(head, emb, e0, Lpre, 0, 0)     # set up the greedy loop at position Lpre (no steps)

    if args.calib_copy_mb > 0:
        nbytes = args.calib_copy_mb << 20
        src, dst = C.c_void_p(), C.c_void_p()
        ev.rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        ev.rt.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
        ev.rt.hipFree.argtypes = [C.c_void_p]
        assert ev.rt.hipMalloc(C.byref(src), nbytes) == 0 and ev.rt.hipMalloc(C.byref(dst), nbytes) == 0
        assert ev.rt.hipMemcpyAsync(dst, src, nbytes, 3, stream) == 0      # hipMemcpyDeviceToDevice
        ev.device_sync()
        ev.rt.hipFree(src); ev.rt.hipFree(dst)
        log(f"[bench] calibration copy: {args.calib_copy_mb} MiB device to device")

    # warmup, then the loop re-seeded at position Lpre (the warmup's rows past Lpre are
    # rewritten before they are read), then exactly K timed steps over KV Lpre .. Lpre+K
    hip.check(L.qwen_hip_talker_greedy_async(g.h, W), "warmup")
    hip.check(L.qwen_hip_talker_sync(g.h), "sync")
    g.greedy(head, emb, e0, Lpre, 0, 0)
    ev.device_sync()
    a, b = ev.event(), ev.event()
    ev.record(a, stream)
    hip.check(L.qwen_hip_talker_greedy_async(g.h, K), "timed steps")
    ev.record(b, stream)
    ms_total = ev.elapsed_ms(a, b)
    ev.device_sync()
    refuse_if_device_error(L, g, args.workload)
    ms = ms_total / K
    L_mid = Lpre + K / 2.0
    kv_bytes = 2 * s.layers * s.kv_dim * 2       # per position, K and V
    step_bytes = weight_bytes(s, prec) + kv_bytes * (L_mid + 1) + s.codec_vocab * s.hidden * 2
    step_gbs = step_bytes / (ms * 1e-3) / 1e9
    log(f"[bench] {K} steps: {ms * 1e3:.1f} us/step, {step_gbs:.0f} GB/s algorithmic "
        f"({100 * step_gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s)")

    # per-kernel averages (HIP events over repeated launches on the same stream)
    kern = {}
    names = ["qkv", "attn", "o_proj", "gate_up", "down", "final_norm"]
    n = args.kernel_launches
    for kid, nm in enumerate(names if n > 0 else []):
        hip.check(L.qwen_hip_talker_launch_kernel(g.h, kid, 0, 10), "kernel warmup")
        ev.record(a, stream)
        hip.check(L.qwen_hip_talker_launch_kernel(g.h, kid, 0, n), "kernel launches")
        ev.record(b, stream)
        kern[nm] = ev.elapsed_ms(a, b) * 1e3 / n
    if kern:
        log("[bench] per-kernel avg us: " + ", ".join(f"{k}={v:.2f}" for k, v in kern.items()))
    kind, klabel = fused_label(L, g, prec, s.hidden)
    roofline = {"bound": "hbm", "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(step_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": klabel,
                "bytes_per_launch": int(step_bytes * K), "avg_us": round(ms_total * 1e3, 1),
                "steps_per_launch": K}
    # HBM bytes per launch from the committed rocprofv3 PMC passes for this workload: the
    # measured bytes per step at the profiled mean KV length, moved to this run's mean KV
    # length by the K/V bytes of the difference, times K.  Only while the kernel's sources
    # are the ones profiled (their sha256 is recorded with the counters): otherwise null.
    try:
        t = json.load(open(os.path.join(ROOT, "profiles", "fused_step_traffic.json")))
        if kind in FUSED_KERNELS and t["workload"] == args.workload and t["kernel"] == klabel:
            if t["source_sha256"] == kernel_source_sha256(kind):
                per_step = t["traffic_bytes_per_step"] + kv_bytes * (L_mid - t["kv_len_mid"])
                roofline["traffic"] = int(per_step * K)
                roofline["traffic_source"] = t["source"]
            else:
                roofline["traffic_stale"] = "the kernel's sources changed since the committed counter passes"
    except (OSError, ValueError, KeyError):
        pass

    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline(s, prec, g, Lpre, tens, args.cpu_seconds)
        except Exception as ex:  # the GPU number stands on its own; report why there is none
            log(f"[bench] cpu baseline failed: {ex}")
            cpu = {"value": None, "unit": "ms/step", "error": str(ex)[:200]}
    g.free()

    out = {
        "metric": "Talker ms/decode-step (0.6B/1.7B, bf16/int8/int4) + achieved HBM GB/s",
        "value": round(ms, 4), "unit": "ms/step", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": prec if prec != "int4" else "q4_0", "data": "synthetic (seeded N(0,0.02) random-init weights)",
        "config": {"workload": args.workload, "batch": 1, "kv_len_start": Lpre, "kv_len_end": Lpre + K,
                   "layers": s.layers, "hidden": s.hidden, "inter": s.inter},
        "tokens_per_s": round(1000.0 / ms, 1),
        "step_bytes": int(step_bytes), "step_hbm_gbs": round(step_gbs, 1),
        "step_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "kernels_us": {k: round(v, 3) for k, v in kern.items()},
        "kv_upload": kv_upload,
        "roofline": roofline, "cpu_baseline": cpu,
    }
    if configs is not None:
        out["configs"] = configs
    print(json.dumps(out), flush=True)


def bench_batch(args):
    """Config 5: B concurrent 1.7B streams on one GPU, each stream's KV length drawn
    uniform in [lo, hi] from a seed (ragged), weights read once per step for all streams
    (int8 / q4_0: MFMA over exact int8 activation pieces; bf16: MFMA over exact bf16
    planes), attention over every stream's own cache.  A step = one batched step
    of all B streams; value = ms per batched step (device-resident inputs, positions
    advancing on the device), tokens_per_s = B / step time.  The KV contents are zeros
    beyond what the steps write (attention reads every byte regardless of value)."""
    from qwen3_tts_amd import hip, synth
    shape_name, prec, B, (lo, hi), dsteps = BATCH_WORKLOADS[args.workload]
    K = args.steps or dsteps
    W = 4 if args.warmup is None else args.warmup
    s = synth.SHAPES[shape_name]
    kv_max = hi + K + W + 16
    rng = np.random.default_rng(0x5EED0002)
    lens = rng.integers(lo, hi + 1, B).astype(np.int32)
    t0 = time.time()
    only = lambda n: n.startswith("talker.model.")  # noqa: E731
    tens = synth.generate(s, 0x5EED0001, 0.0, threads=int(os.environ.get("OMP_NUM_THREADS", "16")), only=only)
    layers = hip.layers_from_tensors(tens, s)
    cos, sin = synth.rope_tables(s.head_dim, s.rope_theta, kv_max)
    fnorm = synth.bf16_to_f32(tens["talker.model.norm.weight"])
    g = hip.Talker(s, layers, fnorm, cos, sin, hip.BF16, kv_max, quantize_to=hip.PREC[prec])
    del layers
    bt = hip.TalkerBatch(g, B)
    log(f"[bench] batch: {B} streams, KV lengths {lens.min()}..{lens.max()} (mean {lens.mean():.0f}), "
        f"init {time.time() - t0:.1f}s")
    emb = tens["talker.model.codec_embedding.weight"]
    E = np.stack([synth.bf16_to_f32(emb[(17 * b + 5) % 2048]) for b in range(B)])
    bt.step(E, lens)                                   # captures the step graph; positions lens+1 after
    L = hip.lib()
    ev = HipEvents()
    stream = L.qwen_hip_talker_batch_stream(bt.h)
    hip.check(L.qwen_hip_talker_batch_step_async(bt.h, W), "batch warmup")
    hip.check(L.qwen_hip_talker_batch_sync(bt.h), "sync")
    ev.device_sync()
    a, b_ = ev.event(), ev.event()
    ev.record(a, stream)
    hip.check(L.qwen_hip_talker_batch_step_async(bt.h, K), "batch timed")
    ev.record(b_, stream)
    ms_total = ev.elapsed_ms(a, b_)
    ev.device_sync()
    ms = ms_total / K
    kv_bytes = 2 * s.layers * s.kv_dim * 2
    mid = lens.astype(np.float64) + 1 + W + K / 2.0        # mean position of the timed steps
    step_bytes = weight_bytes(s, prec) + kv_bytes * float((mid + 1).sum())
    gbs = step_bytes / (ms * 1e-3) / 1e9
    log(f"[bench] batch: {ms * 1e3:.1f} us/step, {B / ms * 1e3:.0f} tokens/s, {gbs:.0f} GB/s algorithmic")
    bt.free()
    g.free()
    out = {
        "metric": "Talker ms/decode-step (0.6B/1.7B, bf16/int8/int4) + achieved HBM GB/s",
        "value": round(ms, 4), "unit": "ms/step", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": prec, "data": "synthetic (seeded N(0,0.02) random-init weights; zero-filled KV of ragged lengths)",
        "config": {"workload": args.workload, "batch": B, "kv_len_min": int(lens.min()), "kv_len_max": int(lens.max()),
                   "kv_len_mean": round(float(lens.mean()), 1), "layers": s.layers, "hidden": s.hidden, "inter": s.inter},
        "tokens_per_s": round(B * 1000.0 / ms, 1), "step_bytes": int(step_bytes), "step_hbm_gbs": round(gbs, 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": f"batched step (MFMA {prec} GEMMs + ragged split-K attention), whole step",
                     "bytes_per_launch": int(step_bytes), "avg_us": round(ms * 1e3, 1), "steps_per_launch": 1},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def bench_grow(args):
    """Config 2: the greedy decode with the KV cache grown from 0 to N positions over N
    steps (no upload), as N / seg launches of seg steps each, every launch timed with HIP
    events; reports ms/step per KV-length segment and the mean over all N steps (value).
    A 16-step launch from position 0 runs first (untimed) and the loop is re-seeded at 0."""
    from qwen3_tts_amd import hip, synth
    shape_name, prec, N, seg = GROW_WORKLOADS[args.workload]
    s = synth.SHAPES[shape_name]
    kv_max = N + 64
    only = lambda n: not n.startswith("talker.code_predictor.")  # noqa: E731
    tens = synth.generate(s, 0x5EED0001, 0.0, threads=int(os.environ.get("OMP_NUM_THREADS", "16")), only=only)
    layers = hip.layers_from_tensors(tens, s)
    cos, sin = synth.rope_tables(s.head_dim, s.rope_theta, kv_max)
    fnorm = synth.bf16_to_f32(tens["talker.model.norm.weight"])
    g = hip.Talker(s, layers, fnorm, cos, sin, hip.BF16, kv_max, quantize_to=hip.PREC[prec])
    head = np.ascontiguousarray(tens["talker.codec_head.weight"])
    emb = np.ascontiguousarray(tens["talker.model.codec_embedding.weight"])
    L = hip.lib()
    ev = HipEvents()
    stream = L.qwen_hip_talker_stream(g.h)
    e0 = synth.bf16_to_f32(emb[1234])
    g.greedy(head, emb, e0, 0, 0, 0)
    hip.check(L.qwen_hip_talker_greedy_async(g.h, 16), "warmup")
    hip.check(L.qwen_hip_talker_sync(g.h), "sync")
    g.greedy(head, emb, e0, 0, 0, 0)                   # re-seed at position 0
    ev.device_sync()
    segs = []
    kv_bytes = 2 * s.layers * s.kv_dim * 2
    total_ms = 0.0
    for i in range(N // seg):
        a, b = ev.event(), ev.event()
        ev.record(a, stream)
        hip.check(L.qwen_hip_talker_greedy_async(g.h, seg), "grow steps")
        ev.record(b, stream)
        ms_total = ev.elapsed_ms(a, b)
        ev.device_sync()
        refuse_if_device_error(L, g, args.workload)
        total_ms += ms_total
        ms = ms_total / seg
        lm = i * seg + seg / 2.0
        gbs = (weight_bytes(s, prec) + kv_bytes * (lm + 1) + s.codec_vocab * s.hidden * 2) / (ms * 1e-3) / 1e9
        segs.append({"kv_from": i * seg, "kv_to": (i + 1) * seg, "ms_per_step": round(ms, 4), "gbs": round(gbs, 1)})
        log(f"[bench] grow: KV {i * seg:5d}..{(i + 1) * seg:5d}: {ms * 1e3:.1f} us/step, {gbs:.0f} GB/s")
    klabel = fused_label(L, g, prec, s.hidden)[1]
    g.free()
    ms = total_ms / N
    byts = sum(weight_bytes(s, prec) + kv_bytes * (j + 1) + s.codec_vocab * s.hidden * 2 for j in range(N)) / N
    gbs = byts / (ms * 1e-3) / 1e9
    out = {
        "metric": "Talker ms/decode-step (0.6B/1.7B, bf16/int8/int4) + achieved HBM GB/s",
        "value": round(ms, 4), "unit": "ms/step", "n_gpus": 1, "steps": N, "warmup": 16,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": prec, "data": "synthetic (seeded N(0,0.02) random-init weights; KV written by the steps themselves)",
        "config": {"workload": args.workload, "batch": 1, "kv_len_start": 0, "kv_len_end": N, "layers": s.layers,
                   "hidden": s.hidden, "inter": s.inter},
        "segments": segs,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": klabel,
                     "bytes_per_launch": int(byts * seg), "avg_us": round(total_ms / (N // seg) * 1e3, 1),
                     "steps_per_launch": seg},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def bench_sampled(args):
    """The Talker frame loop with the reference's default sampling on the device
    (qwen_hip_talker_sample: step, codec head, codec-head rule, qwen_tts_sample with
    temperature 0.9, top-k 50, top-p 1.0, repetition penalty 1.05 over the code0 history,
    next embedding; qwen_tts.c:559, :1649-1721), 1.7B int8, KV from 2048.  It runs on the
    per-kernel step path (the fused kernel's in-kernel head is greedy), so a step is ~140
    launches.  value = ms per step of one K-step call, host wall clock around the call
    (the call's own launches and its final synchronisation included)."""
    from qwen3_tts_amd import hip, synth
    shape_name, prec, Lpre, dsteps = SAMPLED_WORKLOADS[args.workload]
    K = args.steps or dsteps
    W = 16 if args.warmup is None else args.warmup
    s = synth.SHAPES[shape_name]
    kv_max = Lpre + K + W + 64
    only = lambda n: not n.startswith("talker.code_predictor.")  # noqa: E731
    tens = synth.generate(s, 0x5EED0001, 0.0, threads=int(os.environ.get("OMP_NUM_THREADS", "16")), only=only)
    layers = hip.layers_from_tensors(tens, s)
    cos, sin = synth.rope_tables(s.head_dim, s.rope_theta, kv_max)
    fnorm = synth.bf16_to_f32(tens["talker.model.norm.weight"])
    g = hip.Talker(s, layers, fnorm, cos, sin, hip.BF16, kv_max, quantize_to=hip.PREC[prec])
    head = np.ascontiguousarray(tens["talker.codec_head.weight"])
    emb = np.ascontiguousarray(tens["talker.model.codec_embedding.weight"])
    rng = np.random.default_rng(0x5EED0002)
    kvk = synth.f32_to_bf16_rne(rng.normal(0, 1.0, (s.layers, Lpre, s.kv_dim)).astype(np.float32))
    kvv = synth.f32_to_bf16_rne(rng.normal(0, 0.1, (s.layers, Lpre, s.kv_dim)).astype(np.float32))
    hip.check(hip.lib().qwen_hip_talker_upload_kv(g.h, kvk.ctypes.data, kvv.ctypes.data, Lpre, Lpre), "upload_kv")
    del kvk, kvv
    e0 = synth.bf16_to_f32(emb[1234])
    g.sample(head, emb, e0, Lpre, 10, W, 0.9, 50, 1.0, 1.05, (), 1234)          # warmup (uploads the heads)
    t0 = time.perf_counter()
    toks, _, _ = g.sample(head, emb, e0, Lpre, 10, K, 0.9, 50, 1.0, 1.05, (), 4321)
    dt = time.perf_counter() - t0
    g.free()
    n = len(toks)                                     # < K only if EOS came first
    ms = dt * 1e3 / max(n, 1)
    L_mid = Lpre + n / 2.0
    kv_bytes = 2 * s.layers * s.kv_dim * 2
    step_bytes = weight_bytes(s, prec) + kv_bytes * (L_mid + 1) + s.codec_vocab * s.hidden * 2
    gbs = step_bytes / (ms * 1e-3) / 1e9
    log(f"[bench] sampled loop: {n} steps, {ms * 1e3:.1f} us/step, {gbs:.0f} GB/s algorithmic")
    out = {
        "metric": "Talker ms/decode-step (0.6B/1.7B, bf16/int8/int4) + achieved HBM GB/s",
        "value": round(ms, 4), "unit": "ms/step", "n_gpus": 1, "steps": n, "warmup": W,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": prec, "data": "synthetic (seeded N(0,0.02) random-init weights)",
        "config": {"workload": args.workload, "batch": 1, "kv_len_start": Lpre, "layers": s.layers,
                   "hidden": s.hidden, "inter": s.inter, "temperature": 0.9, "top_k": 50, "rep_penalty": 1.05},
        "tokens_per_s": round(1000.0 / ms, 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "sampled frame loop (per-kernel step + codec head + k_sample + gather), whole call",
                     "bytes_per_launch": int(step_bytes * n), "avg_us": round(dt * 1e6, 1), "steps_per_launch": n},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def bench_frames(args):
    """The whole frame loop of qwen_tts_generate on the device (qwen_hip_generate,
    qwen_tts.c:1649-1778): per frame code0 from the codec head with the reference's default
    sampling (temperature 0.9, top-k 50, repetition penalty 1.05), the Code Predictor frame
    (16 passes of 5 layers + 15 lm-head picks, one captured graph), the next input
    (codec + 15 CP embeddings + tts_pad) and one Talker step (fused kernel), with the KV
    cache holding L positions first.  value = ms per frame of one K-frame call (host wall
    clock around the call, its final synchronisation included); frames/s; the reference's
    real-time bar is 12.5 frames/s of audio (80 ms per frame)."""
    from qwen3_tts_amd import hip, synth
    shape_name, prec, Lpre, dframes = FRAME_WORKLOADS[args.workload]
    K = args.steps or dframes
    W = 8 if args.warmup is None else args.warmup
    s = synth.SHAPES[shape_name]
    kv_max = Lpre + K + W + 64
    tens = synth.generate(s, 0x5EED0001, 0.0, threads=int(os.environ.get("OMP_NUM_THREADS", "16")))
    layers = hip.layers_from_tensors(tens, s)
    cos, sin = synth.rope_tables(s.head_dim, s.rope_theta, kv_max)
    fnorm = synth.bf16_to_f32(tens["talker.model.norm.weight"])
    g = hip.Talker(s, layers, fnorm, cos, sin, hip.BF16, kv_max, quantize_to=hip.PREC[prec])
    cp = hip.cp_from_tensors(tens, s, hip.PREC[prec])
    head = np.ascontiguousarray(tens["talker.codec_head.weight"])
    emb = np.ascontiguousarray(tens["talker.model.codec_embedding.weight"])
    rng = np.random.default_rng(0x5EED0002)
    kvk = synth.f32_to_bf16_rne(rng.normal(0, 1.0, (s.layers, Lpre, s.kv_dim)).astype(np.float32))
    kvv = synth.f32_to_bf16_rne(rng.normal(0, 0.1, (s.layers, Lpre, s.kv_dim)).astype(np.float32))
    hip.check(hip.lib().qwen_hip_talker_upload_kv(g.h, kvk.ctypes.data, kvv.ctypes.data, Lpre, Lpre), "upload_kv")
    del kvk, kvv
    h0 = rng.standard_normal(s.hidden).astype(np.float32)
    h0 /= np.sqrt((h0 ** 2).mean())
    pad = (rng.standard_normal(s.hidden) * 0.02).astype(np.float32)
    hip.generate(g, cp, head, emb, pad, h0, Lpre, 0, W, 0.9, 50, 1.0, 1.05, (), 99)        # warmup, graph capture
    t0 = time.perf_counter()
    codes, eos, _, _ = hip.generate(g, cp, head, emb, pad, h0, Lpre, 0, K, 0.9, 50, 1.0, 1.05, (), 4321)
    dt = time.perf_counter() - t0
    fused = bool(hip.lib().qwen_hip_talker_fused(g.h))
    cp.free()
    g.free()
    n = len(codes) + (1 if eos is not None else 0)    # frames whose work ran before EOS ended the utterance
    ms = dt * 1e3 / K
    log(f"[bench] frame loop: {K} frames ({len(codes)} generated{' + EOS' if eos is not None else ''}), "
        f"{ms:.3f} ms/frame, {1000.0 / ms:.0f} frames/s")
    wb = (lambda r, c: r * c * 2) if prec == "bf16" else (lambda r, c: r * c + 4 * r)
    per_layer = 0
    for r, c in [(s.cp_heads * s.cp_head_dim + 2 * s.cp_kv_heads * s.cp_head_dim, s.cp_hidden),
                 (s.cp_hidden, s.cp_heads * s.cp_head_dim), (2 * s.cp_inter, s.cp_hidden), (s.cp_hidden, s.cp_inter)]:
        per_layer += wb(r, c)
    cp_bytes = 16 * s.cp_layers * per_layer + 15 * wb(s.codebook, s.cp_hidden)
    kv_bytes = 2 * s.layers * s.kv_dim * 2
    frame_bytes = weight_bytes(s, prec) + kv_bytes * (Lpre + K / 2.0 + 1) + s.codec_vocab * s.hidden * 2 + cp_bytes
    gbs = frame_bytes / (ms * 1e-3) / 1e9
    out = {
        "metric": "Talker ms/decode-step (0.6B/1.7B, bf16/int8/int4) + achieved HBM GB/s",
        "value": round(ms, 4), "unit": "ms/frame", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": prec, "data": "synthetic (seeded N(0,0.02) random-init weights)",
        "config": {"workload": args.workload, "kv_len_start": Lpre, "layers": s.layers, "cp_layers": s.cp_layers,
                   "hidden": s.hidden, "temperature": 0.9, "top_k": 50, "rep_penalty": 1.05,
                   "talker_step": "fused" if fused else "per-kernel"},
        "frames_per_s": round(1000.0 / ms, 1), "frames_generated": len(codes), "eos": eos is not None,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "frame loop (head + k_sample + CP frame graph + k_frame_embed + k_pstep), whole call",
                     "bytes_per_launch": int(frame_bytes * K), "avg_us": round(dt * 1e6, 1), "steps_per_launch": K},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def prefill_flops(s, S):
    """Algorithmic flops of one prefill of S positions: the four projections per position
    and layer (2 flops per weight), plus causal attention (q.k and P.V over the keys at or
    before each position: 2 x 128 MACs per key per head, each 2 flops)."""
    macs = (s.q_dim + 2 * s.kv_dim) * s.hidden + s.hidden * s.q_dim + 2 * s.inter * s.hidden + s.hidden * s.inter
    attn = 2 * s.heads * s.head_dim * S * (S + 1)       # MACs: S(S+1)/2 keys x 128 x (q.k + P.V) per head
    return s.layers * (2.0 * S * macs + 2.0 * attn)


def bench_prefill(args):
    """Talker prefill (qwen_talker_prefill, qwen_tts_talker.c:730-1038) of S positions on
    the device, for the decode state of the headline workload (1.7B, int8 per-row weights
    quantized on the device): the prefill projections run on the bf16 weights, as the
    reference's do, as bf16 MFMA GEMMs over exact three-plane f32 activations.  Inputs:
    S codec-embedding rows (seeded).  value = ms per prefill (W warmup, K timed, back to
    back on the state's stream, inputs resident).  roofline: algorithmic flops (the
    projections + causal attention; the three activation planes triple the matrix-core
    work, which is not counted) per second against the dense bf16 MFMA peak."""
    from qwen3_tts_amd import hip, synth
    shape_name, prec, S, dk = PREFILL_WORKLOADS[args.workload]
    K = args.steps or dk
    W = 3 if args.warmup is None else args.warmup
    s = synth.SHAPES[shape_name]
    t0 = time.time()
    only = lambda n: n.startswith("talker.model.")  # noqa: E731
    tens = synth.generate(s, 0x5EED0001, 0.0, threads=int(os.environ.get("OMP_NUM_THREADS", "16")), only=only)
    layers = hip.layers_from_tensors(tens, s)
    cos, sin = synth.rope_tables(s.head_dim, s.rope_theta, S + 16)
    fnorm = synth.bf16_to_f32(tens["talker.model.norm.weight"])
    g = hip.Talker(s, layers, fnorm, cos, sin, hip.BF16, S + 16, quantize_to=hip.PREC[prec])
    emb = tens["talker.model.codec_embedding.weight"]
    rng = np.random.default_rng(0x5EED0004)
    E = synth.bf16_to_f32(emb[rng.integers(0, 2048, S)]).astype(np.float32)
    dx = g.prefill(E)                                   # uploads the bf16 copies, sizes the buffers
    log(f"[bench] prefill: S={S}, init {time.time() - t0:.1f}s, dec_x[0:3] {dx[:3]}")
    L = hip.lib()
    ev = HipEvents()
    stream = L.qwen_hip_talker_stream(g.h)
    hip.check(L.qwen_hip_talker_prefill_async(g.h, S, W), "prefill warmup")
    hip.check(L.qwen_hip_talker_sync(g.h), "sync")
    ev.device_sync()
    a, b = ev.event(), ev.event()
    ev.record(a, stream)
    hip.check(L.qwen_hip_talker_prefill_async(g.h, S, K), "prefill timed")
    ev.record(b, stream)
    ms_total = ev.elapsed_ms(a, b)
    ev.device_sync()
    refuse_if_device_error(L, g, args.workload)
    ms = ms_total / K
    fl = prefill_flops(s, S)
    tfs = fl / (ms * 1e-3) / 1e12
    log(f"[bench] prefill: {ms:.3f} ms per prefill of {S} positions, {S / ms * 1e3:.0f} positions/s, "
        f"{tfs:.1f} TFLOP/s algorithmic ({100 * tfs / BF16_MFMA_PEAK_TFS:.1f}% of bf16 MFMA peak)")
    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline_prefill(s, tens, E, args.cpu_seconds)
        except Exception as ex:
            log(f"[bench] cpu baseline failed: {ex}")
            cpu = {"value": None, "unit": "ms/prefill", "error": str(ex)[:200]}
    g.free()
    out = {
        "metric": "Talker prefill ms (prompt of S positions) + achieved TFLOP/s",
        "value": round(ms, 4), "unit": "ms/prefill", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded N(0,0.02) random-init weights, codec-embedding inputs)",
        "config": {"workload": args.workload, "positions": S, "layers": s.layers, "hidden": s.hidden, "inter": s.inter,
                   "decode_precision": prec},
        "positions_per_s": round(S * 1000.0 / ms, 1), "flops_per_prefill": fl,
        "roofline": {"bound": "mfma", "achieved": round(tfs, 2), "peak": BF16_MFMA_PEAK_TFS, "unit": "TFLOP/s",
                     "frac": round(tfs / BF16_MFMA_PEAK_TFS, 4), "traffic": None,
                     "kernel": "prefill (k_pf_gemm projections dominate; pieces, q/k norm + RoPE + KV store, attention)",
                     "flops_per_launch": fl, "avg_us": round(ms * 1e3, 1), "steps_per_launch": 1},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def cpu_baseline_prefill(s, tens, E, seconds):
    """The reference's own qwen_talker_prefill (oracle/_ref, its matmat_bf16 path: no BLAS
    in this image) on the host cores, same weights and inputs."""
    sys.path.insert(0, ROOT)
    from oracle.oracle import RefModel
    from qwen3_tts_amd import synth
    flags = open("/proc/cpuinfo").read()
    variant = "_avx512" if all(f in flags for f in (" avx512f", " avx512bw", " avx512vl")) else ""
    threads = int(os.environ.get("OMP_NUM_THREADS", "16"))
    full = dict(tens)
    full.update(synth.generate(s, 0x5EED0001, 0.0, threads=threads,
                               only=lambda n: not n.startswith("talker.model.")))
    with tempfile.TemporaryDirectory(prefix="qwen_ref_", dir=os.environ.get("TMPDIR", "/tmp")) as d:
        synth.write_model_dir(d, s, tensors=full)
        del full
        ref = RefModel(d, s, prec="bf16", threads=threads, variant=variant)
    t0 = time.perf_counter()
    ref.prefill(E)
    one = time.perf_counter() - t0
    n = int(max(1, min(5, seconds / max(one, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(n):
        ref.prefill(E)
    ms = (time.perf_counter() - t0) / n * 1e3
    log(f"[bench] cpu baseline: {n} reference qwen_talker_prefill calls, S={E.shape[0]}: {ms:.1f} ms ({threads} threads)")
    return {"value": round(ms, 2), "unit": "ms/prefill", "cores": threads, "kind": "reference",
            "sample": f"{n} reference qwen_talker_prefill calls of {E.shape[0]} positions (matmat_bf16 path, "
                      f"{variant.strip('_') or 'avx2'} build, -O3 -ffast-math), same weights and inputs"}


def bench_cp(args):
    """Config 4: the Code Predictor's per-frame work (qwen_cp_predict,
    qwen_tts_code_predictor.c:926-1045) on the device: 16 passes of the 5-layer CP over a
    fresh KV (positions 0..15) + 15 lm-head argmaxes + embedding gathers, captured once as
    a hipGraph; frames replayed back to back on device-resident inputs (talker hidden =
    RMS-normed N(0,1), code0 seeded).  value = ms per frame.  Algorithmic bytes per frame:
    16 x (5 layers of weights + norms) + 15 x one 2048 x 1024 lm head (bf16, or int8 +
    row scales); with the two-position prefill (cp_prefill2, cp.c:816-902) positions 0
    and 1 share one weight sweep, so 15 sweeps.  The CP's 157 MB of bf16 layer weights fit
    in the 256 MB MALL, so HBM traffic is lower than that."""
    from qwen3_tts_amd import hip, synth
    shape_name, prec, dframes, pf2 = CP_WORKLOADS[args.workload]
    K = args.steps or dframes
    W = 20 if args.warmup is None else args.warmup
    s = synth.SHAPES[shape_name]
    t0 = time.time()
    only = lambda n: n.startswith("talker.code_predictor.") or n == "talker.model.codec_embedding.weight"  # noqa: E731
    tens = synth.generate(s, 0x5EED0001, 0.0, threads=int(os.environ.get("OMP_NUM_THREADS", "16")), only=only)
    cp = hip.cp_from_tensors(tens, s, hip.PREC[prec])
    if pf2:
        cp.set_prefill2(1)
    log(f"[bench] cp: init {time.time() - t0:.1f}s")
    rng = np.random.default_rng(0x5EED0002)
    th = rng.standard_normal(s.hidden).astype(np.float32)
    th /= np.sqrt((th ** 2).mean())
    fused = bool(cp.fused(True)) and not pf2             # the default where the CP qualifies
    codes = cp.frame(th, int(rng.integers(0, 2048)))     # captures the frame graph
    L = hip.lib()
    ev = HipEvents()
    stream = L.qwen_hip_cp_stream(cp.h)
    hip.check(L.qwen_hip_cp_frame_async(cp.h, W), "cp warmup")
    hip.check(L.qwen_hip_cp_sync(cp.h), "sync")
    ev.device_sync()
    a, b = ev.event(), ev.event()
    ev.record(a, stream)
    hip.check(L.qwen_hip_cp_frame_async(cp.h, K), "cp timed")
    ev.record(b, stream)
    ms_total = ev.elapsed_ms(a, b)
    ev.device_sync()
    hip.check(L.qwen_hip_cp_sync(cp.h), "cp timed frames")
    ms = ms_total / K
    wb = (lambda r, c: r * c * 2) if prec == "bf16" else (lambda r, c: r * c + 4 * r)   # int8: + row scales
    per_layer = 0
    for r, c in [(s.cp_heads * s.cp_head_dim + 2 * s.cp_kv_heads * s.cp_head_dim, s.cp_hidden),
                 (s.cp_hidden, s.cp_heads * s.cp_head_dim), (2 * s.cp_inter, s.cp_hidden), (s.cp_hidden, s.cp_inter)]:
        per_layer += wb(r, c)
    per_layer += (2 * s.cp_hidden + 2 * s.cp_head_dim) * 4
    sweeps = 15 if pf2 else 16          # the two-position prefill reads the layer weights once for positions 0, 1
    frame_bytes = sweeps * s.cp_layers * per_layer + 15 * wb(s.codebook, s.cp_hidden)
    gbs = frame_bytes / (ms * 1e-3) / 1e9
    log(f"[bench] cp: {ms * 1e3:.1f} us/frame, {gbs:.0f} GB/s algorithmic, codes[0:4] {list(codes[:4])}")
    cp.free()
    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu = cpu_baseline_cp(s, prec, tens, th, args.cpu_seconds)
        except Exception as ex:
            log(f"[bench] cpu baseline failed: {ex}")
            cpu = {"value": None, "unit": "ms/frame", "error": str(ex)[:200]}
    out = {
        "metric": "Talker ms/decode-step (0.6B/1.7B, bf16/int8/int4) + achieved HBM GB/s",
        "value": round(ms, 4), "unit": "ms/frame", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": prec, "data": "synthetic (seeded N(0,0.02) random-init weights)",
        "config": {"workload": args.workload, "cp_layers": s.cp_layers, "cp_hidden": s.cp_hidden,
                   "passes_per_frame": 16, "weight_sweeps_per_frame": sweeps, "lm_heads": 15},
        "frames_per_s": round(1000.0 / ms, 1), "frame_bytes": int(frame_bytes), "frame_gbs": round(gbs, 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": (f"ps::{'rs06b' if prec == 'bf16' else 'rs06'}::k_rstep CP frame, one launch"
                                if fused else "CP frame (per-kernel launches replayed from one hipGraph)"),
                     "bytes_per_launch": int(frame_bytes), "avg_us": round(ms * 1e3, 1), "steps_per_launch": 1},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def bench_cp_batch(args):
    """The Code Predictor's batched pass (qwen_hip_cp_batch_step, the CP twin of the
    batched ragged step, qwen_tts_batch.h): B streams, each one pass of the 5-layer CP at
    its own position (drawn in 0..15, advancing one per step), the layer weights read once
    for all streams, replayed from the batch's hipGraph on device-resident inputs.
    value = ms per batched pass.  Algorithmic bytes per pass: the layers' weights and norms
    once + every stream's K/V rows at its length (bf16) + the appended rows."""
    from qwen3_tts_amd import hip, synth
    shape_name, prec, B = CP_BATCH_WORKLOADS[args.workload]
    K = args.steps or 40
    W = 4 if args.warmup is None else args.warmup
    s = synth.SHAPES[shape_name]
    cp_kv = 64
    if W + K > cp_kv - 20:
        raise SystemExit(f"cp batch: warmup + steps must stay within the CP cache ({cp_kv - 20})")
    t0 = time.time()
    tens = synth.generate(s, 0x5EED0001, 0.0, threads=int(os.environ.get("OMP_NUM_THREADS", "16")),
                          only=lambda n: n.startswith("talker.code_predictor.") or n == "talker.model.codec_embedding.weight")
    cp = hip.cp_from_tensors(tens, s, hip.PREC[prec], cp_kv_max=cp_kv)
    log(f"[bench] cp batch: init {time.time() - t0:.1f}s")
    rng = np.random.default_rng(0x5EED0003)
    pos = rng.integers(0, 16, B).astype(np.int32)
    x = rng.standard_normal((B, s.cp_hidden)).astype(np.float32)
    cp.batch_step(x, pos)                                 # captures the batch graph
    L = hip.lib()
    bt = cp._bh
    stream = L.qwen_hip_talker_batch_stream(bt)
    ev = HipEvents()
    hip.check(L.qwen_hip_talker_batch_step_async(bt, W), "cp batch warmup")
    hip.check(L.qwen_hip_talker_batch_sync(bt), "sync")
    ev.device_sync()
    a, b = ev.event(), ev.event()
    ev.record(a, stream)
    hip.check(L.qwen_hip_talker_batch_step_async(bt, K), "cp batch timed")
    ev.record(b, stream)
    ms_total = ev.elapsed_ms(a, b)
    ev.device_sync()
    ms = ms_total / K
    wb = (lambda r, c: r * c * 2) if prec == "bf16" else (lambda r, c: r * c + 4 * r)   # int8: + row scales
    per_layer = 0
    for r, c in [(s.cp_heads * s.cp_head_dim + 2 * s.cp_kv_heads * s.cp_head_dim, s.cp_hidden),
                 (s.cp_hidden, s.cp_heads * s.cp_head_dim), (2 * s.cp_inter, s.cp_hidden), (s.cp_hidden, s.cp_inter)]:
        per_layer += wb(r, c)
    per_layer += (2 * s.cp_hidden + 2 * s.cp_head_dim) * 4
    kv_row = 2 * s.cp_kv_heads * s.cp_head_dim * 2            # K and V rows of one position, bf16
    # position of stream b at timed step i (the graph's first run took pos, then W warmups)
    kv_pos = sum(int(p) + 1 + W + i + 1 for p in pos for i in range(K)) / K
    step_bytes = s.cp_layers * (per_layer + kv_pos * kv_row + B * kv_row)
    gbs = step_bytes / (ms * 1e-3) / 1e9
    log(f"[bench] cp batch: {ms * 1e3:.1f} us per pass of {B} streams, {gbs:.0f} GB/s algorithmic")
    cp.free()
    out = {
        "metric": "Talker ms/decode-step (0.6B/1.7B, bf16/int8/int4) + achieved HBM GB/s",
        "value": round(ms, 4), "unit": "ms/batched CP pass", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": prec, "data": "synthetic (seeded N(0,0.02) random-init weights, N(0,1) inputs)",
        "config": {"workload": args.workload, "streams": B, "cp_layers": s.cp_layers, "cp_hidden": s.cp_hidden,
                   "start_positions": [int(p) for p in pos]},
        "stream_passes_per_s": round(B * 1000.0 / ms, 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "batched CP pass (pieces + MFMA projections + batched attention, one hipGraph)",
                     "bytes_per_launch": int(step_bytes), "avg_us": round(ms * 1e3, 1), "steps_per_launch": 1},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def cpu_baseline_cp(s, prec, tens, th, seconds):
    """The reference's own qwen_cp_predict (oracle/_ref) on the host cores, same weights."""
    sys.path.insert(0, ROOT)
    from oracle.oracle import RefModel
    from qwen3_tts_amd import synth
    flags = open("/proc/cpuinfo").read()
    variant = "_avx512" if all(f in flags for f in (" avx512f", " avx512bw", " avx512vl")) else ""
    threads = int(os.environ.get("OMP_NUM_THREADS", "16"))
    full = dict(tens)
    full.update(synth.generate(s, 0x5EED0001, 0.0, threads=threads,
                               only=lambda n: not n.startswith("talker.code_predictor.")
                               and n != "talker.model.codec_embedding.weight"))
    with tempfile.TemporaryDirectory(prefix="qwen_ref_", dir=os.environ.get("TMPDIR", "/tmp")) as d:
        synth.write_model_dir(d, s, tensors=full)
        del full
        ref = RefModel(d, s, prec=prec, threads=threads, variant=variant)
    t0 = time.perf_counter()
    ref.cp_predict(th, 7)
    one = time.perf_counter() - t0
    n = int(max(2, min(50, seconds / max(one, 1e-3))))
    t0 = time.perf_counter()
    for i in range(n):
        ref.cp_predict(th, (7 + 31 * i) % 2048)
    ms = (time.perf_counter() - t0) / n * 1e3
    log(f"[bench] cpu baseline: {n} reference qwen_cp_predict frames: {ms:.1f} ms/frame ({threads} threads)")
    return {"value": round(ms, 3), "unit": "ms/frame", "cores": threads, "kind": "reference",
            "sample": f"{n} reference qwen_cp_predict calls ({prec}, {variant.strip('_') or 'avx2'} build, "
                      f"-O3 -ffast-math), same weights"}


def sd_flops(n):
    """Algorithmic multiply-add work (2 flops each) of one decode of n frames: every
    projection, conv and transposed conv as output rows x output channels x (taps x input
    channels), plus the windowed attention; elementwise work is not counted."""
    f = 2 * n * 512 * 512 + 2 * n * 1024 * 3 * 512 + 2 * n * 512 * 1024            # vq, pre-conv, input proj
    att = sum(2 * 2 * 16 * 64 * min(72, t + 1) for t in range(n))
    f += 8 * (2 * n * 3072 * 512 + 2 * n * 512 * 1024 + 2 * n * 2048 * 512 + 2 * n * 512 * 1024) + 8 * att
    f += 2 * n * 1024 * 512                                                         # output proj
    T = n
    for _ in range(2):                                                              # ConvNeXt upsamplers
        T *= 2
        f += 2 * T * 1024 * 1024 + 2 * (2 * T * 4096 * 1024)
    f += 2 * T * 1536 * 7 * 1024                                                    # initial conv
    cin = 1536
    for r, c in zip((8, 5, 4, 3), (768, 384, 192, 96)):
        Tin, T = T, T * r
        f += 2 * T * c * 2 * cin + 3 * (2 * T * c * 7 * c + 2 * T * c * c)
        cin = c
    return f + 2 * T * 96 * 7


def bench_sd(args):
    """The speech decoder: one decode of n frames (codes -> 1920 n samples of 24 kHz audio,
    the reference's one-shot qwen_speech_decoder_decode) on device-resident codes
    (qwen_hip_sd_decode_device), synthetic F32 weights of the real architecture.
    value = ms per decode; roofline = algorithmic MFMA flops over the f32 matrix peak."""
    from qwen3_tts_amd import hip, synth_sd
    n, dk = SD_WORKLOADS[args.workload]
    K = args.steps or dk
    W = 2 if args.warmup is None else args.warmup
    t0 = time.time()
    tens = synth_sd.generate_sd()
    path = synth_sd.write_sd(os.path.join(os.environ.get("TMPDIR", "/tmp"), "qwen3tts_bench_sd"), tensors=tens)
    dec = hip.SpeechDecoder.from_file(path)
    log(f"[bench] sd: weights + device init {time.time() - t0:.1f}s")
    rng = np.random.default_rng(0x5EED0D0E)
    codes = rng.integers(0, 2048, (n, 16)).astype(np.int32)
    ev = HipEvents()
    rt = ev.rt
    rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    dc, da = C.c_void_p(), C.c_void_p()
    assert rt.hipMalloc(C.byref(dc), codes.nbytes) == 0 and rt.hipMalloc(C.byref(da), n * 1920 * 4) == 0
    assert rt.hipMemcpy(dc, codes.ctypes.data, codes.nbytes, 1) == 0
    L = hip.lib()
    stream = L.qwen_hip_sd_stream(dec.h)
    for _ in range(W):
        hip.check(L.qwen_hip_sd_decode_device(dec.h, dc, n, da), "sd warmup")
    ev.device_sync()
    a, b = ev.event(), ev.event()
    ev.record(a, stream)
    for _ in range(K):
        hip.check(L.qwen_hip_sd_decode_device(dec.h, dc, n, da), "sd timed")
    ev.record(b, stream)
    ms = ev.elapsed_ms(a, b) / K
    ev.device_sync()
    fl = sd_flops(n)
    tfs = fl / (ms * 1e-3) / 1e12
    audio_s = n * 1920 / 24000.0
    log(f"[bench] sd: {n} frames ({audio_s:.1f} s of audio) in {ms:.3f} ms, {tfs:.1f} TFLOP/s, "
        f"{audio_s / (ms * 1e-3):.0f}x real time")
    cpu = None
    if not args.no_cpu_baseline:
        try:
            sys.path.insert(0, ROOT)
            from oracle.oracle import RefSpeechDecoder
            threads = int(os.environ.get("OMP_NUM_THREADS", "16"))
            ref = RefSpeechDecoder(path, threads=threads)
            ns = 2
            secs = ref.time_decode(codes[:ns])
            model, ncpu = host_info()
            cpu = {"value": round(secs * 1e3 / ns * n, 1), "unit": "ms/decode", "cores": threads, "kind": "reference",
                   "sample": f"one reference qwen_speech_decoder_decode of the first {ns} frames of the same codes "
                             f"({secs:.2f} s; oracle/_ref build: reference flags, no BLAS, so its convs run as the "
                             f"naive single-thread loops and only the snake uses the {threads}-thread pool), "
                             f"scaled linearly to {n} frames",
                   "host_cpu": model, "host_logical_cpus": ncpu}
            log(f"[bench] sd cpu baseline: {secs:.2f} s for {ns} frames")
        except Exception as ex:  # noqa: BLE001
            cpu = {"value": None, "unit": "ms/decode", "error": str(ex)[:200]}
    dec.free()
    out = {
        "metric": "speech decoder ms/decode (codes -> 24 kHz audio) + achieved MFMA TFLOP/s",
        "value": round(ms, 3), "unit": "ms/decode", "n_gpus": 1, "steps": K, "warmup": W, "ms_per_step": round(ms, 3),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded random-init F32 decoder weights of the 12 Hz codec architecture; random codes)",
        "config": {"workload": args.workload, "frames": n, "samples": n * 1920, "audio_seconds": audio_s},
        "realtime_factor": round(audio_s / (ms * 1e-3), 1),
        "roofline": {"bound": "mfma", "achieved": round(tfs, 2), "peak": F32_MFMA_PEAK_TFS, "unit": "TFLOP/s",
                     "frac": round(tfs / F32_MFMA_PEAK_TFS, 4), "traffic": None,
                     "kernel": "one decode (all kernels; k_sd_gemm carries the flops)", "flops_per_launch": int(fl),
                     "avg_us": round(ms * 1e3, 1), "steps_per_launch": 1},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def bench_sd_stream(args):
    """The speech decoder's exact streaming decode (qwen_hip_sd_stream_decode, the twin of
    qwen_speech_decoder_decode_streaming_st): a stream of n frames fed in chunks of c frames,
    each call taking host codes and returning the chunk's 1920 c samples on the host (so
    every chunk time includes its two small PCIe copies and a device sync).  value = ms for
    the whole stream; also the first chunk's latency (time to first audio) and the mean
    chunk latency.  Timed on the host clock around each call."""
    from qwen3_tts_amd import hip, synth_sd
    n, c, dk = SD_STREAM_WORKLOADS[args.workload]
    K = args.steps or dk
    W = 1 if args.warmup is None else args.warmup
    t0 = time.time()
    tens = synth_sd.generate_sd()
    path = synth_sd.write_sd(os.path.join(os.environ.get("TMPDIR", "/tmp"), "qwen3tts_bench_sd"), tensors=tens)
    dec = hip.SpeechDecoder.from_file(path)
    log(f"[bench] sd-stream: weights + device init {time.time() - t0:.1f}s")
    rng = np.random.default_rng(0x5EED0D0E)
    codes = rng.integers(0, 2048, (n, 16)).astype(np.int32)
    chunks = [codes[i:i + c] for i in range(0, n, c)]
    st = hip.SpeechDecoderStream(dec)
    firsts, totals, per_chunk = [], [], []
    for it in range(W + K):
        st.reset()
        tt = []
        for ch in chunks:
            a = time.perf_counter()
            st.decode(ch)
            tt.append(time.perf_counter() - a)
        if it >= W:
            firsts.append(tt[0] * 1e3)
            totals.append(sum(tt) * 1e3)
            per_chunk.extend(x * 1e3 for x in tt)
    st.free()
    ms = float(np.median(totals))
    audio_s = n * 1920 / 24000.0
    fl = sd_flops(n)
    tfs = fl / (ms * 1e-3) / 1e12
    log(f"[bench] sd-stream: {n} frames in chunks of {c}: {ms:.2f} ms per stream (median of {K}), first chunk "
        f"{np.median(firsts):.2f} ms, chunk mean {np.mean(per_chunk):.2f} ms")
    cpu = None
    if not args.no_cpu_baseline:
        try:
            sys.path.insert(0, ROOT)
            from oracle.oracle import RefSpeechDecoder
            threads = int(os.environ.get("OMP_NUM_THREADS", "16"))
            ref = RefSpeechDecoder(path, threads=threads)
            a = time.perf_counter()
            ref.stream_decode(chunks[:1])
            secs = time.perf_counter() - a
            model, ncpu = host_info()
            cpu = {"value": round(secs * 1e3, 1), "unit": "ms/first chunk", "cores": threads, "kind": "reference",
                   "sample": f"the reference's streaming decode of the first {c}-frame chunk of the same codes "
                             f"(oracle/_ref, reference flags, no BLAS): its time to first audio",
                   "host_cpu": model, "host_logical_cpus": ncpu}
            log(f"[bench] sd-stream cpu baseline: first chunk {secs:.2f} s")
        except Exception as ex:  # noqa: BLE001
            cpu = {"value": None, "unit": "ms/first chunk", "error": str(ex)[:200]}
    dec.free()
    out = {
        "metric": "speech decoder streaming ms/stream (codes -> 24 kHz audio chunk by chunk) + time to first audio",
        "value": round(ms, 3), "unit": "ms/stream", "n_gpus": 1, "steps": K, "warmup": W, "ms_per_step": round(ms, 3),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded random-init F32 decoder weights of the 12 Hz codec architecture; random codes)",
        "config": {"workload": args.workload, "frames": n, "chunk_frames": c, "chunks": len(chunks),
                   "audio_seconds": audio_s},
        "first_chunk_ms": round(float(np.median(firsts)), 3), "chunk_ms_mean": round(float(np.mean(per_chunk)), 3),
        "chunk_ms_p90": round(float(np.percentile(per_chunk, 90)), 3),
        "realtime_factor": round(audio_s / (ms * 1e-3), 1),
        "roofline": {"bound": "mfma", "achieved": round(tfs, 2), "peak": F32_MFMA_PEAK_TFS, "unit": "TFLOP/s",
                     "frac": round(tfs / F32_MFMA_PEAK_TFS, 4), "traffic": None,
                     "kernel": "one stream (one-shot decode flops over the stream's host-clock time)",
                     "flops_per_launch": int(fl), "avg_us": round(ms * 1e3, 1), "steps_per_launch": 1},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def host_info():
    """CPU model and logical CPU count of this host (/proc/cpuinfo)."""
    model, n = "unknown", 0
    for ln in open("/proc/cpuinfo"):
        if ln.startswith("model name") and model == "unknown":
            model = ln.split(":", 1)[1].strip()
        if ln.startswith("processor"):
            n += 1
    return model, n


def cpu_baseline(s, prec, g, kv_len, tens, seconds):
    """The reference's own qwen_talker_step (oracle/_ref, reference flags) on a bounded
    sample: same weights (written to safetensors and loaded + quantized by the
    reference loader), KV = the device's first kv_len positions; consecutive steps timed
    one by one (clock_gettime around each qwen_talker_step, as the reference times
    itself), first with N threads (OMP_NUM_THREADS, the box's CPU share) for about
    `seconds`, then with 1 thread for about half that.  value = the N-thread median."""
    sys.path.insert(0, ROOT)
    from oracle.oracle import RefModel
    from qwen3_tts_amd import synth
    flags = open("/proc/cpuinfo").read()
    variant = "_avx512" if all(f in flags for f in (" avx512f", " avx512bw", " avx512vl")) else ""
    threads = int(os.environ.get("OMP_NUM_THREADS", "16"))
    t0 = time.time()
    full = dict(tens)
    full.update(synth.generate(s, 0x5EED0001, 0.0, threads=threads,
                               only=lambda n: n.startswith("talker.code_predictor.")))
    # the reference's fastest x86 build (SIMD=avx512bf16: VNNI int8 dots on int8-quantized
    # activations, bf16 dots), timed beside the parity build where the host has the ISA
    fast = "_avx512bf16" if (variant and all(f in flags for f in (" avx512_bf16", " avx512_vnni", " avx512dq"))
                              and os.path.exists(RefModel.lib_path("_avx512bf16"))) else None
    kk, vv = g.download_kv(kv_len)
    emb = tens["talker.model.codec_embedding.weight"]
    e = np.stack([synth.bf16_to_f32(emb[i * 7 + 1]) for i in range(64)])
    out = np.empty(s.hidden, np.float32)

    def timed(ref, build, nt, budget):
        ref.lib.ref_set_threads(nt)
        ref.kv_len = kv_len
        w = np.empty(1, np.float64)
        ref.lib.ref_time_talker_steps_each(ref.h, e.ctypes.data, 1, out.ctypes.data, w.ctypes.data)
        n = int(max(3, min(64, budget / max(w[0], 1e-3))))
        ref.kv_len = kv_len
        ts = np.empty(n, np.float64)
        ref.lib.ref_time_talker_steps_each(ref.h, e.ctypes.data, n, out.ctypes.data, ts.ctypes.data)
        r = {"build": build, "threads": nt, "steps": n, "median_ms": round(float(np.median(ts)) * 1e3, 3),
             "p90_ms": round(float(np.percentile(ts, 90)) * 1e3, 3), "mean_ms": round(float(ts.mean()) * 1e3, 3)}
        log(f"[bench] cpu baseline ({build}): {n} steps at KV {kv_len}, {nt} threads: median {r['median_ms']:.1f} ms, "
            f"p90 {r['p90_ms']:.1f} ms")
        return r

    with tempfile.TemporaryDirectory(prefix="qwen_ref_", dir=os.environ.get("TMPDIR", "/tmp")) as d:
        synth.write_model_dir(d, s, tensors=full)
        del full
        ref = RefModel(d, s, prec=prec, threads=threads, variant=variant)
        log(f"[bench] cpu baseline: reference loaded + quantized in {time.time() - t0:.1f}s ({variant or '_avx2'})")
        ref.set_kv(kk, vv, kv_len)
        build = variant.strip("_") or "avx2"
        runs = [timed(ref, build, threads, seconds), timed(ref, build, 1, seconds / 2)]
        compiler = ref.lib.ref_build_info().decode()
        if fast:
            del ref
            ref = RefModel(d, s, prec=prec, threads=threads, variant=fast)
            ref.set_kv(kk, vv, kv_len)
            r = timed(ref, fast.strip("_"), threads, seconds / 2)
            r["note"] = ("the reference's fastest x86 build: activations rounded to bf16 / quantized to int8 "
                         "inside its dot products, so it is a speed figure, not a parity build")
            runs.append(r)
    model, ncpu = host_info()
    return {"value": runs[0]["median_ms"], "unit": "ms/step", "cores": threads, "kind": "reference",
            "sample": f"{runs[0]['steps']} consecutive reference qwen_talker_step calls ({prec}, "
                      f"{build} build, -O3 -ffast-math) from KV length {kv_len}, same weights "
                      f"and KV as the GPU run; median of per-step clock_gettime times",
            "runs": runs, "host_cpu": model, "host_logical_cpus": ncpu, "compiler": compiler}


if __name__ == "__main__":
    main()
