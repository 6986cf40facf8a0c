#!/usr/bin/env python3
"""Benchmark of the quantized-matmul hot path on one MI355X.

Workload ("Q4_0 GEMV at Llama-2-7B layer shapes,
batch 1"): one step = the 7 Q4_0 GEMVs of one Llama-2-7B layer
    q, k, v, o  4096 x 4096      gate, up  11008 x 4096      down  4096 x 11008
= 113,836,032 weight bytes, through the drop-in entry point cuda_matmul_q4_0.
Steps rotate over `--layers` distinct synthetic layers (default 32, 3.64 GB,
far above the 256 MB MALL) so every step streams its weights from HBM.
Inputs are resident in HBM before timing starts.

Printed: ONE JSON line with
    value        aggregate weight GB/s over the K timed steps (HIP events on the
                 library stream around the whole timed region)
    roofline     dominant kernel = the Q4_0 GEMV kernel; achieved = algorithmic
                 weight bytes per launch / mean launch duration, the durations
                 measured with HIP events around each launch in a second pass
    cpu_baseline the reference's own CPU path (matmul_q of src/ai/llm.c,
                 compiled from the reference sources into oracle/_ref/ with its
                 release flags), Q4_0 branch = single-threaded scalar code, on a
                 bounded sample of the same layer shapes
    extra        config-1/3/5 figures (Q8_0 and Q4_K GEMV GB/s, the full 7B
                 decode step's matmul time)

Only the CPU-baseline leg touches oracle/ (the reference build under
oracle/_ref, or the oracle port when that is absent).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "google-classic_amd"))

import holo_mi355x as holo  # noqa: E402
from holo_mi355x import synth  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
Q4_0, Q8_0, Q4_K = holo.TYPE_Q4_0, holo.TYPE_Q8_0, holo.TYPE_Q4_K
BASE_SEED = 20251201

# Llama-2-7B layer: (name, out_dim, in_dim)
LAYER = [("q", 4096, 4096), ("k", 4096, 4096), ("v", 4096, 4096), ("o", 4096, 4096),
         ("gate", 11008, 4096), ("up", 11008, 4096), ("down", 4096, 11008)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# BASELINE configs 1 and 3
CONFIG1 = [("w", 4096, 4096)]                          # Q8_0 GEMV 4096x4096
CONFIG3 = [("gate", 14336, 4096), ("down", 4096, 14336)]  # Q4_K, Llama-3-8B FFN


class Layer:
    """One set of synthetic weight matrices, resident in HBM."""

    def __init__(self, qtype: int, idx: int, config: int, shapes=LAYER):
        self.shapes = shapes
        self.qtype = qtype
        self.mats = []
        for m, (name, out_dim, in_dim) in enumerate(shapes):
            seed = synth.tensor_seed(BASE_SEED, config, idx, m)
            host = synth.blocks(qtype, out_dim, in_dim, seed)
            self.mats.append((name, out_dim, in_dim, holo.DeviceBuffer.from_array(host)))
            del host

    @staticmethod
    def weight_bytes(qtype: int, shapes=LAYER) -> int:
        return sum(holo.row_bytes(qtype, i) * o for _, o, i in shapes)


def run_layer(lib, fn, layer: Layer, xs, ys, per_launch_events=None):
    for j, (name, out_dim, in_dim, W) in enumerate(layer.mats):
        if per_launch_events is not None:
            lib.holo_event_record(per_launch_events[j][0])
        fn(ys[out_dim].ptr, W.ptr, xs[in_dim].ptr, out_dim, in_dim)
        if per_launch_events is not None:
            lib.holo_event_record(per_launch_events[j][1])


def gemv_bench(lib, qtype, layers, steps, warmup, xs, ys):
    """Returns (ms_per_step, GB/s over the timed region, mean per-launch us, bytes/launch)."""
    fn = {Q4_0: lib.cuda_matmul_q4_0, Q8_0: lib.cuda_matmul_q8_0, Q4_K: lib.cuda_matmul_q4_k}[qtype]
    nL = len(layers)
    for i in range(warmup):
        run_layer(lib, fn, layers[i % nL], xs, ys)
    lib.cuda_sync()
    ev = holo.Events()
    ev.start()
    for i in range(steps):
        run_layer(lib, fn, layers[(warmup + i) % nL], xs, ys)
    total_ms = ev.stop()
    lib.cuda_sync()
    holo.check("timed region")
    bytes_step = Layer.weight_bytes(qtype, layers[0].shapes)
    gbs = steps * bytes_step / (total_ms * 1e-3) / 1e9

    # Second pass: events around every launch (kernel durations).
    pairs = [(lib.holo_event_create(), lib.holo_event_create()) for _ in layers[0].shapes]
    durs = []
    for i in range(steps):
        run_layer(lib, fn, layers[i % nL], xs, ys, per_launch_events=pairs)
        lib.cuda_sync()
        durs.extend(lib.holo_event_elapsed_ms(a, b) for a, b in pairs)
    for a, b in pairs:
        lib.holo_event_destroy(a)
        lib.holo_event_destroy(b)
    ev.close()
    mean_us = 1e3 * sum(durs) / len(durs)
    return total_ms / steps, gbs, mean_us, bytes_step / len(layers[0].shapes)


def cpu_baseline(qtype: int, budget_s: float) -> dict:
    """The reference CPU path on the same layer shapes (bounded sample)."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc  # test-infrastructure checker / baseline only
    if orc.ref_available("release"):
        ref = orc.RefBuild("release")
        kind, fn = "reference", (lambda M, v, o, i: ref.matmul(qtype, M, v, o, i))
        what = "oracle/_ref/libholo_ref_release.so matmul_q (reference sources, -O3 -ffast-math -mavx2 -mfma)"
    else:
        o_ = orc.Oracle()
        kind, fn = "port", (lambda M, v, o, i: o_.matmul(qtype, M, v, o, i))
        what = "oracle/liboracle.so restatement of matmul_q"
    mats = []
    for m, (name, out_dim, in_dim) in enumerate(LAYER):
        seed = synth.tensor_seed(BASE_SEED, 2, 0, m)
        mats.append((synth.blocks(qtype, out_dim, in_dim, seed), out_dim, in_dim))
    x = {4096: synth.normal(4096, 11), 11008: synth.normal(11008, 12)}
    bytes_layer = Layer.weight_bytes(qtype)
    for M, o, i in mats:  # warm-up
        fn(M, x[i], o, i)
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 2000):
        t0 = time.perf_counter()
        for M, o, i in mats:
            fn(M, x[i], o, i)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    # Q4_0/Q4_K branches have no OpenMP pragma (llm.c:893-915, quant.c:626-633);
    # Q8_0 runs its AVX2 rows under OpenMP (llm.c:838).
    cores = 1 if qtype in (Q4_0, Q4_K) else (os.cpu_count() or 1)
    return {"value": round(bytes_layer / med / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": kind,
            "sample": f"{len(times)} runs (median) of one Llama-2-7B layer's 7 Q4_0 GEMVs "
                      f"({bytes_layer} weight bytes) with {what}; host has {os.cpu_count()} logical CPUs",
            "ms_per_step": round(med * 1e3, 3)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU-baseline sampling")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--xmode", choices=["i24", "f32"], default="f32",
                    help="GEMV activation mode (holo_gemv_set_xmode)")
    a = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the path is a single-GPU decode "
                                   "GEMV (multi-GPU sharding is a design note, not built)",
                          "n_gpus": a.gpus}), flush=True)
        sys.exit(2)

    lib = holo.load()
    holo.init()
    log(f"device: {lib.cuda_get_device_name().decode()}")

    t0 = time.time()
    layers = [Layer(Q4_0, i, 2) for i in range(a.layers)]
    log(f"generated + uploaded {a.layers} Q4_0 layers ({a.layers * Layer.weight_bytes(Q4_0) / 1e9:.2f} GB) "
        f"in {time.time() - t0:.1f}s")
    xs = {4096: holo.DeviceBuffer.from_array(synth.normal(4096, 1)),
          11008: holo.DeviceBuffer.from_array(synth.normal(11008, 2))}
    ys = {4096: holo.DeviceBuffer(4096 * 4), 11008: holo.DeviceBuffer(11008 * 4)}

    lib.holo_gemv_set_xmode(1 if a.xmode == "i24" else 0)
    ms_step, gbs, mean_us, bytes_launch = gemv_bench(lib, Q4_0, layers, a.steps, a.warmup, xs, ys)
    achieved = bytes_launch / (mean_us * 1e-6) / 1e9
    log(f"Q4_0 layer step: {ms_step * 1e3:.1f} us/step, {gbs:.0f} GB/s; mean launch {mean_us:.2f} us "
        f"-> {achieved:.0f} GB/s per launch")

    extra = {}
    if not a.no_extra:
        other = "f32" if a.xmode == "i24" else "i24"
        lib.holo_gemv_set_xmode(1 if other == "i24" else 0)
        m2, g2, u2, b2 = gemv_bench(lib, Q4_0, layers, a.steps, a.warmup, xs, ys)
        extra[f"q4_0_layer_xmode_{other}"] = {"gbs_back_to_back": round(g2, 1),
                                              "gbs_per_launch": round(b2 / (u2 * 1e-6) / 1e9, 1)}
        log(f"Q4_0 layer step, xmode {other}: {m2 * 1e3:.1f} us/step, {g2:.0f} GB/s")
        lib.holo_gemv_set_xmode(1 if a.xmode == "i24" else 0)
        del layers
        xs[14336] = holo.DeviceBuffer.from_array(synth.normal(14336, 3))
        ys[14336] = holo.DeviceBuffer(14336 * 4)
        # config 1: Q8_0 4096x4096 over 32 copies (570 MB); config 3: Q4_K
        # Llama-3-8B FFN pair over 10 copies (660 MB).
        for qt, cfg, name, shapes, copies in ((Q8_0, 1, "config1_q8_0_4096x4096", CONFIG1, 32),
                                              (Q4_K, 3, "config3_q4_k_llama3_ffn", CONFIG3, 10)):
            ls = [Layer(qt, i, cfg, shapes) for i in range(copies)]
            m, g, u, b = gemv_bench(lib, qt, ls, 4 * copies, copies, xs, ys)
            extra[name] = {"gbs_back_to_back": round(g, 1),
                           "gbs_per_launch": round(b / (u * 1e-6) / 1e9, 1),
                           "mean_launch_us": round(u, 3), "bytes_per_launch": b}
            log(f"{name}: {m * 1e3:.1f} us/step, {g:.0f} GB/s back-to-back, {u:.2f} us/launch")
            del ls

    result = {
        "metric": "Q4_0 GEMV weight GB/s at Llama-2-7B layer shapes (batch 1)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x f32 -> f32" if a.xmode == "f32" else "q4_0 x (f32 as 24-bit fixed point per 32-block) -> f32",
        "data": "synthetic (seeded GGUF Q4_0 blocks, N(0,1) fp32 activations)",
        "config": {"workload": "Llama-2-7B layer: 7 Q4_0 GEMVs (4x 4096x4096, 2x 11008x4096, 1x 4096x11008), "
                               f"rotating over {a.layers} distinct layers",
                   "weight_bytes_per_step": Layer.weight_bytes(Q4_0), "batch": 1,
                   "entry_point": "cuda_matmul_q4_0"},
        "roofline": {"bound": "hbm", "kernel": "holo::gemv_kernel<Q4_0>",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": bytes_launch, "mean_launch_us": round(mean_us, 3)},
        "extra": extra,
    }
    holo.check("bench")
    if not a.no_cpu:
        log("CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(Q4_0, a.cpu_budget)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
