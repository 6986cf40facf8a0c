#!/usr/bin/env python3
"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline ("Q4_0 GEMV at Llama-2-7B layer shapes,
batch 1"): one step = the 7 Q4_0 GEMVs of one Llama-2-7B layer,
    q, k, v, o  4096 x 4096      gate, up  11008 x 4096      down  4096 x 11008
= 113,836,032 weight bytes, issued as a decode loop on MI355X issues them:
holo_batched_qkv (q, k, v in one launch), cuda_matmul_q4_0 (o),
holo_batched_ffn_gate_up (gate and up in one launch, silu(g)*u epilogue) and
cuda_matmul_q4_0 (down).  Steps rotate over --layers distinct synthetic
layers (default 32, 3.64 GB, far above the 256 MB MALL), so each step streams
its weights from HBM; all inputs are resident in HBM before timing starts.
Consecutive steps are captured together in HIP graphs (as a decode loop
captures its layers), so the timed region holds the K steps' kernels and no
per-step host launch.

The printed JSON line carries
  value         aggregate weight GB/s over the K timed steps (HIP events on the
                library stream around the timed region)
  roofline      dominant kernel = the fused gate/up Q4_0 GEMV (50,724,864 weight
                bytes per launch); achieved = those bytes / its mean kernel
                duration, measured in a second pass of the same layers issued
                back to back, with HIP events that the launch itself records
                at the kernel's start and end
                (holo_time_next_launch; the span rocprofv3's kernel trace
                reports), also given with events around the call; traffic =
                HBM bytes per launch from the committed PMC summary
                profiles/traffic_q4_0_gateup_<mode>.json
  cpu_baseline  the reference's own CPU path: matmul_q (src/ai/llm.c:770),
                compiled from the reference sources into oracle/_ref/ with its
                release flags; the Q4_0 branch is single-threaded scalar code;
                a bounded sample of the same layer
  extra         the unfused drop-in layer (7 cuda_matmul_q4_0 calls), configs
                1 and 3 (Q8_0 4096x4096; Q4_K Llama-3-8B FFN; per matrix the
                median kernel time over >= 128 launches and its fraction of
                HBM peak), the Q6_K GEMV (32000x4096 head and 4096x11008
                down), config 4 (the batched prefill products: useful TOP/s
                = 2*M*N*K per kernel time, and its fraction of the dense f16
                and int8 peaks; and a 512-token prompt through the 32 layers
                in one pass, also on a Q4_K_M-style mix of Q4_K and Q6_K
                matrices), config 5 (full synthetic Llama-2-7B Q4_0 decode
                step: end-to-end and matmuls-only ms, as 4 launches a layer
                and as one persistent launch for all 128 layer GEMVs), decode
                attention at 512 / 2048 / 4096 cached positions.  Configs 1,
                3, 4 and 5 carry a cpu_baseline of their own: the reference's
                matmul_q on the same shapes (Q8_0 on its OpenMP threads, Q4_0
                and Q4_K on one core; config 4 as 512 sequential GEMVs, the
                reference's token-by-token prompt loop; config 5 as one
                layer x 32 + the head)

Only the CPU-baseline leg touches oracle/.
"""
from __future__ import annotations

import argparse
import ctypes as C
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

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
F16_PEAK_TFLOPS = 2500.0   # MI355X dense f16 MFMA
I8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA
Q4_0, Q8_0, Q4_K = holo.TYPE_Q4_0, holo.TYPE_Q8_0, holo.TYPE_Q4_K
Q6_K = 14
BASE_SEED = 20251201
DIM, FFN, VOCAB = 4096, 11008, 32000

# Llama-2-7B layer: (name, out_dim, in_dim)
LAYER = [("q", 4096, 4096), ("k", 4096, 4096), ("v", 4096, 4096), ("o", 4096, 4096),
         ("gate", 11008, 4096), ("up", 11008, 4096), ("down", 4096, 11008)]
CONFIG1 = [("w", 4096, 4096)]                             # Q8_0 GEMV
CONFIG3 = [("gate", 14336, 4096), ("down", 4096, 14336)]  # Q4_K, Llama-3-8B FFN
Q6K_SHAPES = [("output", 32000, 4096), ("down", 4096, 11008)]  # Q6_K head and down of a Q4_K_M Llama-2-7B


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def weight_bytes(qtype, shapes):
    return sum(holo.row_bytes(qtype, i) * o for _, o, i in shapes)


class Mats:
    """One set of synthetic weight matrices, resident in HBM."""

    def __init__(self, qtype, idx, config, shapes):
        self.shapes, self.qtype = shapes, qtype
        self.buf = {}
        for m, (name, out_dim, in_dim) in enumerate(shapes):
            host = synth.blocks(qtype, out_dim, in_dim, synth.tensor_seed(BASE_SEED, config, idx, m))
            self.buf[name] = holo.DeviceBuffer.from_array(host)


class Acts:
    """Activation vectors in HBM: inputs x<n>, outputs y<n>, q/k/v/h scratch."""

    def __init__(self):
        self.b = {}
        for n in (DIM, FFN, 14336):
            self.b[f"x{n}"] = holo.DeviceBuffer.from_array(synth.normal(n, n))
        for n in (DIM, FFN, 14336, VOCAB):
            self.b[f"y{n}"] = holo.DeviceBuffer(4 * n)
        for n in ("q", "k", "v", "h"):
            self.b[n] = holo.DeviceBuffer(4 * FFN)

    def __getitem__(self, k):
        return self.b[k].ptr


# ---- layer step ------------------------------------------------------------------------

def layer_fused(lib, L, A, ev=None, kernel_ev=None):
    """The 4 launches of a layer; `ev` = (start, stop) event pairs around each
    launch; `kernel_ev` = (j, start, stop): events on launch j's kernel alone
    (holo_time_next_launch)."""
    b = L.buf
    calls = [
        lambda: lib.holo_batched_qkv(A["q"], A["k"], A["v"], b["q"].ptr, b["k"].ptr, b["v"].ptr, A["x4096"],
                                     DIM, DIM, DIM, Q4_0),
        lambda: lib.cuda_matmul_q4_0(A["y4096"], b["o"].ptr, A["v"], DIM, DIM),
        lambda: lib.holo_batched_ffn_gate_up(A["h"], b["gate"].ptr, b["up"].ptr, A["x4096"], FFN, DIM, Q4_0),
        lambda: lib.cuda_matmul_q4_0(A["y4096"], b["down"].ptr, A["h"], DIM, FFN),
    ]
    for j, c in enumerate(calls):
        if ev and ev[j][0]:
            lib.holo_event_record(ev[j][0])
        if kernel_ev and kernel_ev[0] == j:
            lib.holo_time_next_launch(kernel_ev[1], kernel_ev[2])
        c()
        if ev and ev[j][1]:
            lib.holo_event_record(ev[j][1])


def layer_unfused(lib, L, A):
    """The reference decode loop's pattern: one cuda_matmul_q4_0 per matrix."""
    for name, o, i in LAYER:
        lib.cuda_matmul_q4_0(A[f"y{o}"], L.buf[name].ptr, A[f"x{i}"], o, i)


def capture(lib, fn):
    if lib.holo_graph_begin() != 0:
        raise holo.HoloError("graph capture failed to start")
    fn()
    g = lib.holo_graph_end()
    holo.check("graph capture")
    if not g:
        raise holo.HoloError("graph instantiation failed")
    return g


def time_graphs(lib, graphs, steps, warmup):
    n = len(graphs)
    for i in range(warmup):
        lib.holo_graph_launch(graphs[i % n])
    lib.cuda_sync()
    ev = holo.Events()
    ev.start()
    for i in range(steps):
        lib.holo_graph_launch(graphs[(warmup + i) % n])
    ms = ev.stop()
    lib.cuda_sync()
    ev.close()
    holo.check("timed graphs")
    return ms


MAX_STEPS_PER_GRAPH = 256


def time_steps(lib, layers, step_fn, steps, warmup):
    """Time exactly `steps` layer steps (layer i % len(layers) for step i),
    issued as a decode loop issues its layers: consecutive steps captured
    together in HIP graphs (at most MAX_STEPS_PER_GRAPH per graph), so the
    timed region holds the steps' kernels and no per-step host launch.  The
    `warmup` steps run first, in graphs of their own."""
    def build(first, count):
        out = []
        for g0 in range(0, count, MAX_STEPS_PER_GRAPH):
            n = min(MAX_STEPS_PER_GRAPH, count - g0)
            out.append(capture(lib, lambda g0=g0, n=n: [step_fn(layers[(first + g0 + j) % len(layers)])
                                                        for j in range(n)]))
        return out
    warm = build(0, warmup) if warmup > 0 else []
    timed = build(warmup, steps)
    for g in warm:
        lib.holo_graph_launch(g)
    lib.cuda_sync()
    ev = holo.Events()
    ev.start()
    for g in timed:
        lib.holo_graph_launch(g)
    ms = ev.stop()
    lib.cuda_sync()
    ev.close()
    for g in warm + timed:
        lib.holo_graph_destroy(g)
    holo.check("timed steps")
    return ms


def mean_launch_us(lib, layers, A, steps, which, kernel_only):
    """Mean duration of launch index `which` of the layer step, over `steps`
    layers issued back to back (one synchronisation at the end, as in the
    timed graph pass).  kernel_only: HIP events that the launch records at
    its kernel's start and end (the span rocprofv3's kernel trace measures);
    otherwise events recorded around the call."""
    n = min(steps, 64)
    evs = [(lib.holo_event_create(), lib.holo_event_create()) for _ in range(n)]
    for i in range(n):
        e0, e1 = evs[i]
        if kernel_only:
            layer_fused(lib, layers[i % len(layers)], A, kernel_ev=(which, e0, e1))
        else:
            ev = [(None, None)] * 4
            ev[which] = (e0, e1)
            layer_fused(lib, layers[i % len(layers)], A, ev=ev)
    lib.cuda_sync()
    durs = [lib.holo_event_elapsed_ms(a, b) for a, b in evs]
    for a, b in evs:
        lib.holo_event_destroy(a)
        lib.holo_event_destroy(b)
    holo.check("per-launch pass")
    return 1e3 * statistics.mean(durs)


def kernel_median_us(lib, call, n):
    """Median kernel duration of call(i), i < n, issued back to back with one
    synchronisation at the end: HIP events that each launch records at its
    kernel's start and end (holo_time_next_launch, the span rocprofv3's
    kernel trace measures)."""
    evs = [(lib.holo_event_create(), lib.holo_event_create()) for _ in range(n)]
    for i in range(n):
        lib.holo_time_next_launch(evs[i][0], evs[i][1])
        call(i)
    lib.cuda_sync()
    durs = [lib.holo_event_elapsed_ms(a, b) for a, b in evs]
    for a, b in evs:
        lib.holo_event_destroy(a)
        lib.holo_event_destroy(b)
    holo.check("kernel medians")
    return 1e3 * statistics.median(durs)


def single_gemv_gbs(lib, qtype, sets, steps):
    """Back-to-back launches of one config's matrices, rotating over copies."""
    fn = {Q4_0: lib.cuda_matmul_q4_0, Q8_0: lib.cuda_matmul_q8_0, Q4_K: lib.cuda_matmul_q4_k,
          Q6_K: lib.cuda_matmul_q6_k}[qtype]
    A = sets["acts"]

    def run(k):
        s = sets["mats"][k % len(sets["mats"])]
        for name, o, i in s.shapes:
            fn(A[f"y{o}"], s.buf[name].ptr, A[f"x{i}"], o, i)
    for k in range(4):
        run(k)
    lib.cuda_sync()
    ev = holo.Events()
    ev.start()
    for k in range(steps):
        run(k)
    ms = ev.stop()
    ev.close()
    holo.check("single gemv")
    b = weight_bytes(qtype, sets["mats"][0].shapes)
    return steps * b / (ms * 1e-3) / 1e9, ms * 1e3 / (steps * len(sets["mats"][0].shapes))


def single_gemvs(lib, A, cpu_budget=None):
    """Configs 1 and 3 and the Q6_K GEMV, each over enough copies of its
    matrices to defeat the MALL.  Per matrix shape: the median kernel time
    over >= 128 launches (rotating over the copies) and its fraction of HBM
    peak; per config: the aggregate rate of back-to-back launches and, with a
    CPU budget, the reference CPU path on the same shapes."""
    out = {}
    fn = {Q8_0: lib.cuda_matmul_q8_0, Q4_K: lib.cuda_matmul_q4_k, Q6_K: lib.cuda_matmul_q6_k}
    for qt, cfg, name, shapes, copies in ((Q8_0, 1, "config1_q8_0_4096x4096", CONFIG1, 32),
                                          (Q4_K, 3, "config3_q4_k_llama3_ffn", CONFIG3, 10),
                                          (Q6_K, 6, "q6_k_head_and_down_llama2_7b", Q6K_SHAPES, 4)):
        sets = {"mats": [Mats(qt, i, cfg, shapes) for i in range(copies)], "acts": A}
        g, us = single_gemv_gbs(lib, qt, sets, 4 * copies)
        per = {}
        for mname, o, i in shapes:
            bpl = holo.row_bytes(qt, i) * o
            med = kernel_median_us(lib, lambda k, mname=mname, o=o, i=i: fn[qt](
                A[f"y{o}"], sets["mats"][k % copies].buf[mname].ptr, A[f"x{i}"], o, i), max(128, 4 * copies))
            per[f"{o}x{i}"] = {"kernel_us_median": round(med, 2), "bytes_per_launch": bpl,
                               "gbs": round(bpl / (med * 1e-6) / 1e9, 1),
                               "frac": round(bpl / (med * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        out[name] = {"gbs": round(g, 1), "frac": round(g / HBM_PEAK_GBS, 4), "us_per_launch": round(us, 2),
                     "bytes_per_launch": weight_bytes(qt, shapes) / len(shapes), "per_matrix": per}
        if cpu_budget and qt in (Q8_0, Q4_K):
            out[name]["cpu_baseline"] = cpu_gemvs(qt, cfg, shapes, cpu_budget, 8 if qt == Q8_0 else 2)
        log(f"{name}: {out[name]}")
        del sets
    return out


# ---- config 5: full decode step ----------------------------------------------------------

def decode_step(lib, layers, head, A, ones, matmuls_only, fused=False):
    """Synthetic Llama-2-7B decode step at position 0: RoPE is the identity and
    attention over one cached position returns v, so per layer
      xb = rms(x); q,k,v = W.xb; x += Wo.v; xb = rms(x); h = silu(W1.xb)*(W3.xb);
      x += W2.h
    and after the layers logits = Wout.rms(x).  `matmuls_only` issues the same
    GEMVs on the same buffers without the norms and residual adds.  `fused`
    runs the same step with the norms folded into the q/k/v and gate/up GEMVs
    and the adds into the o and down GEMVs (4 launches per layer, not 8)."""
    x, xb = A["x4096"], A["y4096"]
    if fused:
        for L in layers:
            b = L.buf
            lib.holo_batched_qkv_norm(A["q"], A["k"], A["v"], b["q"].ptr, b["k"].ptr, b["v"].ptr, x, ones.ptr, 1e-5,
                                      xb, DIM, DIM, DIM, Q4_0)
            lib.holo_matmul_add(x, b["o"].ptr, A["v"], x, DIM, DIM, Q4_0)
            lib.holo_batched_ffn_gate_up_norm(A["h"], b["gate"].ptr, b["up"].ptr, x, ones.ptr, 1e-5, xb, FFN, DIM,
                                              Q4_0)
            lib.holo_matmul_add(x, b["down"].ptr, A["h"], x, DIM, FFN, Q4_0)
        lib.cuda_rms_norm(xb, x, ones.ptr, DIM, 1e-5)
        lib.cuda_matmul_q8_0(A["y32000"], head.ptr, xb, VOCAB, DIM)
        return
    for L in layers:
        b = L.buf
        if not matmuls_only:
            lib.cuda_rms_norm(xb, x, ones.ptr, DIM, 1e-5)
        lib.holo_batched_qkv(A["q"], A["k"], A["v"], b["q"].ptr, b["k"].ptr, b["v"].ptr, xb, DIM, DIM, DIM, Q4_0)
        lib.cuda_matmul_q4_0(A["y11008"], b["o"].ptr, A["v"], DIM, DIM)
        if not matmuls_only:
            lib.cuda_vec_add(x, x, A["y11008"], DIM)
            lib.cuda_rms_norm(xb, x, ones.ptr, DIM, 1e-5)
        lib.holo_batched_ffn_gate_up(A["h"], b["gate"].ptr, b["up"].ptr, xb, FFN, DIM, Q4_0)
        lib.cuda_matmul_q4_0(A["y11008"], b["down"].ptr, A["h"], DIM, FFN)
        if not matmuls_only:
            lib.cuda_vec_add(x, x, A["y11008"], DIM)
    if not matmuls_only:
        lib.cuda_rms_norm(xb, x, ones.ptr, DIM, 1e-5)
    lib.cuda_matmul_q8_0(A["y32000"], head.ptr, xb, VOCAB, DIM)


def stream_step_plans(layers, A, ones):
    """The config-5 step's 128 layer GEMVs as one persistent launch each
    (holo_gemv_stream): `matmuls` on the buffers of decode_step(matmuls_only),
    `fused` with the norms in the q/k/v and gate/up staging and the residual
    adds in the o and down stores, in place on x (decode_step(fused))."""
    x, xb = A["x4096"], A["y4096"]
    mm, fz = [], []
    for L in layers:
        b = L.buf
        qkv = [b["q"].ptr, b["k"].ptr, b["v"].ptr]
        gu = [b["gate"].ptr, b["up"].ptr]
        mm += [holo.stream_stage(qkv, [A["q"], A["k"], A["v"]], [DIM] * 3, xb, DIM),
               holo.stream_stage([b["o"].ptr], [A["y11008"]], [DIM], A["v"], DIM),
               holo.stream_stage(gu, [A["h"]], [FFN], xb, DIM, gate_up=True),
               holo.stream_stage([b["down"].ptr], [A["y11008"]], [DIM], A["h"], FFN)]
        fz += [holo.stream_stage(qkv, [A["q"], A["k"], A["v"]], [DIM] * 3, x, DIM, norm_w=ones.ptr),
               holo.stream_stage([b["o"].ptr], [x], [DIM], A["v"], DIM, r=x),
               holo.stream_stage(gu, [A["h"]], [FFN], x, DIM, gate_up=True, norm_w=ones.ptr),
               holo.stream_stage([b["down"].ptr], [x], [DIM], A["h"], FFN, r=x)]
    return holo.StreamPlan(mm, Q4_0), holo.StreamPlan(fz, Q4_0)


def decode_step_stream(lib, plan, head, A, ones, fused):
    """One stream launch for the layers, then (fused) the final norm and the
    Q8_0 head GEMV."""
    if plan.launch() != 0:
        raise holo.HoloError("holo_gemv_stream_launch failed")
    xb = A["y4096"]
    if fused:
        lib.cuda_rms_norm(xb, A["x4096"], ones.ptr, DIM, 1e-5)
    lib.cuda_matmul_q8_0(A["y32000"], head.ptr, xb, VOCAB, DIM)


# ---- config 4 end to end: a prompt through the whole model ------------------------------

class MixedLayer:
    """One synthetic layer in the mix of a Q4_K_M file: Q4_K q/k/o/gate/up,
    Q6_K v and down."""
    TYPES = {"q": Q4_K, "k": Q4_K, "v": Q6_K, "o": Q4_K, "gate": Q4_K, "up": Q4_K, "down": Q6_K}

    def __init__(self, idx):
        self.buf = {name: holo.DeviceBuffer.from_array(
            synth.blocks(self.TYPES[name], o, i, synth.tensor_seed(BASE_SEED, 7, idx, m)))
            for m, (name, o, i) in enumerate(LAYER)}


def prompt_forward_q4_k_m(lib, n_tokens=512):
    """The 512-token prompt of prompt_forward on a Q4_K_M-style Llama-2-7B:
    Q4_K embeddings, q/k/o/gate/up; Q6_K v, down and output head.  Every
    matrix takes the exact batched product (holo_matmul_batch's default);
    its Q6_K matrices are read through a repacked layout, built per call
    (prompt_ms_q6_k_repacked_per_call) or once by holo_llama_prepare before
    the timed prompts (prompt_ms, the load-time form; 1 byte per weight of
    the Q6_K layer matrices, q6_k_prepared_bytes).  Before the batched path,
    every non-Q4_0 matrix of a prompt ran one GEMV per token."""
    layers = [MixedLayer(i) for i in range(32)]
    emb = holo.DeviceBuffer.from_array(synth.blocks(Q4_K, VOCAB, DIM, synth.tensor_seed(BASE_SEED, 7, 32, 0)))
    head = holo.DeviceBuffer.from_array(synth.blocks(Q6_K, VOCAB, DIM, synth.tensor_seed(BASE_SEED, 7, 32, 1)))
    ones = holo.DeviceBuffer.from_array(np.ones(DIM, np.float32))
    T = MixedLayer.TYPES
    L = (holo.LlamaLayer * 32)()
    for i, Ls in enumerate(layers):
        b = Ls.buf
        L[i] = holo.LlamaLayer(ones.ptr, b["q"].ptr, b["k"].ptr, b["v"].ptr, b["o"].ptr, T["q"], T["k"], T["v"],
                               T["o"], ones.ptr, b["gate"].ptr, b["down"].ptr, b["up"].ptr, T["gate"], T["down"],
                               T["up"])
    kv_floats = 32 * n_tokens * DIM
    kc, vc = holo.DeviceBuffer(4 * kv_floats), holo.DeviceBuffer(4 * kv_floats)
    logits = holo.DeviceBuffer(4 * VOCAB)
    m = holo.LlamaModel(n_layers=32, dim=DIM, n_heads=32, n_kv_heads=32, head_dim=128, ffn_dim=FFN, vocab=VOCAB,
                        max_seq=n_tokens, rms_eps=1e-5, rope_base=10000.0, tok_emb=emb.ptr, emb_type=Q4_K,
                        out_norm=ones.ptr, output=head.ptr, out_type=Q6_K, key_cache=kc.ptr, value_cache=vc.ptr,
                        layers=L)
    tokens = np.random.default_rng(6).integers(0, VOCAB, size=n_tokens).astype(np.int32)

    def run():
        rc = lib.holo_llama_forward(C.byref(m), tokens.ctypes.data, n_tokens, 0, logits.ptr, 0)
        if rc != 0:
            raise holo.HoloError(f"holo_llama_forward returned {rc}")

    def timed():
        run()
        lib.cuda_sync()
        ev = holo.Events()
        times = []
        for _ in range(5):  # each prompt timed alone; the median is reported (single prompts vary by up to 20%)
            ev.start()
            run()
            times.append(ev.stop())
        ev.close()
        holo.check("prompt forward q4_k_m")
        return times

    per_call = timed()
    rc = lib.holo_llama_prepare(C.byref(m))
    if rc != 0:
        raise holo.HoloError(f"holo_llama_prepare returned {rc}")
    try:
        times = timed()
    finally:
        lib.holo_llama_release(C.byref(m))
    ms = statistics.median(times)
    q6_bytes = 32 * sum(o * i for name, o, i in LAYER if T[name] == Q6_K)
    return {"prompt_tokens": n_tokens, "prompt_ms": round(ms, 2),
            "prompt_ms_min_max": [round(min(times), 2), round(max(times), 2)],
            "prompt_tokens_per_s": round(n_tokens / (ms * 1e-3), 1),
            "prompt_ms_q6_k_repacked_per_call": round(statistics.median(per_call), 2),
            "q6_k_prepared_bytes": q6_bytes,
            "types": "Q4_K q/k/o/gate/up and embeddings; Q6_K v, down and head"}


def prompt_forward(lib, layers, head, ones, graph_step_ms, n_tokens=512, decode_steps=32):
    """A 512-token prompt through the 32 synthetic Llama-2-7B layers in one pass
    (holo_llama_forward): Q4_0 matmuls on the MFMA prefill GEMM, causal prefill
    attention, KV caches for every position; embeddings tied to the Q8_0 head,
    unit norm weights, random tokens.  The reference runs a prompt as one
    decode step per token (llm.c:1049); the comparison is with the fastest
    decode step here, the graph-captured config-5 step (graph_step_ms), per
    token of the prompt.  The driver's own n = 1 step (not captured, one
    launch per op) is reported beside it."""
    L = (holo.LlamaLayer * 32)()
    for i, Ls in enumerate(layers[:32]):
        b = Ls.buf
        L[i] = holo.LlamaLayer(ones.ptr, b["q"].ptr, b["k"].ptr, b["v"].ptr, b["o"].ptr, Q4_0, Q4_0, Q4_0, Q4_0,
                               ones.ptr, b["gate"].ptr, b["down"].ptr, b["up"].ptr, Q4_0, Q4_0, Q4_0)
    max_seq = n_tokens + decode_steps
    kv_floats = 32 * max_seq * DIM
    kc, vc = holo.DeviceBuffer(4 * kv_floats), holo.DeviceBuffer(4 * kv_floats)
    logits = holo.DeviceBuffer(4 * VOCAB)
    m = holo.LlamaModel(n_layers=32, dim=DIM, n_heads=32, n_kv_heads=32, head_dim=128, ffn_dim=FFN, vocab=VOCAB,
                        max_seq=max_seq, rms_eps=1e-5, rope_base=10000.0, tok_emb=head.ptr, emb_type=Q8_0,
                        out_norm=ones.ptr, output=head.ptr, out_type=Q8_0, key_cache=kc.ptr, value_cache=vc.ptr,
                        layers=L)
    tokens = np.random.default_rng(5).integers(0, VOCAB, size=max_seq).astype(np.int32)
    ev = holo.Events()

    def run(t, pos0):
        rc = lib.holo_llama_forward(C.byref(m), t.ctypes.data, len(t), pos0, logits.ptr, 0)
        if rc != 0:
            raise holo.HoloError(f"holo_llama_forward returned {rc}")

    run(tokens[:n_tokens], 0)  # warm-up (also fills the caches for the decode steps)
    lib.cuda_sync()
    reps = 3
    ev.start()
    for _ in range(reps):
        run(tokens[:n_tokens], 0)
    prompt_ms = ev.stop() / reps
    ev.start()
    for i in range(decode_steps):
        run(tokens[n_tokens + i:n_tokens + i + 1], n_tokens + i)
    step_ms = ev.stop() / decode_steps
    ev.close()
    holo.check("prompt forward")
    out = {"prompt_tokens": n_tokens, "prompt_ms": round(prompt_ms, 2),
           "prompt_tokens_per_s": round(n_tokens / (prompt_ms * 1e-3), 1),
           "driver_decode_step_ms_at_end_of_prompt": round(step_ms, 3)}
    if graph_step_ms:
        out["token_by_token_prompt_ms"] = round(graph_step_ms * n_tokens, 1)
        out["speedup_vs_token_by_token"] = round(graph_step_ms * n_tokens / prompt_ms, 1)
    return out


# ---- config 4: prefill ------------------------------------------------------------------

def decode_attention(lib, kv_lens=(512, 2048, 4096), reps=50):
    """cuda_multi_head_attention at Llama-2-7B shape (32 heads of 128, no
    grouping) over caches of kv_len positions: microseconds per call, issued
    back to back, and the key/value bytes read per second (2 * kv_len * 4096 *
    4 bytes per call)."""
    out = {}
    nh, hd = 32, 128
    q = holo.DeviceBuffer.from_array(synth.normal(nh * hd, 41))
    y = holo.DeviceBuffer(4 * nh * hd)
    for n in kv_lens:
        kc = holo.DeviceBuffer.from_array(synth.normal(n * nh * hd, 42))
        vc = holo.DeviceBuffer.from_array(synth.normal(n * nh * hd, 43))
        for _ in range(5):
            lib.cuda_multi_head_attention(y.ptr, q.ptr, kc.ptr, vc.ptr, n, hd, nh, nh)
        lib.cuda_sync()
        ev = holo.Events()
        ev.start()
        for _ in range(reps):
            lib.cuda_multi_head_attention(y.ptr, q.ptr, kc.ptr, vc.ptr, n, hd, nh, nh)
        ms = ev.stop()
        ev.close()
        holo.check("decode attention")
        us = ms * 1e3 / reps
        out[f"kv_len_{n}"] = {"us_per_call": round(us, 2), "kv_gbs": round(2 * n * nh * hd * 4 / (us * 1e-6) / 1e9, 1),
                              "per_decode_step_32_layers_ms": round(32 * us / 1e3, 3)}
        del kc, vc
    return out


def prefill_tops(lib, reps=10):
    """Config 4 at M = 512, the batched products:
      q8_0: holo_gemm_q4_0_q8_0 (Q8_0 activations, bit-exact specification)
            on the f16 matrix cores (the default), q8_0_int8_mfma the same on
            the int8 matrix cores (identical bits);
      f16:  holo_gemm_q4_0_f16 (f16 activations and dequantised weights);
      exact: holo_matmul_batch_q4_0 (the default of the batched matmuls and
            the prompt forward: fp32-accurate).
    gemm_us is the call (the activation panel pass, the GEMM kernel and the
    stream-ordered workspace), kernel_us the GEMM kernel alone
    (holo_time_next_launch).  Both run on v_mfma_f32_32x32x16_f16; useful work
    is 2*M*N*K."""
    M = 512
    out = {}
    for name, (N, K) in (("11008x4096", (FFN, DIM)), ("4096x11008", (DIM, FFN))):
        W = holo.DeviceBuffer.from_array(synth.blocks(Q4_0, N, K, seed=N + K))
        X = holo.DeviceBuffer.from_array(synth.normal(M * K, seed=K))
        Xq = holo.DeviceBuffer(M * (K // 32) * 34)
        Y = holo.DeviceBuffer(4 * M * N)
        lib.holo_quantize_act_q8_0(Xq.ptr, X.ptr, M, K)
        ev = holo.Events()
        def q8(kind):
            lib.holo_prefill_set_q8_kernel(kind)
            lib.holo_gemm_q4_0_q8_0(Y.ptr, W.ptr, Xq.ptr, M, N, K)
            lib.holo_prefill_set_q8_kernel(0)

        calls = {"q8_0": lambda: q8(0), "q8_0_int8_mfma": lambda: q8(1),
                 "f16": lambda: lib.holo_gemm_q4_0_f16(Y.ptr, W.ptr, X.ptr, M, N, K),
                 "exact": lambda: lib.holo_matmul_batch_q4_0(Y.ptr, W.ptr, X.ptr, M, N, K, None)}
        out[name] = {}
        for prod, call in calls.items():
            call()
            lib.cuda_sync()
            ev.start()
            for _ in range(reps):
                call()
            ms = ev.stop() / reps
            kernel = []
            for _ in range(reps):
                lib.holo_time_next_launch(ev.a, ev.b)
                call()
                lib.cuda_sync()
                kernel.append(float(lib.holo_event_elapsed_ms(ev.a, ev.b)))
            kms = statistics.median(kernel)
            tops = 2.0 * M * N * K / (kms * 1e-3) / 1e12
            out[name][prod] = {"gemm_us": round(ms * 1e3, 2), "kernel_us": round(kms * 1e3, 2),
                               "tops": round(tops, 1), "frac_of_f16_peak": round(tops / F16_PEAK_TFLOPS, 4),
                               "frac_of_int8_peak": round(tops / I8_PEAK_TOPS, 4)}
        ev.start()
        for _ in range(reps):
            lib.holo_quantize_act_q8_0(Xq.ptr, X.ptr, M, K)
        out[name]["q8_0"]["quantize_us"] = round(ev.stop() / reps * 1e3, 2)
        ev.close()
    holo.check("prefill")
    return out


# ---- CPU baseline -------------------------------------------------------------------------

def measured_traffic(xmode: str):
    """HBM bytes per gate/up launch from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by what the counter
    reads for a device-to-device copy of known size); None if no summary
    exists for this activation mode."""
    p = ROOT / "profiles" / f"traffic_q4_0_gateup_{xmode}.json"
    if not p.exists():
        return None
    return json.loads(p.read_text())["traffic_bytes_per_launch"]


def ref_matmul():
    """(kind, matmul(qtype, M, v, out_dim, in_dim), description) of the CPU
    path timed beside the GPU numbers: the reference's own matmul_q
    (src/ai/llm.c:770) compiled into oracle/_ref/ with its release flags when
    that build exists, else the oracle's restatement of it."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc  # checker / baseline only
    if orc.ref_available("release"):
        ref = orc.RefBuild("release")
        return ("reference", lambda t, M, v, o, i: ref.matmul(t, M, v, o, i),
                "oracle/_ref/libholo_ref_release.so: matmul_q of the reference sources built with "
                "-O3 -ffast-math -mavx2 -mfma -fopenmp")
    o_ = orc.Oracle()
    return ("port", lambda t, M, v, o, i: o_.matmul(t, M, v, o, i),
            "oracle/liboracle.so: the oracle's restatement of matmul_q")


def omp_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)


def cpu_median(calls, budget_s: float):
    """Median seconds of one pass over `calls` (after one warm-up pass), over
    as many passes as fit in budget_s (at least 3); (median, passes, total s)."""
    for c in calls:
        c()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 5000):
        t0 = time.perf_counter()
        for c in calls:
            c()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times), sum(times)


def cores_of(qtype) -> int:
    """Threads the reference's matmul_q branch uses: its Q8_0 (and F32) AVX2
    loops carry `#pragma omp parallel for` (llm.c:838); the Q4_0 branch
    (llm.c:893-915) and mat_vec_q4_k (quant.c:626-633) are single-threaded."""
    return omp_threads() if qtype == Q8_0 else 1


def cpu_gemvs(qtype, cfg, shapes, budget_s: float, copies: int) -> dict:
    """The reference CPU path on `copies` copies of a config's matrices (the
    GPU's synthetic weights, the same seeds), one pass = every matrix of every
    copy, so the pass streams more bytes than a host's last-level cache."""
    kind, mm, what = ref_matmul()
    mats = [(synth.blocks(qtype, o, i, synth.tensor_seed(BASE_SEED, cfg, c, m)), o, i)
            for c in range(copies) for m, (_, o, i) in enumerate(shapes)]
    xs = {i: synth.normal(i, i) for _, _, i in shapes}
    med, n, tot = cpu_median([lambda M=M, o=o, i=i: mm(qtype, M, xs[i], o, i) for M, o, i in mats], budget_s)
    b = copies * weight_bytes(qtype, shapes)
    return {"value": round(b / med / 1e9, 3), "unit": "GB/s", "cores": cores_of(qtype), "kind": kind,
            "sample": f"{n} passes (median {med * 1e3:.2f} ms, {tot:.1f} s of CPU work) over {copies} copies of "
                      f"{', '.join(f'{o}x{i}' for _, o, i in shapes)} ({b} weight bytes a pass) with {what}; host "
                      f"has {os.cpu_count()} logical CPUs, OMP_NUM_THREADS="
                      f"{os.environ.get('OMP_NUM_THREADS', 'unset')}"}


def cpu_prefill(budget_s: float, M: int = 512) -> dict:
    """Config 4 on the reference CPU path: it has no batched product, its
    prompt loop runs one decode step per token (llm.c:1049), so M tokens cost
    M sequential matmul_q GEMVs per matrix; the sample times single GEMVs of
    each shape and scales by M."""
    kind, mm, what = ref_matmul()
    out = {}
    for name, (N, K) in (("11008x4096", (FFN, DIM)), ("4096x11008", (DIM, FFN))):
        W = synth.blocks(Q4_0, N, K, seed=N + K)
        x = synth.normal(K, seed=K)
        med, n, tot = cpu_median([lambda: mm(Q4_0, W, x, N, K)], budget_s / 2)
        ms = M * med * 1e3
        out[name] = {"value": round(2.0 * M * N * K / (M * med) / 1e12, 5), "unit": "TOP/s",
                     "ms_for_512_tokens": round(ms, 1), "cores": 1, "kind": kind,
                     "sample": f"{n} GEMVs (median {med * 1e3:.2f} ms, {tot:.1f} s of CPU work) scaled by {M}, "
                               f"with {what}"}
    return out


def cpu_decode_step(budget_s: float) -> dict:
    """Config 5 on the reference CPU path: one layer's 7 Q4_0 GEMVs (1 core)
    and the 32000x4096 Q8_0 head (OpenMP) timed, the step = 32 layers + head."""
    kind, mm, what = ref_matmul()
    mats = [(synth.blocks(Q4_0, o, i, synth.tensor_seed(BASE_SEED, 2, 0, m)), o, i)
            for m, (_, o, i) in enumerate(LAYER)]
    xs = {4096: synth.normal(4096, 11), 11008: synth.normal(11008, 12)}
    head = synth.blocks(Q8_0, VOCAB, DIM, synth.tensor_seed(BASE_SEED, 5, 0, 7))
    t_layer, n1, tot1 = cpu_median([lambda M=M, o=o, i=i: mm(Q4_0, M, xs[i], o, i) for M, o, i in mats],
                                   budget_s * 0.75)
    t_head, n2, tot2 = cpu_median([lambda: mm(Q8_0, head, xs[4096], VOCAB, DIM)], budget_s * 0.25)
    ms = (32 * t_layer + t_head) * 1e3
    b = 32 * weight_bytes(Q4_0, LAYER) + holo.row_bytes(Q8_0, DIM) * VOCAB
    return {"value": round(ms, 1), "unit": "ms per step (matmuls)", "gbs": round(b / (ms * 1e-3) / 1e9, 3),
            "cores": f"1 (Q4_0 layers), {omp_threads()} (Q8_0 head, OpenMP)", "kind": kind,
            "sample": f"{n1} passes over one layer's 7 Q4_0 GEMVs (median {t_layer * 1e3:.1f} ms) x 32 + {n2} "
                      f"head GEMVs (median {t_head * 1e3:.1f} ms), {tot1 + tot2:.1f} s of CPU work, with {what}"}


def cpu_baseline(budget_s: float) -> dict:
    """The reference CPU path on one layer's 7 Q4_0 matrices (bounded sample)."""
    kind, mm, what = ref_matmul()
    mats = [(synth.blocks(Q4_0, o, i, synth.tensor_seed(BASE_SEED, 2, 0, m)), o, i)
            for m, (_, o, i) in enumerate(LAYER)]
    x = {4096: synth.normal(4096, 11), 11008: synth.normal(11008, 12)}
    med, n, tot = cpu_median([lambda M=M, o=o, i=i: mm(Q4_0, M, x[i], o, i) for M, o, i in mats], budget_s)
    b = weight_bytes(Q4_0, LAYER)
    return {"value": round(b / med / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{n} runs (median {med * 1e3:.1f} ms) of one Llama-2-7B layer's 7 Q4_0 GEMVs "
                      f"({b} weight bytes, {tot:.1f} s of CPU work) with {what}; the reference's Q4_0 "
                      f"branch has no OpenMP pragma (llm.c:893-915), so 1 core; host has {os.cpu_count()} "
                      f"logical CPUs"}


# ---- main ----------------------------------------------------------------------------------

def decode_step_config5(lib, layers, A, reps):
    """Config 5: the full decode step (32 layers + the Q8_0 head) as HIP graphs (unfused, fused, matmuls only)
    and with its 128 layer GEMVs in one persistent holo_gemv_stream launch.  Returns (result, fused end-to-end
    ms, head, ones)."""
    head = holo.DeviceBuffer.from_array(synth.blocks(Q8_0, VOCAB, DIM, synth.tensor_seed(BASE_SEED, 5, 0, 7)))
    ones = holo.DeviceBuffer.from_array(np.ones(DIM, np.float32))
    full = capture(lib, lambda: decode_step(lib, layers[:32], head, A, ones, False))
    mm = capture(lib, lambda: decode_step(lib, layers[:32], head, A, ones, True))
    fz = capture(lib, lambda: decode_step(lib, layers[:32], head, A, ones, False, True))
    unfused_ms = time_graphs(lib, [full], reps, 2) / reps
    mm_ms = time_graphs(lib, [mm], reps, 2) / reps
    full_ms = time_graphs(lib, [fz], reps, 2) / reps
    lib.holo_graph_destroy(fz)
    # the same step with the 128 layer GEMVs in one persistent launch
    plan_mm, plan_fz = stream_step_plans(layers[:32], A, ones)
    smm = capture(lib, lambda: decode_step_stream(lib, plan_mm, head, A, ones, False))
    sfz = capture(lib, lambda: decode_step_stream(lib, plan_fz, head, A, ones, True))
    smm_ms = time_graphs(lib, [smm], reps, 2) / reps
    sfz_ms = time_graphs(lib, [sfz], reps, 2) / reps
    if lib.holo_gemv_stream_status() != 0:
        raise holo.HoloError("the persistent decode-step launch could not synchronise")
    for g in (smm, sfz):
        lib.holo_graph_destroy(g)
    plan_mm.close()
    plan_fz.close()
    step_bytes = 32 * weight_bytes(Q4_0, LAYER) + holo.row_bytes(Q8_0, DIM) * VOCAB
    best_mm = min(mm_ms, smm_ms)
    c5 = {
        "matmuls_ms": round(mm_ms, 4), "end_to_end_ms": round(full_ms, 4),
        "end_to_end_unfused_ms": round(unfused_ms, 4),
        "matmuls_stream_ms": round(smm_ms, 4), "end_to_end_stream_ms": round(sfz_ms, 4),
        "weight_bytes": step_bytes, "matmul_weight_gbs": round(step_bytes / (mm_ms * 1e-3) / 1e9, 1),
        "matmul_stream_weight_gbs": round(step_bytes / (smm_ms * 1e-3) / 1e9, 1),
        "end_to_end_weight_gbs": round(step_bytes / (full_ms * 1e-3) / 1e9, 1),
        "frac": round(step_bytes / (best_mm * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "frac_basis": "weight bytes of the step / the faster matmuls-only variant's ms, over 8 TB/s",
        "launches": {"matmuls": 32 * 4 + 1, "end_to_end": 32 * 4 + 2, "end_to_end_unfused": 32 * 8 + 2,
                     "matmuls_stream": 2, "end_to_end_stream": 3}}
    lib.holo_graph_destroy(full)
    lib.holo_graph_destroy(mm)
    log(f"config 5 decode step: matmuls {mm_ms:.3f} ms, end-to-end {full_ms:.3f} ms "
        f"(unfused {unfused_ms:.3f} ms); one stream launch: matmuls {smm_ms:.3f} ms, "
        f"end-to-end {sfz_ms:.3f} ms")
    return c5, full_ms, head, ones


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU-baseline sampling")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--xmode", choices=["mfma", "f32", "i24"], default="mfma", help="GEMV activation mode")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run 3 device-to-device copies of BYTES (HBM counter calibration) and exit")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only run config 4 (prefill GEMM), print its JSON and exit (for profiling)")
    ap.add_argument("--prompt-only", action="store_true",
                    help="only run the 512-token prompt forward over 32 layers, print its JSON and exit")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only run the single-GEMV measurements (configs 1 and 3, Q6_K), print their JSON and exit")
    ap.add_argument("--decode-step-only", action="store_true",
                    help="only run config 5 (the decode step as graphs and as one stream launch) and exit")
    ap.add_argument("--attention-only", action="store_true",
                    help="only run the decode-attention measurement, print its JSON and exit")
    a = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the hot path is a single-GPU decode "
                                   "GEMV (how it would shard is a design note, not built)", "n_gpus": a.gpus}),
              flush=True)
        sys.exit(2)

    lib = holo.load()
    holo.init()
    if a.copy_probe:
        src, dst = holo.DeviceBuffer(a.copy_probe), holo.DeviceBuffer(a.copy_probe)
        ev = holo.Events()
        ev.start()
        for _ in range(3):
            lib.cuda_memcpy_d2d(dst.ptr, src.ptr, a.copy_probe)
        ms = ev.stop() / 3
        holo.check("copy probe")
        print(json.dumps({"copy_bytes": a.copy_probe, "ms": round(ms, 4),
                          "gbs": round(2 * a.copy_probe / (ms * 1e-3) / 1e9, 1)}), flush=True)
        return
    if a.prefill_only:
        print(json.dumps({"config4_prefill_m512": prefill_tops(lib)}), flush=True)
        return
    if a.gemv_only:
        print(json.dumps(single_gemvs(lib, Acts(), None if a.no_cpu else a.cpu_budget / 3)), flush=True)
        return
    if a.attention_only:
        print(json.dumps({"decode_attention_llama2_7b": decode_attention(lib)}), flush=True)
        return
    if a.decode_step_only:
        s = lib.holo_stream_create()
        lib.holo_set_stream(s)  # graphs capture a non-null stream
        c5 = decode_step_config5(lib, [Mats(Q4_0, i, 2, LAYER) for i in range(32)], Acts(), 4)[0]
        print(json.dumps({"config5_decode_step": c5}), flush=True)
        return
    if a.prompt_only:
        layers = [Mats(Q4_0, i, 2, LAYER) for i in range(32)]
        head = holo.DeviceBuffer.from_array(synth.blocks(Q8_0, VOCAB, DIM, synth.tensor_seed(BASE_SEED, 5, 0, 7)))
        ones = holo.DeviceBuffer.from_array(np.ones(DIM, np.float32))
        print(json.dumps({"config4_prompt_forward_512": prompt_forward(lib, layers, head, ones, None)}), flush=True)
        del layers
        print(json.dumps({"prompt_forward_512_q4_k_m": prompt_forward_q4_k_m(lib)}), flush=True)
        return
    stream = lib.holo_stream_create()
    lib.holo_set_stream(stream)  # graphs capture a non-null stream
    lib.holo_gemv_set_xmode({"f32": 0, "i24": 1, "mfma": 2}[a.xmode])
    log(f"device: {lib.cuda_get_device_name().decode(errors='replace')}")

    t0 = time.time()
    layers = [Mats(Q4_0, i, 2, LAYER) for i in range(a.layers)]
    A = Acts()
    log(f"generated + uploaded {a.layers} Q4_0 layers ({a.layers * weight_bytes(Q4_0, LAYER) / 1e9:.2f} GB) "
        f"in {time.time() - t0:.1f}s")

    total_ms = time_steps(lib, layers, lambda L: layer_fused(lib, L, A), a.steps, a.warmup)
    bytes_step = weight_bytes(Q4_0, LAYER)
    gbs = a.steps * bytes_step / (total_ms * 1e-3) / 1e9
    ms_step = total_ms / a.steps
    gu_us = mean_launch_us(lib, layers, A, a.steps, which=2, kernel_only=a.xmode == "mfma")
    gu_call_us = mean_launch_us(lib, layers, A, a.steps, which=2, kernel_only=False)
    gu_bytes = 2 * holo.row_bytes(Q4_0, DIM) * FFN
    achieved = gu_bytes / (gu_us * 1e-6) / 1e9
    log(f"layer step (fused, graph): {ms_step * 1e3:.1f} us/step, {gbs:.0f} GB/s; gate/up kernel {gu_us:.2f} us "
        f"-> {achieved:.0f} GB/s (events around the call: {gu_call_us:.2f} us)")

    extra = {}
    if not a.no_extra:
        # the reference decode loop's pattern: 7 cuda_matmul_q4_0 launches per layer
        ums = time_steps(lib, layers, lambda L: layer_unfused(lib, L, A), a.steps, a.warmup)
        extra["layer_unfused_drop_in"] = {"gbs": round(a.steps * bytes_step / (ums * 1e-3) / 1e9, 1),
                                          "us_per_step": round(ums * 1e3 / a.steps, 2),
                                          "launches_per_step": 7}
        log(f"layer step (7 drop-in launches): {ums * 1e3 / a.steps:.1f} us/step")

        # config 5: full decode step (32 layers + Q8_0 head)
        if a.layers >= 32:
            c5, full_ms, head, ones = decode_step_config5(lib, layers, A, max(3, a.steps // 16))
            extra["config5_decode_step"] = c5
            if not a.no_cpu:
                extra["config5_decode_step"]["cpu_baseline"] = cpu_decode_step(a.cpu_budget / 2)
            extra["config4_prompt_forward_512"] = prompt_forward(lib, layers, head, ones, full_ms)
            log(f"config 4 prompt forward: {extra['config4_prompt_forward_512']}")
            extra["prompt_forward_512_q4_k_m"] = prompt_forward_q4_k_m(lib)
            log(f"prompt forward, Q4_K_M mix: {extra['prompt_forward_512_q4_k_m']}")
            del head

        del layers

        extra.update(single_gemvs(lib, A, None if a.no_cpu else a.cpu_budget / 3))
        extra["config4_prefill_m512"] = prefill_tops(lib)
        if not a.no_cpu:
            extra["config4_prefill_m512"]["cpu_baseline"] = cpu_prefill(a.cpu_budget / 3)
        log(f"config 4 prefill: {extra['config4_prefill_m512']}")
        extra["decode_attention_llama2_7b"] = decode_attention(lib)
        log(f"decode attention: {extra['decode_attention_llama2_7b']}")

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
        "dtype": "q4_0 x f32 -> f32" if a.xmode == "f32" else "q4_0 x (f32 as 22-bit fixed point per 32-block) -> f32 (three int8 planes, int32 block dots on int8 MFMA, fp32 accumulation)",
        "data": "synthetic (seeded GGUF Q4_0 blocks, N(0,1) fp32 activations)",
        "config": {"workload": "Llama-2-7B layer: 7 Q4_0 GEMVs (4x 4096x4096, 2x 11008x4096, 1x 4096x11008) "
                               "as 4 launches (fused q/k/v, o, fused gate/up, down) in a HIP graph, rotating over "
                               f"{a.layers} distinct layers",
                   "weight_bytes_per_step": bytes_step, "batch": 1, "activation_mode": a.xmode},
        "roofline": {"bound": "hbm", "kernel": ("holo::gemv_mfma_kernel<Q4_0, gate/up>" if a.xmode == "mfma" else "holo::gemv_kernel<Q4_0, gate/up>"),
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(a.xmode),
                     "bytes_per_launch": gu_bytes, "mean_launch_us": round(gu_us, 3),
                     "mean_launch_us_events_around_call": round(gu_call_us, 3)},
        "extra": extra,
    }
    if not a.no_cpu:
        log("CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(a.cpu_budget)
    lib.holo_set_stream(None)
    lib.holo_stream_destroy(stream)
    holo.check("bench")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
