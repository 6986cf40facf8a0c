"""Config 5 at full size: the synthetic Llama-2-7B Q4_0 decode step (32
layers of q/k/v/o 4096x4096, gate/up 11008x4096, down 4096x11008, and the
32000x4096 Q8_0 head; 3,782,017,024 weight bytes) as bench.py times it: the
fused launches (norm in the q/k/v and gate/up GEMVs, residual add in the o
and down GEMVs).

The step is the Llama decode dataflow at position 0, where RoPE is the
identity and attention over the one cached position returns v
(src/ai/llm.c:1075-1240 with rms_norm and silu of src/ai/tensor.c:218-256):
  xb = rms(x); q, k, v = W.xb; x += Wo.v; xb = rms(x);
  h = silu(W1.xb) * (W3.xb); x += W2.h;   after 32 layers: logits = Wout.rms(x)
with unit norm weights and eps 1e-5.

Checks:
  teacher-forced, every launch of every layer: the oracle's matmul_q (and
      silu_mul) on the GPU's own input to that launch, rms norms in float64;
      bar 1e-3 normwise and elementwise (the GEMV bar);
  end to end: the final logits against the oracle run through the whole step
      from the same x, untethered (errors compound over 225 GEMVs); bar 1e-3
      normwise;
  the same step captured in a HIP graph and replayed twice gives the eager
      logits bit for bit.
"""
import numpy as np
import pytest

from oracle.oracle import max_rel_err, normwise_err

pytestmark = pytest.mark.gpu

Q4_0, Q8_0 = 2, 8
DIM, FFN, VOCAB, NL = 4096, 11008, 32000, 32
EPS = 1e-5
SHAPES = [("q", DIM, DIM), ("k", DIM, DIM), ("v", DIM, DIM), ("o", DIM, DIM), ("gate", FFN, DIM),
          ("up", FFN, DIM), ("down", DIM, FFN)]
TOL = 1e-3


def rms(x):
    """tensor.c:242-256 in float64, rounded to fp32."""
    x64 = x.astype(np.float64)
    return (x64 / np.sqrt(np.mean(x64 * x64) + EPS)).astype(np.float32)


def check(got, want, what):
    e_n, e_r = normwise_err(got, want), max_rel_err(got, want)
    assert np.all(np.isfinite(got)), what
    assert e_n <= TOL and e_r <= TOL, (what, e_n, e_r)
    return max(e_n, e_r)


@pytest.fixture(scope="module")
def model(holo, synth):
    print("case decode step: generating 32 layers + head (3.78 GB)", flush=True)
    host, dev = [], []
    for l in range(NL):
        h = {n: synth.blocks(Q4_0, o, i, synth.tensor_seed(20251201, 5, l, m)) for m, (n, o, i) in enumerate(SHAPES)}
        host.append(h)
        dev.append({n: holo.DeviceBuffer.from_array(a) for n, a in h.items()})
    head = synth.blocks(Q8_0, VOCAB, DIM, synth.tensor_seed(20251201, 5, NL, 0))
    x0 = synth.normal(DIM, 5005)
    return host, dev, head, holo.DeviceBuffer.from_array(head), x0


class Bufs:
    def __init__(self, holo):
        self.x, self.xb = holo.DeviceBuffer(4 * DIM), holo.DeviceBuffer(4 * DIM)
        self.q, self.k, self.v = (holo.DeviceBuffer(4 * DIM) for _ in range(3))
        self.h, self.logits = holo.DeviceBuffer(4 * FFN), holo.DeviceBuffer(4 * VOCAB)
        self.ones = holo.DeviceBuffer.from_array(np.ones(DIM, np.float32))


def launches(lib, B, L):
    """The 4 fused launches of one layer (bench.py decode_step, fused)."""
    return [
        lambda: lib.holo_batched_qkv_norm(B.q.ptr, B.k.ptr, B.v.ptr, L["q"].ptr, L["k"].ptr, L["v"].ptr, B.x.ptr,
                                          B.ones.ptr, EPS, B.xb.ptr, DIM, DIM, DIM, Q4_0),
        lambda: lib.holo_matmul_add(B.x.ptr, L["o"].ptr, B.v.ptr, B.x.ptr, DIM, DIM, Q4_0),
        lambda: lib.holo_batched_ffn_gate_up_norm(B.h.ptr, L["gate"].ptr, L["up"].ptr, B.x.ptr, B.ones.ptr, EPS,
                                                  B.xb.ptr, FFN, DIM, Q4_0),
        lambda: lib.holo_matmul_add(B.x.ptr, L["down"].ptr, B.h.ptr, B.x.ptr, DIM, FFN, Q4_0),
    ]


def head_launches(lib, B, head):
    lib.cuda_rms_norm(B.xb.ptr, B.x.ptr, B.ones.ptr, DIM, EPS)
    lib.cuda_matmul_q8_0(B.logits.ptr, head.ptr, B.xb.ptr, VOCAB, DIM)


def test_decode_step_teacher_forced_and_end_to_end(holo, oracle, model):
    lib = holo.lib()
    host, dev, head_h, head_d, x0 = model
    B = Bufs(holo)
    B.x.upload(x0)
    worst = 0.0
    for l in range(NL):
        W = host[l]
        mm = lambda n, v: oracle.matmul(Q4_0, W[n], v, *[(o, i) for nn, o, i in SHAPES if nn == n][0])
        c = launches(lib, B, dev[l])
        x_in = B.x.download(np.float32, DIM)
        c[0]()
        lib.cuda_sync()
        xb = rms(x_in)
        for n, buf in (("q", B.q), ("k", B.k), ("v", B.v)):
            worst = max(worst, check(buf.download(np.float32, DIM), mm(n, xb), f"layer {l} {n}"))
        v = B.v.download(np.float32, DIM)
        c[1]()
        lib.cuda_sync()
        x_mid = B.x.download(np.float32, DIM)
        worst = max(worst, check(x_mid, x_in + mm("o", v), f"layer {l} o + residual"))
        c[2]()
        lib.cuda_sync()
        xb = rms(x_mid)
        h = B.h.download(np.float32, FFN)
        worst = max(worst, check(h, oracle.silu_mul(mm("gate", xb), mm("up", xb)), f"layer {l} gate/up"))
        c[3]()
        lib.cuda_sync()
        worst = max(worst, check(B.x.download(np.float32, DIM), x_mid + mm("down", h), f"layer {l} down + residual"))
    head_launches(lib, B, head_d)
    lib.cuda_sync()
    holo.check("decode step")
    x_end = B.x.download(np.float32, DIM)
    logits = B.logits.download(np.float32, VOCAB)
    worst = max(worst, check(logits, oracle.matmul(Q8_0, head_h, rms(x_end), VOCAB, DIM), "head"))
    print(f"  teacher-forced worst error {worst:.2e}", flush=True)

    # untethered: the oracle through the whole step from x0
    x = x0.copy()
    for l in range(NL):
        W = host[l]
        xb = rms(x)
        v = oracle.matmul(Q4_0, W["v"], xb, DIM, DIM)
        x = (x + oracle.matmul(Q4_0, W["o"], v, DIM, DIM)).astype(np.float32)
        xb = rms(x)
        h = oracle.silu_mul(oracle.matmul(Q4_0, W["gate"], xb, FFN, DIM), oracle.matmul(Q4_0, W["up"], xb, FFN, DIM))
        x = (x + oracle.matmul(Q4_0, W["down"], h, DIM, FFN)).astype(np.float32)
    want = oracle.matmul(Q8_0, head_h, rms(x), VOCAB, DIM)
    e2e = normwise_err(logits, want)
    print(f"  end-to-end logits normwise error {e2e:.2e} (hidden state {normwise_err(x_end, x):.2e})", flush=True)
    assert e2e <= TOL


def test_decode_step_graph_replays_match_eager(holo, model):
    lib = holo.lib()
    _, dev, _, head_d, x0 = model
    B = Bufs(holo)

    def step():
        for l in range(NL):
            for c in launches(lib, B, dev[l]):
                c()
        head_launches(lib, B, head_d)

    B.x.upload(x0)
    step()
    lib.cuda_sync()
    eager = B.logits.download(np.float32, VOCAB)
    s = lib.holo_stream_create()
    lib.holo_set_stream(s)
    try:
        assert lib.holo_graph_begin() == 0
        step()
        g = lib.holo_graph_end()
        holo.check("capture")
        assert g
        for rep in range(2):
            B.x.upload(x0)
            lib.holo_graph_launch(g)
            lib.cuda_sync()
            assert np.array_equal(B.logits.download(np.float32, VOCAB).view(np.uint32), eager.view(np.uint32)), rep
            B.x.upload(x0)  # eager work between the replays
            step()
            lib.cuda_sync()
        lib.holo_graph_destroy(g)
    finally:
        lib.holo_set_stream(None)
        lib.holo_stream_destroy(s)
    holo.check("graph replays")


# ---- the same step as one persistent holo_gemv_stream launch ------------------------------

def stream_plans(holo, dev, B, y11008):
    """The two 128-stage plans bench.py's stream_step_plans builds, on the same
    buffer layout: `mm` (the matmuls on xb, o and down writing one shared
    y11008 buffer) and `fz` (norms in the q/k/v and gate/up staging, residual
    adds in the o and down stores, in place on x)."""
    mm, fz = [], []
    for L in dev:
        qkv = [L["q"].ptr, L["k"].ptr, L["v"].ptr]
        gu = [L["gate"].ptr, L["up"].ptr]
        mm += [holo.stream_stage(qkv, [B.q.ptr, B.k.ptr, B.v.ptr], [DIM] * 3, B.xb.ptr, DIM),
               holo.stream_stage([L["o"].ptr], [y11008.ptr], [DIM], B.v.ptr, DIM),
               holo.stream_stage(gu, [B.h.ptr], [FFN], B.xb.ptr, DIM, gate_up=True),
               holo.stream_stage([L["down"].ptr], [y11008.ptr], [DIM], B.h.ptr, FFN)]
        fz += [holo.stream_stage(qkv, [B.q.ptr, B.k.ptr, B.v.ptr], [DIM] * 3, B.x.ptr, DIM, norm_w=B.ones.ptr),
               holo.stream_stage([L["o"].ptr], [B.x.ptr], [DIM], B.v.ptr, DIM, r=B.x.ptr),
               holo.stream_stage(gu, [B.h.ptr], [FFN], B.x.ptr, DIM, gate_up=True, norm_w=B.ones.ptr),
               holo.stream_stage([L["down"].ptr], [B.x.ptr], [DIM], B.h.ptr, FFN, r=B.x.ptr)]
    return holo.StreamPlan(mm, Q4_0), holo.StreamPlan(fz, Q4_0)


def oracle_chain(oracle, host, x0):
    """The decode dataflow of the module docstring on the CPU, untethered."""
    x = x0.copy()
    for W in host:
        xb = rms(x)
        v = oracle.matmul(Q4_0, W["v"], xb, DIM, DIM)
        x = (x + oracle.matmul(Q4_0, W["o"], v, DIM, DIM)).astype(np.float32)
        xb = rms(x)
        h = oracle.silu_mul(oracle.matmul(Q4_0, W["gate"], xb, FFN, DIM), oracle.matmul(Q4_0, W["up"], xb, FFN, DIM))
        x = (x + oracle.matmul(Q4_0, W["down"], h, DIM, FFN)).astype(np.float32)
    return x


def test_stream_bench_plans_full_step(holo, oracle, model):
    """bench.py's two 128-stage stream plans at full size.
    `mm`: the last layer's q, k, v, h and down output (the values the shared
    buffers hold after the launch) against the oracle on the GPU's own inputs,
    and a second launch bit-identical to the first.
    `fz`: the hidden state after 32 layers against the oracle run untethered
    through the whole step from the same x, within the 1e-3 bar, and the head
    logits on it likewise."""
    lib = holo.lib()
    host, dev, head_h, head_d, x0 = model
    B = Bufs(holo)
    y11008 = holo.DeviceBuffer(4 * FFN)
    xb = rms(x0)
    B.xb.upload(xb)
    mm, fz = stream_plans(holo, dev, B, y11008)
    try:
        print("case stream mm plan, 128 stages", flush=True)
        outs = []
        for rep in range(2):
            assert mm.launch() == 0
            lib.cuda_sync()
            holo.check("stream mm")
            assert lib.holo_gemv_stream_status() == 0
            outs.append({"q": B.q.download(np.float32, DIM), "k": B.k.download(np.float32, DIM),
                         "v": B.v.download(np.float32, DIM), "h": B.h.download(np.float32, FFN),
                         "y": y11008.download(np.float32, DIM)})
        W = host[-1]
        g = outs[0]
        worst = 0.0
        for n in ("q", "k", "v"):
            worst = max(worst, check(g[n], oracle.matmul(Q4_0, W[n], xb, DIM, DIM), f"mm layer 31 {n}"))
        worst = max(worst, check(g["h"], oracle.silu_mul(oracle.matmul(Q4_0, W["gate"], xb, FFN, DIM),
                                                         oracle.matmul(Q4_0, W["up"], xb, FFN, DIM)), "mm gate/up"))
        worst = max(worst, check(g["y"], oracle.matmul(Q4_0, W["down"], g["h"], DIM, FFN), "mm down"))
        for n in g:
            assert np.array_equal(outs[1][n].view(np.uint32), g[n].view(np.uint32)), n
        print(f"  mm plan: last layer worst error {worst:.2e}, repeat bit-identical", flush=True)

        print("case stream fz plan, 128 stages + head", flush=True)
        B.x.upload(x0)
        assert fz.launch() == 0
        head_launches(lib, B, head_d)
        lib.cuda_sync()
        holo.check("stream fz")
        assert lib.holo_gemv_stream_status() == 0
        x_end = B.x.download(np.float32, DIM)
        logits = B.logits.download(np.float32, VOCAB)
        assert np.all(np.isfinite(x_end)) and np.all(np.isfinite(logits))
        x_want = oracle_chain(oracle, host, x0)
        e_x = normwise_err(x_end, x_want)
        e_l = normwise_err(logits, oracle.matmul(Q8_0, head_h, rms(x_want), VOCAB, DIM))
        print(f"  fz plan: hidden state {e_x:.2e}, logits {e_l:.2e} normwise vs the oracle chain", flush=True)
        assert e_x <= TOL and e_l <= TOL
    finally:
        mm.close()
        fz.close()


def test_stream_128_stages_every_output(holo, oracle, model):
    """The mm plan's 128 stages with an output buffer of its own for every
    stage (q, k, v, gate/up on xb; o on that layer's v; down on that layer's
    h), so every one of the 224 layer GEMVs is checked against the oracle on
    the GPU's own input, within the 1e-3 bar."""
    print("case stream 128 stages, every output", flush=True)
    lib = holo.lib()
    host, dev, _, _, x0 = model
    xb = rms(x0)
    dxb = holo.DeviceBuffer.from_array(xb)
    outs, stages = [], []
    for L in dev:
        o = {"q": holo.DeviceBuffer(4 * DIM), "k": holo.DeviceBuffer(4 * DIM), "v": holo.DeviceBuffer(4 * DIM),
             "o": holo.DeviceBuffer(4 * DIM), "h": holo.DeviceBuffer(4 * FFN), "y": holo.DeviceBuffer(4 * DIM)}
        outs.append(o)
        stages += [holo.stream_stage([L["q"].ptr, L["k"].ptr, L["v"].ptr], [o["q"].ptr, o["k"].ptr, o["v"].ptr],
                                     [DIM] * 3, dxb.ptr, DIM),
                   holo.stream_stage([L["o"].ptr], [o["o"].ptr], [DIM], o["v"].ptr, DIM),
                   holo.stream_stage([L["gate"].ptr, L["up"].ptr], [o["h"].ptr], [FFN], dxb.ptr, DIM, gate_up=True),
                   holo.stream_stage([L["down"].ptr], [o["y"].ptr], [DIM], o["h"].ptr, FFN)]
    plan = holo.StreamPlan(stages, Q4_0)
    try:
        assert plan.launch() == 0
        lib.cuda_sync()
        holo.check("stream 128")
        assert lib.holo_gemv_stream_status() == 0
        worst = 0.0
        for l, (W, o) in enumerate(zip(host, outs)):
            g = {n: o[n].download(np.float32, FFN if n == "h" else DIM) for n in o}
            for n in ("q", "k", "v"):
                worst = max(worst, check(g[n], oracle.matmul(Q4_0, W[n], xb, DIM, DIM), f"layer {l} {n}"))
            worst = max(worst, check(g["o"], oracle.matmul(Q4_0, W["o"], g["v"], DIM, DIM), f"layer {l} o"))
            worst = max(worst, check(g["h"], oracle.silu_mul(oracle.matmul(Q4_0, W["gate"], xb, FFN, DIM),
                                                             oracle.matmul(Q4_0, W["up"], xb, FFN, DIM)),
                                     f"layer {l} gate/up"))
            worst = max(worst, check(g["y"], oracle.matmul(Q4_0, W["down"], g["h"], DIM, FFN), f"layer {l} down"))
        print(f"  224 GEMVs, worst error {worst:.2e}", flush=True)
    finally:
        plan.close()
