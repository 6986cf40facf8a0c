"""GPU tests of the persistent decode-step kernel (holo_gemv_stream_*): a plan
of dependent GEMV stages run as one launch.

Every stage's output is checked against the CPU oracle run on that stage's
own input (the stream's output of the stage it reads), within the 1e-3 bar,
and against the same GEMVs made as separate calls (holo_batched_qkv,
cuda_matmul_*, holo_batched_ffn_gate_up) within 1e-4 normwise: the stream
kernel scales its activation planes per 16 values where the separate calls
scale them per 32, so the two differ by fixed-point rounding only.  Every
stage of a multi-layer chain reads an earlier stage's output, so a missing
or leaky hand-over, or a weight item of one stage consumed as another's,
shows up as a mismatch far above those bounds.  Repeats of one stage and
graph replays are compared bit for bit.  Stages with the rms_norm folded
into their input (or into their output scale) and the residual add into
their stores are compared with the per-launch fused calls
(holo_batched_*_norm, holo_matmul_add) within 2e-5 and with the CPU oracle
within the 1e-3 bar.  holo_gemv_stream_status() must report no exchange
timeout.
"""
import numpy as np
import pytest

from oracle.oracle import max_rel_err, normwise_err

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K = 2, 8, 12


def _up(holo, a):
    return holo.DeviceBuffer.from_array(np.ascontiguousarray(a))


def _bits(buf, n):
    return buf.download(np.uint32, n)


class Layer:
    """Weights of one decode layer: q, k, v, o, gate, up, down."""

    def __init__(self, holo, synth, t, dim, kv, ffn, seed):
        self.shapes = {"q": (dim, dim), "k": (kv, dim), "v": (kv, dim), "o": (dim, kv),
                       "gate": (ffn, dim), "up": (ffn, dim), "down": (dim, ffn)}
        self.host = {n: synth.blocks(t, o, i, seed + j) for j, (n, (o, i)) in enumerate(self.shapes.items())}
        self.dev = {n: _up(holo, w) for n, w in self.host.items()}
        self.dim, self.kv, self.ffn = dim, kv, ffn


def _bufs(holo, dim, kv, ffn):
    return {"q": holo.DeviceBuffer(4 * dim), "k": holo.DeviceBuffer(4 * kv), "v": holo.DeviceBuffer(4 * kv),
            "o": holo.DeviceBuffer(4 * dim), "h": holo.DeviceBuffer(4 * ffn), "y": holo.DeviceBuffer(4 * dim)}


def _plain_stages(holo, L, x_ptr, out):
    d, kv, f, dev = L.dim, L.kv, L.ffn, L.dev
    return [
        holo.stream_stage([dev["q"].ptr, dev["k"].ptr, dev["v"].ptr], [out["q"].ptr, out["k"].ptr, out["v"].ptr],
                          [d, kv, kv], x_ptr, d),
        holo.stream_stage([dev["o"].ptr], [out["o"].ptr], [d], out["v"].ptr, kv),
        holo.stream_stage([dev["gate"].ptr, dev["up"].ptr], [out["h"].ptr], [f], out["o"].ptr, d, gate_up=True),
        holo.stream_stage([dev["down"].ptr], [out["y"].ptr], [d], out["h"].ptr, f),
    ]


def _plain_separate(lib, t, L, x_ptr, out):
    fn = {Q4_0: lib.cuda_matmul_q4_0, Q4_K: lib.cuda_matmul_q4_k}[t]
    d, kv, f, dev = L.dim, L.kv, L.ffn, L.dev
    lib.holo_batched_qkv(out["q"].ptr, out["k"].ptr, out["v"].ptr, dev["q"].ptr, dev["k"].ptr, dev["v"].ptr, x_ptr,
                         d, kv, d, t)
    fn(out["o"].ptr, dev["o"].ptr, out["v"].ptr, d, kv)
    lib.holo_batched_ffn_gate_up(out["h"].ptr, dev["gate"].ptr, dev["up"].ptr, out["o"].ptr, f, d, t)
    fn(out["y"].ptr, dev["down"].ptr, out["h"].ptr, d, f)


@pytest.mark.parametrize("t,dim,kv,ffn,layers", [(Q4_0, 4096, 4096, 11008, 2), (Q4_0, 512, 256, 1280, 3),
                                                 (Q4_K, 1024, 256, 2816, 2), (Q4_0, 768, 256, 1536, 3)],
                         ids=["q4_0-llama2", "q4_0-small", "q4_k-gqa", "q4_0-768"])
def test_stream_layers_match_separate_calls(holo, synth, oracle, t, dim, kv, ffn, layers):
    """`layers` decode layers chained (each layer's down output is the next
    layer's input): 4 * layers stages in one launch, every output against
    the oracle on its own stage input and against the separate calls."""
    print(f"case stream layers type {t} dim {dim} kv {kv} ffn {ffn} x{layers}", flush=True)
    lib = holo.lib()
    Ls = [Layer(holo, synth, t, dim, kv, ffn, seed=900 + dim + t + 10 * i) for i in range(layers)]
    x = synth.normal(dim, seed=31 + dim)
    dx = _up(holo, x)
    got = [_bufs(holo, dim, kv, ffn) for _ in Ls]
    ref = [_bufs(holo, dim, kv, ffn) for _ in Ls]
    stages, xp_g, xp_r = [], dx.ptr, dx.ptr
    for i, L in enumerate(Ls):
        stages += _plain_stages(holo, L, xp_g, got[i])
        _plain_separate(lib, t, L, xp_r, ref[i])
        xp_g, xp_r = got[i]["y"].ptr, ref[i]["y"].ptr
    plan = holo.StreamPlan(stages, t)
    assert plan.launch() == 0
    lib.cuda_sync()
    holo.check("stream")
    assert lib.holo_gemv_stream_status() == 0
    n = {"q": dim, "k": kv, "v": kv, "o": dim, "h": ffn, "y": dim}
    xin = x
    for i, L in enumerate(Ls):
        g = {name: got[i][name].download(np.float32, n[name]) for name in n}
        r = {name: ref[i][name].download(np.float32, n[name]) for name in n}
        # each stage against the oracle on the stage's own input (un-normalised
        # random layers grow without bound: a later layer can overflow, in the
        # oracle as in the separate calls; such stages are skipped)
        want = {"q": oracle.matmul(t, L.host["q"], xin, dim, dim), "k": oracle.matmul(t, L.host["k"], xin, kv, dim),
                "v": oracle.matmul(t, L.host["v"], xin, kv, dim), "o": oracle.matmul(t, L.host["o"], g["v"], dim, kv),
                "h": oracle.silu_mul(oracle.matmul(t, L.host["gate"], g["o"], ffn, dim),
                                     oracle.matmul(t, L.host["up"], g["o"], ffn, dim)),
                "y": oracle.matmul(t, L.host["down"], g["h"], dim, ffn)}
        for name in n:
            if i > 0 and not np.all(np.isfinite(want[name])):
                continue
            e, m = normwise_err(g[name], want[name]), max_rel_err(g[name], want[name])
            assert e <= 1e-3 and m <= 1e-3, (i, name, e, m)
            # the separate calls' chain drifts from this one by the rounding
            # of each earlier stage (about 1e-5 after four stages): compare
            # the first layer only
            if i == 0:
                e = normwise_err(g[name], r[name])
                print(f"  layer 0 {name}: vs separate calls {e:.2e}", flush=True)
                assert e <= 1e-4, (name, e)
        xin = g["y"]
    plan.close()


def _rms(x, w, eps=1e-5):
    x64 = x.astype(np.float64)
    return (x64 / np.sqrt(np.mean(x64 * x64) + eps) * w).astype(np.float32)


@pytest.mark.parametrize("t,dim,kv,ffn,layers", [(Q4_0, 4096, 4096, 11008, 3), (Q4_K, 1024, 512, 2816, 2)],
                         ids=["q4_0-llama2", "q4_k"])
def test_stream_fused_decode_layers(holo, synth, oracle, t, dim, kv, ffn, layers):
    """The decode dataflow at position 0 (attention over one key returns v):
    per layer xb = rms(x) * w1 -> q, k, v; x += Wo v; xb = rms(x) * w2 ->
    h = silu(W1 xb) * (W3 xb); x += W2 h, with the norms in the stages'
    staging and the adds in their stores, in place on x.  Against the
    per-launch fused calls within 1e-5, and against numpy norms + the
    oracle's GEMVs run through every stage within 1e-3."""
    print(f"case stream fused layers type {t} dim {dim} x{layers}", flush=True)
    lib = holo.lib()
    Ls = [Layer(holo, synth, t, dim, dim if t == Q4_0 else kv, ffn, seed=500 + 10 * i) for i in range(layers)]
    kvd = Ls[0].kv
    rng = np.random.default_rng(7)
    nws = [(1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32) for _ in range(2 * layers)]
    dnw = [_up(holo, w) for w in nws]
    x0 = synth.normal(dim, seed=8)
    xs, xr = _up(holo, x0), _up(holo, x0)
    sb, rb = _bufs(holo, dim, kvd, ffn), _bufs(holo, dim, kvd, ffn)
    xb = holo.DeviceBuffer(4 * dim)
    stages = []
    for i, L in enumerate(Ls):
        d = L.dev
        stages += [
            holo.stream_stage([d["q"].ptr, d["k"].ptr, d["v"].ptr], [sb["q"].ptr, sb["k"].ptr, sb["v"].ptr],
                              [dim, kvd, kvd], xs.ptr, dim, norm_w=dnw[2 * i].ptr),
            holo.stream_stage([d["o"].ptr], [xs.ptr], [dim], sb["v"].ptr, kvd, r=xs.ptr),
            holo.stream_stage([d["gate"].ptr, d["up"].ptr], [sb["h"].ptr], [ffn], xs.ptr, dim, gate_up=True,
                              norm_w=dnw[2 * i + 1].ptr),
            holo.stream_stage([d["down"].ptr], [xs.ptr], [dim], sb["h"].ptr, ffn, r=xs.ptr),
        ]
        lib.holo_batched_qkv_norm(rb["q"].ptr, rb["k"].ptr, rb["v"].ptr, d["q"].ptr, d["k"].ptr, d["v"].ptr, xr.ptr,
                                  dnw[2 * i].ptr, np.float32(1e-5), xb.ptr, dim, kvd, dim, t)
        lib.holo_matmul_add(xr.ptr, d["o"].ptr, rb["v"].ptr, xr.ptr, dim, kvd, t)
        lib.holo_batched_ffn_gate_up_norm(rb["h"].ptr, d["gate"].ptr, d["up"].ptr, xr.ptr, dnw[2 * i + 1].ptr,
                                          np.float32(1e-5), xb.ptr, ffn, dim, t)
        lib.holo_matmul_add(xr.ptr, d["down"].ptr, rb["h"].ptr, xr.ptr, dim, ffn, t)
    plan = holo.StreamPlan(stages, t)
    assert plan.launch() == 0
    lib.cuda_sync()
    holo.check("stream fused")
    assert lib.holo_gemv_stream_status() == 0
    got, ref = xs.download(np.float32, dim), xr.download(np.float32, dim)
    e = normwise_err(got, ref)
    print(f"  vs per-launch fused calls {e:.2e}", flush=True)
    assert e <= 2e-5
    # the CPU chain: numpy norms, the oracle's GEMVs, silu_mul
    x = x0.copy()
    for i, L in enumerate(Ls):
        h = L.host
        xb_ = _rms(x, nws[2 * i])
        v = oracle.matmul(t, h["v"], xb_, kvd, dim)
        x = (x + oracle.matmul(t, h["o"], v, dim, kvd)).astype(np.float32)
        xb_ = _rms(x, nws[2 * i + 1])
        hh = oracle.silu_mul(oracle.matmul(t, h["gate"], xb_, ffn, dim), oracle.matmul(t, h["up"], xb_, ffn, dim))
        x = (x + oracle.matmul(t, h["down"], hh, dim, ffn)).astype(np.float32)
    e = normwise_err(got, x)
    print(f"  vs the CPU chain {e:.2e}", flush=True)
    assert e <= 1e-3
    plan.close()


def test_stream_long_plan(holo, synth):
    """1040 stages in one launch (the stage table, 150 KB, is read from
    device memory stage by stage).  Each of 260 layers reads the same input
    and writes outputs of its own, every one equal to the separate
    calls within 1e-5 and the repeats of one layer bit-equal to each other."""
    print("case stream 1040 stages", flush=True)
    lib = holo.lib()
    t, dim, kv, ffn, nl = Q4_0, 512, 256, 1280, 260
    Ls = [Layer(holo, synth, t, dim, kv, ffn, seed=1300 + 10 * i) for i in range(4)]
    dx = _up(holo, synth.normal(dim, seed=1301))
    got = [_bufs(holo, dim, kv, ffn) for _ in range(nl)]
    ref = [_bufs(holo, dim, kv, ffn) for _ in range(4)]
    stages = []
    for i in range(nl):
        stages += _plain_stages(holo, Ls[i % 4], dx.ptr, got[i])
    for i in range(4):
        _plain_separate(lib, t, Ls[i], dx.ptr, ref[i])
    plan = holo.StreamPlan(stages, t)
    assert plan.launch() == 0
    lib.cuda_sync()
    holo.check("stream long plan")
    assert lib.holo_gemv_stream_status() == 0
    n = {"q": dim, "k": kv, "v": kv, "o": dim, "h": ffn, "y": dim}
    want = [{name: _bits(got[j][name], n[name]) for name in n} for j in range(4)]
    for j in range(4):
        for name in n:
            e = normwise_err(got[j][name].download(np.float32, n[name]), ref[j][name].download(np.float32, n[name]))
            assert e <= 1e-5, (j, name, e)
    for i in range(4, nl):
        for name in n:
            assert np.array_equal(_bits(got[i][name], n[name]), want[i % 4][name]), (i, name)
    plan.close()


def test_stream_ragged_rows(holo, synth, oracle):
    """Row counts that leave short tiles, matrices that share a tile, and
    stages so small that most workgroups have no tile (no slot for most
    waves) between larger ones."""
    print("case stream ragged rows", flush=True)
    lib = holo.lib()
    t, K = Q4_0, 768
    r1, r2, r3, r4 = 100, 36, 301, 7
    W = [synth.blocks(t, r, K, seed=40 + j) for j, r in enumerate((r1, r2, r2))]
    G = synth.blocks(t, r3, K, seed=50)
    U = synth.blocks(t, r3, K, seed=51)
    S = synth.blocks(t, r4, K, seed=53)
    x = synth.normal(K, seed=52)
    dW = [_up(holo, w) for w in W]
    dG, dU, dS, dx = _up(holo, G), _up(holo, U), _up(holo, S), _up(holo, x)
    ys = [holo.DeviceBuffer(4 * r) for r in (r1, r2, r2)]
    hy, sy = holo.DeviceBuffer(4 * r3), holo.DeviceBuffer(4 * r4)
    st = [holo.stream_stage([dS.ptr], [sy.ptr], [r4], dx.ptr, K),
          holo.stream_stage([d.ptr for d in dW], [y.ptr for y in ys], [r1, r2, r2], dx.ptr, K),
          holo.stream_stage([dS.ptr], [sy.ptr], [r4], dx.ptr, K),
          holo.stream_stage([dG.ptr, dU.ptr], [hy.ptr], [r3], dx.ptr, K, gate_up=True),
          holo.stream_stage([dS.ptr], [sy.ptr], [r4], dx.ptr, K)]
    plan = holo.StreamPlan(st, t)
    assert plan.launch() == 0
    lib.cuda_sync()
    holo.check("stream ragged")
    assert lib.holo_gemv_stream_status() == 0
    for w, y, r in zip(list(W) + [S], ys + [sy], (r1, r2, r2, r4)):
        want = oracle.matmul(t, w, x, r, K)
        got = y.download(np.float32, r)
        assert normwise_err(got, want) <= 1e-3 and max_rel_err(got, want) <= 1e-3
    want = oracle.silu_mul(oracle.matmul(t, G, x, r3, K), oracle.matmul(t, U, x, r3, K))
    got = hy.download(np.float32, r3)
    assert normwise_err(got, want) <= 1e-3 and max_rel_err(got, want) <= 1e-3
    plan.close()


def test_stream_rewritten_output(holo, synth, oracle):
    """An output vector written again by a later stage whose tiles put its
    rows on other workgroups (the third matrix of a 3-matrix stage, then a
    single matrix), once over all its rows and once over its first half: the
    final vector holds the last writer's rows and, past them, the earlier
    stage's.  Only the last writer of a row stores it in plain fp32; plain
    stores of one row from two XCDs in one launch would race at L2
    write-back."""
    print("case stream rewritten output", flush=True)
    lib = holo.lib()
    t, K = Q4_0, 512
    A1, A2, A3 = (synth.blocks(t, r, K, seed=60 + j) for j, r in enumerate((256, 256, 512)))
    B, C = synth.blocks(t, 512, K, seed=70), synth.blocks(t, 256, K, seed=71)
    x0, x1 = synth.normal(K, seed=72), synth.normal(K, seed=73)
    dA = [_up(holo, a) for a in (A1, A2, A3)]
    dB, dC, dx0, dx1 = _up(holo, B), _up(holo, C), _up(holo, x0), _up(holo, x1)
    u1, u2, y, z = (holo.DeviceBuffer(4 * n) for n in (256, 256, 512, 512))
    for later, rows, W2 in (("full", 512, B), ("half", 256, C)):
        st = [holo.stream_stage([d.ptr for d in dA], [u1.ptr, u2.ptr, y.ptr], [256, 256, 512], dx0.ptr, K),
              holo.stream_stage([dB.ptr if later == "full" else dC.ptr], [y.ptr], [rows], dx1.ptr, K),
              holo.stream_stage([dA[2].ptr], [z.ptr], [512], dx1.ptr, K)]
        plan = holo.StreamPlan(st, t)
        assert plan.launch() == 0
        lib.cuda_sync()
        holo.check("stream rewritten output")
        assert lib.holo_gemv_stream_status() == 0
        first = oracle.matmul(t, A3, x0, 512, K)
        want = first.copy()
        want[:rows] = oracle.matmul(t, W2, x1, rows, K)
        got = y.download(np.float32, 512)
        for name, g, w in (("y", got, want), ("u1", u1.download(np.float32, 256), oracle.matmul(t, A1, x0, 256, K)),
                           ("z", z.download(np.float32, 512), oracle.matmul(t, A3, x1, 512, K))):
            e, m = normwise_err(g, w), max_rel_err(g, w)
            assert e <= 1e-3 and m <= 1e-3, (later, name, e, m)
        plan.close()


def test_stream_rewrite_while_read(holo, synth, oracle):
    """A vector rewritten by a later stage that depends on nothing after the
    stage still reading the old contents (y = A x; z = B y; y = C x): a fast
    workgroup may store the new y while a slow one still copies the old one,
    so every stage output has exchange buffers of its own.  z must be B (A x)
    and the final y must be C x, over repeated launches."""
    print("case stream rewrite while read", flush=True)
    lib = holo.lib()
    t, K = Q4_0, 1024
    A, B, Cm = (synth.blocks(t, 1024, K, seed=80 + j) for j in range(3))
    x = synth.normal(K, seed=83)
    dA, dB, dC, dx = _up(holo, A), _up(holo, B), _up(holo, Cm), _up(holo, x)
    y, z = holo.DeviceBuffer(4 * 1024), holo.DeviceBuffer(4 * 1024)
    plan = holo.StreamPlan([holo.stream_stage([dA.ptr], [y.ptr], [1024], dx.ptr, K),
                            holo.stream_stage([dB.ptr], [z.ptr], [1024], y.ptr, K),
                            holo.stream_stage([dC.ptr], [y.ptr], [1024], dx.ptr, K)], t)
    ya = oracle.matmul(t, A, x, 1024, K)
    want_z, want_y = oracle.matmul(t, B, ya, 1024, K), oracle.matmul(t, Cm, x, 1024, K)
    for rep in range(3):
        assert plan.launch() == 0
        lib.cuda_sync()
        holo.check("stream rewrite while read")
        assert lib.holo_gemv_stream_status() == 0
        for name, got, want in (("z", z.download(np.float32, 1024), want_z), ("y", y.download(np.float32, 1024), want_y)):
            e, m = normwise_err(got, want), max_rel_err(got, want)
            assert e <= 1e-3 and m <= 1e-3, (rep, name, e, m)
    plan.close()


def test_stream_graph_replays(holo, synth):
    """A plan launch captured in a HIP graph replays bit for bit like the
    eager launch, with eager launches of the same plan between replays (each
    launch advances the plan's launch counter, so every launch's exchange tags
    differ from the words the previous one left behind)."""
    print("case stream graph replays", flush=True)
    lib = holo.lib()
    t = Q4_0
    L = Layer(holo, synth, t, 1024, 512, 2816, seed=77)
    x = synth.normal(1024, seed=78)
    dx = _up(holo, x)
    eager, out = _bufs(holo, 1024, 512, 2816), _bufs(holo, 1024, 512, 2816)
    pe = holo.StreamPlan(_plain_stages(holo, L, dx.ptr, eager), t)
    po = holo.StreamPlan(_plain_stages(holo, L, dx.ptr, out), t)
    assert pe.launch() == 0
    lib.cuda_sync()
    s = lib.holo_stream_create()
    lib.holo_set_stream(s)
    try:
        assert lib.holo_graph_begin() == 0
        assert po.launch() == 0
        g = lib.holo_graph_end()
        holo.check("capture")
        assert g
        n = {"q": 1024, "k": 512, "v": 512, "o": 1024, "h": 2816, "y": 1024}
        for rep in range(3):
            lib.cuda_memset(out["y"].ptr, 0, 4 * 1024)
            assert lib.holo_graph_launch(g) == 0
            lib.cuda_sync()
            for name in n:
                assert np.array_equal(_bits(out[name], n[name]), _bits(eager[name], n[name])), (rep, name)
            assert pe.launch() == 0
            lib.cuda_sync()
        lib.holo_graph_destroy(g)
    finally:
        lib.holo_set_stream(None)
        lib.holo_stream_destroy(s)
    assert lib.holo_gemv_stream_status() == 0
    pe.close()
    po.close()


def test_stream_rejects_unsupported(holo, synth):
    """Shapes and types outside the kernel's set are rejected at plan
    creation, with nothing launched."""
    lib = holo.lib()
    W = _up(holo, synth.blocks(Q4_0, 16, 320, seed=1))  # 10 blocks per row: not a multiple of 8
    x = _up(holo, synth.normal(320, seed=2))
    y = holo.DeviceBuffer(64)
    with pytest.raises(holo.HoloError):
        holo.StreamPlan([holo.stream_stage([W.ptr], [y.ptr], [16], x.ptr, 320)], Q4_0)
    W8 = _up(holo, synth.blocks(Q8_0, 16, 512, seed=3))
    x8 = _up(holo, synth.normal(512, seed=4))
    with pytest.raises(holo.HoloError):
        holo.StreamPlan([holo.stream_stage([W8.ptr], [y.ptr], [16], x8.ptr, 512)], Q8_0)
    W2 = _up(holo, synth.blocks(Q4_0, 16, 512, seed=5))
    with pytest.raises(holo.HoloError):  # a residual on a gate/up stage
        holo.StreamPlan([holo.stream_stage([W2.ptr, W2.ptr], [y.ptr], [16], x8.ptr, 512, gate_up=True,
                                           r=y.ptr)], Q4_0)
    # exchange rules: a later input that overlaps an earlier output other than
    # exactly, an output over its own stage's input, two outputs of one stage
    # in one vector
    W3 = _up(holo, synth.blocks(Q4_0, 512, 512, seed=6))
    big = holo.DeviceBuffer(4 * 2048)
    x512 = _up(holo, synth.normal(512, seed=7))
    first = holo.stream_stage([W3.ptr], [big.ptr], [512], x512.ptr, 512)
    with pytest.raises(holo.HoloError):  # reads from the middle of stage 0's output
        holo.StreamPlan([first, holo.stream_stage([W3.ptr], [y.ptr], [16], big.ptr + 256, 512)], Q4_0)
    with pytest.raises(holo.HoloError):  # reads past what stage 0 wrote
        W4 = _up(holo, synth.blocks(Q4_0, 16, 1024, seed=8))
        holo.StreamPlan([first, holo.stream_stage([W4.ptr], [y.ptr], [16], big.ptr, 1024)], Q4_0)
    with pytest.raises(holo.HoloError):  # an output over its own input
        holo.StreamPlan([holo.stream_stage([W3.ptr], [x512.ptr], [512], x512.ptr, 512)], Q4_0)
    with pytest.raises(holo.HoloError):  # two outputs of one stage in one vector
        holo.StreamPlan([holo.stream_stage([W3.ptr, W3.ptr], [big.ptr, big.ptr], [512, 512], x512.ptr, 512)], Q4_0)
    W5 = _up(holo, synth.blocks(Q4_0, 256, 512, seed=9))
    with pytest.raises(holo.HoloError):  # reads past what the last writer (256 rows) stored
        holo.StreamPlan([first, holo.stream_stage([W5.ptr], [big.ptr], [256], x512.ptr, 512),
                         holo.stream_stage([W3.ptr], [y.ptr], [16], big.ptr, 512)], Q4_0)
    ok = holo.StreamPlan([first, holo.stream_stage([W3.ptr], [y.ptr], [16], big.ptr, 512)], Q4_0)
    ok.close()
    # caller memory read with plain loads: [y = A x; x = C w] stores over the
    # x that stage 0 may still be reading on a slow workgroup (stage 1 does
    # not wait for stage 0), so it is rejected; with a stage between them that
    # copies stage 0's whole output, every workgroup is past stage 0 first
    w512 = _up(holo, synth.normal(512, seed=10))
    over_x = holo.stream_stage([W3.ptr], [x512.ptr], [512], w512.ptr, 512)
    with pytest.raises(holo.HoloError):
        holo.StreamPlan([first, over_x], Q4_0)
    mid = holo.DeviceBuffer(4 * 512)
    ok = holo.StreamPlan([first, holo.stream_stage([W3.ptr], [mid.ptr], [512], big.ptr, 512), over_x], Q4_0)
    ok.close()
    with pytest.raises(holo.HoloError):  # a later output over a norm weight read by stage 0
        holo.StreamPlan([holo.stream_stage([W3.ptr], [big.ptr], [512], x512.ptr, 512, norm_w=w512.ptr),
                         holo.stream_stage([W3.ptr], [w512.ptr], [512], mid.ptr, 512)], Q4_0)
    with pytest.raises(holo.HoloError):  # a norm weight in an earlier stage's output
        holo.StreamPlan([first, holo.stream_stage([W3.ptr], [mid.ptr], [512], x512.ptr, 512, norm_w=big.ptr)],
                        Q4_0)
    with pytest.raises(holo.HoloError):  # a residual that overlaps its own output at another offset
        holo.StreamPlan([holo.stream_stage([W3.ptr], [big.ptr + 64], [512], x512.ptr, 512, r=big.ptr)], Q4_0)
    ok = holo.StreamPlan([holo.stream_stage([W3.ptr], [big.ptr], [512], x512.ptr, 512, r=big.ptr)], Q4_0)
    ok.close()
    lib.cuda_sync()
