"""GPU tests of holo_gemv_chain: several dependent GEMV stages in one launch.

Each chain is compared with the same stages made as separate calls
(cuda_matmul_* / holo_batched_qkv / holo_batched_ffn_gate_up), bit for bit,
and with the CPU oracle within the 1e-3 bar.  A stage reads an earlier
stage's output as its activations, so a missing or leaky grid barrier shows
up as a mismatch.  holo_gemv_chain_status() must report no barrier timeout.
"""
import numpy as np
import pytest

from oracle.oracle import max_rel_err, normwise_err

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K = 2, 8, 12


def _up(holo, a):
    return holo.DeviceBuffer.from_array(a)


def _bits(holo, buf, n):
    return buf.download(np.uint32, n)


def _layer(holo, synth, t, dim, kv, ffn, seed):
    """Weights and buffers of one decode layer: q, k, v, o, gate, up, down."""
    shapes = {"q": (dim, dim), "k": (kv, dim), "v": (kv, dim), "o": (dim, kv),
              "gate": (ffn, dim), "up": (ffn, dim), "down": (dim, ffn)}
    host = {n: synth.blocks(t, o, i, seed + j) for j, (n, (o, i)) in enumerate(shapes.items())}
    dev = {n: _up(holo, w) for n, w in host.items()}
    x = synth.normal(dim, seed + 100)
    return shapes, host, dev, x


def _separate(holo, lib, t, shapes, dev, dx, out):
    fn = {Q4_0: lib.cuda_matmul_q4_0, Q4_K: lib.cuda_matmul_q4_k}[t]
    dim, kv, ffn = shapes["q"][0], shapes["k"][0], shapes["gate"][0]
    lib.holo_batched_qkv(out["q"].ptr, out["k"].ptr, out["v"].ptr, dev["q"].ptr, dev["k"].ptr, dev["v"].ptr,
                         dx.ptr, dim, kv, dim, t)
    fn(out["o"].ptr, dev["o"].ptr, out["v"].ptr, dim, kv)
    lib.holo_batched_ffn_gate_up(out["h"].ptr, dev["gate"].ptr, dev["up"].ptr, out["o"].ptr, ffn, dim, t)
    fn(out["y"].ptr, dev["down"].ptr, out["h"].ptr, dim, ffn)


def _chain_stages(holo, shapes, dev, dx, out):
    dim, kv, ffn = shapes["q"][0], shapes["k"][0], shapes["gate"][0]
    return [
        holo.gemv_stage([dev["q"].ptr, dev["k"].ptr, dev["v"].ptr], [out["q"].ptr, out["k"].ptr, out["v"].ptr],
                        [dim, kv, kv], dx.ptr, dim),
        holo.gemv_stage([dev["o"].ptr], [out["o"].ptr], [dim], out["v"].ptr, kv),
        holo.gemv_stage([dev["gate"].ptr, dev["up"].ptr], [out["h"].ptr], [ffn], out["o"].ptr, dim, gate_up=True),
        holo.gemv_stage([dev["down"].ptr], [out["y"].ptr], [dim], out["h"].ptr, ffn),
    ]


def _outputs(holo, shapes):
    dim, kv, ffn = shapes["q"][0], shapes["k"][0], shapes["gate"][0]
    return {"q": holo.DeviceBuffer(4 * dim), "k": holo.DeviceBuffer(4 * kv), "v": holo.DeviceBuffer(4 * kv),
            "o": holo.DeviceBuffer(4 * dim), "h": holo.DeviceBuffer(4 * ffn), "y": holo.DeviceBuffer(4 * dim)}


@pytest.mark.parametrize("t,dim,kv,ffn", [(Q4_0, 4096, 4096, 11008), (Q4_0, 512, 256, 1280),
                                          (Q4_K, 1024, 256, 2816), (Q4_0, 768, 256, 1536)],
                         ids=["q4_0-llama2", "q4_0-small", "q4_k-gqa", "q4_0-768"])
def test_chain_layer_matches_separate_calls(holo, synth, oracle, t, dim, kv, ffn):
    print(f"case chain layer type {t} dim {dim} kv {kv} ffn {ffn}", flush=True)
    lib = holo.lib()
    shapes, host, dev, x = _layer(holo, synth, t, dim, kv, ffn, seed=900 + dim + t)
    dx = _up(holo, x)
    ref, got = _outputs(holo, shapes), _outputs(holo, shapes)
    _separate(holo, lib, t, shapes, dev, dx, ref)
    rc = holo.gemv_chain(_chain_stages(holo, shapes, dev, dx, got), t)
    assert rc == 0
    lib.cuda_sync()
    holo.check("chain")
    assert lib.holo_gemv_chain_status() == 0
    n = {"q": dim, "k": kv, "v": kv, "o": dim, "h": ffn, "y": dim}
    for name in ("q", "k", "v", "o", "h", "y"):
        assert np.array_equal(_bits(holo, got[name], n[name]), _bits(holo, ref[name], n[name])), name
    # the first and last stage against the CPU oracle (teacher-forced input)
    q = got["q"].download(np.float32, dim)
    want_q = oracle.matmul(t, host["q"], x, dim, dim)
    assert normwise_err(q, want_q) <= 1e-3 and max_rel_err(q, want_q) <= 1e-3
    h = got["h"].download(np.float32, ffn)
    y = got["y"].download(np.float32, dim)
    want_y = oracle.matmul(t, host["down"], h, dim, ffn)
    assert normwise_err(y, want_y) <= 1e-3 and max_rel_err(y, want_y) <= 1e-3


def test_chain_ragged_rows(holo, synth, oracle):
    """Row counts that leave short tiles and matrices that share tiles."""
    print("case chain ragged rows", flush=True)
    lib = holo.lib()
    t, K = Q4_0, 768
    r1, r2, r3 = 100, 36, 301
    W = [synth.blocks(t, r, K, seed=40 + j) for j, r in enumerate((r1, r2, r2))]
    G = synth.blocks(t, r3, K, seed=50)
    U = synth.blocks(t, r3, K, seed=51)
    x = synth.normal(K, seed=52)
    dW = [_up(holo, w) for w in W]
    dG, dU, dx = _up(holo, G), _up(holo, U), _up(holo, x)
    ys = [holo.DeviceBuffer(4 * r) for r in (r1, r2, r2)]
    hy = holo.DeviceBuffer(4 * r3)
    st = [holo.gemv_stage([d.ptr for d in dW], [y.ptr for y in ys], [r1, r2, r2], dx.ptr, K),
          holo.gemv_stage([dG.ptr, dU.ptr], [hy.ptr], [r3], dx.ptr, K, gate_up=True)]
    assert holo.gemv_chain(st, t) == 0
    lib.cuda_sync()
    assert lib.holo_gemv_chain_status() == 0
    for w, y, r in zip(W, ys, (r1, r2, r2)):
        want = oracle.matmul(t, w, x, r, K)
        got = y.download(np.float32, r)
        assert normwise_err(got, want) <= 1e-3 and max_rel_err(got, want) <= 1e-3
    want = oracle.silu_mul(oracle.matmul(t, G, x, r3, K), oracle.matmul(t, U, x, r3, K))
    got = hy.download(np.float32, r3)
    assert normwise_err(got, want) <= 1e-3 and max_rel_err(got, want) <= 1e-3


def test_chain_graph_replays(holo, synth):
    """The barrier state survives graph replays: every replay matches the
    eager result, with eager launches between the replays."""
    print("case chain graph replays", flush=True)
    lib = holo.lib()
    t = Q4_0
    shapes, host, dev, x = _layer(holo, synth, t, 1024, 512, 2816, seed=77)
    dx = _up(holo, x)
    eager, out = _outputs(holo, shapes), _outputs(holo, shapes)
    assert holo.gemv_chain(_chain_stages(holo, shapes, dev, dx, eager), t) == 0
    lib.cuda_sync()
    s = lib.holo_stream_create()
    lib.holo_set_stream(s)
    try:
        assert lib.holo_graph_begin() == 0
        assert holo.gemv_chain(_chain_stages(holo, shapes, dev, dx, out), t) == 0
        g = lib.holo_graph_end()
        holo.check("capture")
        assert g
        n = {"q": 1024, "k": 512, "v": 512, "o": 1024, "h": 2816, "y": 1024}
        for rep in range(3):
            lib.cuda_memset(out["y"].ptr, 0, 4 * 1024)
            lib.holo_graph_launch(g)
            lib.cuda_sync()
            for name in n:
                assert np.array_equal(_bits(holo, out[name], n[name]), _bits(holo, eager[name], n[name])), (rep, name)
            # eager work on the same barrier between replays
            assert holo.gemv_chain(_chain_stages(holo, shapes, dev, dx, eager), t) == 0
            lib.cuda_sync()
        lib.holo_graph_destroy(g)
    finally:
        lib.holo_set_stream(None)
        lib.holo_stream_destroy(s)
    assert lib.holo_gemv_chain_status() == 0


def test_chain_rejects_unsupported(holo, synth):
    """Shapes and types outside the MFMA path return HOLO_EINVAL and launch nothing."""
    lib = holo.lib()
    W = _up(holo, synth.blocks(Q4_0, 16, 320, seed=1))  # 10 blocks per row: not a multiple of 8
    x = _up(holo, synth.normal(320, seed=2))
    y = holo.DeviceBuffer(64)
    st = [holo.gemv_stage([W.ptr], [y.ptr], [16], x.ptr, 320)]
    assert holo.gemv_chain(st, Q4_0) == holo.EINVAL
    W8 = _up(holo, synth.blocks(Q8_0, 16, 512, seed=3))
    x8 = _up(holo, synth.normal(512, seed=4))
    assert holo.gemv_chain([holo.gemv_stage([W8.ptr], [y.ptr], [16], x8.ptr, 512)], Q8_0) == holo.EINVAL
    assert holo.gemv_chain([], Q4_0) == holo.EINVAL
    lib.cuda_sync()
    holo.check("rejects")
