"""GPU parity of the fused multi-GEMVs, the prefill path and the remaining
boundary ops, through the C ABI.

Bars:
  * fused GEMVs: as the single GEMVs (relative error 1e-3 normwise and
    elementwise), against the oracle's per-matrix products;
  * prefill: the quantiser and the int8 MFMA product are specified bit for
    bit (oracle_quantize_act_q8_0 / oracle_gemm_q4_0_q8_0): exact equality;
  * non-matmul ops: fp32 arithmetic against float64 numpy, 1e-5 normwise
    (transcendentals: 1e-5 absolute on bounded outputs).
"""
import numpy as np
import pytest

from oracle.oracle import max_rel_err, normwise_err

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
QK = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}


def up(holo, a):
    return holo.DeviceBuffer.from_array(np.ascontiguousarray(a))


def down(buf, n, dtype=np.float32):
    return buf.download(dtype, n)


# ---- fused multi-GEMVs ---------------------------------------------------------------

@pytest.fixture(params=[3, 0], ids=["mfma", "f32"])
def xmode(request, holo):
    holo.lib().holo_gemv_set_xmode(request.param)
    yield request.param
    holo.lib().holo_gemv_set_xmode(2)


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K], ids=["q8_0", "q4_0", "q4_k"])
@pytest.mark.parametrize("dims", [(4096, 1024, 4096), (512, 512, 512), (96, 32, 256 * 3), (37, 13, 256 * 3)],
                         ids=str)
def test_batched_qkv(holo, synth, oracle, t, dims, xmode):
    q_dim, kv_dim, in_dim = dims
    if in_dim % QK[t]:
        pytest.skip("in_dim not a multiple of the block")
    print(f"case qkv type {t} {dims} xmode {xmode}", flush=True)
    Wq, Wk, Wv = (synth.blocks(t, r, in_dim, seed=s) for r, s in ((q_dim, 1), (kv_dim, 2), (kv_dim, 3)))
    x = synth.normal(in_dim, seed=4)
    dW = [up(holo, w) for w in (Wq, Wk, Wv)]
    dx = up(holo, x)
    dy = [holo.DeviceBuffer(4 * r) for r in (q_dim, kv_dim, kv_dim)]
    if t == Q8_0:
        holo.lib().cuda_batched_qkv_q8_0(dy[0].ptr, dy[1].ptr, dy[2].ptr, dW[0].ptr, dW[1].ptr, dW[2].ptr,
                                         dx.ptr, q_dim, kv_dim, in_dim)
    else:
        holo.lib().holo_batched_qkv(dy[0].ptr, dy[1].ptr, dy[2].ptr, dW[0].ptr, dW[1].ptr, dW[2].ptr,
                                    dx.ptr, q_dim, kv_dim, in_dim, t)
    holo.lib().cuda_sync()
    holo.check("qkv")
    for W, y, r in zip((Wq, Wk, Wv), dy, (q_dim, kv_dim, kv_dim)):
        want = oracle.matmul(t, W, x, r, in_dim)
        got = down(y, r)
        assert normwise_err(got, want) <= 1e-3 and max_rel_err(got, want) <= 1e-3


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K], ids=["q8_0", "q4_0", "q4_k"])
@pytest.mark.parametrize("dims", [(11008, 4096), (300, 512), (301, 256 * 3)], ids=str)
def test_batched_gate_up(holo, synth, oracle, t, dims, xmode):
    ffn, in_dim = dims
    print(f"case gate_up type {t} {dims} xmode {xmode}", flush=True)
    W1 = synth.blocks(t, ffn, in_dim, seed=11)
    W3 = synth.blocks(t, ffn, in_dim, seed=12)
    x = synth.normal(in_dim, seed=13)
    d1, d3, dx, dy = up(holo, W1), up(holo, W3), up(holo, x), holo.DeviceBuffer(4 * ffn)
    if t == Q8_0:
        holo.lib().cuda_batched_ffn_gate_up_q8_0(dy.ptr, d1.ptr, d3.ptr, dx.ptr, ffn, in_dim)
    else:
        holo.lib().holo_batched_ffn_gate_up(dy.ptr, d1.ptr, d3.ptr, dx.ptr, ffn, in_dim, t)
    holo.lib().cuda_sync()
    holo.check("gate_up")
    g = oracle.matmul(t, W1, x, ffn, in_dim)
    u = oracle.matmul(t, W3, x, ffn, in_dim)
    want = oracle.silu_mul(g, u)
    got = down(dy, ffn)
    assert normwise_err(got, want) <= 1e-3
    assert max_rel_err(got, want) <= 1e-3


def test_null_matrix_writes_zeros(holo):
    """matmul_q with M == NULL writes zeros (llm.c:772-775)."""
    dy = up(holo, np.full(64, 7.0, np.float32))
    dx = up(holo, np.ones(128, np.float32))
    holo.lib().cuda_matmul_q4_0(dy.ptr, None, dx.ptr, 64, 128)
    holo.lib().cuda_sync()
    assert np.all(down(dy, 64) == 0)


# ---- prefill ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,k", [(3, 64), (64, 4096), (512, 4096), (512, 11008)], ids=str)
def test_quantize_act_bit_exact(holo, synth, oracle, rows, k):
    print(f"case quantize {rows}x{k}", flush=True)
    X = synth.normal(rows * k, seed=rows + k).reshape(rows, k)
    X[0, :32] = 0.0
    dX = up(holo, X)
    dq = holo.DeviceBuffer(rows * (k // 32) * 34)
    holo.lib().holo_quantize_act_q8_0(dq.ptr, dX.ptr, rows, k)
    holo.lib().cuda_sync()
    holo.check("quantize")
    assert np.array_equal(down(dq, rows * (k // 32) * 34, np.uint8), oracle.quantize_act_q8_0(X))


def tile_rows(M):
    """All rows for small M; otherwise the first and last row of every
    32-row band (and the last row of M)."""
    if M <= 96:
        return np.arange(M)
    return np.unique(np.r_[0:M:32, 31:M:32, M - 1])


@pytest.mark.parametrize("M,N,K", [(16, 16, 32), (64, 64, 256), (77, 150, 4096), (512, 11008, 4096),
                                   (512, 4096, 11008)], ids=str)
def test_gemm_q4_0_q8_0_bit_exact(holo, synth, oracle, M, N, K):
    print(f"case gemm {M}x{N}x{K}", flush=True)
    W = synth.blocks(Q4_0, N, K, seed=M + N)
    Xq = oracle.quantize_act_q8_0(synth.normal(M * K, seed=K).reshape(M, K))
    dW, dXq, dY = up(holo, W), up(holo, Xq), holo.DeviceBuffer(4 * M * N)
    holo.lib().holo_gemm_q4_0_q8_0(dY.ptr, dW.ptr, dXq.ptr, M, N, K)
    holo.lib().cuda_sync()
    holo.check("gemm")
    got = down(dY, M * N).reshape(M, N)
    # At the full sizes the oracle runs on a row subset (CPU time) that holds
    # the first and last row of every 32-row band, so every row tile of every
    # tile shape (64 and 128 rows), and every XCD the tiles map to, is checked.
    rows = tile_rows(M)
    want = oracle.gemm_q4_0_q8_0(W, Xq.reshape(M, -1)[rows].copy().reshape(-1), len(rows), N, K)
    assert np.array_equal(got[rows].view(np.uint32), want.reshape(len(rows), N).view(np.uint32))


def f16_bound(K, A):
    """fp32 accumulation on the matrix cores: one rounding per 16-product
    instruction step and per stage, so |y - truth| <= 2 (K/16 + 2) 2^-24 A."""
    return 2.0 * (K / 16 + 2) * 2.0 ** -24 * A


EXACT = 2


def test_matmul_batch_dispatch(holo, synth, oracle):
    """M >= 64: the exact product by default, the f16 product in F16 mode, the
    Q8_0 product in Q8_0 mode; M < 64: one fp32 GEMV per row."""
    N, K = 256, 512
    W = synth.blocks(Q4_0, N, K, seed=1)
    dW = up(holo, W)
    lib = holo.lib()
    assert lib.holo_prefill_get_mode() == EXACT
    for M, mode in ((8, EXACT), (64, EXACT), (64, 0), (64, 1)):
        lib.holo_prefill_set_mode(mode)
        X = synth.normal(M * K, seed=M).reshape(M, K)
        dX, dY = up(holo, X), holo.DeviceBuffer(4 * M * N)
        lib.holo_matmul_batch_q4_0(dY.ptr, dW.ptr, dX.ptr, M, N, K, None)
        lib.cuda_sync()
        lib.holo_prefill_set_mode(EXACT)
        holo.check("batch")
        got = down(dY, M * N).reshape(M, N)
        if M < 64:
            want = np.stack([oracle.matmul(Q4_0, W, X[m], N, K) for m in range(M)])
            assert normwise_err(got, want) <= 1e-3
        elif mode == EXACT:
            truth = oracle.truth_batch(Q4_0, W, X, N, K)
            assert normwise_err(got, truth) <= 1e-5
        elif mode == 0:
            Y, A = oracle.gemm_q4_0_f16(W, X, M, N, K)
            assert np.all(np.abs(got - Y) <= f16_bound(K, A))
        else:
            want = oracle.gemm_q4_0_q8_0(W, oracle.quantize_act_q8_0(X), M, N, K)
            assert np.array_equal(got, want)


@pytest.mark.parametrize("M,N,K", [(64, 128, 256), (77, 150, 4096), (512, 4096, 4096), (512, 11008, 4096),
                                   (512, 4096, 11008), (512, 16384, 4096)], ids=str)
def test_gemm_q4_0_f16(holo, synth, oracle, M, N, K):
    """The f16 product against the float64 truth of the f16-rounded operands
    (oracle_gemm_q4_0_f16), elementwise within the fp32 accumulation bound, and
    against the reference's fp32 GEMV of the same rows within 1e-3."""
    print(f"case gemm f16 {M}x{N}x{K}", flush=True)
    W = synth.blocks(Q4_0, N, K, seed=M + N + 1)
    X = synth.normal(M * K, seed=K + 1).reshape(M, K)
    dW, dX, dY = up(holo, W), up(holo, X), holo.DeviceBuffer(4 * M * N)
    holo.lib().holo_gemm_q4_0_f16(dY.ptr, dW.ptr, dX.ptr, M, N, K)
    holo.lib().cuda_sync()
    holo.check("gemm f16")
    got = down(dY, M * N).reshape(M, N)
    rows = min(M, 16)  # the oracle on a row subset at the full sizes (CPU time)
    Y, A = oracle.gemm_q4_0_f16(W, X[:rows], rows, N, K)
    assert np.all(np.abs(got[:rows] - Y) <= f16_bound(K, A))
    ref = np.stack([oracle.matmul(Q4_0, W, X[m], N, K) for m in range(min(rows, 4))])
    assert normwise_err(got[:len(ref)], ref) <= 1e-3


@pytest.mark.parametrize("M,Ns,K", [(100, (256, 128, 128), 512), (512, (4096, 1024, 1024), 4096),
                                    (64, (384, 384), 256), (77, (150,), 1024), (512, (11008, 11008), 4096)], ids=str)
def test_gemm_multi_matches_single(holo, synth, oracle, M, Ns, K):
    """Several matrices over the same activations in one launch: every output
    bit-identical to its single-matrix launch (Q8_0 and f16 products), and the
    Q8_0 product to the oracle."""
    import ctypes as C
    print(f"case gemm multi {M}x{Ns}x{K}", flush=True)
    lib = holo.lib()
    Ws = [synth.blocks(Q4_0, n, K, seed=7 + i) for i, n in enumerate(Ns)]
    X = synth.normal(M * K, seed=3).reshape(M, K)
    Xq = oracle.quantize_act_q8_0(X)
    dWs = [up(holo, w) for w in Ws]
    dXq, dX = up(holo, Xq), up(holo, X)
    dYs = [holo.DeviceBuffer(4 * M * n) for n in Ns]
    dYb = [holo.DeviceBuffer(4 * M * n) for n in Ns]
    k = len(Ns)
    Yp = (C.c_void_p * k)(*[d.ptr for d in dYs])
    Wp = (C.c_void_p * k)(*[d.ptr for d in dWs])
    Np = (C.c_int * k)(*Ns)
    lib.holo_gemm_q4_0_q8_0_multi(Yp, Wp, Np, k, dXq.ptr, M, K)
    Yb = (C.c_void_p * k)(*[d.ptr for d in dYb])
    lib.holo_prefill_set_mode(0)  # the f16 product
    try:
        lib.holo_matmul_batch_q4_0_multi(Yb, Wp, Np, k, dX.ptr, M, K, None)
    finally:
        lib.holo_prefill_set_mode(EXACT)
    dYf = [holo.DeviceBuffer(4 * M * n) for n in Ns]
    lib.holo_gemm_q4_0_f16_multi((C.c_void_p * k)(*[d.ptr for d in dYf]), Wp, Np, k, dX.ptr, M, K)
    lib.cuda_sync()
    holo.check("gemm multi")
    for i, n in enumerate(Ns):
        dS = holo.DeviceBuffer(4 * M * n)
        lib.holo_gemm_q4_0_q8_0(dS.ptr, dWs[i].ptr, dXq.ptr, M, n, K)
        lib.cuda_sync()
        got = down(dYs[i], M * n)
        assert np.array_equal(got.view(np.uint32), down(dS, M * n).view(np.uint32)), i
        gf = down(dYf[i], M * n)
        assert np.array_equal(down(dYb[i], M * n).view(np.uint32), gf.view(np.uint32)), i
        dF = holo.DeviceBuffer(4 * M * n)
        lib.holo_gemm_q4_0_f16(dF.ptr, dWs[i].ptr, dX.ptr, M, n, K)
        lib.cuda_sync()
        assert np.array_equal(down(dF, M * n).view(np.uint32), gf.view(np.uint32)), i
        rows = min(M, 16)
        want = oracle.gemm_q4_0_q8_0(Ws[i], Xq.reshape(M, -1)[:rows].copy().reshape(-1), rows, n, K)
        assert np.array_equal(got.reshape(M, n)[:rows].view(np.uint32), want.view(np.uint32)), i


@pytest.mark.parametrize("M,mode", [(100, 2), (100, 0), (8, 2), (100, 1)], ids=["exact", "f16", "gemv_rows", "q8_0"])
def test_batch_add_and_swiglu(holo, synth, oracle, M, mode):
    """Y = R + X.W^T and Y = R + (silu(G)*U).W^T with the add in the GEMM's
    store and the SwiGLU in its panel: bit-identical to the unfused sequence
    (cuda_silu_mul, the batched product, an fp32 add), in place and out of
    place; M < 64 runs GEMVs, within 1e-3 of the oracle."""
    print(f"case batch add/swiglu M {M} mode {mode}", flush=True)
    lib = holo.lib()
    N, K = 256, 512
    W = synth.blocks(Q4_0, N, K, seed=31)
    X = synth.normal(M * K, seed=32).reshape(M, K)
    G = synth.normal(M * K, seed=33).reshape(M, K)
    U = synth.normal(M * K, seed=34).reshape(M, K)
    R = synth.normal(M * N, seed=35).reshape(M, N) * 5.0
    dW, dX, dU = up(holo, W), up(holo, X), up(holo, U)
    lib.holo_prefill_set_mode(mode)
    try:
        # unfused reference on the GPU: H = silu(G)*U, T = H.W^T, T2 = X.W^T
        dG, dH = up(holo, G), holo.DeviceBuffer(4 * M * K)
        lib.cuda_silu_mul(dH.ptr, dG.ptr, dU.ptr, M * K)
        dT, dT2 = holo.DeviceBuffer(4 * M * N), holo.DeviceBuffer(4 * M * N)
        lib.holo_matmul_batch_q4_0(dT.ptr, dW.ptr, dH.ptr, M, N, K, None)
        lib.holo_matmul_batch_q4_0(dT2.ptr, dW.ptr, dX.ptr, M, N, K, None)
        dY, dR = holo.DeviceBuffer(4 * M * N), up(holo, R)
        lib.holo_matmul_batch_q4_0_add(dY.ptr, dW.ptr, dX.ptr, dR.ptr, M, N, K)
        dS = up(holo, R)  # in place: S += X.W^T
        lib.holo_matmul_batch_q4_0_add(dS.ptr, dW.ptr, dX.ptr, dS.ptr, M, N, K)
        dG2, dZ = up(holo, G), up(holo, R)  # in place: Z += swiglu(G, U).W^T
        lib.holo_matmul_batch_q4_0_swiglu_add(dZ.ptr, dW.ptr, dG2.ptr, dU.ptr, dZ.ptr, M, N, K)
        lib.cuda_sync()
        holo.check("batch add")
    finally:
        lib.holo_prefill_set_mode(EXACT)
    t2 = down(dT2, M * N).reshape(M, N)
    want = (R + t2).astype(np.float32)
    got = down(dY, M * N).reshape(M, N)
    if M >= 64:
        assert np.array_equal(got, want)
        assert np.array_equal(down(dZ, M * N).reshape(M, N), (R + down(dT, M * N).reshape(M, N)).astype(np.float32))
    else:
        ref = R + np.stack([oracle.matmul(Q4_0, W, X[m], N, K) for m in range(M)])
        assert normwise_err(got, ref) <= 1e-3
        h = (G / (1.0 + np.exp(-G.astype(np.float64))) * U).astype(np.float32)
        refz = R + np.stack([oracle.matmul(Q4_0, W, h[m], N, K) for m in range(M)])
        assert normwise_err(down(dZ, M * N).reshape(M, N), refz) <= 1e-3
    assert np.array_equal(down(dS, M * N).reshape(M, N), got)


def test_gemm_multi_rejects(holo, synth):
    import ctypes as C
    lib = holo.lib()
    d = holo.DeviceBuffer(4 * 64 * 256)
    w = up(holo, synth.blocks(Q4_0, 200, 256, seed=1))
    q = holo.DeviceBuffer(64 * 8 * 34)
    Yp = (C.c_void_p * 2)(d.ptr, d.ptr)
    Wp = (C.c_void_p * 2)(w.ptr, w.ptr)
    lib.holo_last_error()
    lib.holo_gemm_q4_0_q8_0_multi(Yp, Wp, (C.c_int * 2)(200, 200), 2, q.ptr, 64, 256)  # N not a multiple of 128
    assert lib.holo_last_error() == 100001
    lib.holo_gemm_q4_0_q8_0_multi(Yp, Wp, (C.c_int * 2)(128, 128), 4, q.ptr, 64, 256)  # too many matrices
    assert lib.holo_last_error() == 100001


# ---- decode-layer fusions -----------------------------------------------------------------

def rms_norm_np(x, w, eps):
    x64 = x.astype(np.float64)
    return (x64 / np.sqrt(np.mean(x64 * x64) + eps) * w).astype(np.float32)


@pytest.mark.parametrize("t,dim,kv", [(Q4_0, 4096, 1024), (Q4_K, 4096, 4096), (Q4_0, 11008, 512), (Q8_0, 2048, 512)],
                         ids=["q4_0", "q4_k", "q4_0_long", "q8_0"])
def test_qkv_and_gate_up_with_norm(holo, synth, oracle, t, dim, kv):
    """holo_batched_qkv_norm / _gate_up_norm against cuda_rms_norm followed by
    the plain fused GEMV (1e-5 normwise: only the norm's summation order
    differs) and against the oracle on numpy's norm (1e-3).  in_dim 11008 and
    Q8_0 run the unfused route through xb."""
    print(f"case norm-fused type {t} dim {dim}", flush=True)
    lib = holo.lib()
    eps = 1e-5
    x = synth.normal(dim, seed=5) * 3.0
    w = (1.0 + 0.1 * synth.normal(dim, seed=6)).astype(np.float32)
    Ws = [synth.blocks(t, n, dim, seed=10 + i) for i, n in enumerate((dim, kv, kv))]
    dWs = [up(holo, m) for m in Ws]
    dx, dw = up(holo, x), up(holo, w)
    dxb = holo.DeviceBuffer(4 * dim)
    outs = [holo.DeviceBuffer(4 * n) for n in (dim, kv, kv)]
    refs = [holo.DeviceBuffer(4 * n) for n in (dim, kv, kv)]
    lib.holo_batched_qkv_norm(outs[0].ptr, outs[1].ptr, outs[2].ptr, dWs[0].ptr, dWs[1].ptr, dWs[2].ptr, dx.ptr,
                              dw.ptr, eps, dxb.ptr, dim, kv, dim, t)
    lib.cuda_rms_norm(dxb.ptr, dx.ptr, dw.ptr, dim, eps)
    lib.holo_batched_qkv(refs[0].ptr, refs[1].ptr, refs[2].ptr, dWs[0].ptr, dWs[1].ptr, dWs[2].ptr, dxb.ptr,
                         dim, kv, dim, t)
    lib.cuda_sync()
    holo.check("qkv norm")
    xn = rms_norm_np(x, w, eps)
    for i, n in enumerate((dim, kv, kv)):
        got = down(outs[i], n)
        assert normwise_err(got, down(refs[i], n)) <= 1e-5, i
        assert normwise_err(got, oracle.matmul(t, Ws[i], xn, n, dim)) <= 1e-3, i
    # gate/up: silu(W1 xn) * (W3 xn)
    ffn = kv
    dg = holo.DeviceBuffer(4 * ffn)
    lib.holo_batched_ffn_gate_up_norm(dg.ptr, dWs[1].ptr, dWs[2].ptr, dx.ptr, dw.ptr, eps, dxb.ptr, ffn, dim, t)
    lib.cuda_sync()
    holo.check("gate_up norm")
    g = oracle.matmul(t, Ws[1], xn, ffn, dim).astype(np.float64)
    u = oracle.matmul(t, Ws[2], xn, ffn, dim).astype(np.float64)
    assert normwise_err(down(dg, ffn), g / (1.0 + np.exp(-g)) * u) <= 1e-3


@pytest.mark.parametrize("t,out_dim,in_dim", [(Q4_0, 4096, 4096), (Q4_0, 4096, 11008), (Q8_0, 1024, 4096),
                                              (Q4_K, 2048, 4096), (0, 256, 512)],
                         ids=["q4_0", "q4_0_down", "q8_0", "q4_k", "f32"])
def test_matmul_add(holo, synth, oracle, t, out_dim, in_dim):
    """y = r + W.v with the add in the GEMV's store: in place (y is r) and out
    of place, bit-identical to each other, and within 1e-3 of the oracle.  F32
    runs the unfused route (out of place only)."""
    print(f"case matmul_add type {t} {out_dim}x{in_dim}", flush=True)
    lib = holo.lib()
    W = synth.blocks(t, out_dim, in_dim, seed=21) if t else synth.normal(out_dim * in_dim, seed=21)
    v = synth.normal(in_dim, seed=22)
    r = synth.normal(out_dim, seed=23) * 10.0
    dW, dv, dr = up(holo, W), up(holo, v), up(holo, r)
    dy = holo.DeviceBuffer(4 * out_dim)
    lib.holo_matmul_add(dy.ptr, dW.ptr, dv.ptr, dr.ptr, out_dim, in_dim, t)
    lib.cuda_sync()
    holo.check("matmul_add")
    got = down(dy, out_dim)
    want = r.astype(np.float64) + (oracle.matmul(t, W, v, out_dim, in_dim) if t else
                                   W.reshape(out_dim, in_dim).astype(np.float64) @ v)
    assert normwise_err(got, want) <= 1e-3
    if t:
        lib.holo_matmul_add(dr.ptr, dW.ptr, dv.ptr, dr.ptr, out_dim, in_dim, t)  # in place
        lib.cuda_sync()
        holo.check("matmul_add in place")
        assert np.array_equal(down(dr, out_dim), got)
    else:
        lib.holo_last_error()
        lib.holo_matmul_add(dr.ptr, dW.ptr, dv.ptr, dr.ptr, out_dim, in_dim, t)
        assert lib.holo_last_error() == 100001  # in place only for the block formats


# ---- remaining boundary ops --------------------------------------------------------------

def test_vector_and_activation_ops(holo, synth):
    n = 5000
    a, b = synth.normal(n, seed=1), synth.normal(n, seed=2)
    da, db, dd = up(holo, a), up(holo, b), holo.DeviceBuffer(4 * n)
    L = holo.lib()
    L.cuda_vec_add(dd.ptr, da.ptr, db.ptr, n); L.cuda_sync()
    assert np.array_equal(down(dd, n), a + b)
    L.cuda_vec_mul(dd.ptr, da.ptr, db.ptr, n); L.cuda_sync()
    assert np.array_equal(down(dd, n), a * b)
    L.cuda_vec_scale(dd.ptr, da.ptr, 0.5, n); L.cuda_sync()
    assert np.array_equal(down(dd, n), a * np.float32(0.5))
    dot = L.cuda_vec_dot(da.ptr, db.ptr, n)
    assert abs(dot - float(np.dot(a.astype(np.float64), b))) < 1e-3
    a64 = a.astype(np.float64)
    silu = a64 / (1 + np.exp(-a64))
    L.cuda_silu_mul(dd.ptr, da.ptr, db.ptr, n); L.cuda_sync()
    assert normwise_err(down(dd, n), silu * b) < 1e-5
    dc = up(holo, a); L.cuda_silu(dc.ptr, n); L.cuda_sync()
    assert normwise_err(down(dc, n), silu) < 1e-5
    dc = up(holo, a); L.cuda_gelu(dc.ptr, n); L.cuda_sync()
    gelu = 0.5 * a64 * (1 + np.tanh(0.7978845608 * (a64 + 0.044715 * a64 ** 3)))
    assert normwise_err(down(dc, n), gelu) < 1e-5
    dc = up(holo, a); L.cuda_relu(dc.ptr, n); L.cuda_sync()
    assert np.array_equal(down(dc, n), np.maximum(a, 0))
    holo.check("vector ops")


def test_norm_softmax_argmax(holo, synth):
    n = 4096
    x, w = synth.normal(n, seed=3), synth.normal(n, seed=4)
    dx, dw, dd = up(holo, x), up(holo, w), holo.DeviceBuffer(4 * n)
    L = holo.lib()
    L.cuda_rms_norm(dd.ptr, dx.ptr, dw.ptr, n, 1e-5); L.cuda_sync()
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 ** 2) + 1e-5) * w
    assert normwise_err(down(dd, n), want) < 1e-5
    L.cuda_layer_norm(dd.ptr, dx.ptr, dw.ptr, None, n, 1e-5); L.cuda_sync()   # the reference's layer norm = RMS norm
    assert normwise_err(down(dd, n), want) < 1e-5
    L.cuda_softmax(dd.ptr, dx.ptr, n); L.cuda_sync()
    e = np.exp(x64 - x64.max())
    assert normwise_err(down(dd, n), e / e.sum()) < 1e-5
    v = synth.normal(32000, seed=5)
    v[12345] = 99.0
    v[20000] = 99.0
    dvv = up(holo, v)
    assert L.cuda_argmax(dvv.ptr, 32000) == 12345              # first index of the maximum
    holo.check("norm/softmax/argmax")


def test_attention_and_rope(holo, synth):
    L = holo.lib()
    hd, nh, nkv, kv_len = 128, 8, 2, 37
    q = synth.normal(nh * hd, seed=6)
    kc = synth.normal(kv_len * nkv * hd, seed=7)
    vc = synth.normal(kv_len * nkv * hd, seed=8)
    dq, dk, dv, dd = up(holo, q), up(holo, kc), up(holo, vc), holo.DeviceBuffer(4 * nh * hd)
    L.cuda_multi_head_attention(dd.ptr, dq.ptr, dk.ptr, dv.ptr, kv_len, hd, nh, nkv); L.cuda_sync()
    K = kc.reshape(kv_len, nkv, hd).astype(np.float64)
    V = vc.reshape(kv_len, nkv, hd).astype(np.float64)
    want = np.zeros((nh, hd))
    for h in range(nh):
        g = h // (nh // nkv)
        s = K[:, g, :] @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
        p = np.exp(s - s.max()); p /= p.sum()
        want[h] = p @ V[:, g, :]
    assert normwise_err(down(dd, nh * hd), want.ravel()) < 1e-5
    datt = holo.DeviceBuffer(4 * kv_len)
    L.cuda_attention_single(dd.ptr, dq.ptr, dk.ptr, dv.ptr, datt.ptr, kv_len, hd, 1, nkv * hd); L.cuda_sync()
    s = K[:, 1, :] @ q[:hd] / np.sqrt(hd); p = np.exp(s - s.max()); p /= p.sum()
    assert normwise_err(down(dd, hd), p @ V[:, 1, :]) < 1e-5
    # RoPE on pairs (i, i + hd/2)
    kk = synth.normal(nkv * hd, seed=9)
    dq2, dk2 = up(holo, q), up(holo, kk)
    pos, base = 17, 10000.0
    L.cuda_rope_apply(dq2.ptr, dk2.ptr, pos, hd, nh, nkv, base); L.cuda_sync()

    def rope(a, nheads):
        a = a.reshape(nheads, hd).astype(np.float64).copy()
        i = np.arange(hd // 2)
        th = pos / base ** (2 * i / hd)
        c, s_ = np.cos(th), np.sin(th)
        x0, x1 = a[:, :hd // 2].copy(), a[:, hd // 2:].copy()
        a[:, :hd // 2], a[:, hd // 2:] = x0 * c - x1 * s_, x0 * s_ + x1 * c
        return a.ravel()
    assert normwise_err(down(dq2, nh * hd), rope(q, nh)) < 1e-5
    assert normwise_err(down(dk2, nkv * hd), rope(kk, nkv)) < 1e-5
    # attention_scores / attention_apply
    S, T = 3, 5
    Q = synth.normal(S * hd, seed=10).reshape(S, hd)
    Kt = synth.normal(T * hd, seed=11).reshape(T, hd)
    ds = holo.DeviceBuffer(4 * S * T)
    dQ, dKt = up(holo, Q), up(holo, Kt)   # keep the buffers alive across the calls
    L.cuda_attention_scores(ds.ptr, dQ.ptr, dKt.ptr, S, T, hd, 0.125); L.cuda_sync()
    sc = Q.astype(np.float64) @ Kt.T * 0.125
    assert normwise_err(down(ds, S * T), sc.ravel()) < 1e-5
    do = holo.DeviceBuffer(4 * S * hd)
    L.cuda_attention_apply(do.ptr, ds.ptr, dKt.ptr, S, T, hd); L.cuda_sync()
    assert normwise_err(down(do, S * hd), (down(ds, S * T).reshape(S, T) @ Kt).ravel()) < 1e-5
    holo.check("attention/rope")


@pytest.mark.parametrize("t", [0, 1, Q8_0, Q4_0, Q6_K], ids=["f32", "f16", "q8_0", "q4_0", "q6_k"])
def test_embeddings_and_dense_gemv(holo, synth, oracle, t):
    dim, vocab = 512, 40
    if t == 0:
        E = synth.normal(vocab * dim, seed=1)
        rows = E.reshape(vocab, dim)
    elif t == 1:
        rows16 = (synth.normal(vocab * dim, seed=1) * np.float32(0.1)).astype(np.float16)
        E = rows16.view(np.uint16)
        rows = rows16.astype(np.float32).reshape(vocab, dim)
    else:
        E = synth.blocks(t, vocab, dim, seed=2)
        rows = oracle.dequant(t, E, vocab * dim).reshape(vocab, dim)
    dE, dd = up(holo, E), holo.DeviceBuffer(4 * dim)
    fn = {0: "cuda_get_embedding_f32", 1: "cuda_get_embedding_f16", Q8_0: "cuda_get_embedding_q8_0",
          Q4_0: "cuda_get_embedding_q4_0", Q6_K: "cuda_get_embedding_q6_k"}[t]
    for tok in (0, 7, vocab - 1):
        getattr(holo.lib(), fn)(dd.ptr, dE.ptr, tok, dim, vocab)
        holo.lib().cuda_sync()
        assert np.array_equal(down(dd, dim), rows[tok]), tok        # bit-exact dequant of one row
    if t in (0, 1, Q6_K):
        x = synth.normal(dim, seed=3)
        dx, dy = up(holo, x), holo.DeviceBuffer(4 * vocab)
        holo.lib().holo_matmul(dy.ptr, dE.ptr, dx.ptr, vocab, dim, t)
        holo.lib().cuda_sync()
        want = rows.astype(np.float64) @ x
        assert normwise_err(down(dy, vocab), want) < 1e-5
    holo.check("embedding")


@pytest.mark.parametrize("M,N,K", [(64, 256, 512), (77, 150, 4096), (200, 640, 1056), (512, 11008, 4096),
                                   (512, 4096, 11008)], ids=str)
def test_gemm_q4_0_q8_0_int8_and_f16_kernels_agree(holo, synth, oracle, M, N, K):
    """The Q8_0 product on the f16 matrix cores (the default) and on the int8
    ones compute the same specification: bit-identical outputs, and equal to
    the oracle on the first and last row of every 32-row band (1056 = 33
    blocks: an odd block count, which the int8 kernel hands to the f16 one)."""
    print(f"case q8 kernels {M}x{N}x{K}", flush=True)
    lib = holo.lib()
    assert lib.holo_prefill_get_q8_kernel() == 0
    W = synth.blocks(Q4_0, N, K, seed=3 * M + N)
    Xq = oracle.quantize_act_q8_0(synth.normal(M * K, seed=K + 1).reshape(M, K))
    dW, dXq = up(holo, W), up(holo, Xq)
    outs = []
    try:
        for kind in (1, 0):
            lib.holo_prefill_set_q8_kernel(kind)
            dY = holo.DeviceBuffer(4 * M * N)
            lib.holo_gemm_q4_0_q8_0(dY.ptr, dW.ptr, dXq.ptr, M, N, K)
            lib.cuda_sync()
            holo.check("q8 kernel")
            outs.append(down(dY, M * N).reshape(M, N))
    finally:
        lib.holo_prefill_set_q8_kernel(0)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    rows = tile_rows(M)
    want = oracle.gemm_q4_0_q8_0(W, Xq.reshape(M, -1)[rows].copy().reshape(-1), len(rows), N, K)
    assert np.array_equal(outs[0][rows].view(np.uint32), want.view(np.uint32))
