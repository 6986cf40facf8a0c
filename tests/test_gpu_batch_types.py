"""GPU parity of the batched products for every weight type the GEMVs serve
(holo_matmul_batch and its multi / add / SwiGLU-add forms, holo_dequant_f16),
through the C ABI.

In HOLO_PREFILL_F16 mode (set for every test here), Q8_0, Q4_K, Q6_K, F16
and F32 weights are dequantised to an f16 panel and multiplied on the f16
product:
  w16 = f16_rne(dequantize_row_*(W))   (quant.c:118-311, bit-exact oracle)
  x16 = f16_rne(x),  Y = sum_k x16 * w16, fp32 accumulation.
Bars:
  * the panel: bit-identical to the oracle's dequant rounded by numpy's
    float16 conversion (round to nearest even, subnormals kept);
  * the product: elementwise within the fp32 accumulation bound
    2 (K/16 + 2) 2^-24 sum_k |x16 w16| of the float64 sum of the rounded
    operands, and within 1e-3 normwise of the reference's fp32 GEMV
    (oracle matmul_q) on the unrounded operands;
  * the multi form, the add in the store and the SwiGLU in the panel:
    bit-identical to the single product and the unfused sequence;
  * M < 64: one GEMV per row, 1e-3 against the oracle.
"""
import ctypes as C

import numpy as np
import pytest

from oracle.oracle import normwise_err

pytestmark = pytest.mark.gpu

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
NAMES = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k"}


def up(holo, a):
    return holo.DeviceBuffer.from_array(np.ascontiguousarray(a))


def down(buf, n, dtype=np.float32):
    return buf.download(dtype, n)


def weights(synth, oracle, t, N, K, seed):
    """(the stream handed to the library, its fp32 dequantisation)."""
    if t == F32:
        w = synth.normal(N * K, seed) * np.float32(0.05)
        return w, w
    if t == F16:
        w16 = (synth.normal(N * K, seed) * np.float32(0.05)).astype(np.float16)
        return w16.view(np.uint16), w16.astype(np.float32)
    b = synth.blocks(t, N, K, seed)
    return b, oracle.dequant(t, b, N * K)


def f16_bound(K, A):
    return 2.0 * (K / 16 + 2) * 2.0 ** -24 * A


@pytest.fixture(autouse=True)
def f16_mode(holo):
    """These tests hold the f16 product (HOLO_PREFILL_F16) to its bound; the
    default exact product is tested in test_gpu_batch_exact.py."""
    holo.lib().holo_prefill_set_mode(0)
    yield
    holo.lib().holo_prefill_set_mode(2)


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q6_K, F32, F16], ids=lambda t: NAMES[t])
def test_dequant_f16_bit_exact(holo, synth, oracle, t):
    n = 256 * 1031
    print(f"case dequant f16 {NAMES[t]} n {n}", flush=True)
    src, w = weights(synth, oracle, t, 1, n, seed=40 + t)
    want = w.astype(np.float16).view(np.uint16)
    ds, dd = up(holo, src), holo.DeviceBuffer(2 * n)
    holo.lib().holo_dequant_f16(dd.ptr, ds.ptr, n, t)
    holo.lib().cuda_sync()
    holo.check("dequant f16")
    assert np.array_equal(down(dd, n, np.uint16), want)


def test_dequant_f16_subnormal_scales(holo, synth, oracle):
    """Q8_0 blocks with scales across the f16 range, subnormals included, so
    that many weights round to f16 subnormals or to zero."""
    nb = 4096
    rng = np.random.default_rng(5)
    blk = np.zeros((nb, 34), np.uint8)
    d = rng.integers(0, 0x3C00, nb).astype(np.uint16)
    d[: nb // 4] = rng.integers(0, 0x0400, nb // 4)  # subnormal scales
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = rng.integers(0, 256, (nb, 32))
    src = blk.reshape(-1)
    want = oracle.dequant(Q8_0, src, nb * 32).astype(np.float16).view(np.uint16)
    ds, dd = up(holo, src), holo.DeviceBuffer(2 * nb * 32)
    holo.lib().holo_dequant_f16(dd.ptr, ds.ptr, nb * 32, Q8_0)
    holo.lib().cuda_sync()
    holo.check("dequant f16 subnormal")
    got = down(dd, nb * 32, np.uint16)
    assert np.count_nonzero((want & 0x7C00) == 0) > 1000  # the case is exercised
    assert np.array_equal(got, want)


CASES = [(Q4_K, 128, 512, 2048), (Q6_K, 96, 384, 1024), (Q8_0, 64, 256, 512), (F16, 80, 256, 256),
         (F32, 70, 200, 128), (Q4_K, 512, 4096, 14336), (Q6_K, 512, 4096, 11008), (Q8_0, 512, 11008, 4096)]


@pytest.mark.parametrize("t,M,N,K", CASES, ids=[f"{NAMES[t]}-{m}x{n}x{k}" for t, m, n, k in CASES])
def test_matmul_batch(holo, synth, oracle, t, M, N, K):
    print(f"case matmul batch {NAMES[t]} {M}x{N}x{K}", flush=True)
    src, w = weights(synth, oracle, t, N, K, seed=M + N + K)
    X = synth.normal(M * K, seed=K + 3).reshape(M, K)
    dW, dX, dY = up(holo, src), up(holo, X), holo.DeviceBuffer(4 * M * N)
    holo.lib().holo_matmul_batch(dY.ptr, dW.ptr, dX.ptr, M, N, K, t)
    holo.lib().cuda_sync()
    holo.check("matmul batch")
    got = down(dY, M * N).reshape(M, N)
    rows = min(M, 24)  # float64 truth on a row subset at the full sizes (CPU time)
    x16 = X[:rows].astype(np.float16).astype(np.float64)
    w16 = w.reshape(N, K).astype(np.float16).astype(np.float64)
    truth = x16 @ w16.T
    A = np.abs(x16) @ np.abs(w16).T
    err = np.abs(got[:rows] - truth)
    print(f"  max |err| / bound {np.max(err / np.maximum(f16_bound(K, A), 1e-30)):.3f}", flush=True)
    assert np.all(err <= f16_bound(K, A))
    if t in (Q8_0, Q4_K, Q6_K):
        ref = np.stack([oracle.matmul(t, src, X[m], N, K) for m in range(4)])
        e = normwise_err(got[:4], ref)
        print(f"  vs the reference GEMV {e:.2e}", flush=True)
        assert e <= 1e-3


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q8_0], ids=lambda t: NAMES[t])
def test_matmul_batch_multi_and_fused(holo, synth, oracle, t):
    """Three matrices in one launch equal three single launches bit for bit;
    the add in the store and the SwiGLU in the panel equal the unfused
    sequence (cuda_silu_mul, the product, an fp32 add), in place."""
    print(f"case matmul batch multi/fused {NAMES[t]}", flush=True)
    lib = holo.lib()
    M, K, Ns = 100, 512, (256, 128, 128)
    srcs = [weights(synth, oracle, t, n, K, seed=60 + i)[0] for i, n in enumerate(Ns)]
    X = synth.normal(M * K, seed=61).reshape(M, K)
    dWs, dX = [up(holo, s) for s in srcs], up(holo, X)
    dYm = [holo.DeviceBuffer(4 * M * n) for n in Ns]
    k = len(Ns)
    lib.holo_matmul_batch_multi((C.c_void_p * k)(*[d.ptr for d in dYm]), (C.c_void_p * k)(*[d.ptr for d in dWs]),
                                (C.c_int * k)(*Ns), k, dX.ptr, M, K, t)
    singles = []
    for i, n in enumerate(Ns):
        d = holo.DeviceBuffer(4 * M * n)
        lib.holo_matmul_batch(d.ptr, dWs[i].ptr, dX.ptr, M, n, K, t)
        singles.append(d)
    N = Ns[0]
    G = synth.normal(M * K, seed=62).reshape(M, K)
    U = synth.normal(M * K, seed=63).reshape(M, K)
    R = synth.normal(M * N, seed=64).reshape(M, N) * 5.0
    dG, dU, dH = up(holo, G), up(holo, U), holo.DeviceBuffer(4 * M * K)
    lib.cuda_silu_mul(dH.ptr, dG.ptr, dU.ptr, M * K)
    dT = holo.DeviceBuffer(4 * M * N)
    lib.holo_matmul_batch(dT.ptr, dWs[0].ptr, dH.ptr, M, N, K, t)
    dS = up(holo, R)
    lib.holo_matmul_batch_add(dS.ptr, dWs[0].ptr, dX.ptr, dS.ptr, M, N, K, t)
    dZ = up(holo, R)
    lib.holo_matmul_batch_swiglu_add(dZ.ptr, dWs[0].ptr, dG.ptr, dU.ptr, dZ.ptr, M, N, K, t)
    lib.cuda_sync()
    holo.check("batch multi/fused")
    for i, n in enumerate(Ns):
        assert np.array_equal(down(dYm[i], M * n).view(np.uint32), down(singles[i], M * n).view(np.uint32)), i
    y0 = down(singles[0], M * N).reshape(M, N)
    assert np.array_equal(down(dS, M * N).reshape(M, N), (R + y0).astype(np.float32))
    assert np.array_equal(down(dZ, M * N).reshape(M, N), (R + down(dT, M * N).reshape(M, N)).astype(np.float32))


@pytest.mark.parametrize("t", [Q4_K, Q6_K], ids=lambda t: NAMES[t])
def test_matmul_batch_few_rows(holo, synth, oracle, t):
    """M < 64: one GEMV per row (and per row for the add, through a scratch
    row, in place)."""
    lib = holo.lib()
    M, N, K = 5, 96, 512
    src, _ = weights(synth, oracle, t, N, K, seed=70)
    X = synth.normal(M * K, seed=71).reshape(M, K)
    R = synth.normal(M * N, seed=72).reshape(M, N)
    dW, dX, dY, dS = up(holo, src), up(holo, X), holo.DeviceBuffer(4 * M * N), up(holo, R)
    lib.holo_matmul_batch(dY.ptr, dW.ptr, dX.ptr, M, N, K, t)
    lib.holo_matmul_batch_add(dS.ptr, dW.ptr, dX.ptr, dS.ptr, M, N, K, t)
    lib.cuda_sync()
    holo.check("batch few rows")
    ref = np.stack([oracle.matmul(t, src, X[m], N, K) for m in range(M)])
    assert normwise_err(down(dY, M * N).reshape(M, N), ref) <= 1e-3
    assert normwise_err(down(dS, M * N).reshape(M, N), R + ref) <= 1e-3


def test_matmul_batch_multi_types(holo, synth, oracle):
    """q/k/v of different types (Q4_K, Q4_0, Q6_K) in one launch: each output
    bit-identical to its own single-type call -- the Q4_0 panel holds the same
    f16 values the Q4_0 kernel unpacks, and the accumulation order is the
    same -- and within the f16 bound of the float64 truth."""
    lib = holo.lib()
    M, K = 100, 512
    types, Ns = (Q4_K, Q4_0, Q6_K), (256, 128, 128)
    srcs, ws = zip(*[weights(synth, oracle, t, n, K, seed=80 + i) for i, (t, n) in enumerate(zip(types, Ns))])
    X = synth.normal(M * K, seed=81).reshape(M, K)
    dWs, dX = [up(holo, s) for s in srcs], up(holo, X)
    dYm = [holo.DeviceBuffer(4 * M * n) for n in Ns]
    k = len(Ns)
    lib.holo_matmul_batch_multi_types((C.c_void_p * k)(*[d.ptr for d in dYm]), (C.c_void_p * k)(*[d.ptr for d in dWs]),
                                      (C.c_int * k)(*types), (C.c_int * k)(*Ns), k, dX.ptr, M, K)
    singles = []
    for i, n in enumerate(Ns):
        d = holo.DeviceBuffer(4 * M * n)
        lib.holo_matmul_batch(d.ptr, dWs[i].ptr, dX.ptr, M, n, K, types[i])
        singles.append(d)
    lib.cuda_sync()
    holo.check("batch multi types")
    x16 = X.astype(np.float16).astype(np.float64)
    for i, n in enumerate(Ns):
        got = down(dYm[i], M * n).reshape(M, n)
        assert np.array_equal(got.view(np.uint32), down(singles[i], M * n).reshape(M, n).view(np.uint32)), i
        w16 = ws[i].reshape(n, K).astype(np.float16).astype(np.float64)
        assert np.all(np.abs(got - x16 @ w16.T) <= f16_bound(K, np.abs(x16) @ np.abs(w16).T)), i
