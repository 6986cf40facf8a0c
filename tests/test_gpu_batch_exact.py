"""GPU parity of the exact batched product (HOLO_PREFILL_EXACT, the default of
holo_matmul_batch* and of the prompt forward), through the C ABI.

The product (prefill_exact.hip) holds the activations as two f16 halves
(x = xh + xl to 2^-22), the weights as the blocks' exact integers with
their fp32 scales, and accumulates in fp32.  Its truth is the float64 product
of the fp32 activations and the bit-exact dequantised weights (the reference's
dequantize_row_* restated in the oracle, quant.c:118-311), the quantity the
reference's fp32 forward approximates one token at a time (llm.c:1049).
Bars:
  * elementwise |got - truth| <= (nb + 70) 2^-24 sum_k |x w| (the split, the
    matrix core's fp32 accumulation of a block's 64 products and one fp32
    rounding per block), with nb = K / 32; doubled for Q4_K, whose min term
    adds a block sum of x;
  * normwise against the truth <= 1e-5, and against the reference's own fp32
    GEMV (oracle matmul_q) <= 1e-5 on a few rows;
  * the multi form, mixed types, the add in the store and the SwiGLU in the
    activation halves: bit-identical to the single product and the unfused
    sequence.
"""
import ctypes as C

import numpy as np
import pytest

from oracle.oracle import normwise_err

pytestmark = pytest.mark.gpu

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
NAMES = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k"}
EXACT = 2


def up(holo, a):
    return holo.DeviceBuffer.from_array(np.ascontiguousarray(a))


def down(buf, n, dtype=np.float32):
    return buf.download(dtype, n)


def weights(synth, oracle, t, N, K, seed):
    """(the stream handed to the library, its fp32 dequantisation [N][K])."""
    if t == F32:
        w = synth.normal(N * K, seed) * np.float32(0.05)
        return w, w.reshape(N, K)
    if t == F16:
        w16 = (synth.normal(N * K, seed) * np.float32(0.05)).astype(np.float16)
        return w16.view(np.uint16), w16.astype(np.float32).reshape(N, K)
    b = synth.blocks(t, N, K, seed)
    return b, oracle.dequant(t, b, N * K).reshape(N, K)


def check_rows(got, X, w, rows, t, K):
    """got[rows] against the float64 truth, elementwise and normwise."""
    Xr = X[rows].astype(np.float64)
    W = w.astype(np.float64)
    truth = Xr @ W.T
    A = np.abs(Xr) @ np.abs(W).T
    bound = (K / 32 + 70) * 2.0 ** -24 * A * (2.0 if t == Q4_K else 1.0)
    err = np.abs(got[rows] - truth)
    e_n = normwise_err(got[rows], truth)
    print(f"  max |err| / bound {np.max(err / np.maximum(bound, 1e-30)):.3f}, normwise {e_n:.2e}", flush=True)
    assert np.all(err <= bound)
    assert e_n <= 1e-5


@pytest.fixture(autouse=True)
def exact_mode(holo):
    lib = holo.lib()
    assert lib.holo_prefill_get_mode() == EXACT  # the default
    yield
    lib.holo_prefill_set_mode(EXACT)


CASES = [(Q4_0, 64, 128, 256), (Q4_0, 77, 150, 4096), (Q4_0, 66, 256, 1056), (Q4_0, 512, 11008, 4096),
         (Q4_0, 512, 4096, 11008), (Q8_0, 100, 256, 512), (Q8_0, 70, 192, 1056), (Q8_0, 512, 4096, 4096),
         (Q4_K, 128, 512, 2048), (Q4_K, 512, 14336, 4096), (Q4_K, 512, 4096, 14336), (Q6_K, 96, 384, 1024),
         (Q6_K, 65, 200, 256),
         (Q6_K, 512, 4096, 11008), (F16, 80, 256, 256), (F16, 512, 1024, 4096), (F32, 70, 200, 128)]


@pytest.mark.parametrize("t,M,N,K", CASES, ids=[f"{NAMES[t]}-{m}x{n}x{k}" for t, m, n, k in CASES])
def test_exact_product(holo, synth, oracle, t, M, N, K):
    print(f"case exact product {NAMES[t]} {M}x{N}x{K}", flush=True)
    src, w = weights(synth, oracle, t, N, K, seed=M + N + K)
    X = synth.normal(M * K, seed=K + 5).reshape(M, K)
    dW, dX, dY = up(holo, src), up(holo, X), holo.DeviceBuffer(4 * M * N)
    holo.lib().holo_matmul_batch(dY.ptr, dW.ptr, dX.ptr, M, N, K, t)
    holo.lib().cuda_sync()
    holo.check("exact product")
    got = down(dY, M * N).reshape(M, N)
    assert np.all(np.isfinite(got))
    # at the full sizes: the first and last row of every 32-row band, so every
    # row tile (64 or 128 rows) and the XCD it maps to is checked
    rows = np.arange(M) if M * N * K <= 64 * 4096 * 4096 else np.unique(np.r_[0:M:32, 31:M:32, 0:4, M - 4:M])
    check_rows(got, X, w, rows, t, K)
    if t in (Q4_0, Q8_0, Q4_K, Q6_K):
        ref = np.stack([oracle.matmul(t, src, X[m], N, K) for m in range(3)])
        e = normwise_err(got[:3], ref)
        print(f"  vs the reference fp32 GEMV {e:.2e}", flush=True)
        assert e <= 1e-5


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q4_K, Q6_K, F16], ids=lambda t: NAMES[t])
def test_exact_multi_and_fused(holo, synth, oracle, t):
    """Three matrices in one launch equal three single launches bit for bit;
    Y = R + X.W^T (add in the store, in place) and Y = R + (silu(G)*U).W^T
    (SwiGLU in the activation halves) equal the unfused sequence
    (cuda_silu_mul, the product, an fp32 add)."""
    print(f"case exact multi/fused {NAMES[t]}", flush=True)
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
    holo.check("exact multi/fused")
    for i, n in enumerate(Ns):
        assert np.array_equal(down(dYm[i], M * n).view(np.uint32), down(singles[i], M * n).view(np.uint32)), i
    y0 = down(singles[0], M * N).reshape(M, N)
    assert np.array_equal(down(dS, M * N).reshape(M, N), (R + y0).astype(np.float32))
    assert np.array_equal(down(dZ, M * N).reshape(M, N), (R + down(dT, M * N).reshape(M, N)).astype(np.float32))


def test_exact_multi_types(holo, synth, oracle):
    """q/k/v of different types (a Q4_K_M file's Q4_K, Q4_K, Q6_K, and a Q4_0
    and Q8_0 mix): each output bit-identical to its own single-type call and
    within the bound of the float64 truth."""
    lib = holo.lib()
    M, K = 100, 512
    for types in ((Q4_K, Q4_K, Q6_K), (Q4_0, Q4_0, Q8_0)):
        print(f"case exact multi types {[NAMES[t] for t in types]}", flush=True)
        Ns = (256, 128, 128)
        srcs, ws = zip(*[weights(synth, oracle, t, n, K, seed=80 + i) for i, (t, n) in enumerate(zip(types, Ns))])
        X = synth.normal(M * K, seed=81).reshape(M, K)
        dWs, dX = [up(holo, s) for s in srcs], up(holo, X)
        dYm = [holo.DeviceBuffer(4 * M * n) for n in Ns]
        k = len(Ns)
        lib.holo_matmul_batch_multi_types((C.c_void_p * k)(*[d.ptr for d in dYm]),
                                          (C.c_void_p * k)(*[d.ptr for d in dWs]), (C.c_int * k)(*types),
                                          (C.c_int * k)(*Ns), k, dX.ptr, M, K)
        singles = []
        for i, n in enumerate(Ns):
            d = holo.DeviceBuffer(4 * M * n)
            lib.holo_matmul_batch(d.ptr, dWs[i].ptr, dX.ptr, M, n, K, types[i])
            singles.append(d)
        lib.cuda_sync()
        holo.check("exact multi types")
        for i, n in enumerate(Ns):
            got = down(dYm[i], M * n).reshape(M, n)
            assert np.array_equal(got.view(np.uint32), down(singles[i], M * n).reshape(M, n).view(np.uint32)), i
            check_rows(got, X, ws[i], np.arange(M), types[i], K)


@pytest.mark.parametrize("t,K", [(Q4_0, 11008), (Q6_K, 11008), (Q4_K, 16384)], ids=["q4_0-11008", "q6_k-11008",
                                                                                      "q4_k-16384"])
def test_exact_swiglu_long_rows(holo, synth, oracle, t, K):
    """The SwiGLU split of rows longer than 4096 (the down projection's 11008,
    and the longest row the split takes): Y = R + (silu(G)*U).W^T equals
    cuda_silu_mul, the product and an fp32 add bit for bit, within the bound
    of the float64 truth."""
    print(f"case exact swiglu long rows {NAMES[t]} K {K}", flush=True)
    lib = holo.lib()
    M, N = 72, 128
    src, w = weights(synth, oracle, t, N, K, seed=K + t)
    G = synth.normal(M * K, seed=K + 31).reshape(M, K)
    U = synth.normal(M * K, seed=K + 32).reshape(M, K)
    R = synth.normal(M * N, seed=K + 33).reshape(M, N)
    dW, dG, dU, dH = up(holo, src), up(holo, G), up(holo, U), holo.DeviceBuffer(4 * M * K)
    lib.cuda_silu_mul(dH.ptr, dG.ptr, dU.ptr, M * K)
    dT = holo.DeviceBuffer(4 * M * N)
    lib.holo_matmul_batch(dT.ptr, dW.ptr, dH.ptr, M, N, K, t)
    dZ = up(holo, R)
    lib.holo_matmul_batch_swiglu_add(dZ.ptr, dW.ptr, dG.ptr, dU.ptr, dZ.ptr, M, N, K, t)
    lib.cuda_sync()
    holo.check("exact swiglu long rows")
    H = down(dH, M * K).reshape(M, K)
    T = down(dT, M * N).reshape(M, N)
    assert np.array_equal(down(dZ, M * N).reshape(M, N), (R + T).astype(np.float32))
    check_rows(T, H, w, np.r_[0:4, M - 4:M], t, K)


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q4_K, Q6_K, F16], ids=lambda t: NAMES[t])
def test_exact_product_row_range(holo, synth, oracle, t):
    """Rows far from unit scale: the split scales each row by a power of two
    (largest magnitude into [2^14, 2^15)) and the store scales back, so rows
    near 1e5 (past f16's 65504), 1e30, 1e-6 and 1e-30 (whose low halves would
    be f16 subnormals or zero unscaled) keep the same elementwise bound and
    1e-5 normwise against the float64 truth as unit rows; a zero row gives
    zeros.  The fused add and SwiGLU forms take the same split."""
    print(f"case exact product row range {NAMES[t]}", flush=True)
    M, N, K = 64, 256, 512
    src, w = weights(synth, oracle, t, N, K, seed=90 + t)
    X = synth.normal(M * K, seed=91).reshape(M, K)
    scales = {0: 1e5, 1: 7e4, 2: 1e30, 3: 1e-6, 4: 1e-30, 5: 0.0}
    for r, f in scales.items():
        X[r] *= np.float32(f)
    dW, dX, dY = up(holo, src), up(holo, X), holo.DeviceBuffer(4 * M * N)
    lib = holo.lib()
    lib.holo_matmul_batch(dY.ptr, dW.ptr, dX.ptr, M, N, K, t)
    lib.cuda_sync()
    holo.check("exact product row range")
    got = down(dY, M * N).reshape(M, N)
    assert np.all(np.isfinite(got))
    assert np.all(got[5] == 0.0)
    for r in range(M):
        if r == 5:
            continue
        check_rows(got, X, w, np.array([r]), t, K)
    # SwiGLU in the split with a large up row: silu(g) * u past f16 range
    G = synth.normal(M * K, seed=92).reshape(M, K)
    U = synth.normal(M * K, seed=93).reshape(M, K)
    U[0] *= np.float32(1e6)
    U[1] *= np.float32(1e-7)
    dG, dU, dH, dT = up(holo, G), up(holo, U), holo.DeviceBuffer(4 * M * K), holo.DeviceBuffer(4 * M * N)
    lib.cuda_silu_mul(dH.ptr, dG.ptr, dU.ptr, M * K)
    lib.holo_matmul_batch(dT.ptr, dW.ptr, dH.ptr, M, N, K, t)
    Z = np.zeros((M, N), np.float32)
    dZ = up(holo, Z)
    lib.holo_matmul_batch_swiglu_add(dZ.ptr, dW.ptr, dG.ptr, dU.ptr, dZ.ptr, M, N, K, t)
    lib.cuda_sync()
    holo.check("exact swiglu row range")
    H = down(dH, M * K).reshape(M, K)
    T = down(dT, M * N).reshape(M, N)
    assert np.all(np.isfinite(T))
    assert np.array_equal(down(dZ, M * N).reshape(M, N), (Z + T).astype(np.float32))
    for r in (0, 1, 2):
        check_rows(T, H, w, np.array([r]), t, K)


@pytest.mark.parametrize("M,N,K", [(100, 384, 1024), (512, 4096, 4096)], ids=["whole-tiles", "parts"])
def test_prepared_q6_k(holo, synth, oracle, M, N, K):
    """holo_prefill_prepare keeps a repacked copy of a Q6_K matrix: products
    on it (plain, add form, a captured graph replayed twice) give the bits of
    the per-call repack, and so does the plain product after release.  It
    rejects another type, a K that is not a multiple of 256, and a second
    shape for a registered matrix."""
    print(f"case prepared q6_k {M}x{N}x{K}", flush=True)
    lib = holo.lib()
    src, w = weights(synth, oracle, Q6_K, N, K, seed=M + N + K + 1)
    X = synth.normal(M * K, seed=K + 23).reshape(M, K)
    R = synth.normal(M * N, seed=K + 24).reshape(M, N)
    dW, dX = up(holo, src), up(holo, X)

    def product():
        dY = holo.DeviceBuffer(4 * M * N)
        lib.holo_matmul_batch(dY.ptr, dW.ptr, dX.ptr, M, N, K, Q6_K)
        dS = up(holo, R)
        lib.holo_matmul_batch_add(dS.ptr, dW.ptr, dX.ptr, dS.ptr, M, N, K, Q6_K)
        lib.cuda_sync()
        holo.check("prepared product")
        return down(dY, M * N).reshape(M, N), down(dS, M * N).reshape(M, N)

    y0, s0 = product()
    check_rows(y0, X, w, np.unique(np.r_[0:M:32, 31:M:32, M - 1]), Q6_K, K)
    assert lib.holo_prefill_prepare(dW.ptr, N, K, Q6_K) == 0
    try:
        assert lib.holo_prefill_prepare(dW.ptr, N, K, Q6_K) == 0  # registered with this shape: no-op
        for args in ((dW.ptr, N, K, Q4_0), (dW.ptr, N, 1000, Q6_K), (dW.ptr, N - 32, K, Q6_K)):
            assert lib.holo_prefill_prepare(*args) == holo.EINVAL
            assert lib.holo_last_error() == holo.EINVAL
        y1, s1 = product()
        assert np.array_equal(y1.view(np.uint32), y0.view(np.uint32))
        assert np.array_equal(s1.view(np.uint32), s0.view(np.uint32))
        s = lib.holo_stream_create()
        lib.holo_set_stream(s)
        try:
            dG = holo.DeviceBuffer(4 * M * N)
            assert lib.holo_graph_begin() == 0
            lib.holo_matmul_batch(dG.ptr, dW.ptr, dX.ptr, M, N, K, Q6_K)
            g = lib.holo_graph_end()
            holo.check("capture")
            assert g
            for rep in range(2):
                lib.holo_graph_launch(g)
                lib.cuda_sync()
                got = down(dG, M * N).reshape(M, N)
                assert np.array_equal(got.view(np.uint32), y0.view(np.uint32)), rep
            lib.holo_graph_destroy(g)
        finally:
            lib.holo_set_stream(None)
    finally:
        lib.holo_prefill_release(dW.ptr)
    y2, _ = product()
    assert np.array_equal(y2.view(np.uint32), y0.view(np.uint32))


def _sweep_shapes():
    """Seeded small shapes per type: M from 64 (the batched path's least) to
    ragged row tiles, N ragged against the 32-, 64- and 256-column tiles, K
    from one block (one superblock for Q4_K/Q6_K) to a few hundred."""
    rng = np.random.default_rng(2024)
    out = []
    for t in (Q4_0, Q8_0, Q4_K, Q6_K, F16):
        step = 256 if t in (Q4_K, Q6_K) else 32
        for _ in range(6):
            M = int(rng.choice([64, 65, 96, 127, 130, 200]))
            N = int(rng.choice([8, 31, 64, 100, 200, 257, 330]))
            K = step * int(rng.integers(1, 5 if step == 256 else 25))
            if (t, M, N, K) not in out:
                out.append((t, M, N, K))
    return out


SWEEP = _sweep_shapes()


@pytest.mark.parametrize("t,M,N,K", SWEEP, ids=[f"{NAMES[t]}-{m}x{n}x{k}" for t, m, n, k in SWEEP])
def test_exact_product_shape_sweep(holo, synth, oracle, t, M, N, K):
    """Every row of a ragged small product within the elementwise bound of
    the float64 truth (and 1e-5 normwise), two calls bit-identical."""
    print(f"case exact sweep {NAMES[t]} {M}x{N}x{K}", flush=True)
    lib = holo.lib()
    src, w = weights(synth, oracle, t, N, K, seed=7 * M + 3 * N + K)
    X = synth.normal(M * K, seed=M + K).reshape(M, K)
    dW, dX = up(holo, src), up(holo, X)
    outs = []
    for _ in range(2):
        dY = holo.DeviceBuffer(4 * M * N)
        lib.holo_matmul_batch(dY.ptr, dW.ptr, dX.ptr, M, N, K, t)
        lib.cuda_sync()
        holo.check("exact sweep")
        outs.append(down(dY, M * N).reshape(M, N))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    check_rows(outs[0], X, w, np.arange(M), t, K)


PART_CASES = [(Q4_0, 192, 11008, 2048), (Q8_0, 320, 6656, 2048), (Q4_K, 256, 8448, 2048),
              (Q4_0, 512, 4096, 4096), (Q4_K, 512, 4096, 4096), (Q4_0, 320, 2112, 2048),
              (Q6_K, 256, 8448, 2048), (Q6_K, 512, 4096, 4096)]


@pytest.mark.parametrize("t,M,N,K", PART_CASES, ids=[f"{NAMES[t]}-{m}x{n}x{k}" for t, m, n, k in PART_CASES])
def test_exact_part_shapes(holo, synth, oracle, t, M, N, K):
    """Shapes whose stages split tiles unevenly between workgroups: tiles in
    four and in five parts (192x11008x2048, 320x6656x2048, 256x8448x2048, at
    the launch's two workgroups per CU on 256 CUs), where the last workgroup
    of a run either finds every other part counted (and adds them to its own
    accumulators) or stores its part and counts; the 4096-wide o/v shape, whose
    parts are mapped to XCDs; a last column tile 64 wide (2112).  Two calls
    give the same bits, and the first and last row of every 32-row band are
    within the bound of the float64 truth."""
    print(f"case exact parts {NAMES[t]} {M}x{N}x{K}", flush=True)
    lib = holo.lib()
    src, w = weights(synth, oracle, t, N, K, seed=3 * M + N + K)
    X = synth.normal(M * K, seed=K + 17).reshape(M, K)
    dW, dX = up(holo, src), up(holo, X)
    outs = []
    for _ in range(2):
        dY = holo.DeviceBuffer(4 * M * N)
        lib.holo_matmul_batch(dY.ptr, dW.ptr, dX.ptr, M, N, K, t)
        lib.cuda_sync()
        holo.check("exact parts")
        outs.append(down(dY, M * N).reshape(M, N))
    assert np.all(np.isfinite(outs[0]))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    check_rows(outs[0], X, w, np.unique(np.r_[0:M:32, 31:M:32, M - 1]), t, K)


@pytest.mark.parametrize("t,M,N,K", [(Q4_0, 512, 4096, 11008), (Q8_0, 200, 512, 8192), (F16, 100, 320, 4096),
                                     (Q6_K, 512, 4096, 11008)],
                         ids=["q4_0-512x4096x11008", "q8_0-200x512x8192", "f16-100x320x4096", "q6_k-512x4096x11008"])
def test_exact_split_k_deterministic(holo, synth, oracle, t, M, N, K):
    """Few column tiles and a long K take the K-split form (parts summed in
    part order by the last part to arrive, counted on per-tile counters that
    return to zero): two eager calls and three graph replays (with eager
    work between them) give the same bits, within the bound of the truth."""
    print(f"case exact split-K {NAMES[t]} {M}x{N}x{K}", flush=True)
    lib = holo.lib()
    src, w = weights(synth, oracle, t, N, K, seed=M + 7 * N + K)
    X = synth.normal(M * K, seed=K + 9).reshape(M, K)
    dW, dX = up(holo, src), up(holo, X)
    outs = []
    for _ in range(2):
        dY = holo.DeviceBuffer(4 * M * N)
        lib.holo_matmul_batch(dY.ptr, dW.ptr, dX.ptr, M, N, K, t)
        lib.cuda_sync()
        holo.check("exact split-K eager")
        outs.append(down(dY, M * N).reshape(M, N))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    check_rows(outs[0], X, w, np.unique(np.r_[0:M:37, M - 1]), t, K)
    s = lib.holo_stream_create()
    lib.holo_set_stream(s)
    try:
        dG = holo.DeviceBuffer(4 * M * N)
        assert lib.holo_graph_begin() == 0
        lib.holo_matmul_batch(dG.ptr, dW.ptr, dX.ptr, M, N, K, t)
        g = lib.holo_graph_end()
        holo.check("capture")
        assert g
        for rep in range(3):
            lib.holo_graph_launch(g)
            lib.cuda_sync()
            got = down(dG, M * N).reshape(M, N)
            assert np.array_equal(got.view(np.uint32), outs[0].view(np.uint32)), rep
            dE = holo.DeviceBuffer(4 * M * N)  # eager work between the replays
            lib.holo_matmul_batch(dE.ptr, dW.ptr, dX.ptr, M, N, K, t)
            lib.cuda_sync()
            assert np.array_equal(down(dE, M * N).reshape(M, N).view(np.uint32), outs[0].view(np.uint32)), rep
        lib.holo_graph_destroy(g)
    finally:
        lib.holo_set_stream(None)
        lib.holo_stream_destroy(s)
    holo.check("exact split-K graph")
