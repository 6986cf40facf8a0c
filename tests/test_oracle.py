"""Pins the CPU oracle (oracle/holo_oracle.c) before it is trusted as the
parity checker of the HIP kernels.

Three kinds of evidence, chosen so a plausible transcription mistake (a
swapped nibble, a wrong scale bit, a dropped -8, a transposed index) fails:
  1. the reference's own outputs: tests/golden/reference_vectors.npz holds
     vectors produced by executing the reference CPU code (quant.c + llm.c
     compiled from /root/reference, see tests/golden/make_golden.py), and,
     when oracle/_ref is built in this container, fresh random cases are
     compared against it directly;
  2. closed forms fixed by the mathematics or by IEEE 754: all 65536 f16
     codes vs numpy.float16, one-hot activations (dot = one weight), the
     all-ones activation (dot = row sum), d*q exact products, fp64 truth;
  3. the documented Q4_K scale layout: each scale bit reaches exactly the
     sub-block and magnitude the reference's unpack (quant.c:290-297) gives,
     which differs from llama.cpp's get_scale_min_k4.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle.oracle import RefBuild, max_rel_err, normwise_err, ref_available

GOLD = np.load(Path(__file__).resolve().parent / "golden" / "reference_vectors.npz")
Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
NAMES = {Q8_0: "q8_0", Q4_0: "q4_0", Q4_K: "q4_k", Q6_K: "q6_k"}
QK = {Q8_0: 32, Q4_0: 32, Q4_K: 256, Q6_K: 256}
BLK = {Q8_0: 34, Q4_0: 18, Q4_K: 144, Q6_K: 210}


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---- f16 -> f32 ----------------------------------------------------------------

def test_f16_all_codes_vs_numpy(oracle):
    got = np.array([oracle.f16_to_f32(h) for h in range(65536)], dtype=np.float32)
    want = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(want)[~nan])  # zeros, subnormals, normals, inf


def test_f16_all_codes_vs_reference_table(oracle):
    got = bits([oracle.f16_to_f32(h) for h in range(65536)])
    assert np.array_equal(got, GOLD["f16_table"])  # NaN payloads included


def test_f32_to_f16_rne_vs_numpy(oracle):
    rng = np.random.default_rng(5)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(0.01),
        rng.standard_normal(5000).astype(np.float32) * np.float32(1e-5),    # f16 subnormal range
        rng.standard_normal(5000).astype(np.float32) * np.float32(3e4),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, 2.0 ** -25, 2.0 ** -24, 1.5 * 2.0 ** -24,
                  5.960464477539063e-08, 6.103515625e-05, np.inf, -np.inf], dtype=np.float32),
    ])
    got = np.array([oracle.f32_to_f16(float(x)) for x in xs], dtype=np.uint16)
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---- dequantisation ---------------------------------------------------------------

@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q6_K], ids=lambda t: NAMES[t])
def test_dequant_matches_reference_vectors(oracle, t):
    blk = GOLD[f"{NAMES[t]}_blocks"]
    n = blk.size // BLK[t] * QK[t]
    assert np.array_equal(bits(oracle.dequant(t, blk, n)), GOLD[f"{NAMES[t]}_dequant"])


@pytest.mark.skipif(not ref_available("strict"), reason="oracle/_ref not built (no /root/reference)")
@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q6_K], ids=lambda t: NAMES[t])
def test_dequant_matches_reference_build_random(oracle, synth, t):
    ref = RefBuild("strict")
    n = QK[t] * 3001
    blk = synth.blocks(t, 1, n, seed=99 + t)
    assert np.array_equal(bits(oracle.dequant(t, blk, n)), bits(ref.dequant(t, blk, n)))


def test_dequant_q4_0_one_hot(oracle):
    """w = d * (nibble - 8): low nibble of byte j -> element j, high -> j + 16."""
    blk = np.zeros((32, 18), dtype=np.uint8)
    for e in range(32):
        blk[e, 0:2] = (0x00, 0x40)                    # d = 2.0
        blk[e, 2:] = 0x88                             # every weight 0
        j = e & 15
        blk[e, 2 + j] = (0x8F if e < 16 else 0xF8)    # element e gets nibble 15
    w = oracle.dequant(Q4_0, blk.reshape(-1), 32 * 32).reshape(32, 32)
    want = np.zeros((32, 32), dtype=np.float32)
    np.fill_diagonal(want, 2.0 * 7)
    assert np.array_equal(w, want)


def test_dequant_q8_0_closed_form(oracle):
    rng = np.random.default_rng(1)
    blk = np.zeros((64, 34), dtype=np.uint8)
    d = rng.uniform(1e-3, 10, 64).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(64, 2)
    q = rng.integers(-127, 128, (64, 32)).astype(np.int8)
    blk[:, 2:] = q.view(np.uint8)
    w = oracle.dequant(Q8_0, blk.reshape(-1), 64 * 32).reshape(64, 32)
    assert np.array_equal(w, d.astype(np.float32)[:, None] * q.astype(np.float32))  # exact products


def _q4_k_unpack_expected(byte, bit):
    """(kind, sub-block, value) a single set bit of the packed scales reaches
    under the reference CPU layout (quant.c:290-297)."""
    if byte < 4:
        return ("sc", byte, 1 << bit) if bit < 6 else ("sc", byte + 4, 1 << (bit - 6))
    if byte < 8:
        j = byte - 4
        return ("m", j, 1 << bit) if bit < 6 else ("m", j + 4, 1 << (bit - 6))
    j = byte - 8 + 4
    return ("sc", j, 1 << (bit + 2)) if bit < 4 else ("m", j, 1 << (bit - 4 + 2))


def test_q4_k_scale_layout_from_reference_vectors(oracle):
    """Every scale bit: d = dmin = 1, all nibbles 1, so weights are sc - m."""
    out = GOLD["q4_k_scale_sweep_out"].view(np.float32).reshape(96, 8, 32)
    got = oracle.dequant(Q4_K, GOLD["q4_k_scale_sweep"], 96 * 256).reshape(96, 8, 32)
    assert np.array_equal(got, out)
    for byte in range(12):
        for bit in range(8):
            kind, j, val = _q4_k_unpack_expected(byte, bit)
            want = np.zeros((8, 32), dtype=np.float32)
            want[j, :] = val if kind == "sc" else -val
            assert np.array_equal(out[byte * 8 + bit], want), (byte, bit)
    # llama.cpp's get_scale_min_k4 would put byte 8 bit 0 into sc[4] bit 0
    # (value 1); the reference CPU layout puts it in bit 2 (value 4).
    assert out[8 * 8 + 0][4, 0] == 4.0


def test_q4_k_qs_layout_from_reference_vectors(oracle):
    """qs[16j+l]: low nibble -> 32j+l, high nibble -> 32j+l+16 (quant.c:300-308)."""
    out = GOLD["q4_k_qs_sweep_out"].view(np.float32).reshape(128, 256)
    got = oracle.dequant(Q4_K, GOLD["q4_k_qs_sweep"], 128 * 256).reshape(128, 256)
    assert np.array_equal(got, out)
    for byte in range(128):
        j, l = divmod(byte, 16)
        sc = 1.0 if j < 4 else 4.0
        want = np.zeros(256, dtype=np.float32)
        want[32 * j + l] = sc * 1
        want[32 * j + l + 16] = sc * 2
        assert np.array_equal(out[byte], want), byte


# ---- matrix-vector products -----------------------------------------------------------

@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q6_K], ids=lambda t: NAMES[t])
def test_matmul_matches_reference_vectors(oracle, t):
    n = NAMES[t]
    W, x = GOLD[f"mm_{n}_W"], GOLD[f"mm_{n}_x"]
    got = oracle.matmul(t, W, x, 24, x.size)
    # scalar build = the summation order the oracle restates: bit-exact
    assert np.array_equal(bits(got), GOLD[f"mm_{n}_scalar"])
    # AVX2 / -ffast-math builds reorder the sums: fp32 rounding only
    for b in ("strict", "release"):
        assert normwise_err(got, GOLD[f"mm_{n}_{b}"].view(np.float32)) < 1e-5


@pytest.mark.skipif(not ref_available("scalar"), reason="oracle/_ref not built (no /root/reference)")
@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q6_K], ids=lambda t: NAMES[t])
def test_matmul_matches_reference_build_random(oracle, synth, t):
    K = QK[t] * 16
    W = synth.blocks(t, 33, K, seed=55 + t)
    x = synth.normal(K, seed=66 + t)
    got = oracle.matmul(t, W, x, 33, K)
    assert np.array_equal(bits(got), bits(RefBuild("scalar").matmul(t, W, x, 33, K)))
    assert normwise_err(got, RefBuild("release").matmul(t, W, x, 33, K)) < 1e-5


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q6_K], ids=lambda t: NAMES[t])
def test_matmul_one_hot_and_ones(oracle, synth, t):
    K = QK[t] * 4
    W = synth.blocks(t, 9, K, seed=3 + t)
    Wd = oracle.dequant(t, W, 9 * K).reshape(9, K)
    for k in (0, 5, 17, K - 1):
        e = np.zeros(K, dtype=np.float32)
        e[k] = 1.0
        assert np.array_equal(oracle.matmul(t, W, e, 9, K), Wd[:, k])  # one weight, exact
    ones = np.ones(K, dtype=np.float32)
    assert normwise_err(oracle.matmul(t, W, ones, 9, K), Wd.astype(np.float64).sum(1)) < 1e-6


@pytest.mark.parametrize("t", [Q8_0, Q4_0, Q4_K, Q6_K], ids=lambda t: NAMES[t])
def test_matmul_vs_fp64_truth(oracle, synth, t):
    K = 4096
    W = synth.blocks(t, 64, K, seed=11 + t)
    x = synth.normal(K, seed=12 + t)
    got = oracle.matmul(t, W, x, 64, K)
    truth = oracle.truth(t, W, x, 64, K)
    assert normwise_err(got, truth) < 1e-5
    assert max_rel_err(got, truth) < 1e-4


def test_in_dim_truncates_like_reference(oracle, synth):
    """in_dim not a multiple of 32: in_dim/32 blocks per row (llm.c:895)."""
    W = synth.blocks(Q4_0, 3, 96, seed=1)
    x = synth.normal(100, seed=2)
    assert np.array_equal(oracle.matmul(Q4_0, W, x, 3, 100), oracle.matmul(Q4_0, W, x, 3, 96))


# ---- build-defined: activation quantiser and int8 product ---------------------------------

def _quantize_numpy(X):
    """Independent numpy statement of the Q8_0 activation quantiser spec."""
    X = X.astype(np.float32).reshape(X.shape[0], -1, 32)
    amax = np.abs(X).max(axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    t = (X * idv[:, :, None]).astype(np.float32)
    q = np.clip(np.sign(t) * np.floor(np.abs(t) + np.float32(0.5)), -127, 127).astype(np.int8)
    return d, q


def test_quantize_act_spec_and_invariants(oracle, synth):
    X = synth.normal(7 * 256, seed=8).reshape(7, 256)
    X[3, 32:64] = 0.0                      # an all-zero block: d = 0, q = 0
    X[5, 0] = 100.0                        # a block dominated by one value
    blk = oracle.quantize_act_q8_0(X).reshape(7, 8, 34)
    d16 = blk[:, :, 0:2].copy().view(np.float16)[..., 0]
    q = blk[:, :, 2:].view(np.int8)
    d32, qn = _quantize_numpy(X)
    assert np.array_equal(q, qn)
    assert np.array_equal(d16, d32.astype(np.float16))
    assert np.abs(q.astype(int)).max() <= 127
    err = np.abs(X.reshape(7, 8, 32) - d32[:, :, None] * q)
    assert np.all(err <= d32[:, :, None] * 0.5 * (1 + 1e-6) + 1e-30)
    assert np.all(q[3, 1] == 0) and d16[3, 1] == 0


def test_gemm_q4_0_q8_0_vs_integer_truth(oracle, synth):
    M, N, K = 9, 13, 256
    W = synth.blocks(Q4_0, N, K, seed=21)
    Xq = oracle.quantize_act_q8_0(synth.normal(M * K, seed=22).reshape(M, K))
    Y = oracle.gemm_q4_0_q8_0(W, Xq, M, N, K)
    # integer block dots from the dequantised int values
    wb = W.reshape(N, K // 32, 18)
    qlo = (wb[:, :, 2:] & 15).astype(np.int64) - 8
    qhi = (wb[:, :, 2:] >> 4).astype(np.int64) - 8
    qw = np.concatenate([qlo, qhi], axis=2)                 # [N][b][32]
    dw = wb[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    xb = Xq.reshape(M, K // 32, 34)
    qx = xb[:, :, 2:].view(np.int8).astype(np.int64)
    dx = xb[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    I = np.einsum("mbk,nbk->mnb", qx, qw)
    truth = np.einsum("mnb,nb,mb->mn", I.astype(np.float64), dw, dx)
    assert normwise_err(Y, truth) < 1e-6
    # one-block case: Y = I * (dw * dx) exactly as specified
    Y1 = oracle.gemm_q4_0_q8_0(W.reshape(N, K // 32, 18)[:, :1].copy().reshape(-1),
                               Xq.reshape(M, K // 32, 34)[:, :1].copy().reshape(-1), M, N, 32)
    want1 = (I[:, :, 0].astype(np.float32) * (dw[:, 0].astype(np.float32)[None, :] *
                                              dx[:, 0].astype(np.float32)[:, None]).astype(np.float32))
    assert np.array_equal(Y1, want1.astype(np.float32))


def _fma_f32(a, b, c):
    """fmaf(a, b, c) for float32 a, b, c from exact rationals: the float64 sum
    is used only where it equals the exact value, so the final conversion to
    float32 is the single rounding fmaf specifies."""
    from fractions import Fraction
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    s = float(a) * float(b) + float(c)
    assert Fraction(s) == exact, "float64 sum inexact for this case"
    return np.float32(s)


def test_gemm_q4_0_q8_0_block_order_fma(oracle, synth):
    """acc = fmaf((float)I_b, dw_b*dx_b, acc) over blocks b in order, evaluated
    exactly step by step; a mul-then-add accumulation differs on this input."""
    M, N, K = 6, 7, 32 * 9
    W = synth.blocks(Q4_0, N, K, seed=31)
    Xq = oracle.quantize_act_q8_0(synth.normal(M * K, seed=32).reshape(M, K))
    Y = oracle.gemm_q4_0_q8_0(W, Xq, M, N, K)
    wb = W.reshape(N, K // 32, 18)
    qw = np.concatenate([(wb[:, :, 2:] & 15).astype(np.int64) - 8, (wb[:, :, 2:] >> 4).astype(np.int64) - 8], axis=2)
    dw = wb[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    xb = Xq.reshape(M, K // 32, 34)
    qx = xb[:, :, 2:].view(np.int8).astype(np.int64)
    dx = xb[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    I = np.einsum("mbk,nbk->mnb", qx, qw)
    want = np.zeros((M, N), np.float32)
    muladd = np.zeros((M, N), np.float32)
    for m in range(M):
        for n in range(N):
            acc = np.float32(0)
            acc2 = np.float32(0)
            for b in range(K // 32):
                s = np.float32(dw[n, b] * dx[m, b])
                assert float(s) == float(dw[n, b]) * float(dx[m, b])  # the scale product is exact
                acc = _fma_f32(np.float32(I[m, n, b]), s, acc)
                acc2 = np.float32(acc2 + np.float32(np.float32(I[m, n, b]) * s))
            want[m, n] = acc
            muladd[m, n] = acc2
    assert np.array_equal(Y.view(np.uint32), want.view(np.uint32))
    assert not np.array_equal(Y.view(np.uint32), muladd.view(np.uint32))


def test_silu_mul_vs_numpy(oracle, synth):
    g = synth.normal(1000, seed=1) * np.float32(4)
    u = synth.normal(1000, seed=2)
    want = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
    assert normwise_err(oracle.silu_mul(g, u), want) < 1e-6


# ---- the f16 prefill product ----------------------------------------------------------------

def test_gemm_q4_0_f16_closed_form(oracle):
    """Inputs exact in f16: scale 1 and nibble 9 make every weight 1, so each
    output is the row's plain sum; nibble 0 with scale 2 makes every weight -16."""
    M, N, K = 3, 2, 64
    W = np.zeros((N, K // 32, 18), np.uint8)
    W[0, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    W[0, :, 2:] = 0x99
    W[1, :, 0:2] = np.frombuffer(np.float16(2.0).tobytes(), np.uint8)
    W[1, :, 2:] = 0x00
    X = (np.arange(M * K, dtype=np.float32).reshape(M, K) % 7 - 3) * 0.25  # exact in f16
    Y, A = oracle.gemm_q4_0_f16(W.reshape(-1), X, M, N, K)
    assert np.array_equal(Y[:, 0], X.sum(1).astype(np.float64))
    assert np.array_equal(Y[:, 1], -16.0 * X.sum(1).astype(np.float64))
    assert np.array_equal(A[:, 0], np.abs(X).sum(1).astype(np.float64))


def test_gemm_q4_0_f16_vs_reference_matmul(oracle, synth):
    """Against the reference-pinned fp32 GEMV of the same rows: the two differ
    only by the f16 rounding of each activation and weight (relative 2^-11
    each) and the fp32 GEMV's own rounding, so |Y - y| <= 2^-10 A (+ fp32)."""
    M, N, K = 5, 48, 1024
    W = synth.blocks(Q4_0, N, K, seed=71)
    X = synth.normal(M * K, seed=72).reshape(M, K)
    Y, A = oracle.gemm_q4_0_f16(W, X, M, N, K)
    for m in range(M):
        y = oracle.matmul(Q4_0, W, X[m], N, K).astype(np.float64)
        assert np.all(np.abs(Y[m] - y) <= 2.0 ** -10 * A[m] + 1e-6 * A[m])


def test_gemm_q4_0_f16_vs_numpy_float16(oracle, synth):
    """numpy's float16 conversion (its own round-to-nearest-even) of both
    operands, summed in float64: equal to within float64 rounding."""
    M, N, K = 4, 16, 256
    W = synth.blocks(Q4_0, N, K, seed=81)
    X = synth.normal(M * K, seed=82).reshape(M, K)
    Y, _ = oracle.gemm_q4_0_f16(W, X, M, N, K)
    blk = W.reshape(N, K // 32, 18)
    d = blk[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float32)
    qs = blk[:, :, 2:]
    q = np.concatenate([qs & 0xF, qs >> 4], axis=2).astype(np.float32) - 8.0   # k = 0..15 low, 16..31 high nibbles
    w16 = (d[:, :, None] * q).astype(np.float16).astype(np.float64).reshape(N, K)
    x16 = X.astype(np.float16).astype(np.float64)
    want = x16 @ w16.T
    assert np.all(np.abs(Y - want) <= 1e-12 * (np.abs(x16) @ np.abs(w16).T))
