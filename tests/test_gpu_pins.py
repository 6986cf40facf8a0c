"""GPU pins that close the gaps between the oracle's checks and the GPU
kernels: every f16 code through the GPU's scale conversion, the Q4_K one-hot
scale and quant sweeps through dequant and GEMV, in_dim truncation, and the
zero-fills inside a captured graph.

References: f16 table quant.c:40-82; Q4_K scale unpack quant.c:290-297;
truncation to whole blocks llm.c:895 (nb = in_dim / 32) and
cuda_ops.cu:624,699; NULL matrix -> zeros llm.c:772-775.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle.oracle import max_rel_err, normwise_err

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.npz"
Q4_0, Q8_0, Q4_K = 2, 8, 12
TOL = 1e-3


def _dequant(holo, qtype, blocks, n):
    d_in = holo.DeviceBuffer.from_array(blocks)
    d_out = holo.DeviceBuffer(n * 4)
    holo.lib().holo_dequant(d_out.ptr, d_in.ptr, n, qtype)
    holo.lib().cuda_sync()
    holo.check("holo_dequant")
    return d_out.download(np.float32, n)


def _gemv(holo, qtype, W, x, out_dim, in_dim):
    dW, dx = holo.DeviceBuffer.from_array(W), holo.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    dy = holo.DeviceBuffer(out_dim * 4)
    fn = {Q4_0: "cuda_matmul_q4_0", Q8_0: "cuda_matmul_q8_0", Q4_K: "cuda_matmul_q4_k"}[qtype]
    getattr(holo.lib(), fn)(dy.ptr, dW.ptr, dx.ptr, out_dim, in_dim)
    holo.lib().cuda_sync()
    holo.check(fn)
    return dy.download(np.float32, out_dim)


def test_f16_every_code_as_q8_0_scale(holo, oracle):
    """All 65,536 f16 codes as the scale d of Q8_0 blocks whose first quant
    is 1: element 0 of each block is the conversion itself, compared with the
    reference's own table (executed into the golden fixture); the other 31
    quants are fixed non-zero values, so every product d*q is compared with
    the oracle.  Bit-exact except NaN codes, whose quiet bit the two sides
    may set differently (both must be NaN)."""
    print("case f16 every code", flush=True)
    z = np.load(GOLDEN)
    codes = np.arange(65536, dtype=np.uint32)
    blocks = np.zeros((65536, 34), np.uint8)
    blocks[:, 0] = codes & 0xFF
    blocks[:, 1] = codes >> 8
    q = np.array([1] + [(-1) ** j * ((7 * j) % 128) for j in range(1, 32)], np.int8)
    blocks[:, 2:] = q.view(np.uint8)
    blocks = blocks.reshape(-1)
    n = 65536 * 32
    got = _dequant(holo, Q8_0, blocks, n).view(np.uint32).reshape(65536, 32)
    want = oracle.dequant(Q8_0, blocks, n).view(np.uint32).reshape(65536, 32)
    nan = ((codes >> 10) & 0x1F == 0x1F) & ((codes & 0x3FF) != 0)
    table = z["f16_table"]
    assert np.array_equal(got[~nan, 0], table[~nan])
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(np.isnan(got[nan].view(np.float32)))
    print(f"  {int((~nan).sum())} codes bit-exact; {int(nan.sum())} NaN codes NaN", flush=True)


@pytest.mark.parametrize("sweep", ["scale", "qs"])
def test_q4_k_one_hot_sweeps(holo, oracle, sweep):
    """The reference-executed one-hot sweeps of the golden fixture: each of
    the 12 scale bytes x 8 bits (q4_k_scale_sweep) and each quant byte's bits
    (q4_k_qs_sweep) set alone, through holo_dequant (bit-exact against the
    reference's dequantize_row_q4_k outputs) and through cuda_matmul_q4_k
    with the superblocks as the rows of a [n][256] matrix (within 1e-3 of
    the oracle and of the fp64 truth), in the MFMA and fp32 activation
    modes."""
    z = np.load(GOLDEN)
    blocks, out = z[f"q4_k_{sweep}_sweep"], z[f"q4_k_{sweep}_sweep_out"]
    rows = blocks.size // 144
    print(f"case q4_k {sweep} sweep: {rows} superblocks", flush=True)
    got = _dequant(holo, Q4_K, blocks, rows * 256)
    assert np.array_equal(got.view(np.uint32), out)
    x = np.random.default_rng(3).standard_normal(256).astype(np.float32)
    want = oracle.matmul(Q4_K, blocks, x, rows, 256)
    truth = oracle.truth(Q4_K, blocks, x, rows, 256)
    for xmode in (2, 0):
        holo.lib().holo_gemv_set_xmode(xmode)
        try:
            y = _gemv(holo, Q4_K, blocks, x, rows, 256)
        finally:
            holo.lib().holo_gemv_set_xmode(2)
        e = (normwise_err(y, want), max_rel_err(y, want), normwise_err(y, truth), max_rel_err(y, truth))
        print(f"  xmode {xmode}: vs oracle {e[0]:.2e} {e[1]:.2e}; vs fp64 {e[2]:.2e} {e[3]:.2e}", flush=True)
        assert max(e) <= TOL


# (type, out_dim, in_dim): in_dim past whole blocks; the reference uses
# in_dim / QK blocks and ignores the rest of v (llm.c:895, quant.c:626-633).
TRUNC = [(Q4_0, 300, 4096 + 17), (Q4_0, 64, 32 * 7 + 31), (Q8_0, 300, 4096 + 31), (Q8_0, 50, 32 * 5 + 1),
         (Q4_K, 260, 4096 + 255), (Q4_K, 40, 256 * 3 + 100)]


@pytest.mark.parametrize("qtype,out_dim,in_dim", TRUNC, ids=[f"{t}-{o}x{i}" for t, o, i in TRUNC])
def test_in_dim_truncates_to_whole_blocks(holo, synth, oracle, qtype, out_dim, in_dim):
    qk = 256 if qtype == Q4_K else 32
    whole = in_dim // qk * qk
    print(f"case truncation type {qtype} {out_dim}x{in_dim} ({whole} used)", flush=True)
    W = synth.blocks(qtype, out_dim, whole, seed=in_dim)
    x = synth.normal(in_dim, seed=in_dim + 1)
    x[whole:] = 1e30  # the tail must not be read into any dot
    want = oracle.matmul(qtype, W, x, out_dim, in_dim)
    truth = oracle.truth(qtype, W, x[:whole], out_dim, whole)
    for xmode in (2, 0):
        holo.lib().holo_gemv_set_xmode(xmode)
        try:
            got = _gemv(holo, qtype, W, x, out_dim, in_dim)
        finally:
            holo.lib().holo_gemv_set_xmode(2)
        e = (normwise_err(got, want), max_rel_err(got, want), normwise_err(got, truth), max_rel_err(got, truth))
        print(f"  xmode {xmode}: vs oracle {e[0]:.2e} {e[1]:.2e}; vs fp64 {e[2]:.2e} {e[3]:.2e}", flush=True)
        assert np.all(np.isfinite(got)) and max(e) <= TOL


def test_in_dim_below_one_block_writes_zeros(holo):
    print("case in_dim below one block", flush=True)
    dy = holo.DeviceBuffer.from_array(np.full(37, 7.0, np.float32))
    dx = holo.DeviceBuffer.from_array(np.ones(31, np.float32))
    dW = holo.DeviceBuffer(64)
    for fn in ("cuda_matmul_q4_0", "cuda_matmul_q8_0"):
        dy.upload(np.full(37, 7.0, np.float32))
        getattr(holo.lib(), fn)(dy.ptr, dW.ptr, dx.ptr, 37, 31)
        holo.lib().cuda_sync()
        holo.check(fn)
        assert np.array_equal(dy.download(np.float32, 37), np.zeros(37, np.float32)), fn


def test_zero_fills_inside_a_captured_graph(holo, synth, oracle):
    """A decode-step fragment captured into a HIP graph with a NULL-matrix
    GEMV (zeros, llm.c:772-775), a NULL Q6_K GEMV, cuda_memset and a real
    GEMV between them; the outputs are poisoned before each of four replays,
    with eager work and synchronisations in between, and every replay must
    write the zeros and the product again."""
    print("case zero fills in a graph", flush=True)
    lib = holo.lib()
    W = synth.blocks(Q4_0, 256, 4096, seed=77)
    x = synth.normal(4096, seed=78)
    want = oracle.matmul(Q4_0, W, x, 256, 4096)
    dW, dx = holo.DeviceBuffer.from_array(W), holo.DeviceBuffer.from_array(x)
    a, b, c, y = (holo.DeviceBuffer(4 * 256) for _ in range(4))
    junk = np.full(256, 3.5, np.float32)
    s = lib.holo_stream_create()
    lib.holo_set_stream(s)
    try:
        assert lib.holo_graph_begin() == 0
        lib.cuda_matmul_q4_0(a.ptr, None, dx.ptr, 256, 4096)
        lib.cuda_matmul_q4_0(y.ptr, dW.ptr, dx.ptr, 256, 4096)
        lib.cuda_matmul_q6_k(b.ptr, None, dx.ptr, 256, 4096)
        lib.cuda_memset(c.ptr, 0, 4 * 256)
        g = lib.holo_graph_end()
        holo.check("capture")
        assert g
        for rep in range(4):
            for buf in (a, b, c, y):
                buf.upload(junk)
            lib.cuda_matmul_q4_0(c.ptr, dW.ptr, dx.ptr, 256, 4096)  # eager work between replays
            lib.cuda_sync()
            assert lib.holo_graph_launch(g) == 0
            lib.cuda_sync()
            holo.check(f"replay {rep}")
            for name, buf in (("null q4_0", a), ("null q6_k", b), ("memset", c)):
                assert np.array_equal(buf.download(np.float32, 256), np.zeros(256, np.float32)), (rep, name)
            got = y.download(np.float32, 256)
            assert normwise_err(got, want) <= TOL and max_rel_err(got, want) <= TOL
        lib.holo_graph_destroy(g)
    finally:
        lib.holo_set_stream(None)
        lib.holo_stream_destroy(s)
