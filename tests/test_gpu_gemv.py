"""GPU parity of the fused dequant+GEMV entry points against the CPU oracle.

Bar: dot products within relative error 1e-3 with
fp32 accumulation.  Both measures are asserted:
  normwise  ||gpu - oracle||_inf / ||oracle||_inf <= 1e-3
  elementwise max |gpu - oracle| / |oracle| over outputs with
            |oracle| >= 0.05 * rms(oracle)  <= 1e-3
and the same two against the fp64 truth over the same dequantised weights.
"""
import numpy as np
import pytest

from oracle.oracle import max_rel_err, normwise_err

pytestmark = pytest.mark.gpu

TOL = 1e-3

Q4_0, Q8_0, Q4_K = 2, 8, 12
NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k"}

# (type, out_dim, in_dim): small and ragged cases, then the benchmark shapes.
CASES = [
    (Q4_0, 1, 32), (Q4_0, 3, 64), (Q4_0, 37, 96), (Q4_0, 65, 2048 + 32), (Q4_0, 130, 4096),
    (Q8_0, 1, 32), (Q8_0, 5, 96), (Q8_0, 33, 2080), (Q8_0, 129, 4096),
    (Q4_K, 1, 256), (Q4_K, 7, 512), (Q4_K, 45, 2304), (Q4_K, 130, 4096),
    # MFMA path: rows ending in an 8-unit segment (24 and 136 units), a
    # ragged last tile, and in_dim 16384 (4 items per wave)
    (Q4_0, 23, 256 * 3), (Q8_0, 19, 256 * 3), (Q4_0, 33, 256 * 17), (Q4_K, 9, 256 * 3), (Q8_0, 40, 16384),
    # BASELINE.json configs 1-3 and the config-5 head
    (Q8_0, 4096, 4096), (Q4_0, 4096, 4096), (Q4_0, 11008, 4096), (Q4_0, 4096, 11008),
    (Q4_K, 14336, 4096), (Q4_K, 4096, 14336), (Q8_0, 32000, 4096),
    # in_dim beyond the LDS staging limit (x read from global memory)
    (Q4_0, 64, 32 * 600), (Q4_K, 32, 256 * 70),
]


def _run(holo, synth, qtype, out_dim, in_dim, seed):
    W = synth.blocks(qtype, out_dim, in_dim, seed)
    x = synth.normal(in_dim, seed ^ 0xABCDEF)
    dW = holo.DeviceBuffer.from_array(W)
    dx = holo.DeviceBuffer.from_array(x)
    dy = holo.DeviceBuffer(out_dim * 4)
    fn = {Q4_0: "cuda_matmul_q4_0", Q8_0: "cuda_matmul_q8_0", Q4_K: "cuda_matmul_q4_k"}[qtype]
    getattr(holo.lib(), fn)(dy.ptr, dW.ptr, dx.ptr, out_dim, in_dim)
    holo.lib().cuda_sync()
    holo.check(fn)
    return W, x, dy.download(np.float32, out_dim)


@pytest.mark.parametrize("xmode", [3, 1, 0], ids=["mfma", "i24", "f32"])
@pytest.mark.parametrize("qtype,out_dim,in_dim", CASES,
                         ids=[f"{NAMES[t]}-{o}x{i}" for t, o, i in CASES])
def test_gemv_parity(holo, synth, oracle, qtype, out_dim, in_dim, xmode):
    print(f"case {NAMES[qtype]} {out_dim}x{in_dim} xmode={xmode}", flush=True)
    holo.lib().holo_gemv_set_xmode(xmode)
    try:
        W, x, got = _run(holo, synth, qtype, out_dim, in_dim, seed=out_dim * 7919 + in_dim)
    finally:
        holo.lib().holo_gemv_set_xmode(2)
    want = oracle.matmul(qtype, W, x, out_dim, in_dim)
    truth = oracle.truth(qtype, W, x, out_dim, in_dim)
    e_n, e_r = normwise_err(got, want), max_rel_err(got, want)
    t_n, t_r = normwise_err(got, truth), max_rel_err(got, truth)
    print(f"  vs oracle normwise {e_n:.2e} elementwise {e_r:.2e}; vs fp64 {t_n:.2e} {t_r:.2e}", flush=True)
    assert np.all(np.isfinite(got))
    assert e_n <= TOL and e_r <= TOL
    assert t_n <= TOL and t_r <= TOL


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0, Q4_K, 14], ids=["q4_0", "q8_0", "q4_k", "q6_k"])
def test_dequant_bit_exact(holo, synth, oracle, qtype):
    # Q4_0/Q8_0: an odd block count, so the last block starts on a 4-byte
    # boundary and its dword window must not run past the buffer.
    n = 32 * 32793 if qtype in (Q4_0, Q8_0) else 256 * 4099
    print(f"case dequant type {qtype} n={n}", flush=True)
    blocks = synth.blocks(qtype, 1, n, seed=1234 + qtype)
    want = oracle.dequant(qtype, blocks, n)
    d_in = holo.DeviceBuffer.from_array(blocks)
    d_out = holo.DeviceBuffer(n * 4)
    holo.lib().holo_dequant(d_out.ptr, d_in.ptr, n, qtype)
    holo.lib().cuda_sync()
    holo.check("holo_dequant")
    got = d_out.download(np.float32, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# Q6_K (cuda_matmul_q6_k): odd superblock counts put every other row at a
# 2-byte (not 4-byte) offset; odd out_dim leaves a wave with one row.
Q6_K = 14
Q6_CASES = [(1, 256), (3, 512), (37, 256 * 9), (130, 4096), (4096, 4096), (4096, 11008), (11008, 4096),
            (32000, 4096), (5, 256 * 43)]


@pytest.mark.parametrize("out_dim,in_dim", Q6_CASES, ids=[f"{o}x{i}" for o, i in Q6_CASES])
@pytest.mark.parametrize("x_offset", [0, 1], ids=["x16", "x4"])
def test_gemv_q6_k_parity(holo, synth, oracle, out_dim, in_dim, x_offset):
    """x_offset 1 shifts the activations by one float, off 16-byte alignment
    (the per-weight kernel); 0 runs the 64-weight task kernel."""
    print(f"case q6_k {out_dim}x{in_dim} x_offset={x_offset}", flush=True)
    seed = out_dim * 7919 + in_dim
    W = synth.blocks(Q6_K, out_dim, in_dim, seed)
    x = synth.normal(in_dim, seed ^ 0xABCDEF)
    dW = holo.DeviceBuffer.from_array(W)
    dx = holo.DeviceBuffer.from_array(np.concatenate([np.zeros(x_offset, np.float32), x]))
    dy = holo.DeviceBuffer(out_dim * 4)
    holo.lib().cuda_matmul_q6_k(dy.ptr, dW.ptr, dx.ptr + 4 * x_offset, out_dim, in_dim)
    holo.lib().cuda_sync()
    holo.check("cuda_matmul_q6_k")
    got = dy.download(np.float32, out_dim)
    want = oracle.matmul(Q6_K, W, x, out_dim, in_dim)
    truth = oracle.truth(Q6_K, W, x, out_dim, in_dim)
    e_n, e_r = normwise_err(got, want), max_rel_err(got, want)
    t_n, t_r = normwise_err(got, truth), max_rel_err(got, truth)
    print(f"  vs oracle normwise {e_n:.2e} elementwise {e_r:.2e}; vs fp64 {t_n:.2e} {t_r:.2e}", flush=True)
    assert np.all(np.isfinite(got))
    assert e_n <= TOL and e_r <= TOL
    assert t_n <= TOL and t_r <= TOL
