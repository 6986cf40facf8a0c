"""holo_gemm_q4_0_q8_0_noalloc: the allocation-free variant of
holo_gemm_q4_0_q8_0 (its activation panel in the library's fixed device
array instead of an allocated workspace).  Through the C ABI it must give
the bit-identical output of the allocating entry point (the product is
fully specified, so both are also bit-exact to the oracle), on two calls in
a row whose second is smaller (the array keeps the first call's contents),
and reject a call too large for the array without touching the output."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_0 = 2


def _product(holo, fn, W, Xq, M, N, K):
    dY = holo.DeviceBuffer.from_array(np.full(M * N, np.nan, np.float32))
    rc = getattr(holo.lib(), fn)(dY.ptr, W.ptr, Xq.ptr, M, N, K)
    holo.lib().cuda_sync()
    holo.check(fn)
    return rc, dY.download(np.float32, M * N).reshape(M, N)


@pytest.mark.parametrize("M,N,K", [(512, 4096, 11008), (96, 640, 2048)], ids=["first-512x4096x11008", "then-96x640x2048"])
def test_noalloc_matches_allocating_entry(holo, synth, oracle, M, N, K):
    print(f"case noalloc gemm {M}x{N}x{K}", flush=True)
    W = synth.blocks(Q4_0, N, K, seed=N + 3 * K)
    X = synth.normal(M * K, seed=M + K).reshape(M, K)
    Xq = oracle.quantize_act_q8_0(X)
    dW, dXq = holo.DeviceBuffer.from_array(W), holo.DeviceBuffer.from_array(Xq)
    rc, got = _product(holo, "holo_gemm_q4_0_q8_0_noalloc", dW, dXq, M, N, K)
    assert rc == 0
    _, ref = _product(holo, "holo_gemm_q4_0_q8_0", dW, dXq, M, N, K)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    rows = np.r_[0:8, M - 8:M]  # oracle on a subset of rows (the CPU product is slow)
    want = oracle.gemm_q4_0_q8_0(W, Xq.reshape(M, -1)[rows].reshape(-1), len(rows), N, K)
    assert np.array_equal(got[rows].view(np.uint32), want.view(np.uint32))


def test_noalloc_rejects_past_its_scratch(holo, synth):
    print("case noalloc rejects", flush=True)
    M, N, K = 1024, 128, 16384  # panel of 1024*16384*33/16 bytes > 24 MiB
    W = holo.DeviceBuffer(N * (K // 32) * 18)
    Xq = holo.DeviceBuffer(M * (K // 32) * 34)
    dY = holo.DeviceBuffer.from_array(np.full(M * N, 5.0, np.float32))
    rc = holo.lib().holo_gemm_q4_0_q8_0_noalloc(dY.ptr, W.ptr, Xq.ptr, M, N, K)
    assert rc == holo.EINVAL
    assert holo.lib().holo_last_error() == holo.EINVAL
    holo.lib().cuda_sync()
    assert np.all(dY.download(np.float32, M * N) == 5.0)
