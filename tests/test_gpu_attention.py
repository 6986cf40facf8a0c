"""GPU parity of decode attention (cuda_multi_head_attention, and the one-row
case of holo_attention_prefill) on the key-split kernels, through the C ABI.

softmax((q . k_p) / sqrt(hd)) . v over positions p < kv_len, grouped-query
heads (cuda_ops.cu:1813-1952).  Bar: fp32 arithmetic against float64 numpy,
1e-5 normwise per call.  Cases cover one range and many, ranges with several
64-key passes (the range count is capped), the last pass partly filled, head
sizes from 12 to 128 and one outside the split kernel (head_dim 130, the
single-workgroup kernel), and caches beyond 12288 positions.
"""
import numpy as np
import pytest

from oracle.oracle import normwise_err

pytestmark = pytest.mark.gpu


def up(holo, a):
    return holo.DeviceBuffer.from_array(np.ascontiguousarray(a))


def down(buf, n):
    return buf.download(np.float32, n)


def want_attention(q, K, V, nh, nkv, hd, kv_len):
    Q = q.reshape(nh, hd).astype(np.float64)
    out = np.empty((nh, hd))
    for h in range(nh):
        g = h // (nh // nkv)
        s = K[:kv_len, g] @ Q[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V[:kv_len, g]
    return out.reshape(-1)


@pytest.mark.parametrize("hd,nh,nkv,kv_len", [
    (128, 32, 32, 1), (128, 32, 32, 37), (128, 32, 32, 64), (128, 32, 32, 65), (128, 32, 32, 512),
    (128, 8, 2, 4097), (128, 4, 2, 20000), (64, 16, 4, 300), (32, 8, 4, 129), (80, 6, 3, 700),
    (12, 4, 1, 90), (130, 4, 2, 77)])
def test_decode_attention(holo, synth, hd, nh, nkv, kv_len):
    print(f"case decode attention hd {hd} heads {nh}/{nkv} kv_len {kv_len}", flush=True)
    lib = holo.lib()
    kv_dim = nkv * hd
    q = synth.normal(nh * hd, seed=21)
    kc = synth.normal(kv_len * kv_dim, seed=22)
    vc = synth.normal(kv_len * kv_dim, seed=23)
    dq, dk, dv = up(holo, q), up(holo, kc), up(holo, vc)
    d1, d2 = holo.DeviceBuffer(4 * nh * hd), holo.DeviceBuffer(4 * nh * hd)
    lib.cuda_multi_head_attention(d1.ptr, dq.ptr, dk.ptr, dv.ptr, kv_len, hd, nh, nkv)
    lib.cuda_multi_head_attention(d2.ptr, dq.ptr, dk.ptr, dv.ptr, kv_len, hd, nh, nkv)
    lib.cuda_sync()
    holo.check("decode attention")
    got = down(d1, nh * hd)
    K = kc.reshape(kv_len, nkv, hd).astype(np.float64)
    V = vc.reshape(kv_len, nkv, hd).astype(np.float64)
    assert normwise_err(got, want_attention(q, K, V, nh, nkv, hd, kv_len)) <= 1e-5
    assert np.array_equal(got, down(d2, nh * hd))  # the ranges merge in a fixed order


@pytest.mark.parametrize("rows,pos0", [(1, 0), (1, 700), (3, 250), (4, 0)])
def test_prefill_few_rows(holo, synth, rows, pos0):
    """Up to 4 rows: holo_attention_prefill runs each row as a decode call; row
    m sees positions 0 .. pos0 + m."""
    print(f"case prefill rows {rows} pos0 {pos0}", flush=True)
    lib = holo.lib()
    hd, nh, nkv = 128, 8, 2
    kv_dim = nkv * hd
    max_seq = pos0 + rows + 5
    q = synth.normal(rows * nh * hd, seed=31)
    kc = synth.normal(max_seq * kv_dim, seed=32)
    vc = synth.normal(max_seq * kv_dim, seed=33)
    dq, dk, dv = up(holo, q), up(holo, kc), up(holo, vc)
    do = holo.DeviceBuffer(4 * rows * nh * hd)
    lib.holo_attention_prefill(do.ptr, dq.ptr, dk.ptr, dv.ptr, rows, pos0, hd, nh, nkv)
    lib.cuda_sync()
    holo.check("prefill few rows")
    got = down(do, rows * nh * hd).reshape(rows, nh * hd)
    K = kc.reshape(max_seq, nkv, hd).astype(np.float64)
    V = vc.reshape(max_seq, nkv, hd).astype(np.float64)
    for m in range(rows):
        want = want_attention(q[m * nh * hd:(m + 1) * nh * hd], K, V, nh, nkv, hd, pos0 + m + 1)
        assert normwise_err(got[m], want) <= 1e-5, m
