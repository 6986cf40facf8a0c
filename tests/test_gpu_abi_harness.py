"""The drop-in boundary driven from C: tests/abi_harness.c (built by
build()) calls include/cuda_ops.h only, in the order of the reference's GPU
decode loop (src/ai/llm_cuda.c:604-918: seven cuda_matmul_q4_0 per layer,
cuda_rms_norm, cuda_silu_mul, cuda_vec_add, the loop's synchronisation and a
blocking copy back), as a separate process with no Python in the loop.

Checks: its output against the CPU chain (float64 norms, the oracle's
matmul_q and silu_mul) within the 1e-3 bar, and bit for bit against the same
calls made in this process through the ctypes binding (one library, one set
of kernels)."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle.oracle import max_rel_err, normwise_err

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
HARNESS = ROOT / "tests" / "abi_harness"
Q4_0 = 2
NAMES = ("q", "k", "v", "o", "gate", "up", "down")


def _rms(x, w, eps=1e-5):
    x64 = x.astype(np.float64)
    return (x64 / np.sqrt(np.mean(x64 * x64) + eps) * w).astype(np.float32)


def test_c_caller_runs_the_decode_loop(holo, synth, oracle, tmp_path):
    print("case abi harness: 2 layers dim 1024 ffn 2816", flush=True)
    assert HARNESS.exists(), "run build() (google-classic_amd/build.py builds tests/abi_harness)"
    dim, ffn, nl = 1024, 2816, 2
    shapes = {"q": (dim, dim), "k": (dim, dim), "v": (dim, dim), "o": (dim, dim), "gate": (ffn, dim),
              "up": (ffn, dim), "down": (dim, ffn)}
    W = [{n: synth.blocks(Q4_0, o, i, 4000 + 10 * l + j) for j, (n, (o, i)) in enumerate(shapes.items())}
         for l in range(nl)]
    x = synth.normal(dim, seed=4100)
    rng = np.random.default_rng(41)
    norms = (1.0 + 0.1 * rng.standard_normal(2 * nl * dim)).astype(np.float32)
    (tmp_path / "meta.txt").write_text(f"{dim} {ffn} {nl}\n")
    x.tofile(tmp_path / "x.bin")
    norms.tofile(tmp_path / "norm.bin")
    for l in range(nl):
        for n in NAMES:
            np.ascontiguousarray(W[l][n]).tofile(tmp_path / f"L{l}_{n}.bin")
    r = subprocess.run([str(HARNESS), str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    got = np.fromfile(tmp_path / "out.bin", dtype=np.float32)
    got_h = np.fromfile(tmp_path / "h.bin", dtype=np.float32)
    assert got.size == dim and got_h.size == ffn and np.all(np.isfinite(got))

    # the CPU chain
    xc = x.copy()
    for l in range(nl):
        xb = _rms(xc, norms[2 * l * dim:(2 * l + 1) * dim])
        v = oracle.matmul(Q4_0, W[l]["v"], xb, dim, dim)
        xc = (xc + oracle.matmul(Q4_0, W[l]["o"], v, dim, dim)).astype(np.float32)
        xb = _rms(xc, norms[(2 * l + 1) * dim:(2 * l + 2) * dim])
        h = oracle.silu_mul(oracle.matmul(Q4_0, W[l]["gate"], xb, ffn, dim),
                            oracle.matmul(Q4_0, W[l]["up"], xb, ffn, dim))
        xc = (xc + oracle.matmul(Q4_0, W[l]["down"], h, dim, ffn)).astype(np.float32)
    e, m = normwise_err(got, xc), max_rel_err(got, xc)
    print(f"  vs the CPU chain {e:.2e} (max rel {m:.2e})", flush=True)
    assert e <= 1e-3 and m <= 1e-3

    # the same calls in this process
    lib = holo.lib()
    up = holo.DeviceBuffer.from_array
    dW = [{n: up(np.ascontiguousarray(W[l][n])) for n in NAMES} for l in range(nl)]
    dx, dn = up(x), up(norms)
    buf = {n: holo.DeviceBuffer(4 * k) for n, k in (("xb", dim), ("q", dim), ("k", dim), ("v", dim), ("o", dim),
                                                  ("g", ffn), ("u", ffn), ("h", ffn))}
    for l in range(nl):
        L = dW[l]
        lib.cuda_rms_norm(buf["xb"].ptr, dx.ptr, dn.ptr + 4 * 2 * l * dim, dim, np.float32(1e-5))
        for n in ("q", "k", "v"):
            lib.cuda_matmul_q4_0(buf[n].ptr, L[n].ptr, buf["xb"].ptr, dim, dim)
        lib.cuda_matmul_q4_0(buf["o"].ptr, L["o"].ptr, buf["v"].ptr, dim, dim)
        lib.cuda_vec_add(dx.ptr, dx.ptr, buf["o"].ptr, dim)
        lib.cuda_rms_norm(buf["xb"].ptr, dx.ptr, dn.ptr + 4 * (2 * l + 1) * dim, dim, np.float32(1e-5))
        lib.cuda_matmul_q4_0(buf["g"].ptr, L["gate"].ptr, buf["xb"].ptr, ffn, dim)
        lib.cuda_matmul_q4_0(buf["u"].ptr, L["up"].ptr, buf["xb"].ptr, ffn, dim)
        lib.cuda_silu_mul(buf["h"].ptr, buf["g"].ptr, buf["u"].ptr, ffn)
        lib.cuda_matmul_q4_0(buf["o"].ptr, L["down"].ptr, buf["h"].ptr, dim, ffn)
        lib.cuda_vec_add(dx.ptr, dx.ptr, buf["o"].ptr, dim)
    lib.cuda_sync()
    holo.check("abi harness, in-process calls")
    assert np.array_equal(dx.download(np.float32, dim).view(np.uint32), got.view(np.uint32))
    assert np.array_equal(buf["h"].download(np.float32, ffn).view(np.uint32), got_h.view(np.uint32))
