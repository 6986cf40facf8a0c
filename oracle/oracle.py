"""ctypes + numpy wrapper of the CPU oracle (liboracle.so) and of the reference
builds under oracle/_ref/.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU
baseline, never as a product path.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_DIR = HERE / "_ref"
REF_BUILDS = ("release", "strict", "scalar")

TYPE_Q4_0, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K = 2, 8, 12, 14

_P = C.c_void_p
_I = C.c_int


def build(quiet: bool = True) -> None:
    """make -C oracle: liboracle.so, plus oracle/_ref/* when /root/reference exists."""
    r = subprocess.run(["make", "-C", str(HERE)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stdout + r.stderr)
    if not quiet:
        print(r.stdout)


class Oracle:
    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            build()
        l = C.CDLL(str(path))
        l.oracle_f16_to_f32.argtypes = [C.c_uint16]
        l.oracle_f16_to_f32.restype = C.c_float
        l.oracle_f32_to_f16_rne.argtypes = [C.c_float]
        l.oracle_f32_to_f16_rne.restype = C.c_uint16
        for n in ("oracle_dequant_q8_0", "oracle_dequant_q4_0", "oracle_dequant_q4_k", "oracle_dequant_q6_k"):
            getattr(l, n).argtypes = [_P, _P, _I]
            getattr(l, n).restype = None
        for n in ("oracle_matmul_q8_0", "oracle_matmul_q4_0", "oracle_matmul_q4_k", "oracle_matmul_q6_k"):
            getattr(l, n).argtypes = [_P, _P, _P, _I, _I]
            getattr(l, n).restype = None
        l.oracle_matmul_f64.argtypes = [_P, _P, _P, _I, _I]
        l.oracle_q4_k_unpack_scales.argtypes = [_P, _P, _P]
        l.oracle_silu_mul.argtypes = [_P, _P, _P, _I]
        l.oracle_quantize_act_q8_0.argtypes = [_P, _P, _I, _I]
        l.oracle_gemm_q4_0_q8_0.argtypes = [_P, _P, _P, _I, _I, _I]
        l.oracle_gemm_q4_0_f16.argtypes = [_P, _P, _P, _P, _I, _I, _I]
        self.l = l

    _DQ = {TYPE_Q8_0: "oracle_dequant_q8_0", TYPE_Q4_0: "oracle_dequant_q4_0",
           TYPE_Q4_K: "oracle_dequant_q4_k", TYPE_Q6_K: "oracle_dequant_q6_k"}
    _MM = {TYPE_Q8_0: "oracle_matmul_q8_0", TYPE_Q4_0: "oracle_matmul_q4_0",
           TYPE_Q4_K: "oracle_matmul_q4_k", TYPE_Q6_K: "oracle_matmul_q6_k"}

    def f16_to_f32(self, h: int) -> float:
        return self.l.oracle_f16_to_f32(h)

    def f32_to_f16(self, f: float) -> int:
        return int(self.l.oracle_f32_to_f16_rne(f))

    def dequant(self, qtype: int, blocks: np.ndarray, n: int) -> np.ndarray:
        y = np.empty(n, dtype=np.float32)
        getattr(self.l, self._DQ[qtype])(blocks.ctypes.data, y.ctypes.data, n)
        return y

    def matmul(self, qtype: int, M: np.ndarray, v: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
        v = np.ascontiguousarray(v, dtype=np.float32)
        y = np.empty(out_dim, dtype=np.float32)
        getattr(self.l, self._MM[qtype])(y.ctypes.data, M.ctypes.data, v.ctypes.data, out_dim, in_dim)
        return y

    def matmul_f64(self, W: np.ndarray, v: np.ndarray) -> np.ndarray:
        W = np.ascontiguousarray(W, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        out_dim, in_dim = W.shape
        y = np.empty(out_dim, dtype=np.float64)
        self.l.oracle_matmul_f64(y.ctypes.data, W.ctypes.data, v.ctypes.data, out_dim, in_dim)
        return y

    def truth(self, qtype: int, M: np.ndarray, v: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
        """fp64 dot products over the bit-exact dequantised weights."""
        W = self.dequant(qtype, M, out_dim * in_dim).reshape(out_dim, in_dim)
        return self.matmul_f64(W, v[:in_dim])

    def truth_batch(self, qtype: int, M: np.ndarray, X: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
        """float64 X . W^T over the bit-exact dequantised weights (rows of X)."""
        W = self.dequant(qtype, M, out_dim * in_dim).reshape(out_dim, in_dim).astype(np.float64)
        return np.asarray(X, dtype=np.float64) @ W.T

    def q4_k_unpack_scales(self, sp: bytes):
        a = np.frombuffer(bytes(sp), dtype=np.uint8).copy()
        sc = np.empty(8, np.uint8)
        mn = np.empty(8, np.uint8)
        self.l.oracle_q4_k_unpack_scales(a.ctypes.data, sc.ctypes.data, mn.ctypes.data)
        return sc, mn

    def silu_mul(self, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        out = np.empty_like(g, dtype=np.float32)
        self.l.oracle_silu_mul(out.ctypes.data, np.ascontiguousarray(g, np.float32).ctypes.data,
                               np.ascontiguousarray(u, np.float32).ctypes.data, g.size)
        return out

    def quantize_act_q8_0(self, X: np.ndarray) -> np.ndarray:
        X = np.ascontiguousarray(X, dtype=np.float32)
        rows, k = X.shape
        out = np.empty(rows * (k // 32) * 34, dtype=np.uint8)
        self.l.oracle_quantize_act_q8_0(X.ctypes.data, out.ctypes.data, rows, k)
        return out

    def gemm_q4_0_q8_0(self, W: np.ndarray, Xq: np.ndarray, M: int, N: int, K: int) -> np.ndarray:
        Y = np.empty((M, N), dtype=np.float32)
        self.l.oracle_gemm_q4_0_q8_0(Y.ctypes.data, W.ctypes.data, Xq.ctypes.data, M, N, K)
        return Y

    def gemm_q4_0_f16(self, W: np.ndarray, X: np.ndarray, M: int, N: int, K: int):
        """(Y, A): the float64 truth of the f16-rounded operands and sum |x16 w16|."""
        X = np.ascontiguousarray(X, dtype=np.float32)
        W = np.ascontiguousarray(W)
        Y = np.empty((M, N), dtype=np.float64)
        A = np.empty((M, N), dtype=np.float64)
        self.l.oracle_gemm_q4_0_f16(Y.ctypes.data, A.ctypes.data, X.ctypes.data, W.ctypes.data, M, N, K)
        return Y, A


class RefBuild:
    """One build of the reference CPU path (quant.c + llm.c + tensor.c + gguf.c)."""

    def __init__(self, kind: str):
        path = REF_DIR / f"libholo_ref_{kind}.so"
        if not path.exists():
            raise FileNotFoundError(path)
        l = C.CDLL(str(path))
        l.f16_to_f32.argtypes = [C.c_uint16]
        l.f16_to_f32.restype = C.c_float
        for n in ("dequantize_row_q8_0", "dequantize_row_q4_0", "dequantize_row_q4_k", "dequantize_row_q6_k"):
            getattr(l, n).argtypes = [_P, _P, _I]
            getattr(l, n).restype = None
        l.matmul_q.argtypes = [_P, _P, _P, _I, _I, _I]
        l.matmul_q.restype = None
        self.l = l
        self.kind = kind
        self.path = path

    _DQ = {TYPE_Q8_0: "dequantize_row_q8_0", TYPE_Q4_0: "dequantize_row_q4_0",
           TYPE_Q4_K: "dequantize_row_q4_k", TYPE_Q6_K: "dequantize_row_q6_k"}

    def dequant(self, qtype: int, blocks: np.ndarray, n: int) -> np.ndarray:
        y = np.empty(n, dtype=np.float32)
        getattr(self.l, self._DQ[qtype])(blocks.ctypes.data, y.ctypes.data, n)
        return y

    def matmul(self, qtype: int, M: np.ndarray, v: np.ndarray, out_dim: int, in_dim: int) -> np.ndarray:
        """matmul_q of src/ai/llm.c:770."""
        v = np.ascontiguousarray(v, dtype=np.float32)
        y = np.empty(out_dim, dtype=np.float32)
        self.l.matmul_q(y.ctypes.data, M.ctypes.data, v.ctypes.data, out_dim, in_dim, qtype)
        return y


def ref_available(kind: str = "release") -> bool:
    return (REF_DIR / f"libholo_ref_{kind}.so").exists()


def normwise_err(got: np.ndarray, want: np.ndarray) -> float:
    """||got - want||_inf / ||want||_inf."""
    want = np.asarray(want, dtype=np.float64)
    d = np.max(np.abs(np.asarray(got, dtype=np.float64) - want))
    s = np.max(np.abs(want))
    return float(d / s) if s > 0 else float(d)


def max_rel_err(got: np.ndarray, want: np.ndarray, floor_frac: float = 0.05) -> float:
    """max |got-want|/|want| over outputs with |want| >= floor_frac * rms(want)
    (per-element relative error is unbounded for outputs near zero)."""
    want = np.asarray(want, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    rms = np.sqrt(np.mean(want * want)) if want.size else 0.0
    m = np.abs(want) >= floor_frac * rms
    if not np.any(m):
        return 0.0
    return float(np.max(np.abs(got[m] - want[m]) / np.abs(want[m])))
