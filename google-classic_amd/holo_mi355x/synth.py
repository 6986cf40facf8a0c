"""Binding of libholo_synth.so: seeded synthetic GGUF blocks and activations.

The generator is specified in google-classic_amd/csrc/synth.c (SplitMix64
streams per block, Box-Muller normals, f16 round-to-nearest-even scales).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from . import TYPE_Q4_0, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0, BLOCK

LIB_PATH = Path(__file__).resolve().parent.parent / "libholo_synth.so"
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python google-classic_amd/build.py`")
        l = C.CDLL(str(LIB_PATH))
        for n in ("holo_synth_q8_0", "holo_synth_q4_0", "holo_synth_q4_k", "holo_synth_q6_k"):
            getattr(l, n).argtypes = [C.c_void_p, C.c_int64, C.c_uint64]
            getattr(l, n).restype = None
        l.holo_synth_normal_f32.argtypes = [C.c_void_p, C.c_int64, C.c_uint64]
        l.holo_synth_normal_f32.restype = None
        l.holo_synth_f32_to_f16.argtypes = [C.c_float]
        l.holo_synth_f32_to_f16.restype = C.c_uint16
        l.holo_synth_tensor_seed.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32]
        l.holo_synth_tensor_seed.restype = C.c_uint64
        _lib = l
    return _lib


_FN = {TYPE_Q8_0: "holo_synth_q8_0", TYPE_Q4_0: "holo_synth_q4_0",
       TYPE_Q4_K: "holo_synth_q4_k", TYPE_Q6_K: "holo_synth_q6_k"}


def blocks(qtype: int, rows: int, in_dim: int, seed: int, out: np.ndarray | None = None) -> np.ndarray:
    """rows x in_dim weights as a flat uint8 array of GGUF blocks."""
    qk, bb = BLOCK[qtype]
    nb = rows * (in_dim // qk)
    if out is None:
        out = np.empty(nb * bb, dtype=np.uint8)
    assert out.nbytes >= nb * bb and out.flags.c_contiguous
    getattr(lib(), _FN[qtype])(out.ctypes.data, nb, seed & 0xFFFFFFFFFFFFFFFF)
    return out


def normal(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().holo_synth_normal_f32(out.ctypes.data, n, seed & 0xFFFFFFFFFFFFFFFF)
    return out


def f32_to_f16_bits(x: float) -> int:
    return int(lib().holo_synth_f32_to_f16(float(x)))


def tensor_seed(base: int, config: int, layer: int, matrix: int) -> int:
    return int(lib().holo_synth_tensor_seed(base & 0xFFFFFFFFFFFFFFFF, config, layer, matrix))
