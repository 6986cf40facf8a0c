"""Writes tests/golden/forward_tiny.npz: the reference's own CPU forward on the
tiny Llama file of tests/llama_files.py.

The forward is src/ai/llm.c's llm_load + llm_forward, compiled from the
reference sources into oracle/_ref/libholo_ref_forward.so (oracle/Makefile,
oracle/ref_forward.c).  Cases: a 7-token prompt, an 80-token prompt, and the
same 80 tokens plus one more (one decode step after the prompt).  Stored:
the tokens, the logits after each case, and the key/value caches after the
81-token case (positions 0..80; by causality their first n rows are the
caches after any n-token prefix).

Run in the container that holds /root/reference:
    python3 tests/golden/make_forward_golden.py
"""
from __future__ import annotations

import ctypes as C
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT / "tests"), str(ROOT / "google-classic_amd"), str(ROOT)]

import llama_files as lf  # noqa: E402
from oracle.oracle import REF_DIR  # noqa: E402

OUT = ROOT / "tests" / "golden" / "forward_tiny.npz"
CASES = (7, 80, 81)


def ref_lib():
    lib = C.CDLL(str(REF_DIR / "libholo_ref_forward.so"))
    lib.ref_forward.restype = C.c_int
    lib.ref_forward.argtypes = [C.c_char_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p,
                                C.c_long, C.POINTER(C.c_int)]
    return lib


def run(lib, path, tokens):
    """Logits [vocab] and caches [n_layers][max_seq][kv_dim] after the tokens."""
    c = lf.CFG
    max_seq = c["ctx"]
    logits = np.empty(c["vocab"], np.float32)
    kc = np.zeros((c["n_layers"], max_seq, lf.KV_DIM), np.float32)
    vc = np.zeros_like(kc)
    got = C.c_int(0)
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    rc = lib.ref_forward(str(path).encode(), tok.ctypes.data, len(tok), logits.ctypes.data, c["vocab"],
                         kc.ctypes.data, vc.ctypes.data, kc.size, C.byref(got))
    assert rc == 0 and got.value == max_seq, (rc, got.value)
    return logits, kc, vc


def compute() -> dict:
    lib = ref_lib()
    tokens = lf.prompt(max(CASES))
    out = {"tokens": tokens}
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "tiny.gguf"
        lf.build(path)
        for n in CASES:
            logits, kc, vc = run(lib, path, tokens[:n])
            out[f"logits_{n}"] = logits
            if n == max(CASES):
                out["k_cache"] = kc[:, :n].copy()
                out["v_cache"] = vc[:, :n].copy()
    return out


def main():
    np.savez_compressed(OUT, **compute())
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
