#!/usr/bin/env python3
"""Writes tests/golden/reference_vectors.npz: input/output vectors of the
reference CPU path, produced by running the reference's own C code
(src/ai/quant.c + src/ai/llm.c, compiled from /root/reference into
oracle/_ref/ by oracle/Makefile).  The fixture is data only: inputs (raw GGUF
blocks, activations) and the outputs the reference computed for them.

    make -C oracle ref && python tests/golden/make_golden.py

Contents (all small):
  f16_table            f16_to_f32 of all 65536 codes (quant.c:40-82), as u32 bits
  <t>_blocks           random blocks of type t in {q8_0, q4_0, q4_k, q6_k}
  <t>_dequant          dequantize_row_<t> of those blocks, u32 bits (strict build:
                       source-literal rounding)
  q4_k_scale_sweep     12*8 superblocks: d = 1.0, dmin = 1.0, one bit of the
                       12 scale bytes set, qs = 0x11 everywhere; and their
                       dequantised weights (q4_k_scale_sweep_out)
  q4_k_qs_sweep        128 superblocks: d = 1.0, dmin = 0, all scales = 1,
                       one qs byte = 0x21; and their weights
  mm_<t>_W, mm_<t>_x   a 24 x K matrix and an activation vector
  mm_<t>_<build>       matmul_q (llm.c:770) of the reference builds:
                       scalar (llm.c:876-915 order), strict, release
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "google-classic_amd"))

from oracle.oracle import RefBuild  # noqa: E402
from holo_mi355x import synth  # noqa: E402

Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14
NAMES = {Q8_0: "q8_0", Q4_0: "q4_0", Q4_K: "q4_k", Q6_K: "q6_k"}
QK = {Q8_0: 32, Q4_0: 32, Q4_K: 256, Q6_K: 256}
OUT = Path(__file__).resolve().parent / "reference_vectors.npz"


def main() -> None:
    strict = RefBuild("strict")
    builds = {k: RefBuild(k) for k in ("scalar", "strict", "release")}
    d = {}
    d["f16_table"] = np.array([strict.l.f16_to_f32(h) for h in range(65536)], dtype=np.float32).view(np.uint32)

    for t, name in NAMES.items():
        n = QK[t] * 40
        blk = synth.blocks(t, 1, n, seed=4242 + t)
        d[f"{name}_blocks"] = blk
        d[f"{name}_dequant"] = strict.dequant(t, blk, n).view(np.uint32)

    # Q4_K scale-bit sweep: which (scale|min, sub-block) each bit of the 12
    # packed bytes reaches is visible in the dequantised weights.
    sweep = np.zeros((96, 144), dtype=np.uint8)
    for byte in range(12):
        for bit in range(8):
            b = sweep[byte * 8 + bit]
            b[0:2] = (0x00, 0x3C)       # d = 1.0
            b[2:4] = (0x00, 0x3C)       # dmin = 1.0
            b[4 + byte] = 1 << bit
            b[16:] = 0x11               # every weight nibble = 1
    d["q4_k_scale_sweep"] = sweep.reshape(-1)
    d["q4_k_scale_sweep_out"] = strict.dequant(Q4_K, sweep.reshape(-1), 96 * 256).view(np.uint32)

    qsw = np.zeros((128, 144), dtype=np.uint8)
    for j in range(128):
        b = qsw[j]
        b[0:2] = (0x00, 0x3C)           # d = 1.0, dmin = 0
        b[4:8] = 1                      # scales of sub-blocks 0..3 = 1, mins 0
        b[12:16] = 0x01                 # scales of sub-blocks 4..7 = 1 << 2 | 0 = 4
        b[16 + j] = 0x21                # low nibble 1, high nibble 2
    d["q4_k_qs_sweep"] = qsw.reshape(-1)
    d["q4_k_qs_sweep_out"] = strict.dequant(Q4_K, qsw.reshape(-1), 128 * 256).view(np.uint32)

    for t, name in NAMES.items():
        K = QK[t] * 12
        W = synth.blocks(t, 24, K, seed=777 + t)
        x = synth.normal(K, seed=888 + t)
        d[f"mm_{name}_W"] = W
        d[f"mm_{name}_x"] = x
        for bname, b in builds.items():
            d[f"mm_{name}_{bname}"] = b.matmul(t, W, x, 24, K).view(np.uint32)

    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(d)} arrays)")


if __name__ == "__main__":
    main()
