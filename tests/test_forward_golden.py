"""The prompt-forward fixture (tests/golden/forward_tiny.npz) is the
reference's own CPU forward (src/ai/llm.c llm_load + llm_forward, built into
oracle/_ref/) on the tiny Llama file of tests/llama_files.py.  CPU only:
the fixture reproduces bit for bit from the reference build, and the model
file is deterministic."""
import hashlib

import numpy as np
import pytest

import llama_files as lf
from oracle.oracle import REF_DIR

GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden" / "forward_tiny.npz"


def test_model_file_is_deterministic(tmp_path):
    a, b = tmp_path / "a.gguf", tmp_path / "b.gguf"
    lf.build(a)
    lf.build(b)
    assert hashlib.sha256(a.read_bytes()).digest() == hashlib.sha256(b.read_bytes()).digest()


@pytest.mark.skipif(not (REF_DIR / "libholo_ref_forward.so").exists(), reason="oracle/_ref not built")
def test_fixture_reproduces_from_the_reference():
    import importlib.util
    spec = importlib.util.spec_from_file_location("mfg", GOLDEN.parent / "make_forward_golden.py")
    mfg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mfg)
    got = mfg.compute()
    want = np.load(GOLDEN)
    assert set(got) == set(want.files)
    for k in want.files:
        assert np.array_equal(got[k], want[k]), k


def test_fixture_shapes():
    z = np.load(GOLDEN)
    c = lf.CFG
    assert z["tokens"].shape == (81,) and z["tokens"].max() < c["vocab"]
    for n in (7, 80, 81):
        assert z[f"logits_{n}"].shape == (c["vocab"],) and np.all(np.isfinite(z[f"logits_{n}"]))
    assert z["k_cache"].shape == (c["n_layers"], 81, lf.KV_DIM) == z["v_cache"].shape
