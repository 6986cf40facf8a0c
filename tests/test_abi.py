"""The C-ABI library: it loads without a GPU and exports every function that
include/*.h declares; the reference caller (src/ai/llm_cuda.c) links
against it.  No compute calls (no GPU here)."""
import ctypes as C
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "google-classic_amd" / "libholo_mi355x.so"
HEADERS = [ROOT / "include" / "cuda_ops.h", ROOT / "include" / "holo_mi355x.h", ROOT / "include" / "holo_gguf.h",
           ROOT / "include" / "holo_forward.h"]
REF_CALLER = Path("/root/reference/src/ai/llm_cuda.c")


def declared_functions(header: Path):
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    names = re.findall(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\([^;{]*\)\s*;", text)
    return sorted(set(n for n in names if not n.startswith("HOLO_")))


def test_headers_declare_the_reference_boundary():
    names = declared_functions(HEADERS[0])
    # the 48 functions of the reference include/cuda_ops.h
    assert len(names) == 48
    for n in ("cuda_matmul_q4_0", "cuda_matmul_q8_0", "cuda_matmul_q4_k", "cuda_batched_qkv_q8_0",
              "cuda_batched_ffn_gate_up_q8_0", "cuda_init", "cuda_malloc", "cuda_memcpy_h2d"):
        assert n in names


def test_library_exports_every_declared_symbol():
    assert LIB.exists(), "run python google-classic_amd/build.py"
    lib = C.CDLL(str(LIB))
    missing = [n for h in HEADERS for n in declared_functions(h) if not hasattr(lib, n)]
    assert missing == []


def test_binding_covers_the_headers():
    import holo_mi355x as h
    declared = {n for hd in HEADERS for n in declared_functions(hd)}
    assert declared == set(h._SIGS)


def test_headers_compile_as_c():
    cc = shutil.which("gcc")
    src = "#include \"cuda_ops.h\"\n#include \"holo_mi355x.h\"\n#include \"holo_gguf.h\"\n#include \"holo_forward.h\"\nint main(void){return 0;}\n"
    r = subprocess.run([cc, "-std=c99", "-Wall", "-Werror", "-fsyntax-only", f"-I{ROOT / 'include'}", "-x", "c", "-"],
                       input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.skipif(not REF_CALLER.exists(), reason="reference sources not present")
def test_reference_caller_links_against_the_library(tmp_path):
    """src/ai/llm_cuda.c compiled (unmodified, from /root/reference) against
    this repo's include/cuda_ops.h and linked with libholo_mi355x.so.  The
    caller's one direct CUDA runtime call, cudaDeviceSynchronize()
    (llm_cuda.c:922), is mapped to cuda_sync on the command line."""
    ref = Path("/root/reference")
    work = tmp_path
    # the caller includes "cuda_ops.h" and "llm.h"/"gguf.h" from its own directory;
    # put this repo's header first on the include path
    objs = []
    for src in ("llm_cuda.c", "llm.c", "quant.c", "tensor.c", "gguf.c"):
        o = work / (src + ".o")
        r = subprocess.run(["gcc", "-std=gnu11", "-O1", "-w", "-DHOLO_USE_CUDA", "-DcudaDeviceSynchronize=cuda_sync",
                            f"-I{ROOT / 'include'}", f"-I{ref / 'src' / 'ai'}", f"-I{ref / 'include'}",
                            "-c", str(ref / "src" / "ai" / src), "-o", str(o)], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
        objs.append(str(o))
    main = work / "main.c"
    main.write_text("int llm_cuda_init(void*); int main(void){ return 0; }\n")
    exe = work / "caller"
    r = subprocess.run(["gcc", str(main), *objs, "-o", str(exe), f"-L{LIB.parent}", "-lholo_mi355x",
                        f"-Wl,-rpath,{LIB.parent}", "-lm", "-fopenmp"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_c_harness_is_built_and_linked():
    """tests/abi_harness (built by build()) links the library through its
    rpath, and without arguments prints its usage without touching a GPU."""
    harness = ROOT / "tests" / "abi_harness"
    assert harness.exists(), "run build()"
    r = subprocess.run(["ldd", str(harness)], capture_output=True, text=True)
    assert "libholo_mi355x.so" in r.stdout and "not found" not in r.stdout, r.stdout
    r = subprocess.run([str(harness)], capture_output=True, text=True, timeout=30)
    assert r.returncode == 1 and "usage" in r.stderr
