"""Python binding of libholo_mi355x.so (ctypes) -- host-side mirror of the
reference op boundary include/cuda_ops.h plus the extensions of
include/holo_mi355x.h.

The functions keep the reference's names and argument meaning
(`cuda_matmul_q4_0(dst, M, v, out_dim, in_dim)` with device pointers), so a
test reads like a call sequence of src/ai/llm_cuda.c: cuda_init ->
cuda_malloc/cuda_memcpy_h2d -> cuda_matmul_* -> cuda_sync -> cuda_memcpy_d2h.

There is no CPU fallback: importing succeeds without a GPU (the CPU test suite
checks the exported symbols), but every op runs on the HIP library, and
`load()` raises if the library has not been built.

The process must not also load another HIP runtime (for example torch's
bundled libamdhip64): GPU tests and bench.py use only this binding and numpy.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent.parent
LIB_PATH = PKG_DIR / "libholo_mi355x.so"
ROOT = PKG_DIR.parent
HEADERS = [ROOT / "include" / "cuda_ops.h", ROOT / "include" / "holo_mi355x.h", ROOT / "include" / "holo_gguf.h",
           ROOT / "include" / "holo_forward.h"]

# GGML type ids (reference src/ai/quant.h:19-33)
TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 2, 8, 12, 14
# (block elements, block bytes) per type (reference gguf.c:26-71)
BLOCK = {TYPE_F32: (1, 4), TYPE_F16: (1, 2), TYPE_Q4_0: (32, 18), TYPE_Q8_0: (32, 34),
         TYPE_Q4_K: (256, 144), TYPE_Q6_K: (256, 210)}
TYPE_NAMES = {"f32": TYPE_F32, "f16": TYPE_F16, "q4_0": TYPE_Q4_0, "q8_0": TYPE_Q8_0,
              "q4_k": TYPE_Q4_K, "q6_k": TYPE_Q6_K}


def row_bytes(qtype: int, in_dim: int) -> int:
    """Bytes of one matrix row: in_dim/QK blocks, truncating (cuda_ops.cu:624)."""
    qk, bb = BLOCK[qtype]
    return (in_dim // qk) * bb


def tensor_bytes(qtype: int, n_elem: int) -> int:
    """quant_size of src/ai/llm_cuda.c:121-137 (rounds the block count up)."""
    qk, bb = BLOCK[qtype]
    return ((n_elem + qk - 1) // qk) * bb


_P = C.c_void_p
_I = C.c_int
_SZ = C.c_size_t
_F = C.c_float
_I64 = C.c_int64

# name -> (restype, argtypes)
_SIGS = {
    # runtime (reference cuda_ops.h:18-40)
    "cuda_init": (_I, []),
    "cuda_cleanup": (None, []),
    "cuda_available": (C.c_bool, []),
    "cuda_print_info": (None, []),
    "cuda_get_device_count": (_I, []),
    "cuda_get_free_memory": (_SZ, []),
    "cuda_get_device_name": (C.c_char_p, []),
    "cuda_malloc": (_P, [_SZ]),
    "cuda_free": (None, [_P]),
    "cuda_memcpy_h2d": (None, [_P, _P, _SZ]),
    "cuda_memcpy_d2h": (None, [_P, _P, _SZ]),
    "cuda_memcpy_d2d": (None, [_P, _P, _SZ]),
    "cuda_memcpy_d2d_async": (None, [_P, _P, _SZ]),
    "cuda_memcpy_d2h_async": (None, [_P, _P, _SZ]),
    "cuda_memset": (None, [_P, _I, _SZ]),
    "cuda_sync": (None, []),
    "cuda_sync_copy": (None, []),
    # matmuls (cuda_ops.h:50-66)
    "cuda_matmul_q8_0": (None, [_P, _P, _P, _I, _I]),
    "cuda_matmul_q4_0": (None, [_P, _P, _P, _I, _I]),
    "cuda_matmul_q4_k": (None, [_P, _P, _P, _I, _I]),
    "cuda_matmul_q6_k": (None, [_P, _P, _P, _I, _I]),
    "cuda_matmul_f32": (None, [_P, _P, _P, _I, _I]),
    "cuda_matmul_f16": (None, [_P, _P, _P, _I, _I]),
    "cuda_batched_qkv_q8_0": (None, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I]),
    "cuda_batched_ffn_gate_up_q8_0": (None, [_P, _P, _P, _P, _I, _I]),
    # vector / activation / norm (cuda_ops.h:43-80)
    "cuda_vec_add": (None, [_P, _P, _P, _I]),
    "cuda_vec_mul": (None, [_P, _P, _P, _I]),
    "cuda_vec_scale": (None, [_P, _P, _F, _I]),
    "cuda_vec_dot": (_F, [_P, _P, _I]),
    "cuda_silu": (None, [_P, _I]),
    "cuda_silu_mul": (None, [_P, _P, _P, _I]),
    "cuda_gelu": (None, [_P, _I]),
    "cuda_relu": (None, [_P, _I]),
    "cuda_rms_norm": (None, [_P, _P, _P, _I, _F]),
    "cuda_layer_norm": (None, [_P, _P, _P, _P, _I, _F]),
    "cuda_softmax": (None, [_P, _P, _I]),
    "cuda_softmax_inplace": (None, [_P, _I]),
    # attention / rope / embedding / argmax (cuda_ops.h:83-133)
    "cuda_attention_scores": (None, [_P, _P, _P, _I, _I, _I, _F]),
    "cuda_attention_apply": (None, [_P, _P, _P, _I, _I, _I]),
    "cuda_attention_single": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I]),
    "cuda_multi_head_attention": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "cuda_rope_apply": (None, [_P, _P, _I, _I, _I, _I, _F]),
    "cuda_get_embedding_f32": (None, [_P, _P, _I, _I, _I]),
    "cuda_get_embedding_f16": (None, [_P, _P, _I, _I, _I]),
    "cuda_get_embedding_q8_0": (None, [_P, _P, _I, _I, _I]),
    "cuda_get_embedding_q4_0": (None, [_P, _P, _I, _I, _I]),
    "cuda_get_embedding_q6_k": (None, [_P, _P, _I, _I, _I]),
    "cuda_argmax": (_I, [_P, _I]),
    # extensions (holo_mi355x.h)
    "holo_last_error": (_I, []),
    "holo_error_string": (C.c_char_p, [_I]),
    "holo_set_stream": (None, [_P]),
    "holo_get_stream": (_P, []),
    "holo_event_create": (_P, []),
    "holo_event_record": (None, [_P]),
    "holo_event_elapsed_ms": (_F, [_P, _P]),
    "holo_event_destroy": (None, [_P]),
    "holo_stream_create": (_P, []),
    "holo_stream_destroy": (None, [_P]),
    "holo_graph_begin": (_I, []),
    "holo_graph_end": (_P, []),
    "holo_graph_launch": (_I, [_P]),
    "holo_graph_destroy": (None, [_P]),
    "holo_matmul": (None, [_P, _P, _P, _I, _I, _I]),
    "holo_gemv_set_xmode": (None, [_I]),
    "holo_time_next_launch": (None, [_P, _P]),
    "holo_gemv_stream_create": (_P, [_P, _I, _I]),
    "holo_gemv_stream_launch": (_I, [_P]),
    "holo_gemv_stream_destroy": (None, [_P]),
    "holo_gemv_stream_status": (_I, []),
    "holo_gemv_set_launch": (None, [_I, _I]),
    "holo_dequant": (None, [_P, _P, _I64, _I]),
    "holo_dequant_f16": (None, [_P, _P, _I64, _I]),
    "holo_batched_qkv": (None, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I]),
    "holo_batched_ffn_gate_up": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "holo_quantize_act_q8_0": (None, [_P, _P, _I, _I]),
    "holo_gemm_q4_0_q8_0": (None, [_P, _P, _P, _I, _I, _I]),
    "holo_gemm_q4_0_q8_0_noalloc": (_I, [_P, _P, _P, _I, _I, _I]),
    "holo_matmul_batch_q4_0": (None, [_P, _P, _P, _I, _I, _I, _P]),
    "holo_gemm_q4_0_q8_0_multi": (None, [_P, _P, _P, _I, _P, _I, _I]),
    "holo_matmul_batch_q4_0_multi": (None, [_P, _P, _P, _I, _P, _I, _I, _P]),
    "holo_gemm_q4_0_f16": (None, [_P, _P, _P, _I, _I, _I]),
    "holo_gemm_q4_0_f16_multi": (None, [_P, _P, _P, _I, _P, _I, _I]),
    "holo_prefill_set_mode": (None, [_I]),
    "holo_prefill_set_q8_kernel": (None, [_I]),
    "holo_prefill_get_q8_kernel": (_I, []),
    "holo_prefill_get_mode": (_I, []),
    "holo_batched_qkv_norm": (None, [_P, _P, _P, _P, _P, _P, _P, _P, C.c_float, _P, _I, _I, _I, _I]),
    "holo_batched_ffn_gate_up_norm": (None, [_P, _P, _P, _P, _P, C.c_float, _P, _I, _I, _I]),
    "holo_matmul_add": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "holo_matmul_batch_q4_0_add": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "holo_matmul_batch_q4_0_swiglu_add": (None, [_P, _P, _P, _P, _P, _I, _I, _I]),
    "holo_matmul_batch": (None, [_P, _P, _P, _I, _I, _I, _I]),
    "holo_matmul_batch_multi": (None, [_P, _P, _P, _I, _P, _I, _I, _I]),
    "holo_matmul_batch_multi_types": (None, [_P, _P, _P, _P, _I, _P, _I, _I]),
    "holo_matmul_batch_add": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "holo_matmul_batch_swiglu_add": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I]),
    "holo_prefill_prepare": (_I, [_P, _I, _I, _I]),
    "holo_prefill_release": (None, [_P]),
    # GGUF files (include/holo_gguf.h)
    "holo_gguf_open": (_P, [C.c_char_p]),
    "holo_gguf_close": (None, [_P]),
    "holo_gguf_version": (C.c_uint32, [_P]),
    "holo_gguf_n_tensors": (C.c_uint64, [_P]),
    "holo_gguf_n_kv": (C.c_uint64, [_P]),
    "holo_gguf_data_offset": (C.c_uint64, [_P]),
    "holo_gguf_model": (_P, [_P]),
    "holo_gguf_key": (C.c_char_p, [_P, C.c_uint64]),
    "holo_gguf_value_type": (_I, [_P, C.c_char_p]),
    "holo_gguf_get_string": (C.c_char_p, [_P, C.c_char_p]),
    "holo_gguf_get_int": (_I64, [_P, C.c_char_p, _I64]),
    "holo_gguf_get_float": (_F, [_P, C.c_char_p, _F]),
    "holo_gguf_get_array": (_P, [_P, C.c_char_p, C.POINTER(C.c_uint64), C.POINTER(_I)]),
    "holo_gguf_tensor": (_P, [_P, C.c_uint64]),
    "holo_gguf_find_tensor": (_P, [_P, C.c_char_p]),
    "holo_gguf_load_tensor": (_I, [_P, _P, _P, _SZ]),
    "holo_gguf_upload": (_I, [_P]),
    "holo_gguf_device_base": (_P, [_P]),
    "holo_gguf_device_bytes": (_SZ, [_P]),
    "holo_gguf_device_ptr": (_P, [_P, _P]),
    # prompt forward (include/holo_forward.h)
    "holo_rms_norm_rows": (None, [_P, _P, _P, _I, _I, _F]),
    "holo_rope_rows": (None, [_P, _P, _I, _I, _I, _I, _I, _F]),
    "holo_embedding_rows": (None, [_P, _P, _P, _I, _I, _I]),
    "holo_attention_prefill": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "holo_matmul_rows": (None, [_P, _P, _P, _I, _I, _I, _I, _I]),
    "holo_llama_forward": (_I, [_P, _P, _I, _I, _P, _I]),
    "holo_llama_prepare": (_I, [_P]),
    "holo_llama_release": (None, [_P]),
    "holo_llama_from_gguf": (_I, [_P, _P, _P, _I]),
    "holo_llama_gguf_check": (_I, [_P]),
}

_lib: C.CDLL | None = None


EINVAL, ECHAIN = 100001, 100002


class StreamStage(C.Structure):
    """holo_stream_stage_t (include/holo_mi355x.h): one stage of a
    holo_gemv_stream plan."""
    _fields_ = [("W", C.c_void_p * 3), ("y", C.c_void_p * 3), ("rows", C.c_int * 3), ("nmat", C.c_int),
                ("gate_up", C.c_int), ("x", C.c_void_p), ("in_dim", C.c_int), ("norm_w", C.c_void_p),
                ("eps", C.c_float), ("r", C.c_void_p)]


def stream_stage(W, y, rows, x, in_dim, gate_up=False, norm_w=None, eps=1e-5, r=None) -> StreamStage:
    """A stream stage from device pointers: matrices W, outputs y (one for a
    gate/up pair), their row counts, input x of in_dim values, and the
    optional rms-norm weight of the input and residual of the output."""
    s = StreamStage()
    for i, w in enumerate(W):
        s.W[i] = w
    for i, o in enumerate(y):
        s.y[i] = o
    for i, n in enumerate(rows):
        s.rows[i] = n
    s.nmat = len(W)
    s.gate_up = 1 if gate_up else 0
    s.x = x
    s.in_dim = in_dim
    s.norm_w = norm_w
    s.eps = eps
    s.r = r
    return s


class StreamPlan:
    """A holo_gemv_stream plan (device stage table) for a list of StreamStage."""

    def __init__(self, stages, qtype: int):
        arr = (StreamStage * len(stages))(*stages)
        self.p = lib().holo_gemv_stream_create(C.cast(arr, C.c_void_p), len(stages), qtype)
        if not self.p:
            raise HoloError(f"holo_gemv_stream_create rejected the plan: {lib().holo_last_error()}")

    def launch(self) -> int:
        return lib().holo_gemv_stream_launch(self.p)

    def close(self):
        if self.p:
            lib().holo_gemv_stream_destroy(self.p)
            self.p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GgufTensor(C.Structure):
    """holo_gguf_tensor_t (include/holo_gguf.h), the fields of the reference's
    gguf_tensor_info_t (src/ai/gguf.h:107-118)."""
    _fields_ = [("name", C.c_char * 256), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 4), ("type", C.c_int32),
                ("offset", C.c_uint64), ("n_elements", C.c_uint64), ("size_bytes", C.c_uint64)]


class GgufModel(C.Structure):
    """holo_gguf_model_t (include/holo_gguf.h), the reference's model fields (src/ai/gguf.h:151-165)."""
    _fields_ = [("arch", C.c_char * 64)] + [(n, C.c_uint32) for n in (
        "vocab_size", "context_length", "embedding_length", "block_count", "attention_head_count",
        "attention_head_count_kv", "attention_key_length", "feed_forward_length")] + [
        (n, C.c_float) for n in ("rope_freq_base", "rope_freq_scale", "rms_norm_eps")]


class LlamaLayer(C.Structure):
    """holo_llama_layer_t (include/holo_forward.h)."""
    _fields_ = [("attn_norm", C.c_void_p), ("wq", C.c_void_p), ("wk", C.c_void_p), ("wv", C.c_void_p),
                ("wo", C.c_void_p), ("wq_type", C.c_int), ("wk_type", C.c_int), ("wv_type", C.c_int),
                ("wo_type", C.c_int), ("ffn_norm", C.c_void_p), ("w1", C.c_void_p), ("w2", C.c_void_p),
                ("w3", C.c_void_p), ("w1_type", C.c_int), ("w2_type", C.c_int), ("w3_type", C.c_int)]


class LlamaModel(C.Structure):
    """holo_llama_t (include/holo_forward.h)."""
    _fields_ = [(n, C.c_int) for n in ("n_layers", "dim", "n_heads", "n_kv_heads", "head_dim", "ffn_dim", "vocab",
                                       "max_seq")] + [
        ("rms_eps", C.c_float), ("rope_base", C.c_float), ("tok_emb", C.c_void_p), ("emb_type", C.c_int),
        ("out_norm", C.c_void_p), ("output", C.c_void_p), ("out_type", C.c_int), ("key_cache", C.c_void_p),
        ("value_cache", C.c_void_p), ("layers", C.POINTER(LlamaLayer))]


class HoloError(RuntimeError):
    pass


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load libholo_mi355x.so (once) and attach the C signatures."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise HoloError(f"{p} is not built; run `python google-classic_amd/build.py` "
                        "(or __graft_entry__.build())")
    lib = C.CDLL(str(p))
    missing = []
    for name, (res, args) in _SIGS.items():
        try:
            f = getattr(lib, name)
        except AttributeError:
            missing.append(name)
            continue
        f.restype = res
        f.argtypes = args
    lib.holo_missing_symbols = missing
    _lib = lib
    return lib


def lib() -> C.CDLL:
    return load()


def check(what: str = "") -> None:
    """Raise if the library latched an error since the last check."""
    code = lib().holo_last_error()
    if code:
        raise HoloError(f"{what}: holo error {code}: {lib().holo_error_string(code).decode()}")


def init() -> None:
    if lib().cuda_init() != 0:
        raise HoloError("cuda_init failed: no HIP device")


class DeviceBuffer:
    """A cuda_malloc'd device allocation (freed on close / garbage collection)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = lib().cuda_malloc(max(self.nbytes, 1))
        if not self.ptr:
            raise HoloError(f"cuda_malloc({self.nbytes}) failed")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            lib().cuda_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        lib().cuda_memcpy_h2d(self.ptr + offset, a.ctypes.data, a.nbytes)

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        if out.nbytes:
            lib().cuda_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes)
        return out

    def close(self) -> None:
        if self.ptr and _lib is not None:
            _lib.cuda_free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def matmul(qtype: int, dst: DeviceBuffer, M: DeviceBuffer | None, v: DeviceBuffer, out_dim: int, in_dim: int):
    """gpu_matmul of src/ai/llm_cuda.c:140-163."""
    lib().holo_matmul(dst.ptr, M.ptr if M is not None else None, v.ptr, out_dim, in_dim, qtype)


class Events:
    """HIP events on the library stream, for timing kernels in-process."""

    def __init__(self):
        self.a = lib().holo_event_create()
        self.b = lib().holo_event_create()

    def start(self):
        lib().holo_event_record(self.a)

    def stop(self) -> float:
        lib().holo_event_record(self.b)
        return float(lib().holo_event_elapsed_ms(self.a, self.b))

    def close(self):
        lib().holo_event_destroy(self.a)
        lib().holo_event_destroy(self.b)
