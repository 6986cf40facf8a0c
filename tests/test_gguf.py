"""GGUF parser of libholo_mi355x.so (include/holo_gguf.h), CPU only.

Each file is parsed by the library and, where oracle/_ref is built, by the
reference's own parser (src/ai/gguf.c, compiled from the reference sources
into oracle/_ref/): the tensor table, data offset, metadata answers, model
parameters, tensor bytes and the accept/reject decision must agree.  The
files are written by tests/gguf_files.py, so the expected values are also
known independently of both parsers.

Two inputs divide by zero in the reference (tensor types without a block
size, attention.head_count = 0) and are checked against the library only.
"""
import ctypes as C
import struct

import numpy as np
import pytest

import gguf_files as gf
from oracle.oracle import REF_DIR, ref_available

HAS_REF = ref_available("strict")


@pytest.fixture(scope="module")
def L():
    import holo_mi355x as h
    return h.load()


class RefStr(C.Structure):
    _fields_ = [("len", C.c_uint64), ("data", C.c_char_p)]


class RefValue(C.Structure):
    _fields_ = [("type", C.c_int32), ("pad", C.c_int32), ("u", C.c_uint8 * 24)]


class RefKv(C.Structure):
    _fields_ = [("key", RefStr), ("value", RefValue)]


def _ref():
    import holo_mi355x as h

    class RefCtx(C.Structure):
        _fields_ = [("path", C.c_char * 1024), ("file", C.c_void_p), ("magic", C.c_uint32), ("version", C.c_uint32),
                    ("n_tensors", C.c_uint64), ("n_kv", C.c_uint64), ("kv", C.POINTER(RefKv)),
                    ("tensors", C.POINTER(h.GgufTensor)), ("data_offset", C.c_uint64), ("mmap_base", C.c_void_p),
                    ("mmap_size", C.c_size_t), ("model", h.GgufModel)]

    r = C.CDLL(str(REF_DIR / "libholo_ref_strict.so"))
    r.gguf_open.restype, r.gguf_open.argtypes = C.POINTER(RefCtx), [C.c_char_p]
    r.gguf_close.restype, r.gguf_close.argtypes = None, [C.c_void_p]
    r.gguf_get_int.restype, r.gguf_get_int.argtypes = C.c_int64, [C.c_void_p, C.c_char_p, C.c_int64]
    r.gguf_get_float.restype, r.gguf_get_float.argtypes = C.c_float, [C.c_void_p, C.c_char_p, C.c_float]
    r.gguf_get_string.restype, r.gguf_get_string.argtypes = C.c_char_p, [C.c_void_p, C.c_char_p]
    r.gguf_get_value.restype, r.gguf_get_value.argtypes = C.POINTER(RefValue), [C.c_void_p, C.c_char_p]
    r.gguf_get_array.restype, r.gguf_get_array.argtypes = C.c_void_p, [C.c_void_p, C.c_char_p, C.POINTER(C.c_uint64)]
    r.gguf_find_tensor.restype, r.gguf_find_tensor.argtypes = C.POINTER(h.GgufTensor), [C.c_void_p, C.c_char_p]
    r.gguf_load_tensor.restype, r.gguf_load_tensor.argtypes = C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]
    return r


def _tensor(L, g, i):
    import holo_mi355x as h
    p = L.holo_gguf_tensor(g, i)
    return h.GgufTensor.from_address(p) if p else None


def _model(L, g):
    import holo_mi355x as h
    return h.GgufModel.from_address(L.holo_gguf_model(g))


def _fields(t):
    return (bytes(t.name), t.n_dims, tuple(t.dims), t.type, t.offset, t.n_elements, t.size_bytes)


def _model_fields(m):
    return tuple(getattr(m, f) for f, _ in m._fields_)


def _rich_file(tmp_path, rng, name="rich.gguf"):
    """Every metadata type, arrays of every element type, Llama keys and a
    tensor of each block type the reference tables list."""
    kvs = [("general.architecture", gf.STR, "llama"), ("llama.embedding_length", gf.U32, 256),
           ("llama.block_count", gf.U64, 2), ("llama.attention.head_count", gf.I32, 8),
           ("llama.attention.head_count_kv", gf.U16, 2), ("llama.feed_forward_length", gf.I64, 704),
           ("llama.rope.freq_base", gf.F64, 500000.0), ("llama.attention.layer_norm_rms_epsilon", gf.F32, 1e-6),
           ("llama.context_length", gf.U8, 200), ("k.i8", gf.I8, -5), ("k.i16", gf.I16, -300),
           ("k.bool", gf.BOOL, 1), ("k.f32", gf.F32, 2.5), ("k.str", gf.STR, "hello"), ("k.empty", gf.STR, ""),
           ("k.u64big", gf.U64, 2 ** 63 + 5)]
    for et in (gf.U8, gf.I8, gf.U16, gf.I16, gf.U32, gf.I32, gf.F32, gf.BOOL, gf.U64, gf.I64, gf.F64):
        vals = [int(v) for v in rng.integers(0, 100, size=7)]
        if et in (gf.F32, gf.F64):
            vals = [float(v) / 4 for v in vals]
        if et == gf.BOOL:
            vals = [v & 1 for v in vals]
        kvs.append((f"arr.{et}", gf.ARR, (et, vals)))
    kvs.append(("tokenizer.ggml.tokens", gf.ARR, (gf.STR, ["<s>", "</s>", "", "tok" * 50])))
    kvs.append(("arr.empty", gf.ARR, (gf.U32, [])))
    tensors = []
    for j, (t, dims) in enumerate([(0, [256]), (1, [64, 3]), (2, [256, 16]), (8, [256, 8]), (12, [512, 4]),
                                   (14, [256, 2]), (3, [64, 2]), (29, [5, 7]), (0, [3, 1, 2, 4]), (2, [40, 3]),
                                   (0, [])]):
        n = int(np.prod(dims)) if dims else 1
        data = rng.integers(0, 256, size=gf.size_bytes(t, n), dtype=np.uint8).tobytes()
        tensors.append(gf.Tensor(f"blk.{j}.weight", dims, t, data))
    path = tmp_path / name
    off = gf.write(path, kvs, tensors)
    return path, kvs, tensors, off


def test_parse_matches_what_was_written(L, tmp_path):
    rng = np.random.default_rng(1)
    path, kvs, tensors, off = _rich_file(tmp_path, rng)
    g = L.holo_gguf_open(str(path).encode())
    assert g
    try:
        assert L.holo_gguf_version(g) == 3
        assert L.holo_gguf_n_kv(g) == len(kvs) and L.holo_gguf_n_tensors(g) == len(tensors)
        assert L.holo_gguf_data_offset(g) == off
        assert [L.holo_gguf_key(g, i).decode() for i in range(len(kvs))] == [k for k, _, _ in kvs]
        for k, vt, v in kvs:
            assert L.holo_gguf_value_type(g, k.encode()) == vt
            if vt in (gf.U8, gf.I8, gf.U16, gf.I16, gf.U32, gf.I32, gf.I64):
                assert L.holo_gguf_get_int(g, k.encode(), -7) == v
            elif vt == gf.U64:
                assert L.holo_gguf_get_int(g, k.encode(), -7) == (v - 2 ** 64 if v >= 2 ** 63 else v)
            elif vt in (gf.F32, gf.F64):
                assert L.holo_gguf_get_float(g, k.encode(), -1.0) == np.float32(v)
                assert L.holo_gguf_get_int(g, k.encode(), -7) == -7
            elif vt == gf.STR:
                assert L.holo_gguf_get_string(g, k.encode()).decode() == v
            elif vt == gf.BOOL:
                assert L.holo_gguf_get_int(g, k.encode(), -7) == -7
            elif vt == gf.ARR:
                n, et = C.c_uint64(), C.c_int()
                p = L.holo_gguf_get_array(g, k.encode(), C.byref(n), C.byref(et))
                et_w, items = v
                assert n.value == len(items) and et.value == et_w
                if et_w == gf.STR:
                    arr = (RefStr * len(items)).from_address(p)
                    assert [C.string_at(e.data, e.len).decode() for e in arr] == items
                elif items:
                    raw = C.string_at(p, len(items) * struct.calcsize(gf._FMT[et_w]))
                    assert raw == b"".join(struct.pack(gf._FMT[et_w], x) for x in items)
        assert L.holo_gguf_value_type(g, b"missing") == -1
        assert L.holo_gguf_get_int(g, b"missing", 42) == 42
        for i, t in enumerate(tensors):
            got = _tensor(L, g, i)
            assert got.name.decode() == t.name and got.n_dims == len(t.dims)
            assert list(got.dims)[:len(t.dims)] == t.dims and got.type == t.type
            assert got.offset == t.offset and got.n_elements == t.n_elements and got.size_bytes == t.size
            buf = (C.c_uint8 * max(t.size, 1))()
            assert L.holo_gguf_load_tensor(g, C.addressof(got), buf, t.size) == 0
            assert bytes(buf)[:t.size] == t.data
            if t.size:
                assert L.holo_gguf_load_tensor(g, C.addressof(got), buf, t.size - 1) == -1
            assert L.holo_gguf_find_tensor(g, t.name.encode()) == C.addressof(got)
        assert not L.holo_gguf_find_tensor(g, b"nope")
        m = _model(L, g)
        assert (m.arch, m.embedding_length, m.block_count, m.attention_head_count) == (b"llama", 256, 2, 8)
        assert (m.attention_head_count_kv, m.attention_key_length, m.feed_forward_length) == (2, 32, 704)
        assert (m.context_length, m.vocab_size, m.rope_freq_base) == (200, 32000, 500000.0)
        assert m.rms_norm_eps == np.float32(1e-6) and m.rope_freq_scale == 0.0
        assert not L.holo_gguf_device_base(g) and L.holo_gguf_device_bytes(g) == 0
    finally:
        L.holo_gguf_close(g)


def _same_as_reference(L, r, path, keys=(), check_tensors=True):
    g = L.holo_gguf_open(str(path).encode())
    c = r.gguf_open(str(path).encode())
    assert bool(g) == bool(c), path
    if not g:
        return False
    try:
        ctx = c.contents
        assert (L.holo_gguf_version(g), L.holo_gguf_n_tensors(g), L.holo_gguf_n_kv(g), L.holo_gguf_data_offset(g)) == \
               (ctx.version, ctx.n_tensors, ctx.n_kv, ctx.data_offset)
        assert _model_fields(_model(L, g)) == _model_fields(ctx.model)
        for i in range(ctx.n_kv):
            k = ctx.kv[i].key.data
            assert L.holo_gguf_key(g, i) == k
        for k in list(keys) + [ctx.kv[i].key.data for i in range(ctx.n_kv)]:
            assert L.holo_gguf_get_int(g, k, -99) == r.gguf_get_int(c, k, -99), k
            assert L.holo_gguf_get_float(g, k, -9.5) == r.gguf_get_float(c, k, -9.5), k
            assert L.holo_gguf_get_string(g, k) == r.gguf_get_string(c, k), k
            rv = r.gguf_get_value(c, k)
            assert L.holo_gguf_value_type(g, k) == (rv.contents.type if rv else -1), k
            n1, n2 = C.c_uint64(), C.c_uint64()
            p1 = L.holo_gguf_get_array(g, k, C.byref(n1), None)
            p2 = r.gguf_get_array(c, k, C.byref(n2))
            assert n1.value == n2.value and bool(p1) == bool(p2), k
        if check_tensors:
            for i in range(ctx.n_tensors):
                ours, theirs = _tensor(L, g, i), ctx.tensors[i]
                assert _fields(ours) == _fields(theirs), i
                assert r.gguf_find_tensor(c, theirs.name).contents.offset == ours.offset
                n = ours.size_bytes
                b1, b2 = (C.c_uint8 * max(n, 1))(), (C.c_uint8 * max(n, 1))()
                assert L.holo_gguf_load_tensor(g, C.addressof(ours), b1, n) == \
                       r.gguf_load_tensor(c, C.addressof(theirs), b2, n)
                assert bytes(b1) == bytes(b2)
        return True
    finally:
        L.holo_gguf_close(g)
        r.gguf_close(c)


@pytest.mark.skipif(not HAS_REF, reason="oracle/_ref not built (needs /root/reference)")
def test_agrees_with_reference_parser(L, tmp_path):
    r = _ref()
    rng = np.random.default_rng(2)
    path, kvs, tensors, _ = _rich_file(tmp_path, rng)
    assert _same_as_reference(L, r, path, keys=[b"missing", b"llama.vocab_size"])
    # defaults: no architecture and no model keys; a version-2 file
    p2 = tmp_path / "bare.gguf"
    gf.write(p2, [("x", gf.U32, 1)], [gf.Tensor("w", [32], 2)], version=2)
    assert _same_as_reference(L, r, p2)
    # names longer than 255 bytes, a NUL inside a name, type numbers past the tables
    long = "n" * 300
    p3 = tmp_path / "names.gguf"
    gf.write(p3, [("general.architecture", gf.STR, "qwen2"), ("qwen2.embedding_length", gf.U32, 896),
                  ("qwen2.attention.head_count", gf.U32, 14)],
             [gf.Tensor(long, [32], 2), gf.Tensor("a\x00b", [32], 8), gf.Tensor("big", [64], 31),
              gf.Tensor("t", [7, 9], 0)])
    assert _same_as_reference(L, r, p3)
    # no tensors, no keys
    p4 = tmp_path / "empty.gguf"
    gf.write(p4, [], [])
    assert _same_as_reference(L, r, p4)


def _malformed(tmp_path):
    """(name, bytes) of files both parsers must reject."""
    good, _ = gf.build([("a", gf.U32, 1), ("s", gf.STR, "xy")], [gf.Tensor("w", [32, 2], 2)])
    out = [("magic", b"GGUG" + good[4:]), ("v1", good[:4] + struct.pack("<I", 1) + good[8:]),
           ("v4", good[:4] + struct.pack("<I", 4) + good[8:])]
    for vt, payload in ((13, b""), (gf.ARR, struct.pack("<IQ", gf.ARR, 1)), (gf.ARR, struct.pack("<IQ", 13, 1)),
                        (gf.ARR, struct.pack("<IQ", gf.U8, 10_000_001)), (gf.STR, struct.pack("<Q", 1024 * 1024 + 1))):
        entry = gf.gstr("bad") + struct.pack("<I", vt) + payload
        blob, _ = gf.build([entry], [])
        out.append((f"value{vt}-{len(payload)}", blob))
    blob, _ = gf.build([], [gf.Tensor("w", [1, 1, 1, 1, 1], 0)])
    out.append(("dims5", blob))
    blob, _ = gf.build([("a", gf.U32, 1)], [], n_kv=3)
    out.append(("count", blob))
    return out, good


@pytest.mark.skipif(not HAS_REF, reason="oracle/_ref not built (needs /root/reference)")
def test_rejects_what_the_reference_rejects(L, tmp_path):
    r = _ref()
    bad, good = _malformed(tmp_path)
    for name, blob in bad:
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(blob)
        assert not L.holo_gguf_open(str(p).encode()), name
        assert not r.gguf_open(str(p).encode()), name
    # a file cut at every byte of its header and tensor table: accepted by
    # both exactly when the cut falls after the tensor table
    p = tmp_path / "cut.gguf"
    _, data_offset = gf.build([("a", gf.U32, 1), ("s", gf.STR, "xy")], [gf.Tensor("w", [32, 2], 2)])
    for n in range(0, data_offset + 8):
        p.write_bytes(good[:n])
        a, b = L.holo_gguf_open(str(p).encode()), r.gguf_open(str(p).encode())
        assert bool(a) == bool(b), n
        if a:
            L.holo_gguf_close(a)
            r.gguf_close(b)


def test_rejects_malformed_files(L, tmp_path):
    bad, good = _malformed(tmp_path)
    for name, blob in bad:
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(blob)
        assert not L.holo_gguf_open(str(p).encode()), name
    assert not L.holo_gguf_open(str(tmp_path / "absent.gguf").encode())


def test_inputs_that_divide_by_zero_in_the_reference(L, tmp_path):
    """Types without a block size get size 0; head_count 0 gives key_length 0."""
    p = tmp_path / "iq.gguf"
    gf.write(p, [("general.architecture", gf.STR, "llama"), ("llama.attention.head_count", gf.U32, 0)],
             [gf.Tensor(f"t{t}", [256], t, data=b"") for t in (4, 5, 16, 20, 23)])
    g = L.holo_gguf_open(str(p).encode())
    assert g
    try:
        assert [_tensor(L, g, i).size_bytes for i in range(5)] == [0] * 5
        m = _model(L, g)
        assert m.attention_head_count == 0 and m.attention_key_length == 0 and m.attention_head_count_kv == 0
    finally:
        L.holo_gguf_close(g)


def test_llama_check_rejects_unbuilt_branches(L, tmp_path):
    """holo_llama_gguf_check: a plain Llama file passes; the Qwen (q/k/v
    biases, QK-norm) and Gemma (architecture name, post-norms) branches of
    the reference forward (llm.c:451-521, 1037-1133), which this forward
    does not run, are rejected on the host-side parse."""
    base = [("general.architecture", gf.STR, "llama"), ("llama.block_count", gf.U32, 2)]

    def check(kvs, extra, name):
        ts = [gf.Tensor("token_embd.weight", [32, 4], 0), gf.Tensor("blk.0.attn_q.weight", [32, 32], 0)]
        ts += [gf.Tensor(n, [32], 0) for n in extra]
        path = tmp_path / name
        gf.write(path, kvs, ts)
        g = L.holo_gguf_open(str(path).encode())
        assert g
        try:
            return L.holo_llama_gguf_check(g)
        finally:
            L.holo_gguf_close(g)

    assert check(base, [], "plain.gguf") == 0
    for j, extra in enumerate(["blk.1.attn_q.bias", "blk.0.attn_k.bias", "blk.0.attn_v.bias",
                               "blk.1.attn_q_norm.weight", "blk.0.attn_k_norm.weight",
                               "blk.0.post_attention_norm.weight", "blk.1.post_ffw_norm.weight"]):
        assert check(base, [extra], f"extra{j}.gguf") == -1, extra
    gemma = [("general.architecture", gf.STR, "gemma3"), ("gemma3.block_count", gf.U32, 2)]
    assert check(gemma, [], "gemma.gguf") == -1
    assert L.holo_llama_gguf_check(None) == -1
