"""GPU: holo_gguf_upload puts a GGUF file's tensor data in one HBM arena.

Every tensor's device bytes must equal the file's bytes, and the GEMVs run
on the uploaded weights in place (device pointer = arena base + offset) must
agree with the CPU oracle on the same bytes.  One file is larger than the
64 MiB staging chunk, so the double-buffered copy loop runs several rounds.
"""
import ctypes as C

import numpy as np
import pytest

import gguf_files as gf
from oracle.oracle import max_rel_err, normwise_err

pytestmark = pytest.mark.gpu


def _tensor(holo, g, i):
    return holo.GgufTensor.from_address(holo.lib().holo_gguf_tensor(g, i))


def _download(holo, ptr, n):
    out = np.empty(n, dtype=np.uint8)
    if n:
        holo.lib().cuda_memcpy_d2h(out.ctypes.data, ptr, n)
    return out


@pytest.mark.parametrize("big", [False, True], ids=["small", "multi-chunk"])
def test_upload_places_every_tensor(holo, synth, oracle, tmp_path, big):
    print(f"case gguf upload big={big}", flush=True)
    lib = holo.lib()
    mats = [("wq", 2, 256, 512), ("wk", 8, 128, 512), ("ffn", 12, 96, 1024), ("norm", 0, 1, 512)]
    if big:
        mats.append(("big", 2, 11008, 4096 * 2))  # 50.7 MB of Q4_0 ... plus the rest: beyond one 64 MiB chunk
        mats.append(("big2", 8, 4096, 4096))      # 17.8 MB of Q8_0
    tensors, host = [], {}
    for j, (name, t, rows, cols) in enumerate(mats):
        if t == 0:
            data = synth.normal(rows * cols, seed=j).tobytes()
        else:
            data = synth.blocks(t, rows, cols, seed=10 + j).tobytes()
        host[name] = (t, rows, cols, data)
        tensors.append(gf.Tensor(name, [cols, rows], t, data))
    path = tmp_path / "model.gguf"
    gf.write(path, [("general.architecture", gf.STR, "llama")], tensors)
    g = lib.holo_gguf_open(str(path).encode())
    assert g
    try:
        assert lib.holo_gguf_upload(g) == 0
        holo.check("upload")
        base = lib.holo_gguf_device_base(g)
        assert base and base % 256 == 0
        assert lib.holo_gguf_upload(g) == 0 and lib.holo_gguf_device_base(g) == base  # second call: same arena
        end = max(t.offset + len(t.data) for t in tensors)
        assert lib.holo_gguf_device_bytes(g) == end
        for i, t in enumerate(tensors):
            info = _tensor(holo, g, i)
            dp = lib.holo_gguf_device_ptr(g, C.addressof(info))
            assert dp == base + t.offset and dp % 32 == 0
            assert np.array_equal(_download(holo, dp, len(t.data)), np.frombuffer(t.data, np.uint8)), t.name
        # GEMVs straight from the arena
        fn = {2: lib.cuda_matmul_q4_0, 8: lib.cuda_matmul_q8_0, 12: lib.cuda_matmul_q4_k}
        for i, t in enumerate(tensors):
            qt, rows, cols, data = host[t.name]
            if qt == 0:
                continue
            x = synth.normal(cols, seed=99)
            dx = holo.DeviceBuffer.from_array(x)
            dy = holo.DeviceBuffer(4 * rows)
            info = _tensor(holo, g, i)
            fn[qt](dy.ptr, lib.holo_gguf_device_ptr(g, C.addressof(info)), dx.ptr, rows, cols)
            lib.cuda_sync()
            holo.check(t.name)
            want = oracle.matmul(qt, np.frombuffer(data, np.uint8), x, rows, cols)
            got = dy.download(np.float32, rows)
            assert normwise_err(got, want) <= 1e-3 and max_rel_err(got, want) <= 1e-3, t.name
    finally:
        lib.holo_gguf_close(g)
    holo.check("close")


def test_upload_rejects_a_truncated_file(holo, synth, tmp_path):
    print("case gguf truncated", flush=True)
    lib = holo.lib()
    data = synth.blocks(2, 64, 256, seed=1).tobytes()
    blob, off = gf.build([], [gf.Tensor("w", [256, 64], 2, data)])
    path = tmp_path / "cut.gguf"
    path.write_bytes(blob[:off + len(data) // 2])
    g = lib.holo_gguf_open(str(path).encode())
    assert g  # the header and tensor table are complete
    try:
        assert lib.holo_gguf_upload(g) == -1
        assert not lib.holo_gguf_device_base(g)
    finally:
        lib.holo_gguf_close(g)
    holo.check("truncated")
