"""File -> HBM loading (h3_gpu_tensor_load_bf16/_f32, read_file_bf16,
stream_file_bf16; reference h3_gpu_cuda.cu:426-775), following the
reference's own test (tests/test_cuda_core.c:1278-1347): a 40 MiB bf16
payload behind a 4 KiB header read back bit-exact, the same tensor re-filled
in place, a small load, and a read past the end of the file that must fail.
Added here: unaligned offsets and chunk-straddling sizes, F32, buffered and
O_DIRECT reads, a safetensors file written by the safetensors library, and a
re-fill from an I/O thread while the compute stream runs."""
import os
import shutil
import tempfile
import threading

import numpy as np
import pytest

import h3hip

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(params=["tmp", "repo"])
def folder(request, tmp_path):
    """Two file systems: /tmp (often tmpfs, which refuses O_DIRECT, so the
    buffered path runs) and the repository's own disk."""
    if request.param == "tmp":
        yield tmp_path
    else:
        d = tempfile.mkdtemp(prefix=".load_test_", dir=ROOT)
        yield d
        shutil.rmtree(d, ignore_errors=True)


def write_file(path, header, payload):
    with open(path, "wb") as f:
        f.write(header)
        f.write(payload.tobytes())


def test_reference_file_load_sequence(gpu, folder):
    n = 20 << 20                      # 40 MiB of bf16
    rng = np.random.default_rng(1)
    host = h3hip.f32_to_bf16(rng.uniform(-4, 4, n).astype(np.float32))
    path = os.path.join(folder, "payload.bin")
    write_file(path, b"\xa5" * 4096, host)
    big = gpu.load(path, 4096, n)
    assert np.array_equal(gpu.read_bf16(big), host)
    # re-fill in place after clobbering
    gpu.run("h3_gpu_fill_normal_bf16", big, 0, n, 7, 0.0, 1.0)
    assert not np.array_equal(gpu.read_bf16(big), host)
    gpu.read_file(big, path, 4096, n)
    assert np.array_equal(gpu.read_bf16(big), host)
    gpu.run("h3_gpu_fill_normal_bf16", big, 0, n, 8, 0.0, 1.0)
    gpu.read_file(big, path, 4096, n, stream=True)
    assert np.array_equal(gpu.read_bf16(big), host)
    gpu.free(big)
    small = gpu.load(path, 4096, 1024)
    assert np.array_equal(gpu.read_bf16(small), host[:1024])
    gpu.free(small)
    with pytest.raises(RuntimeError, match="end of file"):
        gpu.load(path, 4096, n + 4096)


@pytest.mark.parametrize("offset,n", [
    (1, 5), (4095, 4097), (12346, (16 << 20) // 2 + 3),
    (8 + 6, (48 << 20) // 2 + 1), (4096 * 3, (16 << 20) // 2)])
@pytest.mark.parametrize("buffered", [False, True])
def test_unaligned_ranges_bf16(gpu, folder, offset, n, buffered, monkeypatch):
    """Offsets off the 4 KiB grid and sizes one past or exactly at the 16 MiB
    staging chunk, read back bit-exact; neighbouring bytes are not taken."""
    if buffered:
        monkeypatch.setenv("H3_HIP_DIRECT_IO", "0")
    rng = np.random.default_rng(offset + n)
    total = offset + 2 * n + 4099
    data = rng.integers(0, 256, total, dtype=np.uint8)
    path = os.path.join(folder, "ragged.bin")
    data.tofile(path)
    t = gpu.load(path, offset, n)
    want = data[offset:offset + 2 * n].view(np.uint16)
    assert np.array_equal(gpu.read_bf16(t), want)
    gpu.free(t)


def test_f32_load(gpu, folder):
    rng = np.random.default_rng(3)
    vals = rng.standard_normal((18 << 20) // 4 + 7).astype(np.float32)
    path = os.path.join(folder, "f32.bin")
    write_file(path, b"hdr", vals)
    t = gpu.load(path, 3, vals.size, dtype="f32")
    assert np.array_equal(gpu.read_f32(t), vals)
    gpu.free(t)


def test_safetensors_file(gpu, folder):
    """A file written by the safetensors library, located through its JSON
    header the way the model layer does, each tensor loaded bit-exact."""
    torch = pytest.importorskip("torch")
    st = pytest.importorskip("safetensors.torch")
    g = torch.Generator().manual_seed(4)
    tensors = {
        "blocks.0.attn.qkv.weight":
            torch.randn(3 * 256, 256, generator=g).to(torch.bfloat16),
        "blocks.0.norm1.weight": torch.randn(256, generator=g).to(
            torch.bfloat16),
        "time.linear_1.bias": torch.randn(333, generator=g),
        "final.weight": torch.randn(96, 2048, generator=g).to(torch.bfloat16),
    }
    path = os.path.join(folder, "model.safetensors")
    st.save_file(tensors, path, metadata={"format": "pt"})
    index = h3hip.safetensors_index(path)
    assert set(index) == set(tensors)
    for name, ref in tensors.items():
        dtype, shape, offset, nbytes = index[name]
        assert shape == tuple(ref.shape)
        if dtype == "BF16":
            t = gpu.load(path, offset, nbytes // 2)
            got = gpu.read_bf16(t)
            want = ref.view(torch.int16).numpy().view(np.uint16).ravel()
        else:
            assert dtype == "F32"
            t = gpu.load(path, offset, nbytes // 4, dtype="f32")
            got = gpu.read_f32(t)
            want = ref.numpy().ravel()
        assert np.array_equal(got, want), name
        gpu.free(t)


def test_read_file_rejects_bad_requests(gpu, folder):
    path = os.path.join(folder, "x.bin")
    np.zeros(64, np.uint16).tofile(path)
    t = gpu.new_bf16(32)
    with pytest.raises(RuntimeError, match="invalid BF16 file read"):
        gpu.read_file(t, path, 0, 31)     # the reference wants the full size
    with pytest.raises(RuntimeError, match="cannot open"):
        gpu.read_file(t, os.path.join(folder, "missing.bin"), 0, 32)
    with pytest.raises(RuntimeError, match="end of file"):
        gpu.read_file(t, path, 100, 32)
    f = gpu.new_f32(32)
    with pytest.raises(RuntimeError, match="invalid BF16 file read"):
        gpu.read_file(f, path, 0, 32)
    gpu.free(t)
    gpu.free(f)


def test_read_file_from_io_thread_while_computing(gpu, folder):
    """h3_gpu.h:67-69: read_file may run on an I/O thread while another
    tensor is in flight.  The main thread keeps running GEMMs whose result is
    checked against the same GEMM run alone."""
    n = 12 << 20
    rng = np.random.default_rng(5)
    host = rng.integers(0, 1 << 16, n, dtype=np.uint16)
    path = os.path.join(folder, "io.bin")
    host.tofile(path)
    dst = gpu.new_bf16(n)
    m = k = 1024
    a = gpu.bf16(rng.standard_normal(m * k).astype(np.float32) * 0.1)
    w = gpu.bf16(rng.standard_normal(k * k).astype(np.float32) * 0.1)
    y = gpu.new_bf16(m * k)
    gpu.run("h3_gpu_linear_bf16", y, a, w, None, m, k, k)
    want = gpu.read_bf16(y)
    errors = []

    def io():
        try:
            for _ in range(3):
                gpu.read_file(dst, path, 0, n)
        except Exception as e:            # reported on the main thread
            errors.append(e)

    th = threading.Thread(target=io)
    th.start()
    for _ in range(20):
        gpu.run("h3_gpu_linear_bf16", y, a, w, None, m, k, k)
    th.join()
    assert not errors, errors
    assert np.array_equal(gpu.read_bf16(y), want)
    assert np.array_equal(gpu.read_bf16(dst), host)
    for t in (dst, a, w, y):
        gpu.free(t)
