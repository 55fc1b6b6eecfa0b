"""The four GPU workloads at their full sizes, through the public API.

Each config's generator is in workloads.py (seeded, synthetic).  Results are
checked against the input bytes and CPU zlib, which is what the oracle is
pinned to for whole streams:
  * 64 MiB float32 strain, zlib level 6: decode bit-exact;
  * 256 MiB text-like, 32 KiB chunks (with history, and independent chunks
    as the config states it): encode round-trips through CPU zlib, within 2 %
    of zlib level 1, and through the GPU decoder;
  * 4096 small mixed files: batch encode, then batch decode of the padded
    slots with the encoder's metadata, every row [len, 0] then [0, 0];
  * 1 GiB mixed stress stream (stored, fixed, run-length and level-9 dynamic
    segments in one zlib stream): decode bit-exact.
"""

import hashlib
import zlib

import numpy as np
import pytest

import workloads

pytestmark = pytest.mark.gpu

# SHA-256 of the generated inputs, so that every run measures the same bytes.
SHA = {
    "c1": "33aaa8b865bd2da79f29d28a737ac49d1bac6cc119835be2850bd8f421126ac9",
    "c2": "adfceb7156b4c9df2a48f59b975bfe5bb7d70db63d0daa942f89ec3f697643c6",
    "c3": "4b3314fda8593b37021a13fc65f8bc980c882dce5e8021247137d4638b32ae03",
    "c3_sizes": "938a0a5a487f764ae9d3770cf4c8267ccbb7be9b339ecb9394ffdca223130035",
    "c4": "652e5fe716a92214ec4b76269bbabaa2832676870912c4e1a24ba9392fde5996",
    "c4_payload": "a98c70aedc518de7edc197841672c5ebd897fe49494d863e44f99326ff77e911",
}


def _sha(data):
    return hashlib.sha256(data).hexdigest()


def _device_bytes(data, device):
    import torch
    return torch.from_numpy(np.frombuffer(data, dtype=np.uint8).copy()).to(device)


def test_strain_64mib_decode(gpu):
    import torch
    import cuda_zlib
    raw = workloads.c1()
    assert _sha(raw) == SHA["c1"]
    payload = zlib.compress(raw, 6)
    out, meta = cuda_zlib.decompress_zlib_checked(payload, len(raw), gpu)
    torch.cuda.synchronize()
    assert int(meta.cpu()[0]) == 0
    assert torch.equal(out, _device_bytes(raw, out.device))


def test_text_256mib_encode(gpu):
    import torch
    import cuda_zlib
    raw = workloads.c2()
    assert _sha(raw) == SHA["c2"]
    enc, meta = cuda_zlib.compress_zlib_padded(raw, gpu, chunk_bytes=32768)
    length, status = (int(v) for v in meta.cpu().numpy())
    assert status == 0
    stream = enc[:length].cpu().numpy().tobytes()
    assert not enc[length:].any()
    assert zlib.decompress(stream) == raw
    assert length <= 1.02 * len(zlib.compress(raw, 1))
    out, dmeta = cuda_zlib.decompress_zlib_checked(stream, len(raw), gpu)
    torch.cuda.synchronize()
    assert int(dmeta.cpu()[0]) == 0
    assert torch.equal(out, _device_bytes(raw, out.device))


def test_text_256mib_encode_independent_chunks(gpu):
    """The config's own mode: every 32 KiB chunk with no history before it."""
    import torch
    import cuda_zlib
    raw = workloads.c2()
    enc, meta = cuda_zlib.compress_zlib_padded(raw, gpu, chunk_bytes=32768,
                                               independent_chunks=True)
    length, status = (int(v) for v in meta.cpu().numpy())
    assert status == 0
    stream = enc[:length].cpu().numpy().tobytes()
    assert not enc[length:].any()
    assert zlib.decompress(stream) == raw
    l1 = len(zlib.compress(raw, 1))
    print("independent chunks: ratio %.4f, zlib L1 %.4f" % (length / len(raw), l1 / len(raw)))
    assert length <= 1.02 * l1
    out, dmeta = cuda_zlib.decompress_zlib_checked(stream, len(raw), gpu)
    torch.cuda.synchronize()
    assert int(dmeta.cpu()[0]) == 0
    assert torch.equal(out, _device_bytes(raw, out.device))


def test_batch_4096_mixed_files(gpu):
    import cuda_zlib
    files = workloads.c3()
    sizes = [len(f) for f in files]
    assert len(files) == 4096 and sizes.count(0) >= 64
    packed = b"".join(files)
    assert _sha(packed) == SHA["c3"]
    assert _sha(",".join(str(n) for n in sizes).encode()) == SHA["c3_sizes"]
    enc, meta = cuda_zlib.compress_zlib_batch_padded(packed, sizes, gpu)
    m = meta.cpu().numpy()
    assert (m[:, 1] == 0).all()
    capacities = [n + 5 * max(1, -(-n // 32768)) + 6 for n in sizes]
    # Every file's slot holds an independent zlib stream.
    host = enc.cpu().numpy().tobytes()
    at = 0
    for i in range(0, len(files), 97):
        at = sum(capacities[:i])
        assert zlib.decompress(host[at:at + int(m[i, 0])]) == files[i]
    out, dmeta = cuda_zlib.decompress_zlib_batch_checked(enc, capacities, sizes, gpu,
                                                         encoded_metadata=meta)
    assert (dmeta.cpu().numpy() == 0).all()
    assert out.cpu().numpy().tobytes() == packed


def test_stress_1gib_mixed_stream_decode(gpu):
    import torch
    import cuda_zlib
    payload, raw = workloads.c4()
    assert len(raw) == 1 << 30
    assert _sha(raw) == SHA["c4"] and _sha(payload) == SHA["c4_payload"]
    out, meta = cuda_zlib.decompress_zlib_checked(payload, len(raw), gpu)
    torch.cuda.synchronize()
    assert int(meta.cpu()[0]) == 0
    assert torch.equal(out, _device_bytes(raw, out.device))
