"""The read-bandwidth calibration probes (the reference's read-bandwidth probe,
src/cuda/read_bandwidth.cu:8-118): argument checks on the host (CPU) and one
real call of each on the GPU.  They write nothing but a 4-byte sink, and only
when their data fold equals a fixed constant; out-of-range page ids are
clamped into the pool."""
import ctypes

import pytest

import kvhp


def test_probe_argument_checks():
    lib = kvhp.load()
    sink = ctypes.c_void_p(0x1000)
    assert lib.kvhp_stream_read(None, 1 << 20, sink, None) == kvhp.KVHP_ERR_INVALID
    assert lib.kvhp_stream_read(ctypes.c_void_p(0x1008), 1 << 20, sink, None) == kvhp.KVHP_ERR_INVALID
    assert lib.kvhp_stream_read(None, 8, sink, None) == kvhp.KVHP_OK   # under one chunk: nothing to read
    ids = ctypes.c_void_p(0x2000)
    assert lib.kvhp_page_read(ctypes.c_void_p(0x1000), 1 << 20, None, 4, 4096, sink,
                              None) == kvhp.KVHP_ERR_INVALID
    rc = lib.kvhp_page_read(ctypes.c_void_p(0x1000), 1 << 20, ids, 4, 1000, sink, None)
    assert rc == kvhp.KVHP_ERR_UNSUPPORTED and "page_bytes" in kvhp.last_error()
    rc = lib.kvhp_page_read(ctypes.c_void_p(0x1000), 1024, ids, 4, 4096, sink, None)
    assert rc == kvhp.KVHP_ERR_INVALID and "smaller than a page" in kvhp.last_error()
    assert lib.kvhp_page_read(ctypes.c_void_p(0x1000), 1 << 20, ids, 0, 4096, sink, None) == kvhp.KVHP_OK


@pytest.mark.gpu
@pytest.mark.parametrize("page_bytes", [2048, 4096, 8192, 16384, 32768])
def test_probes_run(page_bytes):
    import torch
    buf = torch.ones((8 << 20) // 4, dtype=torch.float32, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    kvhp.stream_read(buf, sink)
    npool = buf.numel() * 4 // page_bytes
    # in-range ids, repeats, and ids past either end of the pool (clamped)
    ids = torch.tensor(list(range(0, npool, 3)) + [npool - 1, npool + 5, -7, 0, 0],
                       dtype=torch.int32, device="cuda")
    kvhp.page_read(buf, ids, page_bytes, sink)
    torch.cuda.synchronize()
    assert int(sink[0]) in (0, 0x9E3779B9 - (1 << 32))
    assert torch.all(buf == 1.0)
