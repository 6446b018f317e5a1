"""CPU-side checks of the C ABI: the library loads, exports every function
include/kvhp_c.h declares, and rejects bad arguments on the host before any
GPU work (no compute calls here)."""
import ctypes
import re

import pytest

import kvhp


def _declared_functions():
    text = open(kvhp.HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvhp_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_binding_surface():
    declared = _declared_functions()
    assert declared == sorted(kvhp.exported_symbols())


def test_library_exports_every_declared_symbol():
    lib = kvhp.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.kvhp_abi_version() == 1


def test_kv_view_struct_layout_matches_header():
    # 1 pointer + 4 int64 strides + pointer + 4 int32 = 64 bytes
    assert ctypes.sizeof(kvhp.KVView) == 64


def test_auto_split_policy():
    # chunks of ~L/64 tokens but >= 64 (64-token multiples), grid of at most
    # 6144 workgroups, never more than 256 splits; batches below 8 with at
    # most 512 keys: one split (no merge launch)
    assert kvhp.decode_auto_splits(1, 8, 128, 64) == 1
    expect = {(1, 8, 4096): 64, (1, 8, 16384): 64, (1, 8, 65536): 64, (1, 4, 2176): 34,
              (1, 8, 512): 1, (7, 8, 512): 1, (8, 8, 512): 8, (1, 8, 513): 9, (32, 8, 8193): 22}
    for (b, hkv, L), want in expect.items():
        assert kvhp.decode_auto_splits(b, hkv, 128, L) == want, (b, hkv, L)
    for b, hkv, L in [(1, 8, 100), (3, 2, 600), (64, 8, 32768), (1, 1, 1 << 20), (256, 32, 4096)]:
        s = kvhp.decode_auto_splits(b, hkv, 128, L)
        assert 1 <= s <= 256
        assert s == 1 or b * hkv * s <= 6144
        chunk = -(-L // s) + 63 & ~63    # tokens per split, 64-token multiples
        assert s == -(-L // chunk) and (s == 1 or chunk >= 64)


def test_workspace_sizing():
    # no workspace when a single split covers the sequence
    assert kvhp.decode_workspace_bytes(1, 32, 8, 128, 64, 1) == 0
    # splits * B * Hq * (D + 2) floats, never more than the split_buffer the
    # reference's callers allocate for that split count (test_attention.cpp:124,
    # forward_gpu.cu:100); a request is rounded to 64-token chunks, so 8
    # splits of 600 tokens become 5 chunks of 128
    for b, hq, hkv, d, L, s, used in [(2, 32, 8, 128, 4096, 16, 16), (3, 14, 2, 64, 600, 8, 5),
                                      (1, 32, 4, 64, 2176, 0, None)]:
        n = kvhp.decode_workspace_bytes(b, hq, hkv, d, L, s)
        used = used or kvhp.decode_auto_splits(b, hkv, d, L)
        assert n == used * b * hq * (d + 2) * 4


def test_rows_ksplit_workspace_sizing():
    # the residual projection splits over K only when the batch's x passes
    # 160 KB (B*K > 81920) and N % 16 == 0: the down projection (K = 5632,
    # 16 slices of 352) from 15 rows; fp32 partials slices * B * N
    size = kvhp.gemv_rows_workspace_bytes
    assert size(2048, 5632, 14) == 0
    assert size(2048, 5632, 15) == 16 * 15 * 2048 * 4
    assert size(2048, 5632, 32) == 16 * 32 * 2048 * 4
    assert size(4096, 2816, 32) == 8 * 32 * 4096 * 4     # 8 slices of 352
    assert size(2048, 2048, 32) == 0                      # x of 128 KB: one launch
    assert size(2040, 5632, 32) == 0                      # N not a multiple of 16
    assert size(2048, 5632, 33) == 0 and size(2048, 1000, 32) == 0   # unsupported shapes


def _null_view():
    return kvhp.KVView()


def test_host_validation_errors():
    lib = kvhp.load()
    v = kvhp.KVView()
    v.data = 0x1000
    v.stride_d = 1
    # group size not integral
    rc = lib.kvhp_decode_attention(ctypes.c_void_p(0x1000), ctypes.byref(v), ctypes.byref(v),
                                   ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1000), 1, 6, 4, 64,
                                   128, 0, None, 0, None)
    assert rc == kvhp.KVHP_ERR_INVALID and "multiple" in kvhp.last_error()
    # head_dim beyond 256
    rc = lib.kvhp_decode_attention(ctypes.c_void_p(0x1000), ctypes.byref(v), ctypes.byref(v),
                                   ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1000), 1, 8, 4, 512,
                                   128, 0, None, 0, None)
    assert rc == kvhp.KVHP_ERR_UNSUPPORTED
    # null view data
    nv = _null_view()
    rc = lib.kvhp_decode_attention(ctypes.c_void_p(0x1000), ctypes.byref(nv), ctypes.byref(v),
                                   ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1000), 1, 8, 4, 64,
                                   128, 0, None, 0, None)
    assert rc == kvhp.KVHP_ERR_INVALID
    # mixed paged / strided views
    pv = kvhp.KVView()
    pv.data = 0x1000
    pv.stride_d = 1
    pv.block_table = 0x2000
    pv.max_pages, pv.page_size, pv.num_pages = 4, 16, 4
    rc = lib.kvhp_decode_attention(ctypes.c_void_p(0x1000), ctypes.byref(pv), ctypes.byref(v),
                                   ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1000), 1, 8, 4, 64,
                                   128, 0, None, 0, None)
    assert rc == kvhp.KVHP_ERR_INVALID and "paged" in kvhp.last_error()
    # caller workspace too small for 16 splits (a view the fast path takes)
    v.stride_s, v.stride_h, v.stride_b = 64, 64 * 4096, 4 * 64 * 4096
    rc = lib.kvhp_decode_attention(ctypes.c_void_p(0x1000), ctypes.byref(v), ctypes.byref(v),
                                   ctypes.c_void_p(0x1000), ctypes.c_void_p(0x1000), 1, 8, 4, 64,
                                   4096, 16, ctypes.c_void_p(0x3000), 64, None)
    assert rc == kvhp.KVHP_ERR_WORKSPACE
    # append / prefill argument checks
    rc = lib.kvhp_append_kv(None, None, None, None, 4, 0, 2, 16, 64, None)
    assert rc == kvhp.KVHP_ERR_INVALID
    assert lib.kvhp_append_kv(None, None, None, None, 0, 0, 2, 16, 64, None) == kvhp.KVHP_OK
    rc = lib.kvhp_paged_append_kv(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                  ctypes.c_void_p(16), ctypes.c_void_p(16), 0,
                                  ctypes.c_void_p(16), 1, 1, 2, 64, 4, None)
    assert rc == kvhp.KVHP_ERR_INVALID
    rc = lib.kvhp_flash_prefill(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                ctypes.c_void_p(16), 8, 7, 2, 64, 1, None)
    assert rc == kvhp.KVHP_ERR_INVALID
    rc = lib.kvhp_flash_prefill_paged(ctypes.c_void_p(16), ctypes.c_void_p(16),
                                      ctypes.c_void_p(16), ctypes.c_void_p(16), 8, 8, 2, 64, 1,
                                      None, None, None, 1, 1, None)
    assert rc == kvhp.KVHP_ERR_INVALID
    # zero-length work is a no-op, as in the reference
    assert lib.kvhp_decode_gqa(None, None, None, None, 0, 8, 2, 16, 64, None) == kvhp.KVHP_OK
    assert lib.kvhp_causal_gqa(None, None, None, None, 0, 8, 2, 64, None) == kvhp.KVHP_OK


def test_error_raises_in_binding():
    with pytest.raises(kvhp.KVHPError):
        kvhp._check(kvhp.load().kvhp_append_kv(None, None, None, None, 4, 0, 2, 16, 64, None))


def test_header_is_plain_c(tmp_path):
    """include/kvhp_c.h compiles as strict C11 (no C++ in the ABI) and a C
    program links against libkvhp.so."""
    import os
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no gcc")
    src = tmp_path / "use_abi.c"
    src.write_text('#include "kvhp_c.h"\n'
                   'int main(void) { return kvhp_abi_version() == KVHP_ABI_VERSION ? 0 : 1; }\n')
    inc = os.path.dirname(kvhp.HEADER_PATH)
    libdir = os.path.dirname(kvhp.LIB_PATH)
    subprocess.run([gcc, "-std=c11", "-Wall", "-Wextra", "-pedantic", "-Werror", "-I", inc,
                    str(src), "-L", libdir, "-lkvhp", "-L/opt/rocm/lib", "-lamdhip64",
                    "-Wl,-rpath," + libdir, "-Wl,--allow-shlib-undefined",
                    "-o", str(tmp_path / "use_abi")], check=True)

