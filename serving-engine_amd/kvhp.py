"""ctypes binding of libkvhp.so, the gfx950 KV-cache hot-path library.

The C ABI is declared in include/kvhp_c.h; this module mirrors it one to one
for Python callers (tests, bench, smoke).  Device memory and streams come from
torch: every tensor argument is a torch tensor on the GPU, every `stream` is a
torch.cuda.Stream (default: the current stream).  Errors raise KVHPError with
the library's kvhp_last_error() message, the Python counterpart of the
std::runtime_error the reference's CUDA_CHECK throws
(src/common/cuda_utils.h:12-21).

There is no CPU fallback: if the library is missing, load() raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libkvhp.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "kvhp_c.h")

PAGE_SIZE = 16
KVHP_OK = 0
KVHP_ERR_INVALID = -1
KVHP_ERR_UNSUPPORTED = -2
KVHP_ERR_WORKSPACE = -3
KVHP_ERR_HIP = -4


class KVHPError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"kvhp error {code}: {msg}")
        self.code = code


class KVView(ctypes.Structure):
    """kvhp_kv_view: strided (block_table == NULL) or paged view of K or V."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("stride_b", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
        ("stride_s", ctypes.c_int64),
        ("stride_d", ctypes.c_int64),
        ("block_table", ctypes.c_void_p),
        ("max_pages", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t
_f32 = ctypes.c_float
_u64 = ctypes.c_uint64

# name -> (restype, argtypes)
_SIGNATURES = {
    "kvhp_last_error": (ctypes.c_char_p, []),
    "kvhp_abi_version": (_i32, []),
    "kvhp_append_kv": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp]),
    "kvhp_paged_append_kv": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32,
                                    _i32, _i32, _vp]),
    "kvhp_paged_gather_kv": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _i32, _i32,
                                    _vp, _vp, _vp]),
    "kvhp_decode_auto_splits": (_i32, [_i32, _i32, _i32, _i32]),
    "kvhp_decode_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "kvhp_decode_workspace_init": (_i32, [_vp, _sz, _vp]),
    "kvhp_decode_attention": (_i32, [_vp, ctypes.POINTER(KVView), ctypes.POINTER(KVView), _vp,
                                     _vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _sz, _vp]),
    "kvhp_build_id": (ctypes.c_char_p, []),
    "kvhp_stream_read": (_i32, [_vp, _sz, _vp, _vp]),
    "kvhp_page_read": (_i32, [_vp, _i64, _vp, _i64, _i32, _vp, _vp]),
    "kvhp_decode_attention_noalloc": (_i32, [_vp, ctypes.POINTER(KVView), ctypes.POINTER(KVView),
                                             _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "kvhp_paged_append_decode": (_i32, [_vp, _vp, _vp, ctypes.POINTER(KVView),
                                        ctypes.POINTER(KVView), _vp, _vp, _vp, _i32, _i32, _i32,
                                        _i32, _i32, _i32, _vp, _sz, _vp]),
    "kvhp_append_decode": (_i32, [_vp, _vp, _vp, ctypes.POINTER(KVView), ctypes.POINTER(KVView),
                                  _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _sz,
                                  _vp]),
    "kvhp_decode_gqa": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp]),
    "kvhp_flash_prefill": (_i32, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _vp]),
    "kvhp_flash_prefill_paged": (_i32, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _vp,
                                        _vp, _vp, _i32, _i32, _vp]),
    "kvhp_causal_gqa": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    # model operators
    "kvhp_gemv": (_i32, [_vp, _vp, _vp, _i32, _i32, _vp]),
    "kvhp_gemv_residual": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _vp]),
    "kvhp_rmsnorm_gemv": (_i32, [_vp, _vp, _vp, _f32, _vp, _vp, _i32, _i32, _vp]),
    "kvhp_rmsnorm_gemv_swiglu": (_i32, [_vp, _vp, _vp, _f32, _vp, _i32, _i32, _vp]),
    "kvhp_rmsnorm_qkv_rope_append": (_i32, [_vp, _vp, _vp, _f32, _vp, _f32, _vp, _vp, _vp, _vp,
                                            _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "kvhp_gemv_residual_rows": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "kvhp_gemv_rows_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "kvhp_gemv_residual_rows_ws": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _sz, _vp]),
    "kvhp_rmsnorm_gemv_rows": (_i32, [_vp, _vp, _vp, _f32, _vp, _vp, _i32, _i32, _i32, _vp]),
    "kvhp_rmsnorm_gemv_swiglu_rows": (_i32, [_vp, _vp, _vp, _f32, _vp, _i32, _i32, _i32, _vp]),
    "kvhp_rmsnorm_qkv_rope_append_rows": (_i32, [_vp, _vp, _vp, _f32, _vp, _f32, _vp, _vp, _vp,
                                                 _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                                 _vp]),
    "kvhp_rows_tiled_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "kvhp_rows_tile_weights": (_i32, [_i32, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp]),
    "kvhp_gemv_residual_rows_tiled": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _sz,
                                             _vp]),
    "kvhp_rmsnorm_gemv_rows_tiled": (_i32, [_vp, _vp, _vp, _f32, _vp, _vp, _i32, _i32, _i32,
                                            _vp]),
    "kvhp_rmsnorm_gemv_swiglu_rows_tiled": (_i32, [_vp, _vp, _vp, _f32, _vp, _i32, _i32, _i32,
                                                   _vp]),
    "kvhp_rmsnorm_qkv_rope_append_rows_tiled": (_i32, [_vp, _vp, _vp, _f32, _vp, _f32, _vp, _vp,
                                                       _vp, _vp, _i32, _i32, _i32, _i32, _i32,
                                                       _i32, _i32, _vp]),
    "kvhp_rmsnorm": (_i32, [_vp, _vp, _vp, _i64, _i64, _f32, _vp]),
    "kvhp_apply_rope": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _vp]),
    "kvhp_split_qkv_rope": (_i32, [_vp, _i64, _i32, _i32, _i32, _i64, _f32, _vp, _vp, _vp, _vp]),
    "kvhp_split_qkv_rope_rows": (_i32, [_vp, _i64, _i32, _i32, _i32, _vp, _f32, _vp, _vp, _vp,
                                        _vp]),
    "kvhp_swiglu": (_i32, [_vp, _vp, _vp, _i64, _vp]),
    "kvhp_swiglu_rows": (_i32, [_vp, _vp, _i64, _i64, _vp]),
    "kvhp_embedding": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "kvhp_argmax": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _vp]),
    "kvhp_argmax_rows": (_i32, [_vp, _i64, _i64, _vp, _vp]),
    "kvhp_randn_f16": (_i32, [_vp, _i64, _u64, _u64, _f32, _vp]),
    "kvhp_fill_f16": (_i32, [_vp, _i64, _f32, _vp]),
    # model runner
    "kvhp_llama_create": (_i32, [_vp, _u64, _i32, ctypes.POINTER(ctypes.c_void_p)]),
    "kvhp_llama_destroy": (_i32, [_vp]),
    "kvhp_llama_prefill": (_i32, [_vp, _vp, _i32, _vp, _vp]),
    "kvhp_llama_decode_step": (_i32, [_vp, ctypes.c_int32, _vp, _vp]),
    "kvhp_llama_generate": (_i32, [_vp, _i32, _i32, _vp, _vp]),
    "kvhp_llama_tensor": (_i32, [_vp, _i32, _i32, ctypes.POINTER(ctypes.c_void_p),
                                 ctypes.POINTER(ctypes.c_size_t)]),
    "kvhp_llama_prefill_paged": (_i32, [_vp, _vp, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _vp]),
    "kvhp_llama_prefill_cached": (_i32, [_vp, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _i32, _vp,
                                         _vp, _vp]),
    "kvhp_llama_decode_paged": (_i32, [_vp, _vp, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _i32,
                                       _vp, _vp, _vp]),
    "kvhp_llama_reserve": (_i32, [_vp, _i32, _i32]),
}

_lib: Optional[ctypes.CDLL] = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libkvhp.so (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    # torch's HIP runtime first, so that the library binds to the same one:
    # loaded the other way round, the process holds two HIP runtimes and the
    # library's finds no device once torch's has opened it.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols() -> list:
    return list(_SIGNATURES)


def build_id() -> str:
    """Source hash the loaded library was linked with (kvhp_build_id)."""
    return load().kvhp_build_id().decode()


def source_build_id(root: str = os.path.dirname(os.path.abspath(__file__))) -> str:
    """The same hash over the sources in this tree (Makefile ID_SRCS): the
    library matches the tree when build_id() == source_build_id()."""
    import glob
    import hashlib
    csrc = os.path.join(root, "csrc")
    files = (sorted(glob.glob(os.path.join(csrc, "*.hip"))) +
             sorted(glob.glob(os.path.join(csrc, "*.h"))) +
             [os.path.join(root, "..", "include", "kvhp_c.h")])
    h = hashlib.sha256()
    for f in files:
        with open(f, "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def stream_read(buf, sink, stream=None):
    """Streaming read of the whole tensor `buf` (kvhp_stream_read); sink: a
    device tensor of at least 4 bytes."""
    _check(load().kvhp_stream_read(_ptr(buf), buf.numel() * buf.element_size(), _ptr(sink),
                                   _stream(stream)))


def page_read(pool, page_ids, page_bytes, sink, stream=None):
    """Read the pages page_ids (int32 device tensor) of the device tensor
    `pool` cut into pages of page_bytes (kvhp_page_read); sink: a 4-byte
    device tensor."""
    _check(load().kvhp_page_read(_ptr(pool), pool.numel() * pool.element_size(), _ptr(page_ids),
                                 page_ids.numel(), page_bytes, _ptr(sink), _stream(stream)))


def last_error() -> str:
    return load().kvhp_last_error().decode()


def _check(rc: int) -> None:
    if rc != KVHP_OK:
        raise KVHPError(rc, last_error())


def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    return t.data_ptr()


def _stream(stream) -> Optional[int]:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


# ----------------------------------------------------------------- views --
def strided_view(t, stride_b: int, stride_h: int, stride_s: int, stride_d: int = 1) -> KVView:
    v = KVView()
    v.data = t.data_ptr()
    v.stride_b, v.stride_h, v.stride_s, v.stride_d = stride_b, stride_h, stride_s, stride_d
    v.block_table = None
    v.max_pages = v.page_size = v.num_pages = 0
    return v


def paged_view(pool, block_tables) -> KVView:
    """View over a pool [Hkv][P][16][D] with int32 block tables [B][max_pages]."""
    hkv, p, page, d = pool.shape
    assert page == PAGE_SIZE
    v = KVView()
    v.data = pool.data_ptr()
    v.stride_b = 0
    v.stride_h = p * page * d
    v.stride_s = d
    v.stride_d = 1
    v.block_table = block_tables.data_ptr()
    v.max_pages = block_tables.shape[1]
    v.page_size = page
    v.num_pages = p
    return v


# ------------------------------------------------------------- entry pts --
def append_kv(src_k, src_v, dst_k, dst_v, num_tokens, start_pos, num_kv_heads, max_seq,
              head_dim, stream=None):
    _check(load().kvhp_append_kv(_ptr(src_k), _ptr(src_v), _ptr(dst_k), _ptr(dst_v),
                                 num_tokens, start_pos, num_kv_heads, max_seq, head_dim,
                                 _stream(stream)))


def paged_append_kv(src_k, src_v, pool_k, pool_v, block_tables, start_pos, batch, num_tokens,
                    num_kv_heads, head_dim, stream=None):
    _check(load().kvhp_paged_append_kv(
        _ptr(src_k), _ptr(src_v), _ptr(pool_k), _ptr(pool_v), _ptr(block_tables),
        block_tables.shape[1], _ptr(start_pos), batch, num_tokens, num_kv_heads, head_dim,
        pool_k.shape[1], _stream(stream)))


def paged_gather_kv(pool_k, pool_v, block_tables, seq_lens, max_len, out_k, out_v,
                    stream=None):
    hkv, p, _, d = pool_k.shape
    _check(load().kvhp_paged_gather_kv(
        _ptr(pool_k), _ptr(pool_v), _ptr(block_tables), block_tables.shape[1], _ptr(seq_lens),
        seq_lens.shape[0], hkv, d, p, max_len, _ptr(out_k), _ptr(out_v), _stream(stream)))


def decode_auto_splits(batch, num_kv_heads, head_dim, max_seq_len) -> int:
    return load().kvhp_decode_auto_splits(batch, num_kv_heads, head_dim, max_seq_len)


def decode_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, max_seq_len,
                           num_splits=0) -> int:
    return load().kvhp_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim,
                                              max_seq_len, num_splits)


def decode_workspace_init(ws, stream=None):
    _check(load().kvhp_decode_workspace_init(_ptr(ws), ws.numel() * ws.element_size(),
                                             _stream(stream)))


def decode_attention(q, k_view: KVView, v_view: KVView, seq_lens, out, num_q_heads,
                     num_kv_heads, head_dim, max_seq_len, num_splits=0, workspace=None,
                     stream=None):
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(load().kvhp_decode_attention(
        _ptr(q), ctypes.byref(k_view), ctypes.byref(v_view), _ptr(seq_lens), _ptr(out),
        seq_lens.shape[0], num_q_heads, num_kv_heads, head_dim, max_seq_len, num_splits,
        _ptr(workspace), ws_bytes, _stream(stream)))


def decode_attention_noalloc(q, k_view: KVView, v_view: KVView, seq_lens, out, num_q_heads,
                             num_kv_heads, head_dim, max_seq_len, num_splits=0, stream=None):
    """decode_attention with the split partials in the library's static
    device scratch (no allocation; calls overlapping on one GPU race)."""
    _check(load().kvhp_decode_attention_noalloc(
        _ptr(q), ctypes.byref(k_view), ctypes.byref(v_view), _ptr(seq_lens), _ptr(out),
        seq_lens.shape[0], num_q_heads, num_kv_heads, head_dim, max_seq_len, num_splits,
        _stream(stream)))


def paged_append_decode(q, k_new, v_new, k_view: KVView, v_view: KVView, positions, seq_lens,
                        out, num_q_heads, num_kv_heads, head_dim, max_seq_len, num_splits=0,
                        workspace=None, stream=None):
    """Append row b of k_new / v_new [B][Hkv][D] at positions[b], then decode
    attention over seq_lens[b] keys (one call; paged views)."""
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(load().kvhp_paged_append_decode(
        _ptr(q), _ptr(k_new), _ptr(v_new), ctypes.byref(k_view), ctypes.byref(v_view),
        _ptr(positions), _ptr(seq_lens), _ptr(out), seq_lens.shape[0], num_q_heads,
        num_kv_heads, head_dim, max_seq_len, num_splits, _ptr(workspace), ws_bytes,
        _stream(stream)))


def append_decode(q, k_new, v_new, k_view: KVView, v_view: KVView, positions, seq_lens, out,
                  num_q_heads, num_kv_heads, head_dim, max_seq_len, num_splits=0, workspace=None,
                  stream=None):
    """paged_append_decode for views of either kind (strided views: row
    positions[b] of sequence b, dropped outside [0, max_seq_len))."""
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(load().kvhp_append_decode(
        _ptr(q), _ptr(k_new), _ptr(v_new), ctypes.byref(k_view), ctypes.byref(v_view),
        _ptr(positions), _ptr(seq_lens), _ptr(out), seq_lens.shape[0], num_q_heads,
        num_kv_heads, head_dim, max_seq_len, num_splits, _ptr(workspace), ws_bytes,
        _stream(stream)))


def decode_gqa(q, k_cache, v_cache, out, total_seq_len, num_q_heads, num_kv_heads, max_seq,
               head_dim, stream=None):
    _check(load().kvhp_decode_gqa(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out),
                                  total_seq_len, num_q_heads, num_kv_heads, max_seq, head_dim,
                                  _stream(stream)))


def flash_prefill(q, k, v, out, seq_len, num_q_heads, num_kv_heads, head_dim, batch=1,
                  stream=None):
    _check(load().kvhp_flash_prefill(_ptr(q), _ptr(k), _ptr(v), _ptr(out), seq_len,
                                     num_q_heads, num_kv_heads, head_dim, batch,
                                     _stream(stream)))


def flash_prefill_paged(q, k, v, out, seq_len, num_q_heads, num_kv_heads, head_dim, batch,
                        pool_k, pool_v, block_tables, stream=None):
    _check(load().kvhp_flash_prefill_paged(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), seq_len, num_q_heads, num_kv_heads, head_dim,
        batch, _ptr(pool_k), _ptr(pool_v), _ptr(block_tables), block_tables.shape[1],
        pool_k.shape[1], _stream(stream)))


def causal_gqa(q, k, v, out, seq_len, num_q_heads, num_kv_heads, head_dim, stream=None):
    _check(load().kvhp_causal_gqa(_ptr(q), _ptr(k), _ptr(v), _ptr(out), seq_len, num_q_heads,
                                  num_kv_heads, head_dim, _stream(stream)))


# ------------------------------------------------------ model operators --
def gemv(W, x, y, N, K, stream=None):
    _check(load().kvhp_gemv(_ptr(W), _ptr(x), _ptr(y), N, K, _stream(stream)))


def gemv_residual(W, x, r, y, N, K, stream=None):
    _check(load().kvhp_gemv_residual(_ptr(W), _ptr(x), _ptr(r), _ptr(y), N, K, _stream(stream)))


def rmsnorm_gemv(W, x, norm_w, eps, N, K, y16=None, y32=None, stream=None):
    _check(load().kvhp_rmsnorm_gemv(_ptr(W), _ptr(x), _ptr(norm_w), eps, _ptr(y16), _ptr(y32), N,
                                    K, _stream(stream)))


def rmsnorm_gemv_swiglu(W_gate_up, x, norm_w, eps, out, N, K, stream=None):
    _check(load().kvhp_rmsnorm_gemv_swiglu(_ptr(W_gate_up), _ptr(x), _ptr(norm_w), eps, _ptr(out),
                                           N, K, _stream(stream)))


def rmsnorm_qkv_rope_append(W_qkv, x, norm_w, eps, seq_len, theta, q_out, pool_k, pool_v,
                            block_table, num_q_heads, num_kv_heads, head_dim, K, stream=None):
    """pool_k / pool_v [Hkv][P][16][D]; block_table int32 [max_pages] (one sequence)."""
    _check(load().kvhp_rmsnorm_qkv_rope_append(
        _ptr(W_qkv), _ptr(x), _ptr(norm_w), eps, _ptr(seq_len), theta, _ptr(q_out), _ptr(pool_k),
        _ptr(pool_v), _ptr(block_table), block_table.numel(), pool_k.shape[1], num_q_heads,
        num_kv_heads, head_dim, K, _stream(stream)))


def gemv_residual_rows(W, x, r, y, N, K, batch, stream=None):
    _check(load().kvhp_gemv_residual_rows(_ptr(W), _ptr(x), _ptr(r), _ptr(y), N, K, batch,
                                          _stream(stream)))


def gemv_rows_workspace_bytes(N, K, batch):
    return load().kvhp_gemv_rows_workspace_bytes(N, K, batch)


def gemv_residual_rows_ws(W, x, r, y, N, K, batch, workspace=None, stream=None):
    """gemv_residual_rows with a caller workspace (uint8 tensor): large
    batches split over K; bit-identical output."""
    nbytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check(load().kvhp_gemv_residual_rows_ws(_ptr(W), _ptr(x), _ptr(r), _ptr(y), N, K, batch,
                                             _ptr(workspace), nbytes, _stream(stream)))


def rmsnorm_gemv_rows(W, x, norm_w, eps, N, K, batch, y16=None, y32=None, stream=None):
    _check(load().kvhp_rmsnorm_gemv_rows(_ptr(W), _ptr(x), _ptr(norm_w), eps, _ptr(y16),
                                         _ptr(y32), N, K, batch, _stream(stream)))


def rmsnorm_gemv_swiglu_rows(W_gate_up, x, norm_w, eps, out, N, K, batch, stream=None):
    _check(load().kvhp_rmsnorm_gemv_swiglu_rows(_ptr(W_gate_up), _ptr(x), _ptr(norm_w), eps,
                                                _ptr(out), N, K, batch, _stream(stream)))


def rmsnorm_qkv_rope_append_rows(W_qkv, x, norm_w, eps, positions, theta, q_out, pool_k, pool_v,
                                 block_tables, num_q_heads, num_kv_heads, head_dim, K, batch,
                                 stream=None):
    """pool_k / pool_v [Hkv][P][16][D]; block_tables int32 [batch][max_pages]."""
    _check(load().kvhp_rmsnorm_qkv_rope_append_rows(
        _ptr(W_qkv), _ptr(x), _ptr(norm_w), eps, _ptr(positions), theta, _ptr(q_out),
        _ptr(pool_k), _ptr(pool_v), _ptr(block_tables), block_tables.shape[1], pool_k.shape[1],
        num_q_heads, num_kv_heads, head_dim, K, batch, _stream(stream)))


ROWS_PLAIN, ROWS_SWIGLU, ROWS_QKV = 0, 1, 2


def rows_tiled_bytes(kind, N, K, num_q_heads=0, num_kv_heads=0, head_dim=0):
    return load().kvhp_rows_tiled_bytes(kind, N, K, num_q_heads, num_kv_heads, head_dim)


def rows_tile_weights(kind, W, N, K, W_tiled, num_q_heads=0, num_kv_heads=0, head_dim=0,
                      stream=None):
    """Copy row-major W into the batched projections' tiled layout (W_tiled:
    rows_tiled_bytes bytes, any dtype)."""
    _check(load().kvhp_rows_tile_weights(kind, _ptr(W), N, K, num_q_heads, num_kv_heads,
                                         head_dim, _ptr(W_tiled), _stream(stream)))


def gemv_residual_rows_tiled(Wt, x, r, y, N, K, batch, workspace=None, stream=None):
    nbytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check(load().kvhp_gemv_residual_rows_tiled(_ptr(Wt), _ptr(x), _ptr(r), _ptr(y), N, K, batch,
                                                _ptr(workspace), nbytes, _stream(stream)))


def rmsnorm_gemv_rows_tiled(Wt, x, norm_w, eps, N, K, batch, y16=None, y32=None, stream=None):
    _check(load().kvhp_rmsnorm_gemv_rows_tiled(_ptr(Wt), _ptr(x), _ptr(norm_w), eps, _ptr(y16),
                                               _ptr(y32), N, K, batch, _stream(stream)))


def rmsnorm_gemv_swiglu_rows_tiled(Wt, x, norm_w, eps, out, N, K, batch, stream=None):
    _check(load().kvhp_rmsnorm_gemv_swiglu_rows_tiled(_ptr(Wt), _ptr(x), _ptr(norm_w), eps,
                                                      _ptr(out), N, K, batch, _stream(stream)))


def rmsnorm_qkv_rope_append_rows_tiled(Wt, x, norm_w, eps, positions, theta, q_out, pool_k,
                                       pool_v, block_tables, num_q_heads, num_kv_heads, head_dim,
                                       K, batch, stream=None):
    _check(load().kvhp_rmsnorm_qkv_rope_append_rows_tiled(
        _ptr(Wt), _ptr(x), _ptr(norm_w), eps, _ptr(positions), theta, _ptr(q_out),
        _ptr(pool_k), _ptr(pool_v), _ptr(block_tables), block_tables.shape[1], pool_k.shape[1],
        num_q_heads, num_kv_heads, head_dim, K, batch, _stream(stream)))


def rmsnorm(x, weight, out, rows, dim, eps, stream=None):
    _check(load().kvhp_rmsnorm(_ptr(x), _ptr(weight), _ptr(out), rows, dim, eps, _stream(stream)))


def apply_rope(q, k, seq_len, num_q_heads, num_kv_heads, head_dim, start_pos, theta, stream=None):
    _check(load().kvhp_apply_rope(_ptr(q), _ptr(k), seq_len, num_q_heads, num_kv_heads, head_dim,
                                  start_pos, theta, _stream(stream)))


def split_qkv_rope(qkv, seq_len, num_q_heads, num_kv_heads, head_dim, start_pos, theta, q, k, v,
                   stream=None):
    _check(load().kvhp_split_qkv_rope(_ptr(qkv), seq_len, num_q_heads, num_kv_heads, head_dim,
                                      start_pos, theta, _ptr(q), _ptr(k), _ptr(v),
                                      _stream(stream)))


def split_qkv_rope_rows(qkv, rows, num_q_heads, num_kv_heads, head_dim, positions, theta, q, k,
                        v, stream=None):
    _check(load().kvhp_split_qkv_rope_rows(_ptr(qkv), rows, num_q_heads, num_kv_heads, head_dim,
                                           _ptr(positions), theta, _ptr(q), _ptr(k), _ptr(v),
                                           _stream(stream)))


def swiglu(gate, up, out, count, stream=None):
    _check(load().kvhp_swiglu(_ptr(gate), _ptr(up), _ptr(out), count, _stream(stream)))


def swiglu_rows(gate_up, out, rows, n, stream=None):
    _check(load().kvhp_swiglu_rows(_ptr(gate_up), _ptr(out), rows, n, _stream(stream)))


def embedding(token_ids, table, out, n, hidden, vocab, stream=None):
    _check(load().kvhp_embedding(_ptr(token_ids), _ptr(table), _ptr(out), n, hidden, vocab,
                                 _stream(stream)))


def argmax(logits, n, token, seq_len=None, log=None, log_count=None, stream=None):
    _check(load().kvhp_argmax(_ptr(logits), n, _ptr(token), _ptr(seq_len), _ptr(log),
                              _ptr(log_count), _stream(stream)))


def argmax_rows(logits, rows, n, tokens, stream=None):
    _check(load().kvhp_argmax_rows(_ptr(logits), rows, n, _ptr(tokens), _stream(stream)))


def randn_f16(out, seed, stream_id, std, stream=None):
    _check(load().kvhp_randn_f16(_ptr(out), out.numel(), seed, stream_id, std, _stream(stream)))


def fill_f16(out, value, stream=None):
    _check(load().kvhp_fill_f16(_ptr(out), out.numel(), value, _stream(stream)))


# ------------------------------------------------------------ model runner --
class LlamaConfig(ctypes.Structure):
    """kvhp_llama_config."""

    _fields_ = [("vocab_size", ctypes.c_int), ("hidden_size", ctypes.c_int),
                ("num_layers", ctypes.c_int), ("num_q_heads", ctypes.c_int),
                ("num_kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("ffn_size", ctypes.c_int), ("rms_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("reserved", ctypes.c_int)]


def llama_1b_config() -> LlamaConfig:
    """22 layers, hidden 2048, 32 q / 4 KV heads of 64,
    SwiGLU 5632, vocab 32000, RMSNorm eps 1e-5, RoPE theta 10000."""
    return LlamaConfig(32000, 2048, 22, 32, 4, 64, 5632, 1e-5, 10000.0, 0)


LLAMA_EMBED, LLAMA_LM_HEAD, LLAMA_FINAL_NORM = 0, 1, 2
LLAMA_ATTN_NORM, LLAMA_FFN_NORM, LLAMA_W_QKV, LLAMA_W_O = 10, 11, 12, 13
LLAMA_W_GATE_UP, LLAMA_W_DOWN, LLAMA_POOL_K, LLAMA_POOL_V = 14, 15, 16, 17


class LlamaModel:
    """The C ABI model runner: prefill_gpu / decode_step_gpu / on-device
    greedy generation (host buffers are numpy arrays)."""

    def __init__(self, config: LlamaConfig, seed: int, max_ctx: int):
        import numpy as np
        self._np = np
        self.config = config
        self.max_ctx = max_ctx
        h = ctypes.c_void_p()
        _check(load().kvhp_llama_create(ctypes.byref(config), seed, max_ctx, ctypes.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            load().kvhp_llama_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prefill(self, tokens):
        np = self._np
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.config.vocab_size, np.float32)
        nxt = ctypes.c_int32()
        _check(load().kvhp_llama_prefill(self._h, t.ctypes.data, t.size, logits.ctypes.data,
                                         ctypes.byref(nxt)))
        return int(nxt.value), logits

    def decode_step(self, token: int = -1):
        np = self._np
        logits = np.empty(self.config.vocab_size, np.float32)
        nxt = ctypes.c_int32()
        _check(load().kvhp_llama_decode_step(self._h, token, logits.ctypes.data,
                                             ctypes.byref(nxt)))
        return int(nxt.value), logits

    def generate(self, n_steps: int, use_graph: bool = True):
        """Returns (tokens since the prefill, device milliseconds of the steps)."""
        np = self._np
        out = np.zeros(self.max_ctx + 1, np.int32)
        ms = ctypes.c_float()
        _check(load().kvhp_llama_generate(self._h, n_steps, int(use_graph), out.ctypes.data,
                                          ctypes.byref(ms)))
        return out, float(ms.value)

    def prefill_paged(self, tokens, pool, num_pages: int, block_table, max_pages: int,
                      stream=None):
        """Runner.prefill over a caller-owned pool [L][2][Hkv][num_pages][16][D]
        (torch fp16) and one block-table row (torch int32, device): returns
        (first greedy token, fp32 logits of the last position)."""
        np = self._np
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.config.vocab_size, np.float32)
        nxt = ctypes.c_int32()
        _check(load().kvhp_llama_prefill_paged(self._h, t.ctypes.data, t.size, _ptr(pool),
                                               num_pages, _ptr(block_table), max_pages,
                                               logits.ctypes.data, ctypes.byref(nxt),
                                               _stream(stream)))
        return int(nxt.value), logits

    def prefill_cached(self, tokens, num_cached: int, pool, num_pages: int, block_table,
                       max_pages: int, write_table=None, stream=None):
        """Runner.prefill in the "full" prefix mode: the first num_cached
        positions' K/V are already in the pages; only the rest is forwarded
        (appends through write_table if given)."""
        np = self._np
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.config.vocab_size, np.float32)
        nxt = ctypes.c_int32()
        _check(load().kvhp_llama_prefill_cached(self._h, t.ctypes.data, t.size, num_cached,
                                                _ptr(pool), num_pages, _ptr(block_table),
                                                _ptr(write_table), max_pages, logits.ctypes.data,
                                                ctypes.byref(nxt), _stream(stream)))
        return int(nxt.value), logits

    def decode_paged(self, tokens, pool, num_pages: int, block_tables, max_pages: int, positions,
                     seq_lens, max_seq_len: int, logits, next_tokens, stream=None):
        """Runner.decode_step for tokens.numel() sequences; every argument is a
        device tensor (int32, fp16 pool, fp32 logits [B][V]); asynchronous."""
        _check(load().kvhp_llama_decode_paged(self._h, _ptr(tokens), tokens.numel(), _ptr(pool),
                                              num_pages, _ptr(block_tables), max_pages,
                                              _ptr(positions), _ptr(seq_lens), max_seq_len,
                                              _ptr(logits), _ptr(next_tokens), _stream(stream)))

    def reserve(self, max_batch: int, max_seq_len: int):
        """Size the decode buffers for every decode_paged call up to these
        limits (required before capturing decode_paged in a HIP graph)."""
        _check(load().kvhp_llama_reserve(self._h, max_batch, max_seq_len))

    def tensor(self, layer: int, which: int):
        """Host copy (numpy float16) of a model tensor."""
        np = self._np
        ptr = ctypes.c_void_p()
        n = ctypes.c_size_t()
        _check(load().kvhp_llama_tensor(self._h, layer, which, ctypes.byref(ptr), ctypes.byref(n)))
        out = np.empty(n.value, np.float16)
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipMemcpy.argtypes = [_vp, _vp, _sz, _i32]
        hip.hipMemcpy.restype = _i32
        rc = hip.hipMemcpy(out.ctypes.data, ptr.value, n.value * 2, 2)  # device to host
        if rc != 0:
            raise KVHPError(KVHP_ERR_HIP, f"hipMemcpy device-to-host failed ({rc})")
        return out

    def set_tensor(self, layer: int, which: int, values):
        """Overwrite a model tensor from a host array of its element count
        (synchronous).  Batched decode steps see the new weights after the
        next reserve(), which rebuilds their tiled copies."""
        np = self._np
        ptr = ctypes.c_void_p()
        n = ctypes.c_size_t()
        _check(load().kvhp_llama_tensor(self._h, layer, which, ctypes.byref(ptr), ctypes.byref(n)))
        src = np.ascontiguousarray(values, np.float16).reshape(-1)
        if src.size != n.value:
            raise KVHPError(KVHP_ERR_INVALID, f"tensor holds {n.value} elements, got {src.size}")
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipMemcpy.argtypes = [_vp, _vp, _sz, _i32]
        hip.hipMemcpy.restype = _i32
        rc = hip.hipMemcpy(ptr.value, src.ctypes.data, src.size * 2, 1)  # host to device
        if rc != 0:
            raise KVHPError(KVHP_ERR_HIP, f"hipMemcpy host-to-device failed ({rc})")
