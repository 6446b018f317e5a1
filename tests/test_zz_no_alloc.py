"""kvhp_decode_attention_noalloc (split partials in the library's static
device scratch, no allocation) through the C ABI, against
kvhp_decode_attention on the same inputs: outputs bit for bit, on two calls
in a row, the second smaller (the scratch keeps the first call's partials),
and both against the oracle within the attention tolerance (max-abs 2e-3 /
max-rel 1e-2).  A plan whose partials exceed the scratch is refused before
any launch.
"""
import numpy as np
import pytest

import kvhp
import oracle
from gpu_util import assert_attn_close, from_gpu, make_block_tables, note, sync, to_gpu

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _pool_case(rng, lens, hq, hkv, d):
    """Random fp16 pool [Hkv][P][16][D] on the GPU, seeded random page
    tables; returns (q, k view, v view, seq_lens, oracle reference)."""
    lens = np.asarray(lens, np.int32)
    b = lens.size
    bt, P = make_block_tables(rng, lens)
    gen = torch.Generator(device="cuda").manual_seed(int(rng.integers(1 << 30)))
    pk = torch.randn((hkv, P, 16, d), generator=gen, device="cuda").half()
    pv = torch.randn((hkv, P, 16, d), generator=gen, device="cuda").half()
    q = torch.randn((b, hq, d), generator=gen, device="cuda").half()
    bt_t = to_gpu(bt)
    views = (kvhp.paged_view(pk, bt_t), kvhp.paged_view(pv, bt_t))
    cap = max(int(lens.max()), 1)
    hk, hv = from_gpu(pk).astype(np.float32), from_gpu(pv).astype(np.float32)
    kc = np.zeros((b, hkv, cap, d), np.float32)
    vc = np.zeros_like(kc)
    for i in range(b):
        n = int(lens[i])
        pages = bt[i, :(n + 15) // 16]
        kc[i, :, :n] = hk[:, pages].reshape(hkv, -1, d)[:, :n]
        vc[i, :, :n] = hv[:, pages].reshape(hkv, -1, d)[:, :n]
    ref = oracle.decode_attention(from_gpu(q).astype(np.float32), kc, vc, lens, hq, hkv, d,
                                  nthreads=16)
    return q, views, to_gpu(lens), ref, (pk, pv, bt_t)


def _both(q, views, lens_t, hq, hkv, d, max_len, splits):
    b = lens_t.shape[0]
    a = torch.full((b, hq, d), float("nan"), dtype=torch.float16, device="cuda")
    n = torch.full_like(a, float("nan"))
    kvhp.decode_attention(q, views[0], views[1], lens_t, a, hq, hkv, d, max_len, splits)
    kvhp.decode_attention_noalloc(q, views[0], views[1], lens_t, n, hq, hkv, d, max_len, splits)
    sync()
    return from_gpu(a), from_gpu(n)


def test_noalloc_matches_allocating_entry_point_twice():
    rng = np.random.default_rng(77)
    # call 1: BASELINE config 3 shape (32 sequences, lengths in [128, 8192],
    # 32/8 heads, D=128), auto splits: the device-balanced plan, 11.2 MB of
    # partials in the scratch
    lens1 = rng.integers(128, 8193, size=32).astype(np.int32)
    note(f"noalloc call 1: B=32 sum L={int(lens1.sum())}")
    q, views, lt, ref, keep = _pool_case(rng, lens1, 32, 8, 128)
    a, n = _both(q, views, lt, 32, 8, 128, int(lens1.max()), 0)
    assert np.array_equal(a.view(np.uint16), n.view(np.uint16)), "call 1: outputs differ"
    assert_attn_close(n.astype(np.float32), ref, "noalloc call 1")
    del keep, views
    # call 2, smaller: 4 sequences (one empty), 32/4 heads of 64, 4 explicit
    # splits; the scratch still holds call 1's partials
    lens2 = np.array([700, 33, 0, 2000], np.int32)
    note(f"noalloc call 2: lens {lens2.tolist()}")
    q, views, lt, ref, keep = _pool_case(rng, lens2, 32, 4, 64)
    a, n = _both(q, views, lt, 32, 4, 64, int(lens2.max()), 4)
    assert np.array_equal(a.view(np.uint16), n.view(np.uint16)), "call 2: outputs differ"
    assert_attn_close(n.astype(np.float32), ref, "noalloc call 2")


def test_noalloc_refuses_plans_beyond_the_scratch():
    """256 sequences x 32 heads x 64 splits x (128 + 2) floats = 272 MB of
    partials: refused with KVHP_ERR_WORKSPACE before any launch.  (Every
    length is 0, so nothing would be read even if a launch happened.)"""
    b, hq, hkv, d = 256, 32, 8, 128
    k = torch.zeros((hkv, 16, d), dtype=torch.float16, device="cuda")
    view = kvhp.strided_view(k, 0, 16 * d, d)
    out = torch.zeros((b, hq, d), dtype=torch.float16, device="cuda")
    lens = torch.zeros(b, dtype=torch.int32, device="cuda")
    with pytest.raises(kvhp.KVHPError) as e:
        kvhp.decode_attention_noalloc(torch.zeros((b, hq, d), dtype=torch.float16, device="cuda"),
                                      view, view, lens, out, hq, hkv, d, 65536, 64)
    assert e.value.code == kvhp.KVHP_ERR_WORKSPACE, e.value
    assert "static scratch" in str(e.value)
    sync()


def _pool_only(rng, lens, hq, hkv, d):
    """A random fp16 pool and seeded page tables on the GPU (no oracle)."""
    lens = np.asarray(lens, np.int32)
    bt, P = make_block_tables(rng, lens)
    gen = torch.Generator(device="cuda").manual_seed(int(rng.integers(1 << 30)))
    pk = torch.randn((hkv, P, 16, d), generator=gen, device="cuda").half()
    pv = torch.randn((hkv, P, 16, d), generator=gen, device="cuda").half()
    bt_t = to_gpu(bt)
    q = torch.empty((lens.size, hq, d), dtype=torch.float16, device="cuda")
    return q, (kvhp.paged_view(pk, bt_t), kvhp.paged_view(pv, bt_t)), to_gpu(lens), (pk, pv, bt_t)


def test_noalloc_captured_in_a_graph_replays_bit_exact():
    """Two noalloc calls captured in one HIP graph on a side stream -- a
    32-sequence batch on the device-balanced plan (D=128, auto splits) and a
    4-sequence batch with 4 fixed splits (32/4 heads of 64) -- sharing the
    static scratch one after the other.  The first call on a device resolves
    the scratch address and its kernels' occupancy, so one eager call of each
    runs first (the header asks for that).  Three replays, each with new q
    values and eager work and a synchronisation in between: every replay's
    outputs equal kvhp_decode_attention run eagerly on the same inputs, bit
    for bit."""
    rng = np.random.default_rng(2027)
    lens_a = rng.integers(128, 4097, size=32).astype(np.int32)
    lens_b = np.array([700, 33, 0, 2000], np.int32)
    cases = [(_pool_only(rng, lens_a, 32, 8, 128), 32, 8, 128, int(lens_a.max()), 0),
             (_pool_only(rng, lens_b, 32, 4, 64), 32, 4, 64, int(lens_b.max()), 4)]
    outs = [torch.full((c[0][0].shape[0], c[1], c[3]), float("nan"), dtype=torch.float16,
                       device="cuda") for c in cases]

    def run_noalloc():
        for ((q, views, lt, _), hq, hkv, d, ml, sp), o in zip(cases, outs):
            kvhp.decode_attention_noalloc(q, views[0], views[1], lt, o, hq, hkv, d, ml, sp)

    gen = torch.Generator(device="cuda").manual_seed(5)
    for (q, _, _, _), *_ in cases:
        q.copy_(torch.randn(q.shape, generator=gen, device="cuda").half())
    note("noalloc graph: eager first calls")
    run_noalloc()
    sync()
    g = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    note("noalloc graph: capture")
    with torch.cuda.graph(g, stream=cs):
        run_noalloc()
    torch.cuda.current_stream().wait_stream(cs)
    sync()
    for r in range(3):
        for (q, _, _, _), *_ in cases:
            q.copy_(torch.randn(q.shape, generator=gen, device="cuda").half())
        for o in outs:
            o.fill_(float("nan"))
        note(f"noalloc graph: replay {r}")
        g.replay()
        sync()
        for i, (((q, views, lt, _), hq, hkv, d, ml, sp), o) in enumerate(zip(cases, outs)):
            want = torch.full_like(o, float("nan"))
            kvhp.decode_attention(q, views[0], views[1], lt, want, hq, hkv, d, ml, sp)
            sync()
            assert np.array_equal(from_gpu(o).view(np.uint16), from_gpu(want).view(np.uint16)), \
                f"replay {r}, call {i}: graph output differs from the eager call"
    del g


_FIRST_CALL_SCRIPT = r"""
import sys
sys.path[:0] = sys.argv[1:]
import torch, kvhp
hq, hkv, d, L = 32, 8, 128, 300
k = torch.randn((1, hkv, L, d), device="cuda").half()
view = kvhp.strided_view(k, hkv * L * d, L * d, d)
q = torch.randn((1, hq, d), device="cuda").half()
lens = torch.tensor([L], dtype=torch.int32, device="cuda")
out = torch.zeros((1, hq, d), dtype=torch.float16, device="cuda")
torch.cuda.synchronize()
cs = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
err = None
with torch.cuda.stream(cs):
    g.capture_begin()
    try:
        kvhp.decode_attention_noalloc(q, view, view, lens, out, hq, hkv, d, L, 4)
    except kvhp.KVHPError as e:
        err = e
    finally:
        g.capture_end()
torch.cuda.synchronize()
del g
assert err is not None and err.code == kvhp.KVHP_ERR_INVALID and "first call" in str(err), err
kvhp.decode_attention_noalloc(q, view, view, lens, out, hq, hkv, d, L, 4)   # outside capture
want = torch.zeros_like(out)
kvhp.decode_attention(q, view, view, lens, want, hq, hkv, d, L, 4)
torch.cuda.synchronize()
assert torch.equal(out, want)
print("first-call rule ok", flush=True)
"""


def test_noalloc_first_call_under_capture_is_refused():
    """In a fresh process (the scratch address not yet resolved): a first
    noalloc call under graph capture is refused with KVHP_ERR_INVALID before
    anything is enqueued; the next call outside capture works and matches
    kvhp_decode_attention bit for bit."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    paths = [os.path.join(root, "serving-engine_amd"), os.path.join(root, "oracle"), here]
    note("noalloc first call under capture (subprocess)")
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_SCRIPT] + paths, capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "first-call rule ok" in r.stdout
