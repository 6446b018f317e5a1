"""GPU parity of the KV writes and the paged gather: bit-exact against the
oracle (oracle/kvhp_oracle.c), through the C ABI."""
import numpy as np
import pytest

import kvhp
import oracle
from gpu_util import from_gpu, make_block_tables, note, sync, to_gpu, to_gpu_f16

pytestmark = pytest.mark.gpu


def _src(rng, shape):
    return oracle.normal_f16(rng, shape, 2.0)


def test_append_reference_shapes_bit_exact():
    """Shapes of tests/test_kv_cache.cpp:43-96 (seed 101 there): T 1..37,
    start 0..49, Hkv 1..4, D in {16,32,48,64}, slack after max_seq; plus
    overflow (positions >= max_seq dropped) and a D=12 unvectorised case."""
    import torch
    rng = np.random.default_rng(101)
    for i in range(27):
        t = 1 if i == 0 else int(rng.integers(1, 38))
        start = 0 if i == 0 else int(rng.integers(0, 50))
        hkv = int(rng.integers(1, 5))
        d = 16 * int(rng.integers(1, 5)) if i < 26 else 12
        max_seq = start + t + int(rng.integers(0, 30))
        if i % 6 == 5:
            max_seq = start + max(1, t // 2)   # overflowing append
        note(f"append case {i}: T={t} start={start} Hkv={hkv} D={d} max_seq={max_seq}")
        sk, sv = _src(rng, (t, hkv, d)), _src(rng, (t, hkv, d))
        dk = torch.zeros((hkv, max_seq, d), dtype=torch.float16, device="cuda")
        dv = torch.zeros_like(dk)
        kvhp.append_kv(to_gpu_f16(sk), to_gpu_f16(sv), dk, dv, t, start, hkv, max_seq, d)
        sync()
        ek = np.zeros((hkv, max_seq, d), np.uint16)
        ev = np.zeros_like(ek)
        oracle.append_kv(sk.view(np.uint16), sv.view(np.uint16), ek, ev, t, start, hkv,
                         max_seq, d)
        assert np.array_equal(from_gpu(dk).view(np.uint16), ek), i
        assert np.array_equal(from_gpu(dv).view(np.uint16), ev), i


@pytest.mark.parametrize("b,t,hkv,d", [(4, 1, 8, 128), (3, 37, 2, 64), (1, 2048, 8, 128),
                                       (5, 5, 4, 64)])
def test_paged_append_bit_exact(b, t, hkv, d):
    import torch
    rng = np.random.default_rng(200 + b * t)
    lens = rng.integers(0, 300, size=b).astype(np.int32)
    lens[0] = 0
    cap_lens = lens + t
    bt, P = make_block_tables(rng, cap_lens)
    if b > 1:
        bt[-1, -1] = -1                                  # unused column stays -1
    sk, sv = _src(rng, (b, t, hkv, d)), _src(rng, (b, t, hkv, d))
    pool0 = _src(rng, (hkv, P, 16, d))                   # pre-existing pool content
    note(f"paged_append B={b} T={t} Hkv={hkv} D={d} P={P}")
    pk, pv = to_gpu_f16(pool0), to_gpu_f16(pool0.copy())
    kvhp.paged_append_kv(to_gpu_f16(sk), to_gpu_f16(sv), pk, pv, to_gpu(bt), to_gpu(lens),
                         b, t, hkv, d)
    sync()
    ek = pool0.view(np.uint16).copy()
    ev = pool0.view(np.uint16).copy()
    oracle.paged_append(sk.view(np.uint16), sv.view(np.uint16), ek, ev, bt, lens, b, t, hkv, d)
    assert np.array_equal(from_gpu(pk).view(np.uint16), ek)
    assert np.array_equal(from_gpu(pv).view(np.uint16), ev)
    del torch


def test_paged_append_drops_out_of_range():
    import torch
    hkv, d = 2, 64
    bt = np.array([[1, -1], [5, 0]], np.int32)          # -1 and 5 are invalid ids
    start = np.array([14, 30], np.int32)
    rng = np.random.default_rng(3)
    src = _src(rng, (2, 4, hkv, d))
    pool = np.zeros((hkv, 2, 16, d), np.float16)
    pk, pv = to_gpu_f16(pool), to_gpu_f16(pool)
    note("paged_append drop rules")
    kvhp.paged_append_kv(to_gpu_f16(src), to_gpu_f16(src), pk, pv, to_gpu(bt), to_gpu(start),
                         2, 4, hkv, d)
    sync()
    ek = np.zeros((hkv, 2, 16, d), np.uint16)
    ev = ek.copy()
    oracle.paged_append(src.view(np.uint16), src.view(np.uint16), ek, ev, bt, start, 2, 4, hkv, d)
    assert np.array_equal(from_gpu(pk).view(np.uint16), ek)
    assert np.count_nonzero(ek) > 0
    del torch


@pytest.mark.parametrize("t,start,hkv,d,max_seq", [
    (2048, 0, 8, 128, 2048), (16, 5, 4, 32, 40), (333, 31, 2, 64, 400), (100, 7, 3, 256, 120),
    (17, 0, 1, 128, 17), (64, 48, 8, 64, 90)])
def test_append_runs_bit_exact(t, start, hkv, d, max_seq):
    """Appends of 16 or more tokens run by 16-token runs (one wave per run and
    KV head): page-aligned and unaligned starts, partial last runs, every
    vectorised head dim (32..256) and positions past max_seq dropped."""
    import torch
    rng = np.random.default_rng(t * 7 + start + d)
    sk, sv = _src(rng, (t, hkv, d)), _src(rng, (t, hkv, d))
    pre = _src(rng, (hkv, max_seq, d))
    note(f"append runs T={t} start={start} Hkv={hkv} D={d} max_seq={max_seq}")
    dk, dv = to_gpu_f16(pre), to_gpu_f16(pre.copy())
    kvhp.append_kv(to_gpu_f16(sk), to_gpu_f16(sv), dk, dv, t, start, hkv, max_seq, d)
    sync()
    ek = pre.view(np.uint16).copy()
    ev = pre.view(np.uint16).copy()
    oracle.append_kv(sk.view(np.uint16), sv.view(np.uint16), ek, ev, t, start, hkv, max_seq, d)
    assert np.array_equal(from_gpu(dk).view(np.uint16), ek)
    assert np.array_equal(from_gpu(dv).view(np.uint16), ev)


@pytest.mark.parametrize("t,d", [(16, 32), (50, 64), (129, 128), (40, 256)])
def test_paged_append_runs_bit_exact(t, d):
    """Paged appends of 16 or more tokens (runs): sequences starting on and
    off a page boundary, a negative start (rows before position 0 dropped),
    a run crossing into a -1 table entry and an id outside the pool
    (dropped), and a sequence running past max_pages (dropped)."""
    import torch
    rng = np.random.default_rng(500 + t + d)
    hkv, b, max_pages = 3, 5, 12
    start = np.array([0, 9, -5, 16 * max_pages - t // 2, 33], np.int32)
    P = b * max_pages
    bt = rng.permutation(P).astype(np.int32).reshape(b, max_pages)
    bt[1, (9 + t // 2) // 16] = -1
    bt[4, 2] = P + 3
    sk, sv = _src(rng, (b, t, hkv, d)), _src(rng, (b, t, hkv, d))
    pool0 = _src(rng, (hkv, P, 16, d))
    note(f"paged append runs T={t} D={d}")
    pk, pv = to_gpu_f16(pool0), to_gpu_f16(pool0.copy())
    kvhp.paged_append_kv(to_gpu_f16(sk), to_gpu_f16(sv), pk, pv, to_gpu(bt), to_gpu(start),
                         b, t, hkv, d)
    sync()
    ek = pool0.view(np.uint16).copy()
    ev = pool0.view(np.uint16).copy()
    oracle.paged_append(sk.view(np.uint16), sv.view(np.uint16), ek, ev, bt, start, b, t, hkv, d)
    assert np.array_equal(from_gpu(pk).view(np.uint16), ek)
    assert np.array_equal(from_gpu(pv).view(np.uint16), ev)
    del torch


@pytest.mark.parametrize("b,hkv,d,maxlen", [(3, 2, 64, 100), (8, 8, 128, 700), (2, 1, 40, 33),
                                            (4, 3, 32, 50), (2, 2, 256, 90)])
def test_paged_gather_bit_exact(b, hkv, d, maxlen):
    import torch
    rng = np.random.default_rng(300 + b)
    lens = rng.integers(0, maxlen + 20, size=b).astype(np.int32)
    bt, P = make_block_tables(rng, np.maximum(lens, 1))
    pool_k = _src(rng, (hkv, P, 16, d))
    pool_v = _src(rng, (hkv, P, 16, d))
    note(f"paged_gather B={b} Hkv={hkv} D={d} max_len={maxlen}")
    ok = torch.full((b, hkv, maxlen, d), 7.0, dtype=torch.float16, device="cuda")
    ov = torch.full_like(ok, 7.0)
    kvhp.paged_gather_kv(to_gpu_f16(pool_k), to_gpu_f16(pool_v), to_gpu(bt), to_gpu(lens),
                         maxlen, ok, ov)
    sync()
    ek, ev = oracle.paged_gather(pool_k.view(np.uint16), pool_v.view(np.uint16), bt, lens, maxlen)
    assert np.array_equal(from_gpu(ok).view(np.uint16), ek)
    assert np.array_equal(from_gpu(ov).view(np.uint16), ev)


@pytest.mark.parametrize("d", [64, 40])
def test_paged_gather_invalid_page_ids_read_as_zero(d):
    """Block-table entries outside [0, P) (-1, P, a huge id) gather zeros for
    their rows, on the page-per-wave kernel (D = 64) and the per-chunk one
    (D = 40); rows past the length are zero, past max_len unwritten."""
    import torch
    rng = np.random.default_rng(90 + d)
    hkv, P, maxlen = 2, 6, 70
    bt = np.array([[0, -1, 3, 9], [5, 2, 1 << 30, 4]], np.int32)
    lens = np.array([64, 57], np.int32)
    pool_k = _src(rng, (hkv, P, 16, d))
    pool_v = _src(rng, (hkv, P, 16, d))
    note(f"paged_gather invalid ids D={d}")
    ok = torch.full((2, hkv, maxlen, d), 7.0, dtype=torch.float16, device="cuda")
    ov = torch.full_like(ok, 7.0)
    kvhp.paged_gather_kv(to_gpu_f16(pool_k), to_gpu_f16(pool_v), to_gpu(bt), to_gpu(lens),
                         maxlen, ok, ov)
    sync()
    ek, ev = oracle.paged_gather(pool_k.view(np.uint16), pool_v.view(np.uint16), bt, lens, maxlen)
    assert np.array_equal(from_gpu(ok).view(np.uint16), ek)
    assert np.array_equal(from_gpu(ov).view(np.uint16), ev)
    assert not ek[0, :, 16:32].any() and not ek[1, :, 32:48].any()


def test_config3_scale_append_gather_round_trip():
    """Config-3 scale (32 sequences, lengths U[128,8192], 8 KV heads, D=128,
    ~545 MB pool): appending every token through random block tables and
    gathering back reproduces the tokens exactly (checked on the GPU)."""
    import torch
    rng = np.random.default_rng(2024)
    b, hkv, d = 32, 8, 128
    lens = rng.integers(128, 8193, size=b).astype(np.int32)
    bt, P = make_block_tables(rng, lens)
    maxlen = int(lens.max())
    note(f"config3 round trip: sum L={int(lens.sum())} pages={P}")
    g = torch.Generator(device="cuda").manual_seed(7)
    src_k = torch.randn((b, maxlen, hkv, d), generator=g, device="cuda").half()
    src_v = torch.randn((b, maxlen, hkv, d), generator=g, device="cuda").half()
    pk = torch.zeros((hkv, P, 16, d), dtype=torch.float16, device="cuda")
    pv = torch.zeros_like(pk)
    zero = torch.zeros(b, dtype=torch.int32, device="cuda")
    kvhp.paged_append_kv(src_k, src_v, pk, pv, to_gpu(bt), zero, b, maxlen, hkv, d)
    ok = torch.empty((b, hkv, maxlen, d), dtype=torch.float16, device="cuda")
    ov = torch.empty_like(ok)
    lens_d = to_gpu(lens)
    kvhp.paged_gather_kv(pk, pv, to_gpu(bt), lens_d, maxlen, ok, ov)
    sync()
    pos = torch.arange(maxlen, device="cuda")[None, :] < lens_d[:, None].long()
    mask = pos[:, None, :, None].expand(b, hkv, maxlen, d)
    ek = src_k.permute(0, 2, 1, 3)
    ev = src_v.permute(0, 2, 1, 3)
    assert torch.equal(ok.view(torch.int16)[mask], ek.contiguous().view(torch.int16)[mask])
    assert torch.equal(ov.view(torch.int16)[mask], ev.contiguous().view(torch.int16)[mask])
    assert int(torch.count_nonzero(ok.view(torch.int16)[~mask])) == 0
