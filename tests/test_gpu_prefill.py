"""GPU parity of causal flash prefill against the oracle's restatement of the
reference cpu::causal_gqa (src/cpu/ops.cpp:223-284), through the C ABI.

Tolerance: max-abs 2e-3 / max-rel 1e-2 (see gpu_util.assert_attn_close).
Long prompts are checked on a seeded sample of rows (rows are independent, so
each sampled row is an exact per-row check), always including the first and
last rows and the 64-row block edges.
"""
import numpy as np
import pytest

import kvhp
import oracle
from gpu_util import (assert_attn_close, from_gpu, make_block_tables, note, sync, to_gpu,
                      to_gpu_f16, uniform_f16)

pytestmark = pytest.mark.gpu


def _prefill(q, k, v, hq, hkv, d, batch=1):
    import torch
    s = q.shape[-3]
    out = torch.full(q.shape, float("nan"), dtype=torch.float16, device="cuda")
    kvhp.flash_prefill(to_gpu_f16(q), to_gpu_f16(k), to_gpu_f16(v), out, s, hq, hkv, d, batch)
    sync()
    return from_gpu(out).astype(np.float32)


def test_prefill_reference_shapes():
    """tests/test_attention.cpp:180-291: 25 shapes, Hkv=2, G 7 or 1..7, D=64,
    S in {1, 15, 17, 65, rand<=120}, U(-1,1) inputs."""
    rng = np.random.default_rng(702)
    for i in range(25):
        g = 7 if i % 3 == 0 else int(rng.integers(1, 8))
        hkv, d = 2, 64
        hq = hkv * g
        s = [1, 15, 17, 65][i] if i < 4 else int(rng.integers(1, 121))
        q = uniform_f16(rng, (s, hq, d))
        k, v = uniform_f16(rng, (s, hkv, d)), uniform_f16(rng, (s, hkv, d))
        note(f"prefill ref case {i}: S={s} G={g}")
        got = _prefill(q, k, v, hq, hkv, d)
        ref = oracle.causal_gqa(q.astype(np.float32), k.astype(np.float32),
                                v.astype(np.float32), hq, hkv, d, nthreads=8)
        assert_attn_close(got, ref, f"case {i}")


@pytest.mark.parametrize("s", [1, 2, 63, 64, 65, 200, 512])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (32, 4, 64)])
def test_prefill_baseline_heads_full_check(s, hq, hkv, d):
    rng = np.random.default_rng(s * 13 + d)
    q = oracle.normal_f16(rng, (s, hq, d))
    k, v = oracle.normal_f16(rng, (s, hkv, d)), oracle.normal_f16(rng, (s, hkv, d))
    note(f"prefill S={s} Hq={hq} Hkv={hkv} D={d}")
    got = _prefill(q, k, v, hq, hkv, d)
    ref = oracle.causal_gqa(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32),
                            hq, hkv, d, nthreads=8)
    assert_attn_close(got, ref, f"S={s}")


def _sample_rows(rng, s, n=24):
    fixed = {0, 1, 2, 63, 64, 65, 127, 128, s // 2, s - 2, s - 1}
    rows = set(r for r in fixed if 0 <= r < s)
    rows |= set(int(x) for x in rng.integers(0, s, size=n))
    return sorted(rows)


def _edge_rows(rng, s, n=24):
    """Both rows at every 32-row boundary (the query blocks of the short-prompt
    kernel; every 64-row block edge of the long-prompt kernel is among them),
    plus the first and last rows and a seeded sample."""
    rows = set(_sample_rows(rng, s, n))
    for e in range(32, s, 32):
        rows.update((e - 1, e))
    return sorted(rows)


def _check_rows(got, q, k, v, hq, hkv, d, rows, what):
    """Every head of each listed row against the oracle (rows are independent,
    so each is an exact per-row check)."""
    ref = oracle.causal_gqa_rowlist(q.astype(np.float32), k.astype(np.float32),
                                    v.astype(np.float32), hq, hkv, d, rows, nthreads=16)
    assert_attn_close(got[rows], ref, f"{what} ({len(rows)} rows)")


@pytest.mark.parametrize("s", [2048, 8192])
def test_prefill_config4_sampled_rows(s):
    """BASELINE config 4 (32/8 heads, D=128, N(0,1)) at S=2048 and 8192; every
    head of both rows at each 32-row block edge and of a seeded row sample is
    checked against the oracle."""
    rng = np.random.default_rng(4 + s)
    hq, hkv, d = 32, 8, 128
    q = oracle.normal_f16(rng, (s, hq, d))
    k, v = oracle.normal_f16(rng, (s, hkv, d)), oracle.normal_f16(rng, (s, hkv, d))
    note(f"prefill config4 S={s}")
    got = _prefill(q, k, v, hq, hkv, d)
    _check_rows(got, q, k, v, hq, hkv, d, _edge_rows(rng, s), f"S={s}")


def test_prefill_batched():
    rng = np.random.default_rng(77)
    b, s, hq, hkv, d = 3, 150, 16, 4, 128
    q = oracle.normal_f16(rng, (b, s, hq, d))
    k, v = oracle.normal_f16(rng, (b, s, hkv, d)), oracle.normal_f16(rng, (b, s, hkv, d))
    note("prefill batched B=3")
    got = _prefill(q, k, v, hq, hkv, d, batch=b)
    for i in range(b):
        ref = oracle.causal_gqa(q[i].astype(np.float32), k[i].astype(np.float32),
                                v[i].astype(np.float32), hq, hkv, d, nthreads=8)
        assert_attn_close(got[i], ref, f"batch {i}")


# Short prompts with G <= 4 run the two-key-group kernel (two wave groups
# split every 64-key tile and merge their softmax states at the end), with
# causal blocks paired into one workgroup (two passes) once the pairs fill the
# CUs, one block per workgroup below that.  Cases: G = 1 / 2 / 4, D = 64 /
# 128, odd block counts (the middle pair is a single block), partial last
# tiles, a pair whose two blocks end in the same tile, and a batch.
@pytest.mark.parametrize("s,hq,hkv,d,batch", [
    (1, 4, 4, 128, 1), (96, 4, 4, 128, 1), (333, 4, 4, 64, 1), (1000, 4, 4, 128, 1),
    (100, 8, 4, 128, 1), (513, 8, 4, 64, 1), (640, 8, 4, 128, 1),
    (33, 16, 4, 128, 1), (224, 16, 4, 64, 1), (777, 16, 4, 128, 2),
])
def test_prefill_pair_pass_full_check(s, hq, hkv, d, batch):
    rng = np.random.default_rng(7 * s + hq + d)
    q = oracle.normal_f16(rng, (batch, s, hq, d))
    k, v = oracle.normal_f16(rng, (batch, s, hkv, d)), oracle.normal_f16(rng, (batch, s, hkv, d))
    note(f"prefill pair pass S={s} Hq={hq} Hkv={hkv} D={d} B={batch}")
    got = _prefill(q, k, v, hq, hkv, d, batch=batch)
    for i in range(batch):
        ref = oracle.causal_gqa(q[i].astype(np.float32), k[i].astype(np.float32),
                                v[i].astype(np.float32), hq, hkv, d, nthreads=8)
        assert_attn_close(got[i], ref, f"batch {i}")


@pytest.mark.parametrize("s,hq,hkv,d", [(8192, 32, 8, 128), (2048, 32, 8, 128), (2560, 32, 8, 128),
                                        (333, 14, 2, 64), (70, 6, 3, 96), (515, 8, 4, 128),
                                        (200, 4, 4, 64)])
def test_prefill_paged_writes_pages_bit_exact(s, hq, hkv, d):
    """flash_prefill_paged writes K/V rows into the pages exactly as the paged
    append does (config 4: K/V written into 16-token pages as produced), and
    its attention output matches the oracle: at S >= 2048 (config 4, the path
    bench.py times) on both rows of every 32-row block edge, every head."""
    import torch
    rng = np.random.default_rng(s + d)
    q = oracle.normal_f16(rng, (s, hq, d))
    k, v = oracle.normal_f16(rng, (s, hkv, d)), oracle.normal_f16(rng, (s, hkv, d))
    bt, P = make_block_tables(rng, [s])
    pool0 = oracle.normal_f16(rng, (hkv, P, 16, d))
    pk, pv = to_gpu_f16(pool0), to_gpu_f16(pool0.copy())
    out = torch.empty((s, hq, d), dtype=torch.float16, device="cuda")
    note(f"prefill paged S={s} Hq={hq} D={d}")
    kvhp.flash_prefill_paged(to_gpu_f16(q), to_gpu_f16(k), to_gpu_f16(v), out, s, hq, hkv, d,
                             1, pk, pv, to_gpu(bt))
    sync()
    ek = pool0.view(np.uint16).copy()
    ev = pool0.view(np.uint16).copy()
    oracle.paged_append(k[None].view(np.uint16), v[None].view(np.uint16), ek, ev, bt,
                        np.array([0], np.int32), 1, s, hkv, d)
    assert np.array_equal(from_gpu(pk).view(np.uint16), ek)
    assert np.array_equal(from_gpu(pv).view(np.uint16), ev)
    rows = _edge_rows(rng, s, 8) if s >= 2048 else _sample_rows(rng, s, 8)
    _check_rows(from_gpu(out).astype(np.float32), q, k, v, hq, hkv, d, rows, f"paged S={s}")


@pytest.mark.parametrize("s", [1, 300, 2048])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (32, 4, 64)])
def test_prefill_known_answers(s, hq, hkv, d):
    """Answers fixed by the mathematics, not by the oracle: row 0 attends to
    key 0 alone, so it returns v[0] of its KV head bit for bit (the reference
    KAT, tests/test_cpu_ops.cpp:112-136); with V constant per KV head every
    row of head h returns the constant of KV head h // G (the GQA map)."""
    g = hq // hkv
    rng = np.random.default_rng(s + d)
    note(f"prefill KATs S={s} Hq={hq} Hkv={hkv} D={d}")
    q = oracle.normal_f16(rng, (s, hq, d))
    k, v = oracle.normal_f16(rng, (s, hkv, d)), oracle.normal_f16(rng, (s, hkv, d))
    got = _prefill(q, k, v, hq, hkv, d)
    want = np.stack([v[0, h // g] for h in range(hq)]).astype(np.float32)
    np.testing.assert_array_equal(got[0], want, err_msg="row 0 must return v[0]")
    vc = np.empty((s, hkv, d), np.float16)
    for kh in range(hkv):
        vc[:, kh] = (kh + 1) / 8.0
    got = _prefill(q, k, vc, hq, hkv, d)
    want = np.broadcast_to(np.stack([np.full(d, (h // g + 1) / 8.0) for h in range(hq)]),
                           (s, hq, d))
    assert_attn_close(got, want, "GQA head map")


def test_causal_gqa_api_routes_to_prefill():
    import torch
    rng = np.random.default_rng(45)
    s, hq, hkv, d = 90, 14, 2, 64
    q = uniform_f16(rng, (s, hq, d))
    k, v = uniform_f16(rng, (s, hkv, d)), uniform_f16(rng, (s, hkv, d))
    out = torch.empty((s, hq, d), dtype=torch.float16, device="cuda")
    note("causal_gqa api")
    kvhp.causal_gqa(to_gpu_f16(q), to_gpu_f16(k), to_gpu_f16(v), out, s, hq, hkv, d)
    sync()
    ref = oracle.causal_gqa(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32),
                            hq, hkv, d)
    assert_attn_close(from_gpu(out).astype(np.float32), ref, "causal_gqa")


@pytest.mark.parametrize("s,hq,hkv,d,batch", [
    (2560, 32, 8, 128, 1), (4096, 32, 8, 128, 1), (2048, 32, 8, 128, 2), (6144, 32, 8, 128, 1),
    (5000, 16, 4, 64, 1),
])
def test_prefill_key_group_choice_shapes(s, hq, hkv, d, batch):
    """Prompt sizes on either side of the key-group choice (one unit per wave
    for 129..256 and 385+ block pairs, two key groups for up to 128 and
    257..384; paired or one block per workgroup): both rows at every 32-row
    block edge and a seeded sample, every head, against the oracle."""
    rng = np.random.default_rng(11 * s + d + batch)
    q = oracle.normal_f16(rng, (batch, s, hq, d))
    k, v = oracle.normal_f16(rng, (batch, s, hkv, d)), oracle.normal_f16(rng, (batch, s, hkv, d))
    note(f"prefill key-group choice S={s} Hq={hq} Hkv={hkv} D={d} B={batch}")
    got = _prefill(q, k, v, hq, hkv, d, batch=batch)
    for i in range(batch):
        _check_rows(got[i], q[i], k[i], v[i], hq, hkv, d, _edge_rows(rng, s, 8), f"S={s} batch {i}")
