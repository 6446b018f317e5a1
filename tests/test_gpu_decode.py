"""GPU parity of split-K decode attention against the oracle, through the C ABI.

Tolerance: max-abs 2e-3 / max-rel 1e-2 (see gpu_util.assert_attn_close).
"""
import numpy as np
import pytest

import kvhp
import oracle
from gpu_util import (assert_attn_close, contiguous_from_tokens, from_gpu, make_block_tables,
                      note, sync, to_gpu, to_gpu_f16, uniform_f16)

pytestmark = pytest.mark.gpu


def _run_contig(q, kc, vc, lens, hq, hkv, d, cap, splits=0, workspace=None):
    """q [B][Hq][D], kc/vc [B][Hkv][cap][D] (fp16 numpy) -> GPU output fp32."""
    import torch
    b = q.shape[0]
    kt, vt = to_gpu_f16(kc), to_gpu_f16(vc)
    kview = kvhp.strided_view(kt, hkv * cap * d, cap * d, d)
    vview = kvhp.strided_view(vt, hkv * cap * d, cap * d, d)
    out = torch.full((b, hq, d), float("nan"), dtype=torch.float16, device="cuda")
    kvhp.decode_attention(to_gpu_f16(q), kview, vview, to_gpu(np.asarray(lens, np.int32)), out,
                          hq, hkv, d, cap, splits, workspace)
    sync()
    return from_gpu(out).astype(np.float32)


def test_decode_reference_shapes():
    """tests/test_attention.cpp:34-175: 25 shapes, B 1..3, Hkv=2, G 7 or 1..7,
    D=64, lengths {1, 17, 513, rand<=600}, U(-1,1) inputs."""
    rng = np.random.default_rng(701)
    for i in range(25):
        b = 1 if i % 4 == 0 else int(rng.integers(1, 4))
        hkv = 2
        g = 7 if i % 3 == 0 else int(rng.integers(1, 8))
        hq, d = hkv * g, 64
        lens = np.array([1 if i == 0 else 17 if i == 1 else 513 if i == 2
                         else int(rng.integers(1, 601)) for _ in range(b)], np.int32)
        cap = int(lens.max())
        q = uniform_f16(rng, (b, hq, d))
        kc, vc = uniform_f16(rng, (b, hkv, cap, d)), uniform_f16(rng, (b, hkv, cap, d))
        note(f"decode ref case {i}: B={b} G={g} lens={lens.tolist()}")
        got = _run_contig(q, kc, vc, lens, hq, hkv, d, cap)
        ref = oracle.decode_attention(q.astype(np.float32), kc.astype(np.float32),
                                      vc.astype(np.float32), lens, hq, hkv, d)
        assert_attn_close(got, ref, f"case {i}")


@pytest.mark.parametrize("L", [1, 15, 16, 63, 64, 65, 1000, 4096])
@pytest.mark.parametrize("splits", [1, 4, 16, 64, 0])
def test_decode_d128_splits(L, splits):
    """32 q / 8 KV heads, D=128 at ragged lengths and
    every split count of the config-2 sweep; N(0,1) inputs."""
    rng = np.random.default_rng(1000 + L)
    hq, hkv, d = 32, 8, 128
    q = oracle.normal_f16(rng, (1, hq, d))
    kc, vc = oracle.normal_f16(rng, (1, hkv, L, d)), oracle.normal_f16(rng, (1, hkv, L, d))
    note(f"decode d128 L={L} splits={splits}")
    got = _run_contig(q, kc, vc, [L], hq, hkv, d, L, splits)
    ref = oracle.decode_attention(q.astype(np.float32), kc.astype(np.float32),
                                  vc.astype(np.float32), np.array([L], np.int32), hq, hkv, d,
                                  nthreads=8)
    assert_attn_close(got, ref, f"L={L} splits={splits}")


@pytest.mark.parametrize("d,L,splits", [(64, 1, 1), (64, 40, 1), (64, 96, 1), (64, 160, 1),
                                         (64, 224, 2), (64, 700, 3), (128, 33, 1), (128, 129, 1),
                                         (128, 515, 0)])
def test_decode_four_wave_splits(d, L, splits):
    """Fixed-chunk splits run four waves that take the split's 32-token steps
    round robin and fold their (m, l, O) in LDS: splits of 1..7 steps (waves
    with no step among them), D=64 multi-split and D=128 single splits."""
    rng = np.random.default_rng(3000 + 7 * L + d)
    hq, hkv = 32, 4 if d == 64 else 8
    q = oracle.normal_f16(rng, (1, hq, d))
    kc, vc = oracle.normal_f16(rng, (1, hkv, L, d)), oracle.normal_f16(rng, (1, hkv, L, d))
    note(f"decode four-wave d={d} L={L} splits={splits}")
    got = _run_contig(q, kc, vc, [L], hq, hkv, d, L, splits)
    ref = oracle.decode_attention(q.astype(np.float32), kc.astype(np.float32),
                                  vc.astype(np.float32), np.array([L], np.int32), hq, hkv, d,
                                  nthreads=8)
    assert_attn_close(got, ref, f"d={d} L={L} splits={splits}")


def test_config1_append_then_decode():
    """B=1, 32/8 heads, D=64, 511 cached tokens, append one
    K/V row at position 511 with the append kernel, then decode over 512."""
    import torch
    rng = np.random.default_rng(1)
    hq, hkv, d, max_seq = 32, 8, 64, 512
    kc = np.zeros((hkv, max_seq, d), np.float16)
    vc = np.zeros_like(kc)
    kc[:, :511] = oracle.normal_f16(rng, (hkv, 511, d))
    vc[:, :511] = oracle.normal_f16(rng, (hkv, 511, d))
    knew, vnew = oracle.normal_f16(rng, (1, hkv, d)), oracle.normal_f16(rng, (1, hkv, d))
    q = oracle.normal_f16(rng, (1, hq, d))
    kt, vt = to_gpu_f16(kc), to_gpu_f16(vc)
    note("config1 append + decode")
    kvhp.append_kv(to_gpu_f16(knew), to_gpu_f16(vnew), kt, vt, 1, 511, hkv, max_seq, d)
    out = torch.empty((1, hq, d), dtype=torch.float16, device="cuda")
    kvhp.decode_gqa(to_gpu_f16(q), kt, vt, out, 512, hq, hkv, max_seq, d)
    sync()
    kc[:, 511], vc[:, 511] = knew[0], vnew[0]
    assert np.array_equal(from_gpu(kt), kc)
    ref = oracle.decode_attention(q.astype(np.float32), kc[None].astype(np.float32),
                                  vc[None].astype(np.float32), np.array([512], np.int32),
                                  hq, hkv, d)
    assert_attn_close(from_gpu(out).astype(np.float32), ref, "config1")


@pytest.mark.parametrize("L", [16384, 65536])
def test_config2_split_sweep_and_invariance(L):
    """BASELINE config 2 at its two long contexts (16384 and 65536; 4096 is
    in test_decode_d128_splits) with splits {1,4,16,64} and the auto plan:
    every split count matches the oracle, and the outputs of different split
    counts agree with each other."""
    rng = np.random.default_rng(2 if L == 65536 else 16)
    hq, hkv, d = 32, 8, 128
    q = oracle.normal_f16(rng, (1, hq, d))
    kc, vc = oracle.normal_f16(rng, (1, hkv, L, d)), oracle.normal_f16(rng, (1, hkv, L, d))
    ref = oracle.decode_attention(q.astype(np.float32), kc.astype(np.float32),
                                  vc.astype(np.float32), np.array([L], np.int32), hq, hkv, d,
                                  nthreads=8)
    outs = []
    for s in (1, 4, 16, 64, 0):
        note(f"config2 L={L} splits={s or 'auto'}")
        got = _run_contig(q, kc, vc, [L], hq, hkv, d, L, s)
        assert_attn_close(got, ref, f"L={L} splits={s or 'auto'}")
        outs.append(got)
    for o in outs[1:]:
        assert np.max(np.abs(o - outs[0])) <= 2e-3


def _paged_case(rng, b, lens, hq, hkv, d, with_append, fused=False):
    """Builds a paged pool from token-major K/V through the oracle's paged
    append (host), returns GPU output and oracle reference.  with_append: the
    step's new token goes in on the GPU, by the append kernel or (fused) by
    kvhp_paged_append_decode itself."""
    import torch
    lens = np.asarray(lens, np.int32)
    bt, P = make_block_tables(rng, lens + 1)
    T = int(lens.max()) + 1
    tk = oracle.normal_f16(rng, (b, T, hkv, d))
    tv = oracle.normal_f16(rng, (b, T, hkv, d))
    q = oracle.normal_f16(rng, (b, hq, d))
    pk = np.zeros((hkv, P, 16, d), np.uint16)
    pv = np.zeros_like(pk)
    for i in range(b):
        n = int(lens[i]) if with_append else int(lens[i]) + 1
        oracle.paged_append(tk[i:i + 1, :n].view(np.uint16), tv[i:i + 1, :n].view(np.uint16),
                            pk, pv, bt[i:i + 1], np.array([0], np.int32), 1, n, hkv, d)
    pk_t = to_gpu(pk.view(np.float16))
    pv_t = to_gpu(pv.view(np.float16))
    bt_t = to_gpu(bt)
    L1 = lens + 1
    out = torch.empty((b, hq, d), dtype=torch.float16, device="cuda")
    kview, vview = kvhp.paged_view(pk_t, bt_t), kvhp.paged_view(pv_t, bt_t)
    newk = np.ascontiguousarray(tk[np.arange(b), lens])
    newv = np.ascontiguousarray(tv[np.arange(b), lens])
    if with_append and fused:
        kvhp.paged_append_decode(to_gpu_f16(q), to_gpu_f16(newk), to_gpu_f16(newv), kview, vview,
                                 to_gpu(lens), to_gpu(L1), out, hq, hkv, d, int(L1.max()))
    else:
        if with_append:   # the step's new token goes in with the GPU append kernel
            kvhp.paged_append_kv(to_gpu_f16(newk[:, None]), to_gpu_f16(newv[:, None]), pk_t, pv_t,
                                 bt_t, to_gpu(lens), b, 1, hkv, d)
        kvhp.decode_attention(to_gpu_f16(q), kview, vview, to_gpu(L1), out, hq, hkv, d,
                              int(L1.max()))
    sync()
    kc = contiguous_from_tokens(tk.astype(np.float32), L1, int(L1.max()))
    vc = contiguous_from_tokens(tv.astype(np.float32), L1, int(L1.max()))
    ref = oracle.decode_attention(q.astype(np.float32), kc, vc, L1, hq, hkv, d, nthreads=8)
    return from_gpu(out).astype(np.float32), ref


@pytest.mark.parametrize("b,maxlen,hq,hkv,d", [(8, 1500, 32, 8, 128), (5, 300, 14, 2, 64),
                                               (3, 900, 32, 4, 64), (4, 200, 16, 1, 128),
                                               (80, 3000, 32, 8, 128), (70, 900, 32, 4, 64),
                                               (3, 6000, 32, 8, 128)])
def test_paged_decode_with_append(b, maxlen, hq, hkv, d):
    """Ragged paged batches (lengths from 0); batches of 8 or more run the
    balanced split list (above 64 sequences its scan takes two passes); a
    small batch of long sequences takes fixed chunks with >= 64 KB of
    partials per kv head, merged per query head."""
    rng = np.random.default_rng(b * 31 + maxlen)
    lens = rng.integers(0, maxlen, size=b)
    note(f"paged decode B={b} Hq={hq} Hkv={hkv} D={d} lens={lens.tolist()}")
    got, ref = _paged_case(rng, b, lens, hq, hkv, d, with_append=True)
    assert_attn_close(got, ref, "paged")


@pytest.mark.parametrize("case", ["one_long", "many_short", "all_empty_but_one", "mixed_300"])
def test_balanced_split_list_corners(case):
    """The automatic split mode for batches of 8 or more balances on the
    device; its corners: one long sequence among near-empty ones (its split
    count reaches the plan's slots), 300 short sequences (fewer wave slots
    per sequence than sequences), eleven sequences holding only the appended
    token beside one long one, and 300 mixed lengths (cached lengths of 0
    included).  Paged, D=64, against the oracle."""
    rng = np.random.default_rng({"one_long": 11, "many_short": 12, "all_empty_but_one": 13,
                                 "mixed_300": 14}[case])
    hq, hkv, d = 16, 4, 64
    if case == "one_long":
        lens = np.array([6000] + [1] * 8)
    elif case == "many_short":
        lens = rng.integers(1, 40, size=300)
    elif case == "all_empty_but_one":
        lens = np.array([0] * 11 + [2500])
    else:
        lens = rng.integers(0, 700, size=300)
        lens[::7] = 0
    lens = lens.astype(np.int32)
    note(f"balanced corner {case}: B={lens.size} max={int(lens.max())} sum={int(lens.sum())}")
    got, ref = _paged_case(rng, lens.size, lens, hq, hkv, d, with_append=True,
                           fused=case != "many_short")
    assert_attn_close(got, ref, case)


@pytest.mark.parametrize("seed", range(12))
def test_balanced_split_list_random_batches(seed):
    """Randomised batches through the automatic split mode: batch sizes from
    8 (the smallest balanced batch) to 200, length distributions from
    uniform to heavy-tailed (a few long sequences among many short ones),
    with empty sequences, D = 64 or 128 and G = 4 or 8, fused append on
    every other case; every output against the oracle."""
    rng = np.random.default_rng(1000 + seed)
    b = int(rng.choice([8, 9, 16, 31, 64, 200]))
    # host K/V are dense [b][max len]: wide heads only for the smaller batches
    hq, hkv, d = (32, 8, 128) if seed % 2 and b <= 31 else (16, 2, 64)
    kind = seed % 3
    if kind == 0:
        lens = rng.integers(0, 3000, size=b)
    elif kind == 1:                       # heavy tail: most short, a few long
        lens = rng.integers(0, 64, size=b)
        lens[rng.choice(b, size=max(1, b // 10), replace=False)] = rng.integers(2000, 6000)
    else:                                 # near-equal lengths around one value
        lens = rng.integers(1500, 1600, size=b)
    lens[rng.random(b) < 0.1] = 0
    lens = lens.astype(np.int32)
    note(f"balanced random seed={seed}: B={b} kind={kind} D={d} G={hq // hkv} "
         f"max={int(lens.max())} sum={int(lens.sum())}")
    got, ref = _paged_case(rng, b, lens, hq, hkv, d, with_append=True, fused=seed % 2 == 0)
    assert_attn_close(got, ref, f"seed {seed}")


@pytest.mark.parametrize("fused", [False, True])
def test_config3_paged_decode_full_size(fused):
    """BASELINE config 3 at full size: 32 sequences with seeded lengths in
    [128, 8192], 32/8 heads, D=128, 16-token pages on a seeded random
    permutation; one appended token per sequence, then decode -- as two
    calls, or as the one kvhp_paged_append_decode call the bench times."""
    rng = np.random.default_rng(3)
    lens = rng.integers(128, 8193, size=32) - 1   # + the appended token
    note(f"config3 full (fused={fused}): sum L={int(lens.sum()) + 32}")
    got, ref = _paged_case(rng, 32, lens, 32, 8, 128, with_append=True, fused=fused)
    assert_attn_close(got, ref, "config3")


@pytest.mark.parametrize("d", [16, 32, 48, 64])
def test_decode_gqa_legacy_api(d):
    """tests/test_kv_cache.cpp:98-196: single sequence over a head-major
    [Hkv][max_seq][D] cache, D in {16..64}, ctx <= 64, G 1..5, Hkv 1..3."""
    import torch
    rng = np.random.default_rng(102 + d)
    for i in range(6):
        L = 1 if i == 0 else int(rng.integers(1, 65))
        max_seq = L + int(rng.integers(0, 32))
        hkv = int(rng.integers(1, 4))
        hq = hkv * int(rng.integers(1, 6))
        q = uniform_f16(rng, (1, hq, d))
        kc, vc = uniform_f16(rng, (hkv, max_seq, d)), uniform_f16(rng, (hkv, max_seq, d))
        out = torch.empty((hq, d), dtype=torch.float16, device="cuda")
        note(f"decode_gqa D={d} case {i}: L={L} Hq={hq} Hkv={hkv}")
        kvhp.decode_gqa(to_gpu_f16(q), to_gpu_f16(kc), to_gpu_f16(vc), out, L, hq, hkv,
                        max_seq, d)
        sync()
        ref = oracle.decode_attention(q.astype(np.float32), kc[None].astype(np.float32),
                                      vc[None].astype(np.float32), np.array([L], np.int32),
                                      hq, hkv, d)
        assert_attn_close(from_gpu(out)[None].astype(np.float32), ref, f"D={d} case {i}")


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (32, 4, 64), (8, 8, 96)])
def test_decode_known_answers(hq, hkv, d):
    """Answers fixed by the mathematics, not by the oracle:
    * L = 1: softmax over one key is 1, so every query head returns V[0] of
      its KV head bit for bit;
    * all keys equal: uniform weights, the mean of the V rows;
    * one key = 12 x the shared query direction: its score leads by ~12 sqrt(D)
      (every other weight underflows to 0 in fp32), so the output is that
      key's V row bit for bit, whichever split holds it;
    * V constant per KV head: head h returns the constant of KV head h // G
      (the GQA map of decode_attention_split.cu:48-49)."""
    g = hq // hkv
    rng = np.random.default_rng(77 + d)
    note(f"decode KATs Hq={hq} Hkv={hkv} D={d}")
    # L = 1
    cap = 64
    q = oracle.normal_f16(rng, (1, hq, d))
    kc, vc = oracle.normal_f16(rng, (1, hkv, cap, d)), oracle.normal_f16(rng, (1, hkv, cap, d))
    got = _run_contig(q, kc, vc, [1], hq, hkv, d, cap)
    want = np.stack([vc[0, h // g, 0] for h in range(hq)]).astype(np.float32)
    np.testing.assert_array_equal(got[0], want, err_msg="L=1 must return V[0]")
    # all keys equal
    L = 1000
    kc = np.repeat(oracle.normal_f16(rng, (1, hkv, 1, d)), L, axis=2)
    vc = oracle.normal_f16(rng, (1, hkv, L, d))
    got = _run_contig(q, kc, vc, [L], hq, hkv, d, L, splits=4)
    want = np.stack([vc[0, h // g].astype(np.float64).mean(axis=0) for h in range(hq)])
    assert_attn_close(got[0], want, "equal keys -> mean of V")
    # one dominant key, in the middle of a split
    L, j = 777, 333
    u = oracle.normal_f16(rng, (d,))
    q = np.broadcast_to(u, (1, hq, d)).astype(np.float16)
    kc = (0.1 * oracle.normal_f16(rng, (1, hkv, L, d)).astype(np.float32)).astype(np.float16)
    kc[0, :, j] = (12.0 * u.astype(np.float32)).astype(np.float16)
    vc = oracle.normal_f16(rng, (1, hkv, L, d))
    for splits in (1, 4, 16):
        got = _run_contig(q, kc, vc, [L], hq, hkv, d, L, splits=splits)
        want = np.stack([vc[0, h // g, j] for h in range(hq)]).astype(np.float32)
        np.testing.assert_array_equal(got[0], want, err_msg=f"dominant key, splits={splits}")
    # GQA map
    L = 500
    q = oracle.normal_f16(rng, (1, hq, d))
    kc = oracle.normal_f16(rng, (1, hkv, L, d))
    vc = np.empty((1, hkv, L, d), np.float16)
    for kh in range(hkv):
        vc[0, kh] = (kh + 1) / 8.0
    got = _run_contig(q, kc, vc, [L], hq, hkv, d, L)
    want = np.stack([np.full(d, (h // g + 1) / 8.0) for h in range(hq)])
    assert_attn_close(got[0], want, "GQA head map")


@pytest.mark.parametrize("hq,hkv,d", [(24, 2, 128), (8, 8, 96), (12, 4, 256)])
def test_decode_generic_shapes(hq, hkv, d):
    """Shapes outside the MFMA kernel's template set (G=12, D=96, D=256) run
    on the generic kernel with the same results contract."""
    rng = np.random.default_rng(hq + d)
    lens = np.array([1, 77, 300], np.int32)
    cap = 300
    q = oracle.normal_f16(rng, (3, hq, d))
    kc, vc = oracle.normal_f16(rng, (3, hkv, cap, d)), oracle.normal_f16(rng, (3, hkv, cap, d))
    note(f"decode generic Hq={hq} Hkv={hkv} D={d}")
    got = _run_contig(q, kc, vc, lens, hq, hkv, d, cap)
    ref = oracle.decode_attention(q.astype(np.float32), kc.astype(np.float32),
                                  vc.astype(np.float32), lens, hq, hkv, d)
    assert_attn_close(got, ref, "generic")


def test_decode_caller_workspace_reuse_and_empty_sequences():
    """One caller workspace serves consecutive calls (the second smaller, so
    stale partials from the first are present); zero-length sequences write 0."""
    import torch
    rng = np.random.default_rng(4)
    hq, hkv, d, cap = 32, 8, 128, 3000
    ws_bytes = kvhp.decode_workspace_bytes(4, hq, hkv, d, cap, 32)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    kvhp.decode_workspace_init(ws)
    for lens in ([3000, 0, 1234, 65], [100, 7, 0]):
        b = len(lens)
        q = oracle.normal_f16(rng, (b, hq, d))
        kc, vc = oracle.normal_f16(rng, (b, hkv, cap, d)), oracle.normal_f16(rng, (b, hkv, cap, d))
        note(f"workspace reuse lens={lens}")
        got = _run_contig(q, kc, vc, lens, hq, hkv, d, cap, 32, ws)
        ref = oracle.decode_attention(q.astype(np.float32), kc.astype(np.float32),
                                      vc.astype(np.float32), np.array(lens, np.int32), hq, hkv, d)
        assert_attn_close(got, ref, f"lens={lens}")
        assert np.all(got[np.array(lens) == 0] == 0)


@pytest.mark.parametrize("balanced,d,fixed_splits", [(False, 128, 32), (False, 64, 64),
                                                      (True, 128, 0)])
def test_decode_ignores_stale_workspace_slots(balanced, d, fixed_splits):
    """The merge reads every split slot of a sequence before it knows how
    many the sequence used; slots it did not use may hold anything.  A
    caller workspace filled with NaN bytes (and one filled with huge values)
    must not change a single output: short sequences use few of the
    slots, one uses many.  Balanced: a batch of 12 in the automatic split
    mode; otherwise an explicit 32- or 64-way split (both take the
    per-query-head merge: >= 64 KB of partials per kv head)."""
    import torch
    rng = np.random.default_rng(77 + balanced + d)
    hq, hkv, cap = 32, 8, 4096
    lens = [4096, 40, 1, 300, 0, 2000] * (2 if balanced else 1)
    b = len(lens)
    splits = fixed_splits
    ws_bytes = kvhp.decode_workspace_bytes(b, hq, hkv, d, cap, splits)
    q = oracle.normal_f16(rng, (b, hq, d))
    kc, vc = oracle.normal_f16(rng, (b, hkv, cap, d)), oracle.normal_f16(rng, (b, hkv, cap, d))
    ref = oracle.decode_attention(q.astype(np.float32), kc.astype(np.float32),
                                  vc.astype(np.float32), np.array(lens, np.int32), hq, hkv, d)
    outs = []
    for fill in (0xFF, 0x7F):          # NaN bytes; 3.4e38-ish floats
        ws = torch.full((ws_bytes,), fill, dtype=torch.uint8, device="cuda")
        note(f"stale workspace fill=0x{fill:02x} balanced={balanced} d={d}")
        got = _run_contig(q, kc, vc, lens, hq, hkv, d, cap, splits, ws)
        assert np.isfinite(got).all(), f"fill 0x{fill:02x}: non-finite output"
        assert_attn_close(got, ref, f"fill 0x{fill:02x}")
        outs.append(got)
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("hq,hkv,d,tiles", [(32, 8, 128, 1), (32, 4, 64, 1), (12, 4, 96, 1),
                                            (32, 8, 128, 10), (32, 4, 64, 10)])
def test_paged_append_decode_matches_separate_calls(hq, hkv, d, tiles):
    """kvhp_paged_append_decode (one call: the covering split writes the new
    row into its page and attends it from registers) against
    kvhp_paged_append_kv followed by kvhp_decode_attention, bit for bit on
    both the pools and the outputs.  Ragged batch: an empty sequence, rows
    on page boundaries, a new position past the attended length (written,
    not attended), a new position on an unallocated page (dropped; no
    attended key lies on an unallocated page, whose reads would alias
    physical page 0 while other sequences write their rows), and an idle
    row (position -1: nothing written, its cached keys attended).
    D=96 runs the fallback (append kernel, then the generic decode).  The
    pattern tiled 10 times (80 sequences) runs the balanced split list."""
    import torch
    rng = np.random.default_rng(500 + d + tiles)
    lens = np.tile(np.array([1000, 0, 1, 15, 16, 300, 2047, 700], np.int32), tiles)  # cached
    b = lens.size
    bt, P = make_block_tables(rng, lens + 8)
    pos = lens.copy()
    seq = lens + 1
    pos[5::8] = lens[5::8] + 4    # written, beyond the attended keys
    seq[5::8] = lens[5::8]
    pos[7::8] = -1                # idle: nothing written
    seq[7::8] = lens[7::8]
    for i in range(4, b, 8):      # row 16 starts a page that has no id: the write is
        bt[i, pos[i] // 16] = -1  # dropped, and the 16 attended keys stay on page 0
        seq[i] = lens[i]
    pool_k = to_gpu_f16(oracle.normal_f16(rng, (hkv, P, 16, d)))
    pool_v = to_gpu_f16(oracle.normal_f16(rng, (hkv, P, 16, d)))
    k_new = to_gpu_f16(oracle.normal_f16(rng, (b, hkv, d)))
    v_new = to_gpu_f16(oracle.normal_f16(rng, (b, hkv, d)))
    q = to_gpu_f16(oracle.normal_f16(rng, (b, hq, d)))
    bt_t, pos_t, seq_t = to_gpu(bt), to_gpu(pos), to_gpu(seq)
    cap = int(seq.max())
    note(f"append_decode Hq={hq} Hkv={hkv} D={d} lens={lens.tolist()}")

    pk1, pv1 = pool_k.clone(), pool_v.clone()
    out1 = torch.full((b, hq, d), float("nan"), dtype=torch.float16, device="cuda")
    kvhp.paged_append_kv(k_new.view(b, 1, hkv, d), v_new.view(b, 1, hkv, d), pk1, pv1, bt_t, pos_t,
                         b, 1, hkv, d)
    kvhp.decode_attention(q, kvhp.paged_view(pk1, bt_t), kvhp.paged_view(pv1, bt_t), seq_t, out1,
                          hq, hkv, d, cap)
    pk2, pv2 = pool_k.clone(), pool_v.clone()
    out2 = torch.full((b, hq, d), float("nan"), dtype=torch.float16, device="cuda")
    kvhp.paged_append_decode(q, k_new, v_new, kvhp.paged_view(pk2, bt_t),
                             kvhp.paged_view(pv2, bt_t), pos_t, seq_t, out2, hq, hkv, d, cap)
    sync()
    assert torch.equal(pk1, pk2) and torch.equal(pv1, pv2), "pools differ"
    assert torch.equal(out1, out2), "outputs differ"
    assert not torch.equal(pk2, pool_k), "nothing was appended"


@pytest.mark.parametrize("hq,hkv,d,tiles", [(32, 8, 64, 1), (32, 8, 128, 1), (12, 4, 96, 1),
                                            (32, 8, 128, 3), (32, 4, 64, 2)])
def test_strided_append_decode_matches_separate_calls(hq, hkv, d, tiles):
    """kvhp_append_decode on strided views (the reference KVCache layout,
    [B][Hkv][cap][D]): the covering split writes row positions[b] and attends
    it; against the row written separately followed by kvhp_decode_attention,
    bit for bit on both caches and the outputs.  Ragged batch: an empty
    sequence, a new position past the attended length (written, not
    attended), one at the last row of the capacity, one past it (dropped, as
    the reference append drops positions past max_seq), and an idle row
    (position -1: nothing written, its cached keys attended).  D=96 runs the
    fallback (append kernel, then the generic decode); the pattern tiled 3
    times (21 sequences) runs the balanced split list."""
    import torch
    rng = np.random.default_rng(600 + d + tiles)
    cap = 2100
    lens = np.tile(np.array([1000, 0, 511, 300, 2099, 2050, 700], np.int32), tiles)  # cached
    b = lens.size
    pos = lens.copy()
    seq = lens + 1
    seq[1::7] = 0                  # empty: row 0 written, output zeros
    pos[3::7] = lens[3::7] + 4     # written, beyond the attended keys
    seq[3::7] = lens[3::7]
    pos[5::7] = cap + 7            # past the capacity: dropped
    seq[5::7] = lens[5::7]
    pos[6::7] = -1                 # idle: nothing written
    seq[6::7] = lens[6::7]
    kc = to_gpu_f16(oracle.normal_f16(rng, (b, hkv, cap, d)))
    vc = to_gpu_f16(oracle.normal_f16(rng, (b, hkv, cap, d)))
    k_new = to_gpu_f16(oracle.normal_f16(rng, (b, hkv, d)))
    v_new = to_gpu_f16(oracle.normal_f16(rng, (b, hkv, d)))
    q = to_gpu_f16(oracle.normal_f16(rng, (b, hq, d)))
    pos_t, seq_t = to_gpu(pos), to_gpu(seq)
    note(f"strided append_decode Hq={hq} Hkv={hkv} D={d} lens={lens.tolist()}")

    def views(k, v):
        return (kvhp.strided_view(k, hkv * cap * d, cap * d, d),
                kvhp.strided_view(v, hkv * cap * d, cap * d, d))

    k1, v1 = kc.clone(), vc.clone()
    for i in range(b):
        if 0 <= pos[i] < cap:
            k1[i, :, pos[i]] = k_new[i]
            v1[i, :, pos[i]] = v_new[i]
    out1 = torch.full((b, hq, d), float("nan"), dtype=torch.float16, device="cuda")
    kv1, vv1 = views(k1, v1)
    kvhp.decode_attention(q, kv1, vv1, seq_t, out1, hq, hkv, d, cap)
    k2, v2 = kc.clone(), vc.clone()
    out2 = torch.full((b, hq, d), float("nan"), dtype=torch.float16, device="cuda")
    kv2, vv2 = views(k2, v2)
    kvhp.append_decode(q, k_new, v_new, kv2, vv2, pos_t, seq_t, out2, hq, hkv, d, cap)
    sync()
    assert torch.equal(k1, k2) and torch.equal(v1, v2), "caches differ"
    assert torch.equal(out1, out2), "outputs differ"
    assert not torch.equal(k2, kc), "nothing was appended"
    if tiles == 1:   # and against the oracle
        ref = oracle.decode_attention(q.cpu().numpy().astype(np.float32),
                                      k2.cpu().numpy().astype(np.float32),
                                      v2.cpu().numpy().astype(np.float32), seq, hq, hkv, d,
                                      nthreads=8)
        assert_attn_close(out2.cpu().numpy(), ref, "strided append_decode")


@pytest.mark.parametrize("stride_s", [(1 << 23) + 64, (1 << 24) + 8])
def test_decode_row_pitch_beyond_24_bits(stride_s):
    """A strided view whose row pitch needs more than 24 bits (stride_s
    >= 2^23 halfs, still inside the fast kernel's stride_s < 2^26): the
    split kernel's in-page row offsets must keep the pitch's high bits.  L=17
    rows of one KV head (G=4, D=128), each row stride_s halfs apart, rows 1 and
    16 of each page distinct, against the oracle."""
    import torch
    rng = np.random.default_rng(stride_s % 1000)
    hq, hkv, d, L = 4, 1, 128, 17
    q = oracle.normal_f16(rng, (1, hq, d))
    rows_k = oracle.normal_f16(rng, (L, d))
    rows_v = oracle.normal_f16(rng, (L, d))
    n = (L - 1) * stride_s + d
    note(f"decode row pitch {stride_s} halfs ({n * 2 / 2**20:.0f} MiB per tensor)")
    kt = torch.zeros(n, dtype=torch.float16, device="cuda")
    vt = torch.zeros(n, dtype=torch.float16, device="cuda")
    idx = (torch.arange(L, device="cuda")[:, None] * stride_s +
           torch.arange(d, device="cuda")[None, :]).reshape(-1)
    kt[idx] = to_gpu_f16(rows_k).reshape(-1)
    vt[idx] = to_gpu_f16(rows_v).reshape(-1)
    kview = kvhp.strided_view(kt, 0, 0, stride_s)
    vview = kvhp.strided_view(vt, 0, 0, stride_s)
    out = torch.full((1, hq, d), float("nan"), dtype=torch.float16, device="cuda")
    kvhp.decode_attention(to_gpu_f16(q), kview, vview, to_gpu(np.array([L], np.int32)), out,
                          hq, hkv, d, L)
    sync()
    ref = oracle.decode_attention(q.astype(np.float32), rows_k[None, None].astype(np.float32),
                                  rows_v[None, None].astype(np.float32),
                                  np.array([L], np.int32), hq, hkv, d)
    assert_attn_close(from_gpu(out).astype(np.float32), ref, f"stride_s={stride_s}")
    del kt, vt
    torch.cuda.empty_cache()


def test_paged_append_decode_graph_replays():
    """The serving step (kvhp_paged_append_decode) captured in a HIP graph, as
    the bench times it: two batches (ragged, 40 sequences: the balanced
    split list) in one graph over a shared workspace, replayed three times
    with new queries each time and an eager step of a third batch on the
    same workspace between the replays; every replay's outputs and pools
    equal the eager call's bit for bit."""
    import torch
    rng = np.random.default_rng(909)
    hq, hkv, d = 32, 8, 128

    def batch(seed_lens):
        lens = rng.integers(0, 3000, size=40).astype(np.int32)
        lens[:3] = seed_lens
        b = lens.size
        bt, P = make_block_tables(rng, lens + 8)
        return {"b": b, "bt": to_gpu(bt), "pos": to_gpu(lens), "seq": to_gpu(lens + 1),
                "cap": int(lens.max()) + 1,
                "pk": to_gpu_f16(oracle.normal_f16(rng, (hkv, P, 16, d))),
                "pv": to_gpu_f16(oracle.normal_f16(rng, (hkv, P, 16, d))),
                "kn": to_gpu_f16(oracle.normal_f16(rng, (b, hkv, d))),
                "vn": to_gpu_f16(oracle.normal_f16(rng, (b, hkv, d))),
                "q": to_gpu_f16(oracle.normal_f16(rng, (b, hq, d))),
                "out": torch.zeros((b, hq, d), dtype=torch.float16, device="cuda")}

    A, B, C = batch([0, 16, 2999]), batch([1, 15, 64]), batch([7, 300, 2048])
    cap = max(x["cap"] for x in (A, B, C))
    ws = torch.zeros(kvhp.decode_workspace_bytes(40, hq, hkv, d, cap), dtype=torch.uint8,
                     device="cuda")

    def step(x, pk=None, pv=None, out=None):
        pk = x["pk"] if pk is None else pk
        pv = x["pv"] if pv is None else pv
        out = x["out"] if out is None else out
        kvhp.paged_append_decode(x["q"], x["kn"], x["vn"], kvhp.paged_view(pk, x["bt"]),
                                 kvhp.paged_view(pv, x["bt"]), x["pos"], x["seq"], out, hq, hkv,
                                 d, cap, 0, ws)

    step(A)
    step(B)
    sync()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
        step(A)
        step(B)
    torch.cuda.current_stream().wait_stream(s)
    sync()
    for r in range(3):
        note(f"graph replay {r}")
        for x in (A, B):
            x["q"].copy_(to_gpu_f16(oracle.normal_f16(rng, (x["b"], hq, d))))
            x["out"].fill_(float("nan"))
        g.replay()
        sync()
        for x in (A, B):
            # the append is idempotent (same rows at the same positions), so
            # the eager call on copies of the current pools is the reference
            pk, pv = x["pk"].clone(), x["pv"].clone()
            ref = torch.full_like(x["out"], float("nan"))
            step(x, pk, pv, ref)
            sync()
            assert torch.equal(ref, x["out"]), f"replay {r}: outputs differ"
            assert torch.equal(pk, x["pk"]) and torch.equal(pv, x["pv"]), f"replay {r}: pools differ"
        step(C)   # other work on the same workspace between the replays
        sync()
