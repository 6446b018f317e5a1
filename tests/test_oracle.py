"""Pins the CPU oracle (oracle/kvhp_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something that is not its own formula:
  - the reference's own src/cpu/ops.cpp compiled under oracle/_ref (bit-exact),
  - golden fixtures written from that build (tests/golden/ref_cpu_ops.npz),
  - the reference's known-answer tests (tests/test_cpu_ops.cpp:65-136),
  - invariants and closed forms chosen so a dropped term, wrong sign, wrong
    GQA index or transposed operand fails (see each test's docstring).
"""
import itertools
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_cpu_ops.npz")


def f16(rng, shape, scale=1.0):
    return oracle.normal_f16(rng, shape, scale).astype(np.float32)


# --------------------------------------------------------------- fp16 ----
def test_f16_decode_all_patterns():
    """Every binary16 pattern decodes exactly as numpy's IEEE float16 does."""
    bits = np.arange(65536, dtype=np.uint16)
    ours = oracle.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(ours[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(ours[np.isnan(ref)]))
    assert np.array_equal(ours[np.isinf(ref)], ref[np.isinf(ref)])


def test_f16_encode_ties_and_boundaries():
    """RNE encode at every half value, every midpoint (ties to even) and one
    float32 ulp either side of each midpoint, plus overflow and underflow."""
    bits = np.arange(0, 0x7C00, dtype=np.uint16)          # finite non-negative
    vals = bits.view(np.float16).astype(np.float64)
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)  # exact in fp32
    lo = np.nextafter(mids, np.float32(-np.inf))
    hi = np.nextafter(mids, np.float32(np.inf))
    extra = np.array([65504, 65519.99, 65520, 1e9, 2.0**-24, 2.0**-25, 2.0**-25 * 1.0001,
                      2.0**-26, 1e-30, 0.0], np.float32)
    x = np.concatenate([vals.astype(np.float32), mids, lo, hi, extra])
    x = np.concatenate([x, -x])
    ours = oracle.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_f16_encode_random_bits():
    rng = np.random.default_rng(11)
    x = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[np.isfinite(x)]
    assert np.array_equal(oracle.f32_to_f16_bits(x), x.astype(np.float16).view(np.uint16))


# ------------------------------------------------- attention vs reference --
@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no reference tree)")
@pytest.mark.parametrize("s,hq,hkv,d", [(1, 14, 2, 64), (23, 14, 2, 64), (40, 8, 2, 128),
                                        (31, 32, 8, 128), (19, 6, 3, 16), (64, 4, 4, 64)])
def test_causal_bit_exact_vs_reference_build(s, hq, hkv, d):
    rng = np.random.default_rng(1000 + s * 7 + hq)
    q, k, v = f16(rng, (s, hq, d)), f16(rng, (s, hkv, d)), f16(rng, (s, hkv, d))
    ours = oracle.causal_gqa(q, k, v, hq, hkv, d, nthreads=4)
    ref = oracle.ref_causal_gqa(q, k, v, hq, hkv, d)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_causal_rowlist_equals_full_rows():
    """causal_gqa_rowlist (scattered rows of long prompts) returns exactly the
    listed rows of the full causal_gqa, in the listed order, with repeats;
    out-of-range rows are refused."""
    rng = np.random.default_rng(90)
    s, hq, hkv, d = 97, 8, 2, 64
    q, k, v = f16(rng, (s, hq, d)), f16(rng, (s, hkv, d)), f16(rng, (s, hkv, d))
    full = oracle.causal_gqa(q, k, v, hq, hkv, d)
    rows = [96, 0, 31, 32, 63, 64, 5, 5, 95]
    got = oracle.causal_gqa_rowlist(q, k, v, hq, hkv, d, rows, nthreads=3)
    assert np.array_equal(got.view(np.uint32), full[rows].view(np.uint32))
    assert oracle.causal_gqa_rowlist(q, k, v, hq, hkv, d, []).shape == (0, hq, d)
    with pytest.raises(ValueError):
        oracle.causal_gqa_rowlist(q, k, v, hq, hkv, d, [s])


def _golden():
    return np.load(GOLDEN, allow_pickle=False)


def test_causal_golden_fixtures():
    g = _golden()
    seeds = sorted({k.split("_")[1] for k in g.files if k.startswith("causal_")})
    assert len(seeds) >= 7
    for sd in seeds:
        s, hq, hkv, d = (int(x) for x in g[f"causal_{sd}_shape"])
        q = g[f"causal_{sd}_q"].astype(np.float32)
        k = g[f"causal_{sd}_k"].astype(np.float32)
        v = g[f"causal_{sd}_v"].astype(np.float32)
        ours = oracle.causal_gqa(q, k, v, hq, hkv, d)
        assert np.array_equal(ours.view(np.uint32), g[f"causal_{sd}_out"].view(np.uint32)), sd


def test_supporting_ops_golden_fixtures():
    g = _golden()
    assert np.array_equal(oracle.rmsnorm(g["rmsnorm_x"], g["rmsnorm_w"], 1e-5),
                          g["rmsnorm_out"])
    assert np.array_equal(oracle.matmul_transB(g["matmul_a"], g["matmul_b"], nthreads=3),
                          g["matmul_out"])
    start, theta = g["rope_start_theta"]
    rq, rk = oracle.apply_rope(g["rope_q"], g["rope_k"], 4, 2, 64, int(start), float(theta))
    assert np.array_equal(rq, g["rope_q_out"]) and np.array_equal(rk, g["rope_k_out"])
    assert np.array_equal(oracle.swiglu(g["swiglu_gate"], g["swiglu_up"]), g["swiglu_out"])


@pytest.mark.parametrize("m,k,n", [(4, 64, 8), (5, 130, 13), (9, 2048, 33), (256, 100, 7),
                                   (257, 700, 17), (300, 2048, 2560), (37, 5632, 24)])
def test_matmul_vector_form_bit_exact(m, k, n):
    """The AVX2 form of the blocked matmul (4 x 8 tiles, rows in blocks of
    256) equals the scalar restatement of ops.cpp:76-114 bit for bit at tile,
    block and 64-wide K-block remainders, and the reference build where it is
    present."""
    rng = np.random.default_rng(m * 31 + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)
    vec = oracle.matmul_transB(a, b, nthreads=4)
    sca = oracle.matmul_transB(a, b, nthreads=4, scalar=True)
    assert np.array_equal(vec.view(np.uint32), sca.view(np.uint32))
    if oracle.ref_available() and m * k * n < 5e7:
        ref = oracle.matmul_transB(a, b, use_ref=True)
        assert np.array_equal(vec.view(np.uint32), ref.view(np.uint32))


def test_causal_kat_reference():
    """tests/test_cpu_ops.cpp:112-136: q=k=0.5, v[0]=1, v[1]=2 -> row 0 = v[0];
    row 1 sees two equal scores -> (1+2)/2."""
    q = np.full((2, 2, 4), 0.5, np.float32)
    k = np.full((2, 1, 4), 0.5, np.float32)
    v = np.zeros((2, 1, 4), np.float32)
    v[0], v[1] = 1.0, 2.0
    out = oracle.causal_gqa(q, k, v, 2, 1, 4)
    assert np.all(out[0] == 1.0)
    assert np.allclose(out[1], 1.5, atol=1e-6)


def test_rope_kat_reference():
    """tests/test_cpu_ops.cpp:65-96: identity at pos 0; cos1-sin1 / cos1+sin1 at pos 1."""
    q = np.ones((3, 2, 8), np.float32)
    k = np.ones((3, 1, 8), np.float32)
    rq, rk = oracle.apply_rope(q, k, 2, 1, 8, 0, 10000.0)
    assert np.allclose(rq[0], 1.0) and np.allclose(rk[0], 1.0)
    assert abs(rq[1, 0, 0] - (np.cos(1.0) - np.sin(1.0))) < 1e-5
    assert abs(rq[1, 0, 4] - (np.cos(1.0) + np.sin(1.0))) < 1e-5


def test_swiglu_rmsnorm_kat():
    out = oracle.swiglu(np.array([-2, 0, 2], np.float32), np.array([1.5, 3, -0.5], np.float32))
    assert out[1] == 0.0
    assert abs(out[2] - 2.0 / (1 + np.exp(-2.0)) * -0.5) < 1e-6
    x = np.array([[3.0, 4.0]], np.float32)  # rms = sqrt(12.5)
    r = oracle.rmsnorm(x, np.ones(2, np.float32), 0.0)
    assert np.allclose(r, x / np.sqrt(12.5), rtol=1e-6)


# ------------------------------------------------------------- decode ----
def _contig_cache(rng, b, hkv, cap, d):
    return f16(rng, (b, hkv, cap, d)), f16(rng, (b, hkv, cap, d))


def test_decode_is_last_causal_row():
    """Decode over L keys is, bit for bit, the last row of causal attention
    whose final query is the decode query (ops.cpp:242-282)."""
    rng = np.random.default_rng(5)
    hq, hkv, d, L = 8, 2, 64, 37
    q_all, k, v = f16(rng, (L, hq, d)), f16(rng, (L, hkv, d)), f16(rng, (L, hkv, d))
    causal = oracle.causal_gqa(q_all, k, v, hq, hkv, d)
    kc = np.ascontiguousarray(k.transpose(1, 0, 2))[None]
    vc = np.ascontiguousarray(v.transpose(1, 0, 2))[None]
    dec = oracle.decode_attention(q_all[L - 1][None], kc, vc, np.array([L], np.int32), hq, hkv, d)
    assert np.array_equal(dec[0].view(np.uint32), causal[L - 1].view(np.uint32))


def test_decode_kats():
    """L=1 -> V[0] exactly; equal keys -> mean of V; one dominant key -> its V
    row; GQA head map kv = q_head // G checked head by head."""
    rng = np.random.default_rng(6)
    hq, hkv, d, cap = 4, 2, 16, 9
    q = f16(rng, (1, hq, d))
    k, v = _contig_cache(rng, 1, hkv, cap, d)
    out = oracle.decode_attention(q, k, v, np.array([1], np.int32), hq, hkv, d)
    for h in range(hq):
        assert np.array_equal(out[0, h], v[0, h // 2, 0])
    keq = np.repeat(k[:, :, :1], cap, axis=2)
    out = oracle.decode_attention(q, keq, v, np.array([cap], np.int32), hq, hkv, d)
    for h in range(hq):
        assert np.allclose(out[0, h], v[0, h // 2].astype(np.float64).mean(0), atol=2e-6)
    kdom = np.zeros_like(k)
    for h in range(hkv):
        kdom[0, h, 5] = 64.0 * q[0, 2 * h]  # head 2h sees key 5 dominate
    out = oracle.decode_attention(q, kdom, v, np.array([cap], np.int32), hq, hkv, d)
    for h in range(hkv):
        assert np.allclose(out[0, 2 * h], v[0, h, 5], atol=1e-6)
    out = oracle.decode_attention(q, k, v, np.array([0], np.int32), hq, hkv, d)
    assert np.all(out == 0)


def test_decode_textbook_softmax():
    """Against a float64 numpy softmax(qK^T/sqrt(D))V written independently."""
    rng = np.random.default_rng(7)
    b, hq, hkv, d, cap = 3, 6, 2, 32, 50
    q = f16(rng, (b, hq, d))
    k, v = _contig_cache(rng, b, hkv, cap, d)
    lens = np.array([50, 1, 23], np.int32)
    out = oracle.decode_attention(q, k, v, lens, hq, hkv, d, nthreads=3)
    for bi in range(b):
        for h in range(hq):
            kk = k[bi, h // (hq // hkv), :lens[bi]].astype(np.float64)
            vv = v[bi, h // (hq // hkv), :lens[bi]].astype(np.float64)
            s = kk @ q[bi, h].astype(np.float64) / np.sqrt(d)
            p = np.exp(s - s.max())
            ref = (p / p.sum()) @ vv
            assert np.allclose(out[bi, h], ref, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("chunk", [1, 3, 16, 64, 1000])
def test_splitk_invariant_to_split_count(chunk):
    rng = np.random.default_rng(8)
    b, hq, hkv, d, cap = 2, 8, 2, 64, 300
    q = f16(rng, (b, hq, d))
    k, v = _contig_cache(rng, b, hkv, cap, d)
    lens = np.array([300, 129], np.int32)
    ref = oracle.decode_attention(q, k, v, lens, hq, hkv, d)
    out = oracle.decode_attention_splitk(q, k, v, lens, hq, hkv, d, chunk, nthreads=2)
    assert np.allclose(out, ref, atol=2e-6, rtol=2e-6)


def test_lse_merge_brute_force_all_split_points():
    """Every composition of a short key range into contiguous splits merges
    back to the unsplit result; empty splits carry zero weight."""
    rng = np.random.default_rng(9)
    d, L = 8, 6
    q = f16(rng, (d,))
    k, v = f16(rng, (L, d)), f16(rng, (L, d))
    ref = oracle.decode_attention(q[None, None], k[None, None], v[None, None],
                                  np.array([L], np.int32), 1, 1, d)[0, 0]
    for r in range(L):
        for cuts in itertools.combinations(range(1, L), r):
            bounds = (0,) + cuts + (L,)
            parts = [oracle.split_partial(q, k, v, bounds[i], bounds[i + 1])
                     for i in range(len(bounds) - 1)]
            parts.append(oracle.split_partial(q, k, v, 3, 3))  # an empty split
            ms = np.array([p[0] for p in parts], np.float32)
            ls = np.array([p[1] for p in parts])
            os_ = np.stack([p[2] for p in parts])
            assert np.allclose(oracle.lse_merge(ms, ls, os_), ref, atol=2e-6), bounds
    empty = oracle.split_partial(q, k, v, 2, 2)
    assert empty[0] == -np.inf and empty[1] == 0.0
    assert np.all(oracle.lse_merge(np.array([empty[0]], np.float32), np.array([0.0]),
                                   empty[2][None]) == 0)


def test_lse_merge_single_partial_is_normalisation():
    rng = np.random.default_rng(10)
    o = rng.standard_normal((1, 5))
    out = oracle.lse_merge(np.array([3.5], np.float32), np.array([2.0]), o)
    assert np.allclose(out, (o[0] / 2.0).astype(np.float32), rtol=1e-7)


# -------------------------------------------------------- KV movement ----
def _bits(rng, shape):
    return oracle.normal_f16(rng, shape, 2.0).view(np.uint16)


def test_append_matches_reference_index_map():
    """Reference test shapes (tests/test_kv_cache.cpp:49-94): dst[h, start+t] ==
    src[t, h] (a numpy transpose, an independent statement of the map);
    everything else untouched; positions >= max_seq dropped."""
    rng = np.random.default_rng(101)
    for i in range(25):
        t = 1 if i == 0 else int(rng.integers(1, 38))
        start = 0 if i == 0 else int(rng.integers(0, 50))
        hkv = int(rng.integers(1, 5))
        max_seq = start + t + int(rng.integers(0, 30)) - (3 if i % 5 == 4 else 0)
        max_seq = max(max_seq, 1)
        d = 16 * int(rng.integers(1, 5))
        sk, sv = _bits(rng, (t, hkv, d)), _bits(rng, (t, hkv, d))
        dk = np.zeros((hkv, max_seq, d), np.uint16)
        dv = np.zeros((hkv, max_seq, d), np.uint16)
        oracle.append_kv(sk, sv, dk, dv, t, start, hkv, max_seq, d)
        ek = np.zeros_like(dk)
        ev = np.zeros_like(dv)
        n = max(0, min(t, max_seq - start))
        ek[:, start:start + n] = sk[:n].transpose(1, 0, 2)
        ev[:, start:start + n] = sv[:n].transpose(1, 0, 2)
        assert np.array_equal(dk, ek) and np.array_equal(dv, ev)


def test_paged_identity_table_equals_contiguous_layout():
    """With block table [0,1,2,..] the pool [Hkv][P][16][D] is byte-identical
    to the reference's contiguous [Hkv][max_seq][D] (kv_cache.h:9-11)."""
    rng = np.random.default_rng(102)
    hkv, d, pages, t, start = 3, 32, 6, 41, 37
    sk, sv = _bits(rng, (t, hkv, d)), _bits(rng, (t, hkv, d))
    ck = np.zeros((hkv, pages * 16, d), np.uint16)
    cv = np.zeros_like(ck)
    oracle.append_kv(sk, sv, ck, cv, t, start, hkv, pages * 16, d)
    pk = np.zeros((hkv, pages, 16, d), np.uint16)
    pv = np.zeros_like(pk)
    bt = np.arange(pages, dtype=np.int32)[None]
    oracle.paged_append(sk, sv, pk, pv, bt, np.array([start], np.int32), 1, t, hkv, d)
    assert np.array_equal(pk.reshape(ck.shape), ck) and np.array_equal(pv.reshape(cv.shape), cv)


def test_paged_append_gather_round_trip_random_tables():
    rng = np.random.default_rng(103)
    b, hkv, d = 5, 2, 64
    lens = rng.integers(1, 100, size=b).astype(np.int32)
    maxp = int((lens.max() + 15) // 16) + 1
    need = int(sum((L + 15) // 16 for L in lens))
    P = need + 7
    perm = rng.permutation(P).astype(np.int32)
    bt = np.full((b, maxp), -1, np.int32)
    o = 0
    for i, L in enumerate(lens):
        n = (L + 15) // 16
        bt[i, :n] = perm[o:o + n]
        o += n
    T = int(lens.max())
    sk, sv = _bits(rng, (b, T, hkv, d)), _bits(rng, (b, T, hkv, d))
    pk = np.zeros((hkv, P, 16, d), np.uint16)
    pv = np.zeros_like(pk)
    # append each sequence's first lens[b] tokens: use per-sequence calls
    for i in range(b):
        oracle.paged_append(sk[i, :lens[i]], sv[i, :lens[i]], pk, pv, bt[i:i + 1],
                            np.array([0], np.int32), 1, int(lens[i]), hkv, d)
    gk, gv = oracle.paged_gather(pk, pv, bt, lens, T + 3)
    for i in range(b):
        L = lens[i]
        assert np.array_equal(gk[i, :, :L], sk[i, :L].transpose(1, 0, 2))
        assert np.array_equal(gv[i, :, :L], sv[i, :L].transpose(1, 0, 2))
        assert np.all(gk[i, :, L:] == 0) and np.all(gv[i, :, L:] == 0)


def test_paged_append_drop_rules():
    """Out-of-capacity positions and invalid page ids are dropped, not wrapped."""
    hkv, d = 1, 8
    pk = np.zeros((hkv, 2, 16, d), np.uint16)
    pv = np.zeros_like(pk)
    src = np.full((1, 3, hkv, d), 7, np.uint16)
    bt = np.array([[1, -1]], np.int32)
    oracle.paged_append(src, src, pk, pv, bt, np.array([15], np.int32), 1, 3, hkv, d)
    assert np.all(pk[0, 1, 15] == 7)            # pos 15 -> page 1, slot 15
    assert np.count_nonzero(pk) == d            # pos 16 (id -1), 17 dropped
    bt = np.array([[0]], np.int32)
    pk[:] = 0
    oracle.paged_append(src, src, pk, pv, bt, np.array([15], np.int32), 1, 3, hkv, d)
    assert np.count_nonzero(pk) == d            # pos >= max_pages*16 dropped
