"""GPU parity of the model operators (serving-engine_amd/csrc/model_ops.hip)
against the oracle's restatement of the reference CPU ops (src/cpu/ops.cpp:
RMSNorm :26-51, matmul :53-114, RoPE :165-221, SwiGLU :286-297).

As in the reference's own kernel tests (docs/GATES.md: ">= 20 random shapes
including sizes that are not tile multiples and length-1 sequences"), every
op runs on random shapes that include the config-5 sizes (K = 2048, 5632)
and odd ones.  The reference GPU path stores each projection and the RMSNorm
output in fp16, so the oracle side rounds at the same points.  Tolerance:
|g - r| <= 1e-3 + 2e-3 |r| per element (fp16 output rounding plus fp32 vs
double accumulation order).
"""
import numpy as np
import pytest

import kvhp
import oracle
from gpu_util import to_gpu

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

ATOL, RTOL = 1e-3, 2e-3


def _close(got, ref, what):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} out of tolerance, max abs {err.max():.3g}"


def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def _cpu(t):
    return t.float().cpu().numpy()


GEMV_SHAPES = [(1, 8), (7, 24), (64, 512), (100, 2048), (2048, 2048), (2560, 2048), (33, 5632),
               (2048, 5632), (300, 1000), (5, 2056), (129, 4096), (17, 64), (513, 2048),
               (32000, 2048), (1, 2048), (8, 5632), (250, 136), (96, 3000), (4, 16), (3, 520)]


@pytest.mark.parametrize("n,k", GEMV_SHAPES)
def test_gemv_and_residual(n, k):
    rng = np.random.default_rng(n * 7919 + k)
    W = oracle.normal_f16(rng, (n, k), 0.02)
    x = oracle.normal_f16(rng, (k,))
    r = oracle.normal_f16(rng, (n,))
    ref = oracle.matmul_transB(x[None, :].astype(np.float32), W.astype(np.float32), nthreads=8)[0]
    Wd, xd, rd = to_gpu(W), to_gpu(x), to_gpu(r)
    y = torch.empty(n, dtype=torch.float16, device="cuda")
    kvhp.gemv(Wd, xd, y, n, k)
    torch.cuda.synchronize()
    _close(_cpu(y), _f16(ref), f"gemv {n}x{k}")
    y2 = rd.clone()  # in place: y = W x + y
    kvhp.gemv_residual(Wd, xd, y2, y2, n, k)
    torch.cuda.synchronize()
    _close(_cpu(y2), _f16(ref + r.astype(np.float32)), f"gemv_residual {n}x{k}")


@pytest.mark.parametrize("n,k", [(64, 512), (2048, 2048), (32000, 2048), (100, 5632), (9, 40)])
def test_rmsnorm_gemv(n, k):
    rng = np.random.default_rng(n + 31 * k)
    W = oracle.normal_f16(rng, (n, k), 0.02)
    x = oracle.normal_f16(rng, (k,))
    w = (1.0 + oracle.normal_f16(rng, (k,), 0.1).astype(np.float32)).astype(np.float16)
    xn = _f16(oracle.rmsnorm(x[None, :], w, 1e-5))
    ref = oracle.matmul_transB(xn, W.astype(np.float32), nthreads=8)[0]
    Wd, xd, wd = to_gpu(W), to_gpu(x), to_gpu(w)
    y16 = torch.empty(n, dtype=torch.float16, device="cuda")
    y32 = torch.empty(n, dtype=torch.float32, device="cuda")
    kvhp.rmsnorm_gemv(Wd, xd, wd, 1e-5, n, k, y16=y16)
    kvhp.rmsnorm_gemv(Wd, xd, wd, 1e-5, n, k, y32=y32)
    torch.cuda.synchronize()
    _close(_cpu(y16), _f16(ref), "rmsnorm_gemv fp16")
    _close(y32.cpu().numpy(), ref, "rmsnorm_gemv fp32")


@pytest.mark.parametrize("n,k", [(5632, 2048), (64, 2048), (37, 2048), (100, 320), (1, 2048)])
def test_rmsnorm_gemv_swiglu(n, k):
    rng = np.random.default_rng(n * 3 + k)
    Wgu = oracle.normal_f16(rng, (2 * n, k), 0.02)
    x = oracle.normal_f16(rng, (k,))
    w = np.ones(k, np.float16)
    xn = _f16(oracle.rmsnorm(x[None, :], w, 1e-5))
    gu = _f16(oracle.matmul_transB(xn, Wgu.astype(np.float32), nthreads=8)[0])
    ref = oracle.swiglu(gu[:n], gu[n:])
    out = torch.empty(n, dtype=torch.float16, device="cuda")
    kvhp.rmsnorm_gemv_swiglu(to_gpu(Wgu), to_gpu(x), to_gpu(w), 1e-5, out, n, k)
    torch.cuda.synchronize()
    _close(_cpu(out), _f16(ref), f"rmsnorm_gemv_swiglu {n}x{k}")


@pytest.mark.parametrize("hq,hkv,d,k,pos", [(32, 4, 64, 2048, 0), (32, 4, 64, 2048, 2175),
                                           (8, 2, 128, 2048, 37), (4, 4, 64, 256, 5),
                                           (6, 2, 32, 96, 16)])
def test_rmsnorm_qkv_rope_append(hq, hkv, d, k, pos):
    rng = np.random.default_rng(hq * 100 + pos)
    n = (hq + 2 * hkv) * d
    W = oracle.normal_f16(rng, (n, k), 0.02)
    x = oracle.normal_f16(rng, (k,))
    w = (1.0 + oracle.normal_f16(rng, (k,), 0.1).astype(np.float32)).astype(np.float16)
    theta = 10000.0
    # oracle: fp16 norm output, fp16 projection, RoPE in fp32, fp16 again
    xn = _f16(oracle.rmsnorm(x[None, :], w, 1e-5))
    qkv = _f16(oracle.matmul_transB(xn, W.astype(np.float32), nthreads=8)[0])
    q, kk = oracle.apply_rope(qkv[:hq * d], qkv[hq * d:(hq + hkv) * d], hq, hkv, d, pos, theta)
    v = qkv[(hq + hkv) * d:]
    P = pos // 16 + 3
    perm = np.random.default_rng(pos).permutation(P).astype(np.int32)
    pool_k = torch.zeros((hkv, P, 16, d), dtype=torch.float16, device="cuda")
    pool_v = torch.zeros_like(pool_k)
    q_out = torch.empty(hq * d, dtype=torch.float16, device="cuda")
    seq_len = torch.tensor([pos + 1], dtype=torch.int32, device="cuda")
    kvhp.rmsnorm_qkv_rope_append(to_gpu(W), to_gpu(x), to_gpu(w), 1e-5, seq_len, theta, q_out,
                                 pool_k, pool_v, torch.from_numpy(perm).cuda(), hq, hkv, d, k)
    torch.cuda.synchronize()
    _close(_cpu(q_out), _f16(q), "q")
    page, slot = perm[pos // 16], pos % 16
    pk = pool_k.float().cpu().numpy()
    pv = pool_v.float().cpu().numpy()
    _close(pk[:, page, slot, :].reshape(-1), _f16(kk), "k page")
    _close(pv[:, page, slot, :].reshape(-1), v, "v page")
    # nothing else in the pools was written
    mask = np.ones(pk.shape[1:3], bool)
    mask[page, slot] = False
    assert not pk[:, mask].any() and not pv[:, mask].any()


# Batched projections: each batch row against the oracle's GEMV of that row
# (same roundings as the batch-1 kernels), for batch sizes on both sides of
# the 16-row tile and shapes with a partial last row tile.
ROWS_BATCHES = [1, 5, 16, 17, 32]


@pytest.mark.parametrize("batch", ROWS_BATCHES)
@pytest.mark.parametrize("n,k", [(2048, 2048), (2048, 5632), (100, 512), (33, 1056)])
def test_gemv_residual_rows(batch, n, k):
    rng = np.random.default_rng(batch * 1000 + n + k)
    W = oracle.normal_f16(rng, (n, k), 0.02)
    x = oracle.normal_f16(rng, (batch, k))
    r = oracle.normal_f16(rng, (batch, n))
    ref = oracle.matmul_transB(x.astype(np.float32), W.astype(np.float32), nthreads=8)
    y = to_gpu(r)   # in place: y = W x + y
    kvhp.gemv_residual_rows(to_gpu(W), to_gpu(x), y, y, n, k, batch)
    torch.cuda.synchronize()
    _close(_cpu(y), _f16(ref + r.astype(np.float32)), f"gemv_residual_rows B={batch} {n}x{k}")


@pytest.mark.parametrize("batch,n,k", [(15, 2048, 5632), (16, 2048, 5632), (32, 2048, 5632),
                                       (24, 144, 5632), (32, 4096, 2816), (21, 2048, 4224),
                                       (32, 2048, 2048), (17, 2040, 5632)])
def test_gemv_residual_rows_ksplit(batch, n, k):
    """The workspace form splits large batches over K (partials summed in
    slice order by a second launch): its output is bit-identical to the
    single-launch kernel's, in place like the model calls it, and within the
    oracle tolerance.  Shapes with B*K <= 81920 or N % 16 != 0 need no
    workspace and take the single launch."""
    rng = np.random.default_rng(batch * 7 + n + k)
    W = oracle.normal_f16(rng, (n, k), 0.02)
    x = oracle.normal_f16(rng, (batch, k))
    r = oracle.normal_f16(rng, (batch, n))
    need = kvhp.gemv_rows_workspace_bytes(n, k, batch)
    splits = k // 256 if k % 256 == 0 and k // 256 <= 8 else k // 352   # the per-wave K slices
    if batch * k > 81920 and n % 16 == 0:
        assert need == 4 * splits * batch * n
    else:
        assert need == 0
    Wg, xg = to_gpu(W), to_gpu(x)
    y1 = to_gpu(r)
    kvhp.gemv_residual_rows(Wg, xg, y1, y1, n, k, batch)
    ws = torch.full((max(need, 16),), 0xFF, dtype=torch.uint8, device="cuda")   # NaN bytes
    y2 = to_gpu(r)
    kvhp.gemv_residual_rows_ws(Wg, xg, y2, y2, n, k, batch, ws)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), f"B={batch} {n}x{k}: K-split output differs from the single launch"
    ref = oracle.matmul_transB(x.astype(np.float32), W.astype(np.float32), nthreads=8)
    _close(_cpu(y2), _f16(ref + r.astype(np.float32)), f"gemv_residual_rows_ws B={batch} {n}x{k}")
    if need:
        with pytest.raises(kvhp.KVHPError):                 # workspace too small
            kvhp.gemv_residual_rows_ws(Wg, xg, y2, y2, n, k, batch, ws[:need - 16])


@pytest.mark.parametrize("batch", ROWS_BATCHES)
@pytest.mark.parametrize("n,k", [(32000, 2048), (2048, 2048), (77, 512)])
def test_rmsnorm_gemv_rows(batch, n, k):
    rng = np.random.default_rng(batch * 7 + n + k)
    W = oracle.normal_f16(rng, (n, k), 0.02)
    x = oracle.normal_f16(rng, (batch, k), 3.0)
    w = (1.0 + oracle.normal_f16(rng, (k,), 0.1).astype(np.float32)).astype(np.float16)
    xn = _f16(oracle.rmsnorm(x, w, 1e-5))
    ref = oracle.matmul_transB(xn, W.astype(np.float32), nthreads=8)
    y32 = torch.empty((batch, n), dtype=torch.float32, device="cuda")
    y16 = torch.empty((batch, n), dtype=torch.float16, device="cuda")
    kvhp.rmsnorm_gemv_rows(to_gpu(W), to_gpu(x), to_gpu(w), 1e-5, n, k, batch, y32=y32)
    kvhp.rmsnorm_gemv_rows(to_gpu(W), to_gpu(x), to_gpu(w), 1e-5, n, k, batch, y16=y16)
    torch.cuda.synchronize()
    _close(y32.cpu().numpy(), ref, f"rmsnorm_gemv_rows fp32 B={batch}")
    _close(_cpu(y16), _f16(ref), f"rmsnorm_gemv_rows fp16 B={batch}")


@pytest.mark.parametrize("batch", ROWS_BATCHES)
@pytest.mark.parametrize("n,k", [(5632, 2048), (37, 2048), (100, 768)])
def test_rmsnorm_gemv_swiglu_rows(batch, n, k):
    rng = np.random.default_rng(batch * 11 + n * 3 + k)
    Wgu = oracle.normal_f16(rng, (2 * n, k), 0.02)
    x = oracle.normal_f16(rng, (batch, k))
    w = (1.0 + oracle.normal_f16(rng, (k,), 0.1).astype(np.float32)).astype(np.float16)
    xn = _f16(oracle.rmsnorm(x, w, 1e-5))
    gu = _f16(oracle.matmul_transB(xn, Wgu.astype(np.float32), nthreads=8))
    ref = oracle.swiglu(gu[:, :n], gu[:, n:])
    out = torch.empty((batch, n), dtype=torch.float16, device="cuda")
    kvhp.rmsnorm_gemv_swiglu_rows(to_gpu(Wgu), to_gpu(x), to_gpu(w), 1e-5, out, n, k, batch)
    torch.cuda.synchronize()
    _close(_cpu(out), _f16(ref), f"rmsnorm_gemv_swiglu_rows B={batch} {n}x{k}")


@pytest.mark.parametrize("batch", ROWS_BATCHES)
@pytest.mark.parametrize("hq,hkv,d,k", [(32, 4, 64, 2048), (8, 2, 128, 2048), (4, 4, 32, 256)])
def test_rmsnorm_qkv_rope_append_rows(batch, hq, hkv, d, k):
    rng = np.random.default_rng(batch * 13 + hq + d)
    n = (hq + 2 * hkv) * d
    W = oracle.normal_f16(rng, (n, k), 0.02)
    x = oracle.normal_f16(rng, (batch, k))
    w = (1.0 + oracle.normal_f16(rng, (k,), 0.1).astype(np.float32)).astype(np.float16)
    theta = 10000.0
    max_pages = 4
    P = batch * max_pages + 3
    tables = rng.permutation(P)[:batch * max_pages].astype(np.int32).reshape(batch, max_pages)
    pos = rng.integers(0, 16 * max_pages, batch).astype(np.int32)
    if batch > 1:
        pos[1] = -1                                  # an idle row appends nothing
    xn = _f16(oracle.rmsnorm(x, w, 1e-5))
    qkv = _f16(oracle.matmul_transB(xn, W.astype(np.float32), nthreads=8))
    pool_k = torch.zeros((hkv, P, 16, d), dtype=torch.float16, device="cuda")
    pool_v = torch.zeros_like(pool_k)
    q_out = torch.empty((batch, hq * d), dtype=torch.float16, device="cuda")
    kvhp.rmsnorm_qkv_rope_append_rows(to_gpu(W), to_gpu(x), to_gpu(w), 1e-5, to_gpu(pos), theta,
                                      q_out, pool_k, pool_v, to_gpu(tables), hq, hkv, d, k, batch)
    torch.cuda.synchronize()
    pk = pool_k.float().cpu().numpy()
    pv = pool_v.float().cpu().numpy()
    qo = _cpu(q_out)
    written = np.zeros(pk.shape[1:3], bool)
    for b in range(batch):
        p0 = max(int(pos[b]), 0)
        q, kk = oracle.apply_rope(qkv[b, :hq * d], qkv[b, hq * d:(hq + hkv) * d], hq, hkv, d, p0,
                                  theta)
        _close(qo[b], _f16(q), f"q row {b}")
        if pos[b] < 0:
            continue
        page, slot = tables[b, pos[b] // 16], pos[b] % 16
        written[page, slot] = True
        _close(pk[:, page, slot, :].reshape(-1), _f16(kk), f"k page row {b}")
        _close(pv[:, page, slot, :].reshape(-1), qkv[b, (hq + hkv) * d:], f"v page row {b}")
    assert not pk[:, ~written].any() and not pv[:, ~written].any()


def _tiled(kind, W, n, k, hq=0, hkv=0, d=0):
    nb = kvhp.rows_tiled_bytes(kind, n, k, hq, hkv, d)
    tiles = {kvhp.ROWS_QKV: (hq + 2 * hkv) * d // 16 if d else 0,
             kvhp.ROWS_SWIGLU: (n + 7) // 8, kvhp.ROWS_PLAIN: (n + 15) // 16}[kind]
    assert nb == tiles * 32 * k
    Wt = torch.full((nb // 2,), float("nan"), dtype=torch.float16, device="cuda")
    kvhp.rows_tile_weights(kind, W, n, k, Wt, hq, hkv, d)
    return Wt


@pytest.mark.parametrize("batch", [1, 2, 8, 17, 32])
def test_rows_tiled_plain_bit_identical(batch):
    """Weights pre-tiled for the batched projections give bit-identical
    outputs to the row-major calls: residual (8 live rows per tile at N =
    2048, 16 at N = 4096, clamped rows at N = 77), the K-split residual
    (K = 5632, B >= 15) and the fp16 / fp32 RMSNorm projections (the LM-head
    shape included)."""
    rng = np.random.default_rng(300 + batch)
    for n, k in [(2048, 2048), (4096, 2048), (77, 512), (2048, 5632)]:
        W = to_gpu(oracle.normal_f16(rng, (n, k), 0.02))
        x = to_gpu(oracle.normal_f16(rng, (batch, k)))
        r = oracle.normal_f16(rng, (batch, n))
        Wt = _tiled(kvhp.ROWS_PLAIN, W, n, k)
        y1, y2 = to_gpu(r), to_gpu(r)
        kvhp.gemv_residual_rows(W, x, y1, y1, n, k, batch)
        kvhp.gemv_residual_rows_tiled(Wt, x, y2, y2, n, k, batch)
        need = kvhp.gemv_rows_workspace_bytes(n, k, batch)
        ws = torch.full((max(need, 16),), 0xFF, dtype=torch.uint8, device="cuda")
        y3, y4 = to_gpu(r), to_gpu(r)
        kvhp.gemv_residual_rows_ws(W, x, y3, y3, n, k, batch, ws)
        kvhp.gemv_residual_rows_tiled(Wt, x, y4, y4, n, k, batch, ws)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), f"residual B={batch} {n}x{k}"
        assert torch.equal(y3, y4), f"residual (workspace {need} B) B={batch} {n}x{k}"
    for n, k in [(32000, 2048), (100, 768)]:
        W = to_gpu(oracle.normal_f16(rng, (n, k), 0.02))
        x = to_gpu(oracle.normal_f16(rng, (batch, k), 3.0))
        w = to_gpu((1.0 + oracle.normal_f16(rng, (k,), 0.1).astype(np.float32)).astype(np.float16))
        Wt = _tiled(kvhp.ROWS_PLAIN, W, n, k)
        for dt in (torch.float32, torch.float16):
            a = torch.empty((batch, n), dtype=dt, device="cuda")
            b = torch.empty_like(a)
            kw = "y32" if dt == torch.float32 else "y16"
            kvhp.rmsnorm_gemv_rows(W, x, w, 1e-5, n, k, batch, **{kw: a})
            kvhp.rmsnorm_gemv_rows_tiled(Wt, x, w, 1e-5, n, k, batch, **{kw: b})
            torch.cuda.synchronize()
            assert torch.equal(a, b), f"rmsnorm_gemv_rows {dt} B={batch} {n}x{k}"


@pytest.mark.parametrize("batch", [1, 3, 8, 32])
def test_rows_tiled_swiglu_and_qkv_bit_identical(batch):
    """SwiGLU (gate/up rows paired inside a tile; N = 37 runs 8 live rows
    row-major but 16 tiled) and the fused QKV + RoPE + page append (RoPE
    dimension pairs inside a tile; D = 64, 128, 32) on tiled weights match
    the row-major calls bit for bit, including the pages written and an idle
    row."""
    rng = np.random.default_rng(400 + batch)
    for n, k in [(5632, 2048), (37, 2048), (100, 768)]:
        Wgu = to_gpu(oracle.normal_f16(rng, (2 * n, k), 0.02))
        x = to_gpu(oracle.normal_f16(rng, (batch, k)))
        w = to_gpu((1.0 + oracle.normal_f16(rng, (k,), 0.1).astype(np.float32)).astype(np.float16))
        Wt = _tiled(kvhp.ROWS_SWIGLU, Wgu, n, k)
        a = torch.empty((batch, n), dtype=torch.float16, device="cuda")
        b = torch.empty_like(a)
        kvhp.rmsnorm_gemv_swiglu_rows(Wgu, x, w, 1e-5, a, n, k, batch)
        kvhp.rmsnorm_gemv_swiglu_rows_tiled(Wt, x, w, 1e-5, b, n, k, batch)
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"swiglu B={batch} {n}x{k}"
    for hq, hkv, d, k in [(32, 4, 64, 2048), (8, 2, 128, 2048), (4, 4, 32, 256)]:
        n = (hq + 2 * hkv) * d
        W = to_gpu(oracle.normal_f16(rng, (n, k), 0.02))
        x = to_gpu(oracle.normal_f16(rng, (batch, k)))
        w = to_gpu((1.0 + oracle.normal_f16(rng, (k,), 0.1).astype(np.float32)).astype(np.float16))
        Wt = _tiled(kvhp.ROWS_QKV, W, 0, k, hq, hkv, d)
        max_pages, P = 4, 4 * batch + 3
        tables = to_gpu(rng.permutation(P)[:4 * batch].astype(np.int32).reshape(batch, 4))
        pos = rng.integers(0, 64, batch).astype(np.int32)
        if batch > 1:
            pos[1] = -1
        pos = to_gpu(pos)
        outs = []
        for tiled in (False, True):
            pk = torch.zeros((hkv, P, 16, d), dtype=torch.float16, device="cuda")
            pv = torch.zeros_like(pk)
            q = torch.empty((batch, hq * d), dtype=torch.float16, device="cuda")
            fn = kvhp.rmsnorm_qkv_rope_append_rows_tiled if tiled else \
                kvhp.rmsnorm_qkv_rope_append_rows
            fn(Wt if tiled else W, x, w, 1e-5, pos, 10000.0, q, pk, pv, tables, hq, hkv, d, k,
               batch)
            outs.append((q, pk, pv))
        torch.cuda.synchronize()
        for u, v, what in zip(outs[0], outs[1], ("q", "k pages", "v pages")):
            assert torch.equal(u, v), f"qkv {what} B={batch} {hq}/{hkv}x{d}"


def test_rows_tiled_errors():
    W = torch.zeros((64, 1000), dtype=torch.float16, device="cuda")
    Wt = torch.zeros((1 << 16,), dtype=torch.float16, device="cuda")
    assert kvhp.rows_tiled_bytes(kvhp.ROWS_PLAIN, 64, 1000) == 0          # K not 256n / 352n
    assert kvhp.rows_tiled_bytes(7, 64, 2048) == 0                        # unknown kind
    assert kvhp.rows_tiled_bytes(kvhp.ROWS_QKV, 0, 2048, 4, 4, 24) == 0   # head_dim % 16
    with pytest.raises(kvhp.KVHPError):
        kvhp.rows_tile_weights(kvhp.ROWS_PLAIN, W, 64, 1000, Wt)
    with pytest.raises(kvhp.KVHPError):
        kvhp.gemv_residual_rows_tiled(None, W, W, W, 64, 2048, 2)


def test_rows_projection_errors():
    W = torch.zeros((64, 2048), dtype=torch.float16, device="cuda")
    x = torch.zeros((40, 2048), dtype=torch.float16, device="cuda")
    y = torch.zeros((40, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(kvhp.KVHPError):                  # batch above 32
        kvhp.gemv_residual_rows(W, x, y, y, 64, 2048, 33)
    with pytest.raises(kvhp.KVHPError):                  # K not 256*n / 352*n
        kvhp.gemv_residual_rows(W, x, y, y, 64, 1000, 4)


@pytest.mark.parametrize("rows,dim", [(1, 2048), (2048, 2048), (7, 100), (3, 5632), (65, 64)])
def test_rmsnorm_rows(rows, dim):
    rng = np.random.default_rng(rows + dim)
    x = oracle.normal_f16(rng, (rows, dim))
    w = (1.0 + oracle.normal_f16(rng, (dim,), 0.1).astype(np.float32)).astype(np.float16)
    ref = oracle.rmsnorm(x, w, 1e-5)
    out = torch.empty((rows, dim), dtype=torch.float16, device="cuda")
    kvhp.rmsnorm(to_gpu(x), to_gpu(w), out, rows, dim, 1e-5)
    torch.cuda.synchronize()
    _close(_cpu(out), _f16(ref), "rmsnorm rows")


@pytest.mark.parametrize("s,hq,hkv,d,start", [(1, 32, 4, 64, 0), (2048, 32, 4, 64, 0),
                                             (17, 8, 2, 128, 100), (5, 6, 3, 32, 2047)])
def test_rope_and_split_qkv(s, hq, hkv, d, start):
    rng = np.random.default_rng(s + start)
    qkv = oracle.normal_f16(rng, (s, hq + 2 * hkv, d))
    q = np.ascontiguousarray(qkv[:, :hq])
    k = np.ascontiguousarray(qkv[:, hq:hq + hkv])
    v = np.ascontiguousarray(qkv[:, hq + hkv:])
    rq, rk = oracle.apply_rope(q, k, hq, hkv, d, start, 10000.0)
    qd, kd = to_gpu(q), to_gpu(k)
    kvhp.apply_rope(qd, kd, s, hq, hkv, d, start, 10000.0)
    q2 = torch.empty_like(qd)
    k2 = torch.empty_like(kd)
    v2 = torch.empty((s, hkv, d), dtype=torch.float16, device="cuda")
    kvhp.split_qkv_rope(to_gpu(qkv), s, hq, hkv, d, start, 10000.0, q2, k2, v2)
    torch.cuda.synchronize()
    for got, ref, what in ((qd, rq, "rope q"), (kd, rk, "rope k"), (q2, rq, "split q"),
                           (k2, rk, "split k")):
        _close(_cpu(got).reshape(-1), _f16(ref).reshape(-1), what)
    assert np.array_equal(_cpu(v2), v.astype(np.float32))


def test_split_qkv_rope_rows_per_row_positions():
    """Batched decode: row r rotated at positions[r] (negative = idle row,
    rotated as position 0); each row against the oracle's RoPE of that one
    row at that position."""
    hq, hkv, d = 8, 2, 64
    pos = np.array([0, 5, 2047, -1, 16, 4095, 1], np.int32)
    rows = pos.size
    rng = np.random.default_rng(77)
    qkv = oracle.normal_f16(rng, (rows, hq + 2 * hkv, d))
    q2 = torch.empty((rows, hq, d), dtype=torch.float16, device="cuda")
    k2 = torch.empty((rows, hkv, d), dtype=torch.float16, device="cuda")
    v2 = torch.empty((rows, hkv, d), dtype=torch.float16, device="cuda")
    kvhp.split_qkv_rope_rows(to_gpu(qkv), rows, hq, hkv, d, to_gpu(pos), 10000.0, q2, k2, v2)
    torch.cuda.synchronize()
    for r in range(rows):
        q = np.ascontiguousarray(qkv[r:r + 1, :hq])
        k = np.ascontiguousarray(qkv[r:r + 1, hq:hq + hkv])
        rq, rk = oracle.apply_rope(q, k, hq, hkv, d, max(int(pos[r]), 0), 10000.0)
        _close(_cpu(q2[r]).reshape(-1), _f16(rq).reshape(-1), f"row {r} q")
        _close(_cpu(k2[r]).reshape(-1), _f16(rk).reshape(-1), f"row {r} k")
    assert np.array_equal(_cpu(v2), qkv[:, hq + hkv:].astype(np.float32))


@pytest.mark.parametrize("rows,n", [(1, 5632), (2048, 5632), (3, 7)])
def test_swiglu(rows, n):
    rng = np.random.default_rng(rows * n)
    gu = oracle.normal_f16(rng, (rows, 2 * n), 2.0)
    ref = oracle.swiglu(gu[:, :n], gu[:, n:])
    out = torch.empty((rows, n), dtype=torch.float16, device="cuda")
    kvhp.swiglu_rows(to_gpu(gu), out, rows, n)
    flat = torch.empty(rows * n, dtype=torch.float16, device="cuda")
    g = to_gpu(np.ascontiguousarray(gu[:, :n]))
    u = to_gpu(np.ascontiguousarray(gu[:, n:]))
    kvhp.swiglu(g, u, flat, rows * n)
    torch.cuda.synchronize()
    _close(_cpu(out), _f16(ref), "swiglu rows")
    _close(_cpu(flat).reshape(rows, n), _f16(ref), "swiglu flat")


def test_embedding():
    rng = np.random.default_rng(5)
    vocab, hidden = 1000, 2048
    table = oracle.normal_f16(rng, (vocab, hidden), 0.02)
    ids = np.array([0, 999, 5, 5, -1, 1000, 123], np.int32)
    out = torch.empty((ids.size, hidden), dtype=torch.float16, device="cuda")
    kvhp.embedding(torch.from_numpy(ids).cuda(), to_gpu(table), out, ids.size, hidden, vocab)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, t in enumerate(ids):
        exp = table[t] if 0 <= t < vocab else np.zeros(hidden, np.float16)
        assert np.array_equal(got[i].view(np.uint16), exp.view(np.uint16)), i


def test_argmax_ties_nan_and_counters():
    rng = np.random.default_rng(9)
    cases = []
    x = rng.standard_normal(32000).astype(np.float32)
    cases.append((x.copy(), int(np.argmax(x))))
    y = x.copy()
    y[[7, 30000, 123]] = 50.0                   # tie: lowest index wins
    cases.append((y, 7))
    z = x.copy()
    z[[3, 10]] = np.nan
    z[31999] = 60.0                              # NaN never wins
    cases.append((z, 31999))
    w = np.full(5, -np.inf, np.float32)          # all -inf -> index 0
    cases.append((w, 0))
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    seq = torch.tensor([10], dtype=torch.int32, device="cuda")
    log = torch.full((8,), -1, dtype=torch.int32, device="cuda")
    cnt = torch.zeros(1, dtype=torch.int32, device="cuda")
    for logits, want in cases:
        kvhp.argmax(torch.from_numpy(logits).cuda(), logits.size, tok, seq, log, cnt)
        torch.cuda.synchronize()
        assert int(tok.item()) == want
    assert int(seq.item()) == 10 + len(cases)
    assert int(cnt.item()) == len(cases)
    assert log.cpu().numpy()[:len(cases)].tolist() == [c[1] for c in cases]


def test_argmax_rows():
    """One workgroup per row, the same tie and NaN rules as the single-row
    argmax; rows of a length that is not a multiple of 4 (unaligned rows)."""
    rng = np.random.default_rng(10)
    for n in (32000, 1001):
        x = rng.standard_normal((6, n)).astype(np.float32)
        x[1, [40, 9, 700]] = 9.0                 # tie: lowest index wins
        x[2, :] = -np.inf                        # all -inf -> 0
        x[3, [0, 1]] = np.nan
        x[3, n - 1] = 12.0                       # NaN never wins
        want = [int(np.argmax(x[0])), 9, 0, n - 1, int(np.argmax(x[4])), int(np.argmax(x[5]))]
        tok = torch.full((6,), -1, dtype=torch.int32, device="cuda")
        kvhp.argmax_rows(torch.from_numpy(x).cuda(), 6, n, tok)
        torch.cuda.synchronize()
        assert tok.cpu().numpy().tolist() == want, n


def test_randn_and_fill():
    a = torch.empty(1 << 20, dtype=torch.float16, device="cuda")
    b = torch.empty_like(a)
    c = torch.empty_like(a)
    kvhp.randn_f16(a, 1234, 7, 0.02)
    kvhp.randn_f16(b, 1234, 7, 0.02)
    kvhp.randn_f16(c, 1234, 8, 0.02)
    torch.cuda.synchronize()
    assert torch.equal(a, b)                     # deterministic
    assert not torch.equal(a, c)                 # streams differ
    v = a.float().cpu().numpy()
    assert abs(v.mean()) < 2e-4 and abs(v.std() - 0.02) < 2e-4
    assert abs(np.mean(np.abs(v) < 0.02) - 0.6827) < 0.005
    kvhp.fill_f16(a, 1.0)
    torch.cuda.synchronize()
    assert bool((a == 1.0).all())
