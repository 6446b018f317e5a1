"""Shared helpers of the GPU parity tests: device transfer, seeded inputs,
paged-pool construction and the attention tolerance check.

Tolerance (BASELINE): attention outputs within max-abs 2e-3 / max-rel 1e-2
after fp32 accumulation.  Elementwise we require |g - r| <= 2e-3 + 1e-2*|r|,
and in addition the raw max-abs over the tensor must be <= 2e-3; the report
prints both max-abs and max-rel (relative error over |r| >= 1e-2).
"""
import sys

import numpy as np

import oracle

ATOL = 2e-3
RTOL = 1e-2


def torch_dev():
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("GPU test needs a ROCm GPU (torch.cuda.is_available() is False)")
    return torch.device("cuda", 0)


def to_gpu(a: np.ndarray):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch_dev())


def to_gpu_f16(a: np.ndarray):
    import torch
    return to_gpu(np.ascontiguousarray(a, dtype=np.float16))


def from_gpu(t) -> np.ndarray:
    return t.detach().cpu().numpy()


def sync():
    import torch
    torch.cuda.synchronize()


def note(msg: str) -> None:
    """Names the case before a GPU step, flushed, so a lost box still says which."""
    print(msg, flush=True)
    sys.stdout.flush()


def stats(got: np.ndarray, ref: np.ndarray):
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    err = np.abs(got - ref)
    big = np.abs(ref) >= 1e-2
    max_rel = float((err[big] / np.abs(ref[big])).max()) if big.any() else 0.0
    return float(err.max()) if err.size else 0.0, max_rel, err


def assert_attn_close(got, ref, tag=""):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{tag}: non-finite output"
    max_abs, max_rel, err = stats(got, ref)
    bad = err > ATOL + RTOL * np.abs(ref.astype(np.float64))
    assert not bad.any() and max_abs <= ATOL, (
        f"{tag}: max_abs={max_abs:.3e} max_rel={max_rel:.3e} "
        f"violations={int(bad.sum())} first={np.argwhere(bad)[:3].tolist()}")
    return max_abs, max_rel


def uniform_f16(rng, shape, lo=-1.0, hi=1.0):
    """U(lo,hi) rounded to fp16, as the reference tests draw inputs
    (tests/test_attention.cpp:35-36)."""
    return rng.uniform(lo, hi, size=shape).astype(np.float32).astype(np.float16)


def make_block_tables(rng, lens, slack_pages=3, extra_cols=1):
    """Seeded random permutation of physical pages dealt to sequences in order.
    Returns (block_tables int32 [B][max_pages], num_pages); unused entries -1."""
    lens = np.asarray(lens)
    need = [int((L + 15) // 16) for L in lens]
    P = sum(need) + slack_pages
    maxp = max(max(need), 1) + extra_cols
    perm = rng.permutation(P).astype(np.int32)
    bt = np.full((len(lens), maxp), -1, np.int32)
    o = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[o:o + n]
        o += n
    return bt, P


def contiguous_from_tokens(tok, lens, cap):
    """tok [B][T][Hkv][D] -> [B][Hkv][cap][D] float32 (zeros past each length)."""
    b, t, hkv, d = tok.shape
    out = np.zeros((b, hkv, cap, d), np.float32)
    for i in range(b):
        n = min(int(lens[i]), t, cap)
        out[i, :, :n] = tok[i, :n].transpose(1, 0, 2)
    return out
