"""Write the golden fixtures in this directory from the reference's own CPU ops.

The vectors come from the reference source src/cpu/ops.cpp compiled where it
lies by `make -C oracle ref` (oracle/_ref/libref_ops.so, built in this
container only; the reference tree is not present on the GPU box).  Each
fixture stores the seeded inputs and the reference outputs, so the oracle
restatement can be pinned anywhere without the reference tree.

    python tests/golden/make_golden.py

Shapes cover the reference's own test shapes (head_dim 64, group 7, lengths 1,
15, 17, 65: tests/test_attention.cpp:186-198) and the BASELINE head shapes
(32/8 and 32/4 heads, head_dim 64 and 128).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle"))
import oracle  # noqa: E402

CAUSAL_CASES = [
    # (seed, S, Hq, Hkv, D)
    (7001, 1, 14, 2, 64),
    (7002, 15, 14, 2, 64),
    (7003, 17, 4, 2, 64),
    (7004, 65, 2, 2, 64),
    (7005, 6, 32, 8, 128),
    (7006, 8, 32, 4, 64),
    (7007, 9, 3, 1, 48),
]


def _f16(rng, shape):
    return oracle.normal_f16(rng, shape).astype(np.float32)


def main():
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libref_ops.so missing: run `make -C oracle ref` first")
    out = {}
    for seed, s, hq, hkv, d in CAUSAL_CASES:
        rng = np.random.default_rng(seed)
        q = _f16(rng, (s, hq, d))
        k = _f16(rng, (s, hkv, d))
        v = _f16(rng, (s, hkv, d))
        o = oracle.ref_causal_gqa(q, k, v, hq, hkv, d)
        key = f"causal_{seed}"
        out[key + "_shape"] = np.array([s, hq, hkv, d], np.int64)
        # inputs are fp16-exact, so they are stored as float16
        out[key + "_q"] = q.astype(np.float16)
        out[key + "_k"] = k.astype(np.float16)
        out[key + "_v"] = v.astype(np.float16)
        out[key + "_out"] = o

    rng = np.random.default_rng(7101)
    x = rng.standard_normal((3, 2048), dtype=np.float32)
    w = rng.standard_normal(2048, dtype=np.float32)
    out["rmsnorm_x"], out["rmsnorm_w"] = x, w
    out["rmsnorm_out"] = oracle.rmsnorm(x, w, 1e-5, use_ref=True)

    rng = np.random.default_rng(7102)
    a = rng.standard_normal((4, 200), dtype=np.float32)
    b = rng.standard_normal((37, 200), dtype=np.float32)
    out["matmul_a"], out["matmul_b"] = a, b
    out["matmul_out"] = oracle.matmul_transB(a, b, use_ref=True)

    rng = np.random.default_rng(7103)
    q = rng.standard_normal((5, 4, 64), dtype=np.float32)
    k = rng.standard_normal((5, 2, 64), dtype=np.float32)
    out["rope_q"], out["rope_k"] = q, k
    rq, rk = oracle.apply_rope(q, k, 4, 2, 64, 2041, 10000.0, use_ref=True)
    out["rope_start_theta"] = np.array([2041.0, 10000.0])
    out["rope_q_out"], out["rope_k_out"] = rq, rk

    rng = np.random.default_rng(7104)
    g = rng.standard_normal(1000, dtype=np.float32) * 4
    u = rng.standard_normal(1000, dtype=np.float32)
    out["swiglu_gate"], out["swiglu_up"] = g, u
    out["swiglu_out"] = oracle.swiglu(g, u, use_ref=True)

    path = os.path.join(HERE, "ref_cpu_ops.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
