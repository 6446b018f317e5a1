"""bench.py's contract, on the CPU: the metric is BASELINE.json's, more than
one GPU is refused with a message (one GPU per box here), and the
algorithmic bytes behind `value` and `roofline.achieved` follow the decode
byte count of the reference's benchmark (apps/bench_attention.cpp:136-138:
K and V of every cached token, q read and out written) plus the paging
terms (one int32 page id per 16 tokens, one int32 length per sequence),
counted here per sequence and per page rather than by bench.py's vectorised
form."""
import json
import os
import subprocess
import sys

import numpy as np

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_metric_is_baselines():
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        assert bench.METRIC == json.load(f)["metric"]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def _decode_bytes_by_loop(lens, hq, hkv, d):
    total = 0
    for L in lens:
        total += 2 * int(L) * hkv * d * 2          # K and V rows, fp16
        total += 2 * hq * d * 2                    # q read, out written
        total += 4 * len(range(0, int(L), 16))     # one page id per started page
        total += 4                                 # the sequence's length
    return total


def test_config3_step_bytes():
    # 32 lengths U[128, 8192] from seed 3, one appended token each
    lens = np.random.default_rng(3).integers(128, 8193, size=32).astype(np.int64) + 1
    assert int(lens.sum()) == 122822
    d = bench.decode_bytes(lens, 32, 8, 128)
    assert d == _decode_bytes_by_loop(lens, 32, 8, 128) == 503634100
    # the fused append: K and V rows read and written, position and page id per sequence
    assert bench.append_bytes(32, 8, 128) == 32 * (2 * 8 * 128 * 2 * 2 + 2 * 4)
    assert d + bench.append_bytes(32, 8, 128) == 503896500


def test_config1_decode_bytes():
    # config 1: one sequence of 512 keys, 32/8 heads, D=64
    assert bench.decode_bytes([512], 32, 8, 64) == _decode_bytes_by_loop([512], 32, 8, 64)
    assert bench.decode_bytes([512], 32, 8, 64) == 1048576 + 8192 + 32 * 4 + 4
