"""The C++ API (serving-engine_amd/engine/*.h: KVCache, PagedKVCache,
engine::cuda::append_kv_cache / decode_gqa / decode_gqa_split /
flash_prefill_gqa / causal_gqa, KVView, prefill_gpu / decode_step_gpu)
exercised from C++ by tests/cpp/test_engine (and KVView's accessors in a
kernel by tests/cpp/test_kv_view_device),
the way the reference's doctest suites exercise its own engine::cuda
(tests/test_kv_cache.cpp, tests/test_attention.cpp).  The binary is built by
tests/cpp/Makefile (also run by __graft_entry__.build()); it is built here
only when missing."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CPP = os.path.join(HERE, "cpp")
BIN = os.path.join(CPP, "test_engine")


def _binary(path=BIN):
    if not os.path.exists(path):
        subprocess.run(["make", "-s"], cwd=CPP, check=True)
    return path


def _run(mode, timeout):
    r = subprocess.run([_binary(), mode], capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-4000:])
    print(r.stderr[-2000:])
    assert r.returncode == 0, r.stdout[-4000:]
    assert " 0 failures" in r.stdout


def test_cpp_engine_cpu_cases():
    _run("--cpu", 120)


@pytest.mark.gpu
def test_cpp_engine_gpu_cases():
    _run("--gpu", 240)


@pytest.mark.gpu
def test_kv_view_accessors_in_device_code():
    r = subprocess.run([_binary(os.path.join(CPP, "test_kv_view_device"))], capture_output=True,
                       text=True, timeout=120)
    print(r.stdout[-2000:])
    assert r.returncode == 0 and "all ok" in r.stdout, r.stdout[-2000:] + r.stderr[-1000:]
