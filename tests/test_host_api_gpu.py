"""Runs tests/cpp/host_api_test: the C++ BlockPool / KVCacheManager /
paged_attention interface (include/vllm_cpp, the reference's
src/kv_cache_manager.h and src/paged_attention.h) driven as the reference
engine drives it, checked against the CPU oracle inside the program."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "host_api_test")


def test_host_api(cuda):
    assert os.path.exists(BIN), "tests/cpp/host_api_test not built (run __graft_entry__.build())"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert "ALL PASSED" in r.stdout
