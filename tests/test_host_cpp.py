"""The C++ host API (neural-network-engine_amd/host/nne.hpp) through its test
program tests/cpp/test_host_api.cpp, which mirrors the reference's
tests/nn/flash_attention_tests.rs and tests/nn/kv_cache_tests.rs on the GPU
and checks every result against the CPU oracle.  Built by
__graft_entry__.build() (make -C tests/cpp)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "build", "test_host_api")


def run(args, timeout):
    if not os.path.exists(BIN):
        pytest.fail("C++ host-API tests not built: %s is missing (run __graft_entry__.build())" % BIN)
    res = subprocess.run([BIN] + args, capture_output=True, text=True, timeout=timeout)
    print(res.stdout)
    print(res.stderr)
    return res


def test_host_api_cpu_only_parts():
    """Error variants and messages (src/error.rs), Result, layer and RoPE
    argument checks."""
    res = run(["--cpu"], 60)
    assert res.returncode == 0, res.stdout
    assert re.search(r"^0 of 3 tests failed$", res.stdout, re.M)


@pytest.mark.gpu
def test_host_api_on_gpu():
    res = run([], 300)
    assert res.returncode == 0, res.stdout
    assert re.search(r"^0 of \d+ tests failed$", res.stdout, re.M) and "FAIL" not in res.stdout
