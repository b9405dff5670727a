"""The launch planners on the CPU.  Split-K (neural-network-engine_amd/csrc/
splitk_plan.cpp), through tests/cpp/test_split_plan.cpp: for the benchmark's decode
and cross-attention shapes and a seeded sweep of ragged batches (empty
sequences, one long head among short ones, equal lengths, 1-160 sequences,
8-256 slots), the layout chosen (whole heads packed, cut chunks or equal
chunks) must cover every key once, keep each workgroup within its budget and
each head within its part limit, give partial records unique slots inside the
workspace, and use the smallest budget that fits.  The deep kernel's key
splits (csrc/deep_plan.cpp), through tests/cpp/test_deep_plan.cpp.  Built by
__graft_entry__.build() (make -C tests/cpp)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "build", "test_split_plan")


def test_split_plan_invariants():
    if not os.path.exists(BIN):
        pytest.fail("planner test not built: %s is missing (run __graft_entry__.build())" % BIN)
    res = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout
    assert re.search(r"^0 of \d+ checks failed$", res.stdout, re.M)
    m = re.search(r"^sweep layouts: (\d+) packed, (\d+) cut, (\d+) equal$", res.stdout, re.M)
    assert m and all(int(x) > 0 for x in m.groups()), "sweep must reach every layout"


DEEP_BIN = os.path.join(ROOT, "tests", "cpp", "build", "test_deep_plan")


def test_deep_plan_invariants():
    """The deep kernel's key-split plans (csrc/deep_plan.cpp): the ragged
    decode split and the equal split, on named batches (including more
    (sequence, KV head) pairs than CUs, which must return at once) and a
    seeded sweep."""
    if not os.path.exists(DEEP_BIN):
        pytest.fail("planner test not built: %s is missing (run __graft_entry__.build())" % DEEP_BIN)
    res = subprocess.run([DEEP_BIN], capture_output=True, text=True, timeout=60)
    print(res.stdout)
    assert res.returncode == 0, res.stdout
    assert re.search(r"^0 of \d+ checks failed$", res.stdout, re.M)
    m = re.search(r"^ragged plans: (\d+) taken, (\d+) declined; equal splits taken: (\d+)$", res.stdout, re.M)
    assert m and all(int(x) > 0 for x in m.groups()), "sweep must reach every outcome"
