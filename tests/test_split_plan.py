"""The split-K launch planner (neural-network-engine_amd/csrc/splitk_plan.cpp)
on the CPU, through tests/cpp/test_split_plan.cpp: for the benchmark's decode
and cross-attention shapes and a seeded sweep of ragged batches (empty
sequences, one long head among short ones, equal lengths, 1-160 sequences,
8-256 slots), the layout chosen (whole heads packed, cut chunks or equal
chunks) must cover every key once, keep each workgroup within its budget and
each head within its part limit, give partial records unique slots inside the
workspace, and use the smallest budget that fits.  Built by
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
