"""The engine's MoE call sequence replayed by a compiled C program
(tests/harness/moe_harness.c) that links libcoli_hip.so through
include/coli_backend_abi.h, as colibri's engine does: pipe_router per token,
host union, expert_group_issue, a CPU share between issue and take, take, the
weighted scatter (c/colibri.c:4467-4531, 4782-4810, 5520-5541). The program
compares its layer output and routing with the oracle's cref_moe_layer and
exits 0 on parity."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
HARNESS = os.path.join(HERE, "harness", "moe_harness")


@pytest.fixture(scope="module")
def harness():
    if not os.path.exists(HARNESS):
        subprocess.run(["make", "-C", os.path.dirname(HARNESS)], check=True)
    return HARNESS


@pytest.mark.parametrize("fmt", [4, 7])
@pytest.mark.parametrize("S,seed", [(1, 1), (2, 2), (4, 3), (4, 4)])
def test_moe_call_sequence_in_c(harness, fmt, S, seed):
    r = subprocess.run([harness, str(fmt), str(S), str(seed)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS" in r.stdout and "bit-exact" in r.stdout
