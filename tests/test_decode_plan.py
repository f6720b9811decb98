"""Host-side properties of the decode work planner (csrc/decode_plan.cpp):
tests/plan/plan_check.cpp builds plans for random batches and checks that
every planned (row, KV head) context is covered exactly once, by pieces with
valid table slices and split indices, and that balanced plans fit at most four
rounds of wave slots.  Run for both cutting modes (balanced, and fixed chunks
with ORION_DECODE_BALANCE=0)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "orionserve-rs_amd", "csrc")


@pytest.fixture(scope="module")
def plan_check(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("plan") / "plan_check")
    cmd = ["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I" + CSRC, os.path.join(ROOT, "tests", "plan", "plan_check.cpp"),
           os.path.join(CSRC, "decode_plan.cpp"), "-o", exe]
    subprocess.run(cmd, check=True)
    return exe


@pytest.mark.parametrize("balance", ["1", "0"])
def test_decode_plans_cover_every_context_once(plan_check, balance):
    env = dict(os.environ, ORION_DECODE_BALANCE=balance)
    p = subprocess.run([plan_check, "2000"], env=env, capture_output=True, text=True)
    print(p.stdout)
    assert p.returncode == 0, p.stdout
    trials, nbal = p.stdout.split()[0], int(p.stdout.split()[2])
    assert trials == "2000"
    assert (nbal > 0) == (balance == "1")
    assert int(p.stdout.split()[4]) > 0  # packed prefix items were planned and checked
