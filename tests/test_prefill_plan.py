"""Host-side properties of the chunked-prefill work planner
(csrc/prefill_plan.cpp), run on the CPU by tests/plan/prefill_plan_check.cpp:
every (sequence, tile) gets nparts entries whose key ranges tile its keys,
nparts is uniform per sequence, the split-row lists match, and the list is
longest first.  Also pins the plan shapes that the GPU key-part test
(test_gpu_prefill.py KEY_PART_CASES) relies on to cover empty parts and part
boundaries inside a tile of query rows."""
import os
import subprocess

import pytest

from test_gpu_prefill import KEY_PART_CASES

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "orionserve-rs_amd", "csrc")
CUS = 256  # MI355X compute units, what the library passes on the GPU box


@pytest.fixture(scope="module")
def check_exe(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("pplan") / "prefill_plan_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I" + CSRC, os.path.join(ROOT, "tests", "plan", "prefill_plan_check.cpp"),
                    os.path.join(CSRC, "prefill_plan.cpp"), "-o", exe], check=True)
    return exe


def run_case(exe, prefixes, chunks, hq, hkv, d=128):
    p = subprocess.run([exe, "case", str(CUS), str(hq // hkv), str(hkv),
                        ",".join(map(str, prefixes)), ",".join(map(str, chunks)), str(d)],
                       capture_output=True, text=True)
    print(p.stdout)
    assert p.returncode == 0, p.stdout
    return dict(kv.split("=") for kv in p.stdout.split())


def test_random_prefill_plans_are_consistent(check_exe):
    p = subprocess.run([check_exe, "random", "2000"], capture_output=True, text=True)
    print(p.stdout)
    assert p.returncode == 0, p.stdout
    st = dict(kv.split("=") for kv in p.stdout.split()[2:])
    # the random batches do exercise empty parts and straddling boundaries
    assert int(st["empty"]) > 0 and int(st["straddle"]) > 0


def test_key_part_cases_cover_what_the_gpu_test_claims(check_exe):
    prefixes, chunks, hq, hkv, _ = KEY_PART_CASES[0]
    st = run_case(check_exe, prefixes, chunks, hq, hkv)
    assert int(st["parts"]) > 1
    prefixes, chunks, hq, hkv, _ = KEY_PART_CASES[1]
    st = run_case(check_exe, prefixes, chunks, hq, hkv)
    assert int(st["parts"]) > 1 and int(st["empty"]) > 0 and int(st["straddle"]) > 0
    prefixes, chunks, hq, hkv, d = KEY_PART_CASES[2]
    st = run_case(check_exe, prefixes, chunks, hq, hkv, d)
    assert d == 256 and int(st["parts"]) > 1


def test_no_split_when_disabled(check_exe):
    prefixes, chunks, hq, hkv, _ = KEY_PART_CASES[1]
    env = dict(os.environ, ORION_PREFILL_SPLIT="0")
    p = subprocess.run([check_exe, "case", str(CUS), str(hq // hkv), str(hkv),
                        ",".join(map(str, prefixes)), ",".join(map(str, chunks))],
                       capture_output=True, text=True, env=env)
    assert p.returncode == 0, p.stdout
    assert "parts=1 " in p.stdout
