"""Host check of the decode work-placement arithmetic (apertura_amd/csrc/esda_plan.h:
visibility, the prefix table, balanced shares and their segment walk, partial slots,
the merge's split owners, grid splits) -- the functions the attend and merge kernels
call -- over 3,000 random batches including 256-sequence batches, fewer rows than
workgroups, and 256 x 16 kv heads x 16,384 workgroups.  tests/plan_check.cpp is built
with g++; a variant with the batch-256 prefix-table bug planted must fail."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "plan_check.cpp")
INC = os.path.join(ROOT, "apertura_amd", "csrc")


def _build(tmp_path, *defines):
    cxx = os.environ.get("CXX", "g++")
    if not shutil.which(cxx):
        pytest.skip(f"{cxx} not found")
    exe = tmp_path / ("plan_check" + "".join(d.lower() for d in defines))
    cmd = [cxx, "-std=c++17", "-O2", "-Wall", "-Wextra", "-Werror", "-I", INC, SRC, "-o", str(exe)]
    cmd += [f"-D{d}" for d in defines]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def test_plan_arithmetic_over_random_batches(tmp_path):
    exe = _build(tmp_path)
    r = subprocess.run([str(exe), "3000"], capture_output=True, text=True, timeout=600)
    print(r.stdout[-2000:])
    assert r.returncode == 0 and r.stdout.strip().endswith("3000 batches, 0 failures"), r.stdout[-2000:]


def test_planted_prefix_table_bug_is_caught(tmp_path):
    exe = _build(tmp_path, "PLANT_TABLE_BUG")
    r = subprocess.run([str(exe), "64"], capture_output=True, text=True, timeout=600)
    assert r.returncode != 0 and "table[256] never written" in r.stdout, r.stdout[-2000:]
