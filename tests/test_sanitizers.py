"""AddressSanitizer + UndefinedBehaviorSanitizer builds of the host code that parses
untrusted input or checks the GPU: the KV-snapshot container reader
(apertura_amd/csrc/es/safetensors.cpp, driven by tests/safetensors_check.cpp over valid,
malformed and 3,000 mutated files) and the CPU oracle (oracle/oracle.c, driven by
tests/oracle_check.c over every function and edge-case shapes).  Host compilers only
(g++ / gcc); no GPU, no HIP."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-g", "-O1", "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]


def _run(cmd, **kw):
    r = subprocess.run(cmd, capture_output=True, text=True, **kw)
    return r


def _need(tool):
    if not shutil.which(tool):
        pytest.skip(f"{tool} not found")


def test_snapshot_reader_under_asan_ubsan(tmp_path):
    _need("g++")
    exe = tmp_path / "safetensors_check"
    r = _run(["g++", "-std=c++17", *SAN, "-I", os.path.join(ROOT, "apertura_amd", "csrc"),
              os.path.join(ROOT, "tests", "safetensors_check.cpp"),
              os.path.join(ROOT, "apertura_amd", "csrc", "es", "safetensors.cpp"), "-o", str(exe)])
    assert r.returncode == 0, r.stderr
    r = _run([str(exe), str(tmp_path), "3000"], timeout=600)
    print(r.stdout[-1000:])
    assert r.returncode == 0 and r.stdout.strip().endswith("0 failures"), r.stdout[-2000:] + r.stderr[-4000:]


def test_oracle_under_asan_ubsan(tmp_path):
    _need("gcc")
    exe = tmp_path / "oracle_check"
    r = _run(["gcc", "-std=c11", *SAN, "-ffp-contract=off", "-I", os.path.join(ROOT, "oracle"),
              os.path.join(ROOT, "tests", "oracle_check.c"), os.path.join(ROOT, "oracle", "oracle.c"),
              "-o", str(exe), "-lm", "-lpthread"])
    assert r.returncode == 0, r.stderr
    r = _run([str(exe)], timeout=600)
    print(r.stdout[-1000:])
    assert r.returncode == 0 and r.stdout.strip().endswith("0 failures"), r.stdout[-2000:] + r.stderr[-4000:]
