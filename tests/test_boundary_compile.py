"""The drop-in boundary compiles the reference's callers: tests/reference_callers.cpp makes
every ES* call the reference makes (ESAttention.mm, ESGenerationLoop.mm, ESKVCache.mm,
APLocalSession.mm, AperturaResearch/main.mm), with the reference's argument order and
types, and must compile against include/es with mx::array spelled es::Tensor.  A
planted mismatch (an argument order the headers do not take) must fail to compile, so
the check is not vacuous.  Host compiler only; no GPU."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TU = os.path.join(ROOT, "tests", "reference_callers.cpp")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def _compile(source: str):
    cxx = os.environ.get("CXX", "g++")
    if not shutil.which(cxx):
        pytest.skip(f"{cxx} not found")
    cmd = [cxx, "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(ROCM, "include"), "-I", os.path.join(ROOT, "include"), "-x", "c++", "-"]
    return subprocess.run(cmd, input=source, capture_output=True, text=True)


def test_reference_call_sites_compile_against_the_headers():
    r = _compile(open(TU).read())
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("old,new", [
    # updateRaw's prealloc flag and the layer swapped
    ("cache->updateRaw(layerIdx, kRaw, prealloc)", "cache->updateRaw(kRaw, layerIdx, prealloc)"),
    # esDecodeAttnGlobal without its pitch
    ("raw.buffer, raw.len, raw.pitch, kw", "raw.buffer, raw.len, kw"),
    # a compiled-step member the headers would not declare
    ("cache->endStep();", "cache->endSteps();"),
])
def test_a_planted_signature_mismatch_fails_to_compile(old, new):
    src = open(TU).read()
    assert old in src
    r = _compile(src.replace(old, new))
    assert r.returncode != 0


HOST_PROGRAM = r'''
#include "es/ESDecodeAttn.h"
#include "es/ESKVCache.h"
#include <cstdio>
#include <stdexcept>
template <class E, class F> static int expect(F f, const char *what) {
    try { f(); } catch (const E &) { return 0; } catch (...) { std::printf("%s: wrong exception\n", what); return 1; }
    std::printf("%s: no exception\n", what);
    return 1;
}
int main() {
    using namespace es;
    int bad = 0;
    ESKVCache c(4);
    Tensor t = Tensor::wrap(reinterpret_cast<void *>(0x1000), {2, 1, 128}, Dtype::bf16);
    // quantized KV is not built: the reference's runtime_error class for unsupported storage
    bad += expect<std::runtime_error>([&] { c.updateQuant(1, t, t, 64, 4, true); }, "updateQuant");
    bad += expect<std::invalid_argument>([&] { c.updateQuant(7, t, t, 64, 4); }, "updateQuant layer");
    // compiled-step accessors on an empty slot, and malformed step indices
    bad += expect<std::runtime_error>([&] { (void) c.slotK(0); }, "slotK");
    bad += expect<std::runtime_error>([&] { (void) c.takeSlotV(0); }, "takeSlotV");
    bad += expect<std::invalid_argument>([&] { c.beginStep(Tensor{}, Tensor{}); }, "beginStep");
    // ESSharedKV: what one layer type stores, the same type reads back
    ESSharedKV kv;
    kv.store(true, t, t);
    auto got = kv.get(true);
    if (got.first.data != t.data || got.second.data != t.data) { std::printf("ESSharedKV\n"); ++bad; }
    bad += expect<std::bad_optional_access>([&] { (void) kv.get(false); }, "ESSharedKV empty type");
    std::printf(bad ? "FAIL\n" : "OK\n");
    return bad;
}
'''


def test_host_side_behaviour_of_the_added_members(tmp_path):
    """updateQuant throws std::runtime_error, ESSharedKV stores and reads per layer type,
    and the compiled-step accessors reject empty slots and malformed indices -- all on the
    host, through libesda.so (no device call is made)."""
    cxx = os.environ.get("CXX", "g++")
    lib = os.path.join(ROOT, "apertura_amd", "libesda.so")
    if not os.path.exists(lib):
        pytest.skip("libesda.so not built")
    src = tmp_path / "host.cpp"
    src.write_text(HOST_PROGRAM)
    exe = tmp_path / "host"
    r = subprocess.run([cxx, "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
                        "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe), lib,
                        f"-Wl,-rpath,{os.path.dirname(lib)}", "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
                        f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0 and "OK" in run.stdout, run.stdout + run.stderr
