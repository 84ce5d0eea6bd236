"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer:
capi.hip is compiled with the sanitizers on its host side (-Xarch_host) and
linked with a fuzzer (tests/sanitize/capi_fuzz.cpp) that calls every entry
point with random and near-valid descriptors -- wrong ndim and dtypes, zero,
negative and huge sizes and strides, misaligned or null pointers, sizes at
the int32 / int64 limits.  Every call must return an error code (or, past
validation, fail at the launch for want of a device) without a sanitizer
report.  CPU only: where a GPU is visible a validated call would launch on
the fuzzer's fake pointers, so the fuzzer refuses to run there."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"
CLANG = "/opt/rocm/bin/amdclang++"
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]


def _gpu_visible():
    return os.path.exists("/dev/kfd")


@pytest.mark.skipif(not (os.path.exists(HIPCC) and os.path.exists(CLANG)), reason="ROCm compilers not found")
@pytest.mark.skipif(_gpu_visible(), reason="fuzzes with fake device pointers: hosts without a GPU only")
def test_capi_fuzz_under_asan_and_ubsan(tmp_path):
    lib = os.path.join(ROOT, "saga_amd", "libsaga_amd.so")
    if not os.path.exists(lib):
        pytest.skip("libsaga_amd.so not built")
    common = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC",
              "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", os.path.join(ROOT, "include")]
    capi_o, fuzz_o, exe = (str(tmp_path / n) for n in ("capi_asan.o", "fuzz.o", "capi_fuzz"))
    for src, obj in ((os.path.join(ROOT, "saga_amd", "csrc", "capi.hip"), capi_o),
                     (os.path.join(ROOT, "tests", "sanitize", "capi_fuzz.cpp"), fuzz_o)):
        r = subprocess.run([HIPCC, *common, *SAN, "-c", src, "-o", obj], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-3000:]
    # host-only link (no device code): the sanitizer runtimes of the same clang
    r = subprocess.run([CLANG, "-fsanitize=address,undefined", fuzz_o, capi_o, lib, "-L/opt/rocm/lib", "-lamdhip64",
                        f"-Wl,-rpath,{os.path.dirname(lib)}", "-Wl,-rpath,/opt/rocm/lib", "-o", exe],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, "300000"], capture_output=True, text=True, env=env, timeout=300)
    print(r.stdout[-500:])
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-4000:])
    assert "rejected" in r.stdout and "Sanitizer" not in r.stderr, r.stderr[-4000:]
