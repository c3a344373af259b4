"""CPU contract tests of MI355XBackend's caching allocator (pulsatrix::mi355x::CachingAllocator in
pulsatrix_amd/csrc/host/src/caching_allocator.cpp), the cases of the reference's
tests/caching_allocator_test.cpp:44-127: size classes, reuse, statistics, empty_cache, budget
pressure releasing the cache first, device failure -> release -> retry -> bad_alloc, zero bytes and
null, destruction, and the PULSATRIX_HIP_MEMORY_BUDGET_MB budget. The allocator takes its raw
operations as callbacks, so tests/native/caching_allocator_check.cpp drives it with host memory
standing in for HBM."""
import os
import subprocess

import oracle_ctypes as oc

SRC = os.path.join(oc.ROOT, "pulsatrix_amd", "csrc", "host")


def build(tmp_path, extra=()):
    exe = str(tmp_path / "caching_allocator_check")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", *extra, "-I" + os.path.join(SRC, "include"),
                    os.path.join(oc.ROOT, "tests", "native", "caching_allocator_check.cpp"),
                    os.path.join(SRC, "src", "caching_allocator.cpp"), "-o", exe, "-lpthread"], check=True)
    return exe


def test_caching_allocator_contract(tmp_path):
    exe = build(tmp_path)
    env = dict(os.environ, PULSATRIX_HIP_MEMORY_BUDGET_MB="8")
    r = subprocess.run([exe], capture_output=True, text=True, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all allocator checks passed" in r.stdout


def test_caching_allocator_contract_under_address_sanitizer(tmp_path):
    """The same checks with AddressSanitizer and UBSan (host code only): no leak, double free or
    use of a released block."""
    exe = build(tmp_path, ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-g"])
    r = subprocess.run([exe], capture_output=True, text=True, env=dict(os.environ, ASAN_OPTIONS="detect_leaks=1"))
    assert r.returncode == 0, r.stdout + r.stderr
