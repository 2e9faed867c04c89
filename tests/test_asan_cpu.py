"""The C ABI's host code under AddressSanitizer: the CPU tests that drive libpsgdk.so without a GPU (argument
validation, workspace planning, option tables, group checks, the plugin surface) run again in a child process
against the library with capi.cpp built with the host sanitizer (psgd_pro_amd.build --asan), the sanitizer runtime
preloaded. Any heap or stack overrun in those paths ends the child with the sanitizer's report."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_host_code_under_address_sanitizer():
    sys.path.insert(0, ROOT)
    from psgd_pro_amd import build as b
    src = os.path.join(b.CSRC, "capi.cpp")
    if not os.path.exists(b.ASAN_LIB) or os.path.getmtime(b.ASAN_LIB) < max(os.path.getmtime(src),
                                                                              os.path.getmtime(b.LIB)):
        objs = [os.path.join(b.BUILD, os.path.splitext(s)[0] + ".o") for s in b.SOURCES]
        assert all(os.path.exists(o) for o in objs), "build the library first (python -m psgd_pro_amd.build)"
        b.build_asan(objs)
    env = dict(os.environ, PSGDK_LIB=b.ASAN_LIB, LD_PRELOAD=b.asan_runtime(),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0")
    probe = ("import torch; from psgd_pro_amd import _lib; _lib.lib(); "
             "print(next(l.split()[-1] for l in open('/proc/self/maps') if 'libpsgdk' in l))")
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("libpsgdk_asan.so"), (r.stdout + r.stderr)[-2000:]
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
                        "tests/test_lib_cpu.py", "tests/test_plugin_cpu.py"], cwd=ROOT, env=env,
                       capture_output=True, text=True, timeout=600)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert "AddressSanitizer" not in r.stderr, tail
    assert " passed" in r.stdout, tail
