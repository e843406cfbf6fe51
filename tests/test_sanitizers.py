"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only).

libtbe_hip.so is rebuilt with every sanitizer flag on its host compilation
(`fbgemm-ascend_amd/build.py --sanitize`: planner, C-ABI argument checks, launch
set-up) and the oracle with clang's sanitizers (`make -C oracle asan`).  The host
suites that reach them through ctypes (C-ABI planner and rejection paths, the
oracle and its pins, the block_bucketize and permute host contracts) then run in a
child process with clang's ASan runtime preloaded and TBE_HIP_LIB / TBE_ORACLE_LIB
pointing at the sanitized builds.  A positive control checks that the runtime in
that set-up does report an out-of-bounds write.
"""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "fbgemm-ascend_amd")
ASAN_LIB = os.path.join(PKG, "_asan", "libtbe_hip.so")
ASAN_ORACLE = os.path.join(ROOT, "oracle", "_build_asan", "libtbe_oracle.so")
SUITES = ["tests/test_host.py", "tests/test_oracle.py", "tests/test_sparse_ops.py", "tests/test_pooled_ops.py"]


def _build_module():
    sys.path.insert(0, PKG)
    try:
        import build  # fbgemm-ascend_amd/build.py
    finally:
        sys.path.pop(0)
    return build


@pytest.fixture(scope="module")
def sanitized_env():
    if not shutil.which("hipcc") and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not available")
    b = _build_module()
    csrc = os.path.join(PKG, "csrc")
    sources = [os.path.join(csrc, s) for s in b.HIP_SOURCES]
    sources += [os.path.join(csrc, s) for s in os.listdir(csrc) if s.endswith(".h")]
    sources += [os.path.join(ROOT, "include", s) for s in os.listdir(os.path.join(ROOT, "include"))]
    sources.append(os.path.join(ROOT, "oracle", "tbe_oracle.c"))
    newest = max(os.path.getmtime(s) for s in sources)
    if not all(os.path.exists(p) and os.path.getmtime(p) >= newest for p in (ASAN_LIB, ASAN_ORACLE)):
        b.build_sanitized()
    env = dict(os.environ)
    env.update(LD_PRELOAD=b.asan_runtime(), TBE_HIP_LIB=ASAN_LIB, TBE_ORACLE_LIB=ASAN_ORACLE,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    return env


def test_host_suites_clean_under_asan_ubsan(sanitized_env):
    r = subprocess.run([sys.executable, "-m", "pytest", *SUITES, "-m", "not gpu", "-q", "-p", "no:cacheprovider",
                        "-x"], cwd=ROOT, env=sanitized_env, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    assert " passed" in out


def test_sanitized_libraries_are_the_ones_loaded(sanitized_env):
    code = ("import sys; sys.path.insert(0, %r); import __graft_entry__ as g; p = g.load_package(); "
            "o = g.load_oracle(); p.capi.lib(); o.lib(); "
            "maps = open('/proc/self/maps').read(); "
            "print(%r in maps, %r in maps, 'libclang_rt.asan' in maps)") % (ROOT, ASAN_LIB, ASAN_ORACLE)
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=sanitized_env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert r.stdout.split()[-3:] == ["True", "True", "True"], r.stdout


def test_positive_control_reports_overflow(sanitized_env):
    """The same process set-up reports a heap overflow made through the sanitized oracle."""
    code = ("import ctypes, sys; sys.path.insert(0, %r); import __graft_entry__ as g; o = g.load_oracle(); "
            "src = ctypes.create_string_buffer(8192); dst = ctypes.create_string_buffer(4096); "
            "o.lib().oracle_half_to_float_n(ctypes.addressof(src), ctypes.addressof(dst), 2048)") % ROOT
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=sanitized_env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode != 0
    assert "heap-buffer-overflow" in r.stderr, r.stderr[-2000:]
