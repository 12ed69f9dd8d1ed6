"""The CPU test suite under AddressSanitizer and UndefinedBehaviorSanitizer.

The oracle (oracle/_sanitize, ``make -C oracle sanitize``) and the library's
host code (oxidizedmlx_amd/_sanitize, ``python -m oxidizedmlx_amd.build
--sanitize``; device code is not instrumented) are rebuilt with ASan + UBSan
by the ROCm clang and loaded in a child pytest through MLXHIP_ORACLE_LIB and
MLXHIP_LIB, with the clang sanitizer runtime preloaded. This is the build's
counterpart of the reference's valgrind job over its C ABI
(.github/workflows/ci.yml:52-72, --errors-for-leak-kinds=definite,indirect):
any invalid access, use after free or undefined behaviour in those sources
ends the child with an error. Leak checking is off because the interpreter
itself does not free everything at exit; the bounded-memory loops of
tests/test_gpu_lifecycle.py cover leaks of device memory.

A planted heap overflow in a throwaway C file, built with the same flags,
shows that the runtime reports such errors in this setup."""
import os
import subprocess
import sys
import textwrap

import pytest

from oracle import cpu_ref
from oxidizedmlx_amd import build as hb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_CFLAGS = ["-O1", "-g", "-fPIC", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
              "-fno-sanitize-recover=undefined", "-shared-libsan"]


def newest_source(*dirs) -> float:
    t = 0.0
    for d in dirs:
        for base, _, files in os.walk(d):
            for f in files:
                if f.endswith((".c", ".h", ".cpp", ".hpp", ".hip")):
                    t = max(t, os.path.getmtime(os.path.join(base, f)))
    return t


def stale(lib: str, *dirs) -> bool:
    return not os.path.exists(lib) or os.path.getmtime(lib) < newest_source(*dirs)


@pytest.fixture(scope="module")
def sanitized():
    if os.environ.get("LD_PRELOAD"):
        pytest.skip("this process environment already preloads a library; the sanitizer runtime "
                    "must be the first one loaded, so the sanitized run is left to hosts without one")
    inc = os.path.join(ROOT, "include")
    if stale(cpu_ref.SAN_LIB, cpu_ref.HERE, inc):
        cpu_ref.build(sanitize=True)
    if stale(hb.SAN_LIB, hb.CSRC, inc):
        hb.build(verbose=False, sanitize=True)
    env = dict(os.environ)
    env.update(LD_PRELOAD=hb.sanitizer_runtime(), ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", MLXHIP_LIB=hb.SAN_LIB,
               MLXHIP_ORACLE_LIB=cpu_ref.SAN_LIB)
    return env


def run(env, args, timeout=600):
    return subprocess.run([sys.executable, *args], cwd=ROOT, env=env, capture_output=True, text=True,
                          timeout=timeout)


def test_sanitized_builds_are_the_ones_loaded(sanitized):
    code = textwrap.dedent("""
        from oracle import cpu_ref
        from oxidizedmlx_amd import abi
        cpu_ref.load(); abi.load_library()
        maps = open('/proc/self/maps').read()
        print('\\n'.join(sorted({l.split()[-1] for l in maps.splitlines()
                                  if 'libmlx' in l or 'asan' in l})))
    """)
    r = run(sanitized, ["-c", code])
    assert r.returncode == 0, r.stderr[-3000:]
    loaded = r.stdout.split()
    assert hb.SAN_LIB in loaded and cpu_ref.SAN_LIB in loaded, loaded
    assert any("libclang_rt.asan" in p for p in loaded), loaded


def test_planted_overflow_is_reported(sanitized, tmp_path):
    src = tmp_path / "planted.c"
    src.write_text("#include <stdlib.h>\n"
                   "int planted(int n) { int* p = malloc(n * sizeof(int)); int v = p[n]; free(p); return v; }\n")
    so = tmp_path / "libplanted.so"
    subprocess.run(["/opt/rocm/llvm/bin/clang", *SAN_CFLAGS, "-shared", "-o", str(so), str(src)], check=True)
    r = run(sanitized, ["-c", f"import ctypes; ctypes.CDLL({str(so)!r}).planted(4)"])
    assert r.returncode != 0
    assert "heap-buffer-overflow" in r.stderr, r.stderr[-2000:]


def test_cpu_suite_clean_under_asan_ubsan(sanitized):
    r = run(sanitized, ["-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
                        "--ignore=tests/test_sanitizers.py", "tests"])
    tail = (r.stdout[-3000:] + r.stderr[-3000:])
    print(tail)
    assert r.returncode == 0, tail
    assert "AddressSanitizer" not in r.stderr and "runtime error:" not in r.stderr, tail
    assert " passed" in r.stdout
