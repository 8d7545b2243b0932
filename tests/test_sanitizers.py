"""Host code under sanitizers, on the CPU.

The C oracle (the checker) is rebuilt with AddressSanitizer and UBSan and its
tests rerun against that build; the library is rebuilt with AddressSanitizer
on its host code (argument validation, dispatch, launch set-up; the gfx950
code is unchanged) and the C ABI tests rerun against it. Each run is a
subprocess with the matching sanitizer runtime preloaded: gcc's for the
oracle, clang's for the hipcc-built library. No GPU is used.
"""
import glob
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _gcc_runtime(name):
    path = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


def _clang_asan_runtime():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    found = sorted(glob.glob(f"{rocm}/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return found[-1] if found else None


def _run_pytest(files, env_extra):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1",
               **env_extra)
    cmd = [sys.executable, "-m", "pytest", *files, "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider"]
    return subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)


def test_oracle_under_asan_and_ubsan(tmp_path):
    asan, ubsan = _gcc_runtime("libasan.so"), _gcc_runtime("libubsan.so")
    if not (asan and ubsan and shutil.which("make")):
        pytest.skip("gcc sanitizer runtimes or make not available")
    lib = tmp_path / "liboracle_san.so"
    build = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "sanitized", f"SAN_OUT={lib}"],
                           capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = _run_pytest(["tests/test_oracle.py"], {"LD_PRELOAD": f"{asan}:{ubsan}", "ORACLE_LIBRARY": str(lib)})
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-3000:]


def test_c_abi_under_asan(tmp_path):
    runtime = _clang_asan_runtime()
    if runtime is None:
        pytest.skip("clang AddressSanitizer runtime not found")
    from intent_amd.build import build_host_sanitized

    try:
        lib = build_host_sanitized(tmp_path)
    except RuntimeError as error:  # no hipcc here
        pytest.skip(str(error)[:200])
    # the build is instrumented: its host code calls the sanitizer's report hooks
    syms = subprocess.run(["nm", "-D", "--undefined-only", str(lib)], capture_output=True, text=True).stdout
    assert "__asan_report" in syms
    env = {"LD_PRELOAD": runtime, "INTENT_AMD_LIBRARY": str(lib)}
    which = subprocess.run([sys.executable, "-c", "from intent_amd import _native; _native.library(); "
                            "print([l.split()[-1] for l in open('/proc/self/maps') if 'libintent_amd' in l][0])"],
                           cwd=ROOT, env=dict(os.environ, ASAN_OPTIONS="detect_leaks=0", **env), capture_output=True,
                           text=True)
    assert which.stdout.strip() == str(lib), which.stdout + which.stderr
    run = _run_pytest(["tests/test_abi.py", "tests/test_host.py"], env)
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-3000:]
