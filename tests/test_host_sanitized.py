"""The host layer of the C ABI under the address and undefined-behaviour sanitizers (CPU).

kappa_amd/csrc/host.cpp holds every argument check, the workspace layout and the
program choice of the entry points (the failure handling in front of every HIP
call: the reference's ValueErrors, kappa/qwen3/ffn_moe.py:47-48, 239-240, 251-252,
299). tests/sanitize/host_checks.cpp drives it through the cases of test_abi.py,
the documented no-allocation limits, overflow edges and a layout sweep; here it is
built with g++ -fsanitize=address,undefined (no recovery: the first report
aborts) and run."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from conftest import ROOT

CXX = shutil.which(os.environ.get("CXX", "g++"))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]

pytestmark = pytest.mark.skipif(CXX is None, reason="no C++ compiler")


def _build(tmp_path, sources, name):
    exe = str(tmp_path / name)
    cmd = [CXX, "-std=c++17", "-Wall", "-Wextra", "-Werror", *SAN, "-I", os.path.join(ROOT, "include"), "-I",
           os.path.join(ROOT, "kappa_amd", "csrc"), *sources, "-o", exe]  # fmt: skip
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def _run(exe):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    return subprocess.run([exe], capture_output=True, text=True, env=env, timeout=120)


def test_host_layer_is_clean_under_asan_and_ubsan(tmp_path):
    exe = _build(tmp_path, [os.path.join(ROOT, "kappa_amd", "csrc", "host.cpp"),
                            os.path.join(ROOT, "tests", "sanitize", "host_checks.cpp")], "host_checks")  # fmt: skip
    r = _run(exe)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "host checks: ok" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr


def test_the_sanitizers_are_live(tmp_path):
    """The same flags stop a planted out-of-range enum load and a heap overflow, so a
    clean run above means something."""
    src = tmp_path / "planted.cpp"
    src.write_text(
        '#include <stdlib.h>\n#include <string.h>\n#include "kmoe.h"\n'
        "int main(int argc, char**) {\n"
        "  int raw = 7; kmoe_impl i; memcpy(&i, &raw, sizeof i);\n"
        "  if (argc > 1) { char* p = (char*)malloc(8); p[argc + 7] = 1; free(p); return 0; }\n"
        "  volatile kmoe_impl j = i; return j == KMOE_IMPL_RAGGED;\n}\n"
    )
    exe = _build(tmp_path, [str(src)], "planted")
    r = _run(exe)
    assert r.returncode != 0 and "not a valid value for type 'kmoe_impl'" in r.stderr, r.stderr
    r = subprocess.run([exe, "x"], capture_output=True, text=True, timeout=120)
    # whichever sees it first: ASan's shadow check or UBSan's object-size check
    assert r.returncode != 0 and ("heap-buffer-overflow" in r.stderr or "insufficient space" in r.stderr), r.stderr
