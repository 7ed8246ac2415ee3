"""The host-side resolver (furiosa-opt_amd/csrc/mapping.cpp and json.hpp: the parsers of the caller's
MappingSerde JSON, m![..] text and offsets, and the resolution behind every seam op) built with
AddressSanitizer and UndefinedBehaviorSanitizer and driven by tests/host_sanitize/resolver_harness.cpp:
valid mappings through every resolution step, and 100k malformed JSON inputs that must each end in
an exception. Host code only; no GPU code is built with a sanitizer."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_resolver_under_asan_and_ubsan(tmp_path):
    exe = tmp_path / "resolver_harness"
    build = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
             "-fno-omit-frame-pointer", f"-I{ROOT / 'furiosa-opt_amd' / 'csrc'}",
             str(ROOT / "tests" / "host_sanitize" / "resolver_harness.cpp"),
             str(ROOT / "furiosa-opt_amd" / "csrc" / "mapping.cpp"), "-o", str(exe)]
    res = subprocess.run(build, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-4000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300,
                         env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0", "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert run.returncode == 0 and run.stdout.startswith("ok"), (run.stdout + run.stderr)[-4000:]
