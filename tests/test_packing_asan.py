"""The host-side parser of caller-supplied request blocks (laya-cuda_amd/csrc/packing.cpp: layout,
validation, attention tile and head-row lists) built on its own with AddressSanitizer and UBSan and
fed well-formed, corrupted and random blocks by tests/packing_fuzz.cpp (no GPU)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "laya-cuda_amd" / "csrc"


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")
def test_malformed_blocks_under_address_sanitizer(tmp_path):
    exe = tmp_path / "packing_fuzz"
    build = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
             "-fno-sanitize-recover=all", f"-I{CSRC}", str(ROOT / "tests" / "packing_fuzz.cpp"),
             str(CSRC / "packing.cpp"), "-o", str(exe)]
    subprocess.run(build, check=True, capture_output=True, text=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300,
                         env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0", "UBSAN_OPTIONS": "print_stacktrace=1"})
    print(run.stdout, run.stderr[-4000:])
    assert run.returncode == 0, run.stderr[-4000:]
    assert "AddressSanitizer" not in run.stderr and "runtime error" not in run.stderr
    accepted, refused = (int(w) for w in run.stdout.split()[1:6:4])
    assert accepted > 1000 and refused > 1000
