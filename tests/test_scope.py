"""The host scope guard (laya-cuda_amd/csrc/scope.hpp) that keeps per-thread kernel timing from
staying armed after a failed stage launch and drains the stream before the static entry point's
lock is released on an error (no GPU: compiled alone with g++)."""
import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "laya-cuda_amd" / "csrc"

PROGRAM = r"""
#include <cstdio>
#include <stdexcept>
#include "scope.hpp"

struct Timing { void* start = nullptr; };
thread_local Timing timing;  // stands in for the library's per-thread launch_timing

static void launch(bool fail) {  // a stage launch that may throw before taking the events
  if (fail) throw std::runtime_error("invalid tile");
  timing = Timing{};  // a launch that ran consumed the events
}

static void run_stage(bool fail, int* marker) {
  timing = Timing{marker};
  const laya::ScopeExit disarm([&] { timing = Timing{}; });
  launch(fail);
}

int main() {
  int marker = 0, runs = 0;
  run_stage(false, &marker);
  if (timing.start) return 1;
  try {
    run_stage(true, &marker);
    return 2;
  } catch (const std::runtime_error&) {
  }
  if (timing.start) return 3;  // disarmed although the launch threw
  {
    laya::ScopeExit guard([&] { ++runs; });
    guard.release();
  }
  if (runs != 0) return 4;
  try {
    laya::ScopeExit drain([&] { ++runs; });
    throw std::runtime_error("copy failed");
  } catch (const std::runtime_error&) {
  }
  if (runs != 1) return 5;
  std::puts("ok");
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_scope_guard_runs_on_error_and_not_after_release(tmp_path):
    src = tmp_path / "scope_test.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "scope_test"
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", f"-I{CSRC}", str(src), "-o", str(exe)], check=True)
    result = subprocess.run([str(exe)], capture_output=True, text=True)
    assert result.returncode == 0 and result.stdout.strip() == "ok", result.returncode
