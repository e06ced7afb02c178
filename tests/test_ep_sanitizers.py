"""Host sanitizer lane for the C ABI (CPU only).

The plugin EP and the mock ORT host are rebuilt with AddressSanitizer and UndefinedBehaviorSanitizer
(`make -C tests/mock_ort asan`: g++, host code only; the EP links the regular HIP library), and the
CPU tests that drive the EP through the mock host -- factory, claim, compile, allocator and data
transfer contracts, norm / GQA / QMoE claims -- run again against those builds in a child process
with the sanitizer runtime preloaded.  Any report (heap or stack overflow, use after free, double
free, undefined behaviour) fails the lane.  A control plants a heap overflow in a throwaway
snippet built with the same flags and checks that the lane reports it, so a lane that silently
stopped instrumenting would fail too.  (The reference's counterpart is its planted-violation
validation control, rust/tests/validation_control.rs:114-262.)
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
MOCK = ROOT / "tests" / "mock_ort"
SAN_FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
             "-fno-omit-frame-pointer"]
LANE_TESTS = ["tests/test_ep_boundary.py", "tests/test_ep_norm.py", "tests/test_ep_gqa.py",
              "tests/test_ep_qmoe.py", "tests/test_gqa_abi.py"]

pytestmark = pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++ for the lane")


def _runtime_env(log_dir: Path) -> dict:
    gxx = shutil.which("g++")
    asan = subprocess.run([gxx, "-print-file-name=libasan.so"], capture_output=True,
                          text=True, check=True).stdout.strip()
    stdcxx = subprocess.run([gxx, "-print-file-name=libstdc++.so.6"], capture_output=True,
                            text=True, check=True).stdout.strip()
    env = dict(os.environ)
    # libstdc++ is preloaded with the runtime so ASan resolves the C++ throw it intercepts
    # (the interpreter itself does not link libstdc++)
    env["LD_PRELOAD"] = f"{asan}:{stdcxx}"
    env["ASAN_OPTIONS"] = f"detect_leaks=0:abort_on_error=1:log_path={log_dir / 'asan'}"
    env["UBSAN_OPTIONS"] = f"print_stacktrace=1:halt_on_error=1:log_path={log_dir / 'ubsan'}"
    return env


def _reports(log_dir: Path) -> str:
    return "".join(p.read_text(errors="replace") for p in sorted(log_dir.glob("*san.*")))


@pytest.fixture(scope="module")
def asan_builds():
    r = subprocess.run(["make", "-C", str(MOCK), "asan"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    mock = MOCK / "build_asan" / "libmock_ort.so"
    ep = MOCK / "build_asan" / "libonnxruntime_mi355x_ep.so"
    assert mock.exists() and ep.exists()
    return mock, ep


def test_ep_and_mock_host_are_clean_under_asan_and_ubsan(asan_builds, tmp_path):
    mock, ep = asan_builds
    env = _runtime_env(tmp_path)
    env["MI355X_TEST_MOCK_SO"] = str(mock)
    env["MI355X_TEST_EP_SO"] = str(ep)
    r = subprocess.run([sys.executable, "-m", "pytest", *LANE_TESTS, "-q", "-m", "not gpu",
                        "-p", "no:cacheprovider"], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=600)
    reports = _reports(tmp_path)
    assert r.returncode == 0 and not reports, (r.stdout[-3000:] + r.stderr[-3000:] + reports)
    assert " passed" in r.stdout


def test_lane_reports_a_planted_heap_overflow(tmp_path):
    src = tmp_path / "planted.cpp"
    src.write_text('extern "C" int planted(int i) { int* p = new int[4]; p[i] = 1; '
                   'int v = p[0]; delete[] p; return v; }\n')
    so = tmp_path / "libplanted.so"
    subprocess.run(["g++", "-O0", "-g", "-shared", "-fPIC", *SAN_FLAGS, str(src), "-o", str(so)],
                   check=True)
    env = _runtime_env(tmp_path)
    code = f"import ctypes; ctypes.CDLL({str(so)!r}).planted(4)"
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "heap-buffer-overflow" in _reports(tmp_path)
