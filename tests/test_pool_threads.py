"""Concurrency of the pool core, host only (tests/hostcheck/stress_threads.cpp):
8 threads share one pool and run random allocator / fork / beam-fork /
copy-on-write / share / cached-prefix operations on sequences of their own,
each predicting and checking its tables and the exact refcounts of its blocks
while the others run (the C ABI promises that every call is thread-safe,
include/kcmm.h).  Built twice: optimised, and with ThreadSanitizer on the
host build (any data race fails the run)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

SOURCES = [ROOT / "tests/hostcheck/stress_threads.cpp", ROOT / "lattice_amd/csrc/pool_core.cpp",
           ROOT / "lattice_amd/csrc/tiering.cpp"]


def _build(d, name, flags):
    exe = d / name
    subprocess.run(["g++", *flags, "-std=c++17", "-pthread", *map(str, SOURCES), "-o", str(exe)],
                   check=True)
    return exe


@pytest.fixture(scope="module")
def stress_bins(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("no host compiler")
    d = tmp_path_factory.mktemp("stress")
    out = {"o2": _build(d, "stress_o2", ["-O2"])}
    try:
        out["tsan"] = _build(d, "stress_tsan", ["-O1", "-g", "-fsanitize=thread"])
    except subprocess.CalledProcessError:
        out["tsan"] = None
    return out


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_threads_keep_tables_and_refcounts(stress_bins, seed):
    r = subprocess.run([str(stress_bins["o2"]), "8", "6000", str(seed)], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stderr[-2000:]


@pytest.mark.parametrize("seed", [1, 2])
def test_threads_under_thread_sanitizer(stress_bins, seed):
    if stress_bins["tsan"] is None:
        pytest.skip("ThreadSanitizer is not available to the host compiler")
    r = subprocess.run([str(stress_bins["tsan"]), "8", "3000", str(seed)], capture_output=True,
                       text=True, timeout=300)
    assert "ThreadSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stderr[-2000:]
