"""Differential fuzz of the pool core's block tables and reference counts
against the oracle pool, host only (tests/hostcheck/fuzz_pool.cpp: beam forks
through lazily counted shared bases, single forks, copy-on-write, unregister,
frees including blocks a table still holds, share_prefix, cached-prefix
references and append privacy checks, compared step by step)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def fuzz_bin(tmp_path_factory):
    if shutil.which("g++") is None or shutil.which("gcc") is None:
        pytest.skip("no host compiler")
    d = tmp_path_factory.mktemp("fuzz")
    obj = d / "oracle.o"
    subprocess.run(["gcc", "-O2", "-c", str(ROOT / "oracle/oracle.c"), "-o", str(obj)], check=True)
    exe = d / "fuzz_pool"
    subprocess.run(["g++", "-O2", "-std=c++17", str(ROOT / "tests/hostcheck/fuzz_pool.cpp"),
                    str(ROOT / "lattice_amd/csrc/pool_core.cpp"),
                    str(ROOT / "lattice_amd/csrc/tiering.cpp"), str(obj), "-o", str(exe), "-lm"],
                   check=True)
    return exe


@pytest.mark.parametrize("seed", range(1, 25))
def test_pool_matches_oracle_under_random_ops(fuzz_bin, seed):
    r = subprocess.run([str(fuzz_bin), str(seed), "3000"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stderr[-2000:]
