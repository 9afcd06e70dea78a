"""The reference's own C caller of the ABI, examples/kcmm_c_integration.c
(its 20 tests: pool lifecycle, null safety, allocation, sequences, block
tables, VA queries, stats, metrics, tiering-off behaviour, hints,
protection, plus the kcmm_config_t layout asserts at lines 29-40), built by
`make -C oracle ref` from where it lies under /root/reference against this
build's include/kcmm.h, with -Werror.

* CPU: the binary linked to the host-check library (the product's pool code
  over host memory) must report every check passed;
* GPU: the binary linked to lattice_amd/libkcmm.so must do the same on the
  MI355X.

The binaries are built here (this container holds the reference tree) and
travel to the GPU box with the tree; a test skips when its binary is absent.
"""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF_DIR = ROOT / "oracle" / "_ref"


def _run(binary: Path):
    if not binary.exists():
        pytest.skip(f"{binary.name} not built (needs /root/reference at build time)")
    proc = subprocess.run([str(binary)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True, timeout=120)
    out = proc.stdout
    print(out, flush=True)
    assert proc.returncode == 0, out
    assert "[FAIL]" not in out
    results = [l for l in out.splitlines() if l.startswith("Results:")]
    assert results and results[-1].startswith("Results: 22 passed, 0 failed"), results
    return out


def test_reference_c_caller_hostcheck():
    _run(REF_DIR / "kcmm_c_integration_hostcheck")


@pytest.mark.gpu
def test_reference_c_caller_on_gpu():
    _run(REF_DIR / "kcmm_c_integration")
