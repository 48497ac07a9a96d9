"""The reference's own C test programs, run unchanged against this build.

oracle/Makefile (target ref-tests, called by __graft_entry__.build() where the
reference sources are present) compiles test/test_gemm.c and test/test_h.c from
the reference's sources into oracle/_ref/.  Each program dlopens
"./libvkblas_hipblas.so" (test/test_gemm.c:210, test/test_h.c:82), so it runs
from a scratch directory holding links to this build's libvkblas_hipblas.so
and libvkblas_engine.so.  Pass criteria are the programs' own:
  test_gemm: 68 hipblasSgemm cases, 23 strided-batched cases, "ALL PASS" and
             exit 0 (test/test_gemm.c:289-290);
  test_h:    vkblas_gemm_f16 / _bf16 cases, "fails=0" and exit 0
             (test/test_h.c:227-228).
test/test_v9h.c does not compile against ROCm 7's hipBLAS 3 headers (it names
hipblasDatatype_t); its cases are restated in tests/test_gpu_test_h.py.
"""
import os
import subprocess

import pytest

import vkblas_amd as vk

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_BIN = os.path.join(REPO, "oracle", "_ref")


def _run(prog, tmp_path, args=()):
    exe = os.path.join(REF_BIN, prog)
    if not os.path.exists(exe):
        pytest.skip(f"{exe} not built (make -C oracle ref-tests needs the reference sources)")
    for lib in (vk.LIB_PATH, vk.ENGINE_PATH):
        if not os.path.exists(lib):
            pytest.fail(f"{lib} is not built")
        os.symlink(lib, tmp_path / os.path.basename(lib))
    print(f"[reference program] {prog} in {tmp_path}", flush=True)
    r = subprocess.run([exe, *args], cwd=tmp_path, capture_output=True, text=True, timeout=240)
    return r


def test_reference_test_gemm(tmp_path):
    r = _run("test_gemm", tmp_path)
    lines = r.stdout.splitlines()
    cases = [ln for ln in lines if ln.rstrip().endswith(("PASS", "FAIL")) and "|" in ln]
    assert r.returncode == 0, f"rc={r.returncode}\n{r.stdout[-4000:]}\n{r.stderr[-2000:]}"
    assert "ALL PASS (0 failures)" in r.stdout, r.stdout[-4000:]
    assert len(cases) == 17 * 4 + 3 + 5 * 4 + 3, len(cases)
    assert not any(ln.rstrip().endswith("FAIL") for ln in cases)


def test_reference_test_h(tmp_path):
    r = _run("test_h", tmp_path)
    assert r.returncode == 0, f"rc={r.returncode}\n{r.stdout[-4000:]}\n{r.stderr[-2000:]}"
    assert "fails=0" in r.stdout, r.stdout[-4000:]
    ok = [ln for ln in r.stdout.splitlines() if ln.endswith(" OK")]
    # every case the program prints ran on the engine (rc=0): none fell back with an error
    assert ok and all(" rc=0 " in ln for ln in ok), r.stdout[-4000:]
    assert sum(ln.startswith("BATCH") for ln in ok) == 2 * 4 * 3
