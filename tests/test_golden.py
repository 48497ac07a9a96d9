"""The CPU oracle against the committed golden fixtures (tests/golden/).

The fixtures hold exactly-summed answers computed without the oracle
(tests/golden/make_golden.py).  The oracle sums in double, in k order, as
test/test_gemm.c:32-58 and test/test_h.c:63-79 do; for these sizes that double
sum rounds to the same float32 as the exact one, so the comparison is bitwise.
"""
import json
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gemm_golden.npz")


def load_cases():
    z = np.load(GOLDEN)   # allow_pickle stays False
    index = json.loads(str(z["index"]))
    return [(c, {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(c["name"] + "/")}) for c in index]


CASES = load_cases()


def test_fixture_inventory():
    names = {c["name"] for c, _ in CASES}
    kinds = {c["kind"] for c, _ in CASES}
    assert kinds == {"f32cm", "f16rm"}
    for m, n, k in ((3, 5, 7), (33, 65, 17), (1, 64, 64), (64, 1, 64)):
        for v in ("NN", "NT", "TN", "TT"):
            assert f"f32cm_{m}x{n}x{k}_{v}" in names
    assert {"closed_alpha0", "closed_outer_k1", "closed_identity", "closed_integers"} <= names


@pytest.mark.parametrize("case", [c for c in CASES if c[0]["kind"] == "f32cm"], ids=lambda c: c[0]["name"])
def test_oracle_f32_cm_matches_golden(case):
    meta, a = case
    C = a["C"].copy()
    oracle.ref_gemm_cm(meta["ta"], meta["tb"], meta["m"], meta["n"], meta["k"], meta["alpha"], a["A"], meta["lda"],
                       a["B"], meta["ldb"], meta["beta"], C, meta["ldc"])
    assert np.array_equal(C.view(np.uint32), a["out"].view(np.uint32))


@pytest.mark.parametrize("case", [c for c in CASES if c[0]["kind"] == "f16rm"], ids=lambda c: c[0]["name"])
def test_oracle_f16_rm_matches_golden(case):
    meta, a = case
    args = (meta["op_a"], meta["op_b"], meta["M"], meta["N"], meta["K"], a["A"], meta["lda"], a["B"], meta["ldb"],
            meta["alpha"], meta["beta"])
    C16 = a["C"].copy()
    oracle.ref_gemm_f16_rm(*args, C16, meta["ldc"], threads=1)
    assert np.array_equal(C16, a["out16"])
    C32 = a["Cf"].copy()
    oracle.ref_gemm_f16f32_rm(*args, C32, meta["ldc"], threads=1)
    assert np.array_equal(C32.view(np.uint32), a["out32"].view(np.uint32))


def test_golden_check_catches_planted_mistakes():
    """A transposed operand or a dropped k term in the oracle would not match
    the fixtures: apply both mistakes to the oracle's call and see it fail."""
    meta, a = next(c for c in CASES if c[0]["name"] == "f32cm_33x65x17_NT")
    C = a["C"].copy()
    # wrong transpose flag on B (reads B as K x N instead of N x K), same ld
    oracle.ref_gemm_cm(0, 0, 33, 65, 17, 1.0, a["A"], meta["lda"], a["B"], 65, 0.0, C, meta["ldc"])
    assert not np.array_equal(C, a["out"])
    C = a["C"].copy()
    oracle.ref_gemm_cm(0, 1, 33, 65, 16, 1.0, a["A"], meta["lda"], a["B"], meta["ldb"], 0.0, C, meta["ldc"])
    assert not np.array_equal(C, a["out"])
