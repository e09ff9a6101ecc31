"""libnnc_hip.so against the reference's golden vectors, every case, through the
C-ABI. Bar: bit-exact for data movement / integer / comparison ops and the
ops whose arithmetic order is reproduced exactly; otherwise the reference's
pass rule with the floating-point bar: |got - ref| <= 1e-4 or <= 1e-3 * |ref|."""

from __future__ import annotations

import numpy as np
import pytest

import caserun
from conftest import GOLDEN

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-4, 1e-3


def _batched_expected(case, oracle_lib, abi):
    """True batched MatMul from the oracle's 2-D path, one batch at a time."""
    a = case["tensors"]["a"]
    b = case["tensors"]["b"]
    out = case["tensors"]["out"]
    M, N = out.shape[-2:]
    K = a.shape[-1]
    A = a.reshape(-1, M, K)
    B = b.reshape(-1, K, N)
    res = np.zeros((A.shape[0], M, N), np.float32)
    for q in range(A.shape[0]):
        c2 = {"name": "slice", "op": "nnc_matmul",
              "tensors": {"a": A[q].copy(), "b": B[q % B.shape[0]].copy(), "out": np.zeros((M, N), np.float32)},
              "args": [("t", "a"), ("t", "b"), ("t", "out")], "outputs": ["out"]}
        res[q] = caserun.run_case(oracle_lib, c2, abi)["out"]
    return {"out": res.reshape(out.shape)}


@pytest.mark.parametrize("case", GOLDEN, ids=[c["name"] for c in GOLDEN])
def test_hip_matches_reference(case, hip, dmem, abi, oracle_lib):
    from nnc_py_amd import runtime
    print(f"case {case['name']} op {case['op']}", flush=True)
    got = caserun.run_case(hip, case, abi, dmem)
    expected = case["expected"]
    if case.get("hip") == "batched":
        expected = _batched_expected(case, oracle_lib, abi)
    for key, exp in expected.items():
        g = got[key]
        if case["bar"] == "exact":
            if not caserun.same_bits(g, exp):
                bad = np.nonzero(g.view(np.uint8).reshape(g.size, -1).any(1)
                                 != exp.view(np.uint8).reshape(exp.size, -1).any(1))[0]
                diff = np.nonzero(g.ravel().view(np.uint8) != exp.ravel().view(np.uint8))[0][:5]
                pytest.fail(f"{key}: not bit-exact; first differing bytes {diff}; "
                            f"got {g.ravel()[:6]} want {exp.ravel()[:6]} ({len(bad)})")
        else:
            bad = caserun.fp_violations(g, exp, ATOL, RTOL)
            assert bad.size == 0, (
                f"{key}: {bad.size}/{g.size} outside atol {ATOL} / rtol {RTOL}; first "
                f"{bad[:5]}: got {g.ravel()[bad[:5]]} want {exp.ravel()[bad[:5]]}")
    if case["name"].endswith("_mismatch"):
        code, _ = runtime.last_error()
        assert code != 0, "shape mismatch must be reported"
