"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the
oracle): the oracle must reproduce them bit for bit (CPU), and the gfx950 rows the
resolver picks must match them within the parity bound (GPU)."""
import glob
import os

import numpy as np
import pytest

import libr3d_amd as R
import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fixtures_present():
    assert len(FIXTURES) >= 6


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_oracle_reproduces_fixture(path):
    f = _load(path)
    q, sc = O.quant_act_fp8(f["x"], 128)
    assert np.array_equal(sc, f["AS"])
    if not bool(f["a_edited"]):
        assert np.array_equal(q, f["A"])
    if str(f["dtype"]) == "mxfp4a8":
        Y, Yf, S = O.quant_dot_mxfp4a8(f["A"], f["AS"], f["B"], f["BS"])
    else:
        Y, Yf, S = O.quant_dot_fp8a8(f["A"], f["AS"], f["B"], f["BS"], int(f["rblk"]))
    assert np.array_equal(Y, f["Y"])
    assert np.array_equal(Yf.view(np.uint32), f["Yf"].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_rows_match_fixture(gpu, path):
    from tests import gpu_util as gu
    f = _load(path)
    dtype = str(f["dtype"])
    M, K = f["A"].shape
    N = f["B"].shape[0]
    group = 32 if dtype == "mxfp4a8" else 128
    row = R.resolve("gemm_nt_q", {"dtype": dtype, "M": M, "N": N, "K": K, "group": group})["name"]
    rc, Y, guards = gu.run_row(row, dtype, f["A"], f["AS"], f["B"], f["BS"], M, N, K, gpu)
    assert rc == R.RAD_OK and guards
    c = gu.compare(Y, f["Y"], f["Yf"], f["S"], K, f["S8"])
    assert c["sentinel_left"] == 0 and c["nan_mismatch"] == 0 and c["inf_mismatch"] == 0, c
    assert c["max_viol"] <= 1.0, c
