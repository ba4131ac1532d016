"""A failed arm hands its launch to the next one on the same operands, as the reference's
entries do (src/r3d_gemm_mxfp4.hip:1666-1670 skinny -> tile, :2118-2122 q8x -> legacy
walk; this build's split K -> the unsplit tile walk), instead of returning RAD_E_DEVICE at issue time.  The failures are forced from the
host with the test lever R3D_GFX950_FAIL_ARM, which makes the named arms report a launch
failure without launching anything; each setting runs in a child process (the lever is
read once per process), whose calls must still succeed, log the failure, and match the
oracle within the bar of tests/test_gpu_gemm.py.  The same child runs the tile rows' K split
with each of its two kernels (R3D_GFX950_SPLITK_KERNEL), and the e4m3 prefill on its
four-wave tile (R3D_GFX950_F8_TILE), against the same bar."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

_CHILD = r"""
import json, sys
sys.path.insert(0, %r)
import numpy as np
import torch
import libr3d_amd as R
import oracle as O
from tests import gpu_util as gu
from tests.test_gpu_gemm import _mx_case, _f8_case
dev = torch.device("cuda:0")
out = []
for row, dtype, M, N, K, *sc in %r:
    if dtype == "mxfp4a8":
        A, AS, B, BS = _mx_case(M, N, K, M + N)
        Yr, Yf, S = O.quant_dot_mxfp4a8(A, AS, B, BS, nthreads=8)
    else:
        A, AS, B, BS = _f8_case(M, N, K, M + N, 1)
        Yr, Yf, S = O.quant_dot_fp8a8(A, AS, B, BS, 1, nthreads=8)
    S8 = O.group8_mag(dtype, A, AS, B, BS, 1, nthreads=8)
    rc, Y, guards = gu.run_row(row, dtype, A, AS, B, BS, M, N, K, dev,
                               scratch=sc[0] if sc else None)
    c = gu.compare(Y, Yr, Yf, S, K, S8)
    out.append([row, M, rc, guards, c["max_viol"], c["sentinel_left"], c["nan_mismatch"]])
print("RESULT " + json.dumps(out))
"""

MX_DEC, MX_TILE, F8_DEC = "gemm_nt_q_mxfp4_decode", "gemm_nt_q_mxfp4", "gemm_nt_q_fp8a8_decode"


@pytest.mark.parametrize("arms,cases,logged", [
    # the quad GEMV fails: M <= 4 runs on the 16-row GEMV
    ("quad", [(MX_DEC, "mxfp4a8", 1, 300, 1024), (F8_DEC, "fp8a8", 3, 300, 1024)],
     "quad decode GEMV launch FAILED"),
    # the line GEMV fails: M = 5..16 runs on the 16-row GEMV
    ("lines", [(MX_DEC, "mxfp4a8", 9, 300, 1024), (F8_DEC, "fp8a8", 16, 300, 1024)],
     "line decode GEMV launch FAILED"),
    # the skinny band's passes fail: the prefill pipeline takes M = 17..64
    ("skinny", [(MX_TILE, "mxfp4a8", 40, 1000, 2048)], "skinny line GEMV launch FAILED"),
    # split K fails (hook-sized scratch handed over): the whole K walk recomputes Y
    ("splitk", [(MX_TILE, "mxfp4a8", 40, 1000, 2048, "hook"),
                ("gemm_nt_q_fp8a8", "fp8a8", 64, 520, 4096, "hook")],
     "split-K prefill launch FAILED"),
    # the decode rows' split fails: the line GEMV (M = 9) and the 16-row GEMV (M = 4 on
    # activation rows the quad GEMV cannot stage) take the launch
    ("splitk", [(MX_DEC, "mxfp4a8", 9, 1024, 65536, "hook"),
                (F8_DEC, "fp8a8", 4, 3200, 21504, "hook")],
     "split-K decode launch FAILED"),
])
def test_failed_arm_falls_back(gpu, arms, cases, logged):
    env = dict(os.environ, R3D_GFX950_FAIL_ARM=arms, R3D_DEBUG_GEMM="1")
    p = subprocess.run([sys.executable, "-c", _CHILD % (ROOT, cases)], env=env,
                       capture_output=True, text=True, timeout=300)
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-2000:]
    assert logged in p.stderr, p.stderr[-2000:]
    line = [l for l in p.stdout.splitlines() if l.startswith("RESULT ")][-1]
    for row, M, rc, guards, viol, unwritten, nan_mm in json.loads(line[7:]):
        assert rc == 0 and guards, (row, M, rc)
        assert viol <= 1.0 and unwritten == 0 and nan_mm == 0, (row, M, viol, unwritten)


@pytest.mark.parametrize("env,cases,kernel", [
    # up to M = 64 the split runs the skinny-band GEMV by default; the lever keeps the
    # prefill tile of 64 tokens (one token group a wave), which must meet the same bar
    ({"R3D_GFX950_SPLITK_KERNEL": "tile"},
     [(MX_TILE, "mxfp4a8", 40, 1000, 2048, "hook"), (MX_TILE, "mxfp4a8", 17, 300, 9216, "hook"),
      ("gemm_nt_q_fp8a8", "fp8a8", 33, 700, 2688, "hook")], "split-K prefill"),
    ({}, [(MX_TILE, "mxfp4a8", 40, 1000, 2048, "hook"),
          ("gemm_nt_q_fp8a8", "fp8a8", 33, 700, 2688, "hook")], "split-K skinny GEMV"),
    # the e4m3 prefill's 128 x 256 four-wave tile forced at shapes its cost rule leaves to
    # the 128 x 128 one: ragged tokens and weight rows, one and several steps, both sides
    # of a 256-token tile
    ({"R3D_GFX950_F8_TILE": "256"},
     [("gemm_nt_q_fp8a8", "fp8a8", 300, 1000, 1024), ("gemm_nt_q_fp8a8", "fp8a8", 129, 130, 128),
      ("gemm_nt_q_fp8a8", "fp8a8", 513, 388, 2688)], "fp8a8 prefill, 128 x 256 on four waves"),
])
def test_split_kernel_lever(gpu, env, cases, kernel):
    env = dict(os.environ, R3D_DEBUG_GEMM="1", **env)
    p = subprocess.run([sys.executable, "-c", _CHILD % (ROOT, cases)], env=env,
                       capture_output=True, text=True, timeout=300)
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-2000:]
    assert kernel + " launched" in p.stderr, p.stderr[-2000:]
    line = [l for l in p.stdout.splitlines() if l.startswith("RESULT ")][-1]
    for row, M, rc, guards, viol, unwritten, nan_mm in json.loads(line[7:]):
        assert rc == 0 and guards, (row, M, rc)
        assert viol <= 1.0 and unwritten == 0 and nan_mm == 0, (row, M, viol, unwritten)
