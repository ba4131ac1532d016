"""GPU parity at BASELINE.json's full config shapes, on the configs' own distributions
(libr3d_amd.synth), against the CPU oracle.

Bar (besides the per-element bound of tests/test_gpu_gemm.py): per output row
rel_l2 <= 2^-8 (one bf16 ulp) and whole-tensor rel_l2 <= 2e-3.  C3 (M=2048 prefill) is
checked on a seeded sample of activation rows: the kernel computes all 2048, the oracle
the sampled ones.
"""
import numpy as np
import pytest
import torch

import libr3d_amd as R
from libr3d_amd import synth
import oracle as O

pytestmark = pytest.mark.gpu

ROW_REL_MAX = 2.0 ** -8
TENSOR_REL_MAX = 2e-3
NT = 16


def _run(row, dtype, A, AS, B, BS, M, N, K, gpu):
    from tests import gpu_util as gu
    rc, Y, guards = gu.run_row(row, dtype, A, AS, B, BS, M, N, K, gpu)
    assert rc == R.RAD_OK, rc
    assert guards
    return Y


def _grade(Y, A, AS, B, BS, K, dtype, rblk=1):
    from tests import gpu_util as gu
    if dtype == "mxfp4a8":
        Yr, Yf, S = O.quant_dot_mxfp4a8(A, AS, B, BS, nthreads=NT)
    else:
        Yr, Yf, S = O.quant_dot_fp8a8(A, AS, B, BS, rblk, nthreads=NT)
    S8 = O.group8_mag(dtype, A, AS, B, BS, rblk, nthreads=NT)
    c = gu.compare(Y, Yr, Yf, S, K, S8)
    assert c["sentinel_left"] == 0 and c["nan_mismatch"] == 0 and c["inf_mismatch"] == 0, c
    assert c["max_viol"] <= 1.0, c
    assert c["row_rel_l2_max"] <= ROW_REL_MAX, c
    assert c["rel_l2"] <= TENSOR_REL_MAX, c
    print("  rel_l2 %.3e  row_rel_l2_max %.3e  max_abs %.3e  max_viol %.3f" % (
        c["rel_l2"], c["row_rel_l2_max"], c["max_abs"], c["max_viol"]))
    return c


def test_c0_mxfp4_gemv(gpu):
    M, K, N = 1, 4096, 4096
    _, A, AS = synth.activations(M, K, 0x5EED)
    B, BS = synth.mxfp4_weights(N, K, 0x5EED + 1)
    Y = _run("gemm_nt_q_mxfp4_decode", "mxfp4a8", A, AS, B, BS, M, N, K, gpu)
    _grade(Y, A, AS, B, BS, K, "mxfp4a8")


def test_c1_fp8_gemv(gpu):
    M, K, N = 1, 5376, 21504
    A, AS = synth.fp8_activations_per_token(M, K, 0x5EED + 10)
    B, BS = synth.fp8_weights(N, K, 0x5EED + 11)
    Y = _run("gemm_nt_q_fp8a8_decode", "fp8a8", A, AS, B, BS, M, N, K, gpu)
    _grade(Y, A, AS, B, BS, K, "fp8a8")


C2_SHAPES = {"gate_up": (5376, 21504), "down": (21504, 5376), "qkv": (5376, 8192)}


@pytest.mark.parametrize("shape", sorted(C2_SHAPES))
@pytest.mark.parametrize("M", [1, 4, 16])
def test_c2_mxfp4_decode(gpu, shape, M):
    K, N = C2_SHAPES[shape]
    _, A, AS = synth.activations(M, K, 0x5EED + 20 + M)
    B, BS = synth.mxfp4_weights(N, K, 0x5EED + 21 + K)
    Y = _run("gemm_nt_q_mxfp4_decode", "mxfp4a8", A, AS, B, BS, M, N, K, gpu)
    _grade(Y, A, AS, B, BS, K, "mxfp4a8")


def test_c3_mxfp4_prefill_sampled(gpu):
    M, K, N = 2048, 5376, 21504
    _, A, AS = synth.activations(M, K, 0x5EED + 30)
    B, BS = synth.mxfp4_weights(N, K, 0x5EED + 31)
    Y = _run("gemm_nt_q_mxfp4", "mxfp4a8", A, AS, B, BS, M, N, K, gpu)
    rows = np.sort(np.random.default_rng(3).choice(M, size=12, replace=False))
    _grade(Y[rows], A[rows], AS[rows], B, BS, K, "mxfp4a8")


@pytest.mark.parametrize("rblk", [1, 128])
def test_c3_shape_fp8a8_prefill_sampled(gpu, rblk):
    """The fp8a8 generic row at config 3's shape (M=2048, K=5376, N=21504) on config 1's
    weight law, both weight-scale grids."""
    M, K, N = 2048, 5376, 21504
    A, AS = synth.fp8_activations_per_token(M, K, 0x5EED + 35)
    B, BS = synth.fp8_weights(N, K, 0x5EED + 36)
    if rblk == 128:
        BS = BS[::128].copy()                 # one scale row per 128 weight rows
    Y = _run("gemm_nt_q_fp8a8", "fp8a8", A, AS, B, BS, M, N, K, gpu)
    rows = np.sort(np.random.default_rng(5).choice(M, size=12, replace=False))
    _grade(Y[rows], A[rows], AS[rows], B, BS, K, "fp8a8", rblk)


def test_c4_lm_head_fp8(gpu):
    M, K, N = 4, 5376, 262144
    A, AS = synth.fp8_activations_per_token(M, K, 0x5EED + 40)
    B, BS = synth.fp8_weights(N, K, 0x5EED + 41)
    Y = _run("gemm_nt_q_fp8a8_decode", "fp8a8", A, AS, B, BS, M, N, K, gpu)
    _grade(Y, A, AS, B, BS, K, "fp8a8")
