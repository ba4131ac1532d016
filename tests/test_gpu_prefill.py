"""GPU parity of the mxfp4 prefill GEMM (block-scaled MFMA over a direct-to-LDS ring) and
of the bf16-in gemm_nt_q_mxfp4a16 row, through the C ABI on guarded operands.

gemm_nt_q_mxfp4 (e4m3 + f32 a_scale per 128) is held to the per-element bound of
tests/test_gpu_gemm.py against oracle.quant_dot_mxfp4a8 at shapes that walk every tile
edge: ragged M and N, one K step, odd and even step counts, every tile width the planner
picks.

gemm_nt_q_mxfp4a16 has no reference counterpart.  Its two stages are checked apart:
  * the mxfp8 quantiser (bf16 -> e4m3 + E8M0 per 32) must leave in the launch scratch
    exactly the bytes of oracle.quant_act_mxfp8, edge values included (zeros, NaN,
    +-inf, bf16 subnormals, the largest finite bf16, rounding ties);
  * the GEMM must match oracle.dot_mx8_mxfp4 on those codes within
    |y - y_oracle| <= ulp_bf16 + 2*K*2^-24*S + 2^-10*S8 (S8 with the per-32 scales).
"""
import numpy as np
import pytest
import torch

import libr3d_amd as R
from libr3d_amd import synth
import oracle as O

pytestmark = pytest.mark.gpu

MX_TILE, A16 = "gemm_nt_q_mxfp4", "gemm_nt_q_mxfp4a16"


def _gu():
    from tests import gpu_util
    return gpu_util


def _mx_case(M, N, K, seed):
    rng = np.random.default_rng(seed)
    A = synth.random_e4m3_codes((M, K), rng)
    AS = (0.001 + 0.01 * rng.random((M, K // 128))).astype(np.float32)
    B = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    BS = rng.integers(115, 140, size=(N, K // 32)).astype(np.uint8)
    return A, AS, B, BS


# every tile width the planner picks (bn 256/224/192/128) shows up across these N
@pytest.mark.parametrize("M,N,K", [(17, 300, 128), (128, 256, 256), (129, 448, 384),
                                   (300, 700, 640), (512, 1000, 1152), (260, 64, 512),
                                   (1000, 2176, 256)])
def test_mxfp4a8_prefill_shapes(gpu, M, N, K):
    gu = _gu()
    A, AS, B, BS = _mx_case(M, N, K, M * 7 + N + K)
    rc, Y, guards = gu.run_row(MX_TILE, "mxfp4a8", A, AS, B, BS, M, N, K, gpu)
    assert rc == R.RAD_OK and guards
    Yr, Yf, S = O.quant_dot_mxfp4a8(A, AS, B, BS, nthreads=16)
    S8 = O.group8_mag("mxfp4a8", A, AS, B, BS, nthreads=16)
    c = gu.compare(Y, Yr, Yf, S, K, S8)
    assert c["sentinel_left"] == 0, c
    assert c["nan_mismatch"] == 0 and c["inf_mismatch"] == 0, c
    assert c["max_viol"] <= 1.0, c
    assert c["rel_l2"] <= 3e-2, c


def run_a16(X, B, BS, M, N, K, dev, scratch_bytes=None):
    """Launch gemm_nt_q_mxfp4a16 on guarded operands; returns (rc, Y, Q, SX, guards_ok)."""
    gu = _gu()
    gX, gB, gBS = gu.Guarded(X, dev), gu.Guarded(B, dev), gu.Guarded(BS, dev)
    gY = gu.y_buffer(M, N, dev)
    ops = R.GemmOperands(gX.t, None, gB.t, gBS.t, gY.t, dtype="mxfp4a16", N=N, K=K,
                         group=32, M=M)
    need = R.row_scratch_bytes(A16, ops)
    assert need == ((M * K + 255) // 256) * 256 + M * (K // 32)
    nbytes = need if scratch_bytes is None else scratch_bytes
    gS = gu.Guarded(np.zeros(max(nbytes, 1), np.uint8), dev, fill=0x5A)
    ops.set_scratch(gS.t, nbytes)
    rc = R.launch_row(A16, ops, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    Y = gY.t.cpu().numpy().view(np.uint16).reshape(M, N)
    raw = gS.t.cpu().numpy()
    qb = ((M * K + 255) // 256) * 256
    Q = raw[:M * K].reshape(M, K) if nbytes >= need else None
    SX = raw[qb:qb + M * (K // 32)].reshape(M, K // 32) if nbytes >= need else None
    ok = all(g.guards_intact() for g in (gX, gB, gBS, gY, gS))
    return rc, Y, Q, SX, ok


def _bf16_acts(M, K, seed, edges=False):
    rng = np.random.default_rng(seed)
    X = synth.bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    if edges:
        X = X.copy()
        X[0, :32] = 0                                          # all-zero block -> e = 0
        X[0, 32:64] = 0x8000                                   # -0 block
        X[1, 5] = 0x7FC0                                       # NaN (never the max)
        X[1, 40] = 0x7F80                                      # +inf block -> e = 0, clamps
        X[1, 70] = 0xFF80                                      # -inf
        X[2, :32] = np.arange(1, 33, dtype=np.uint16)          # bf16 subnormals only
        X[2, 32:64] = 0x7F7F                                   # largest finite bf16
        X[3, :32] = synth.bf16_bits(np.float32(448.0) * np.ones(32, np.float32))
        X[3, 0] = synth.bf16_bits(np.array([464.0], np.float32))[0]   # above the range
        X[4, :32] = synth.bf16_bits((np.arange(32) - 16).astype(np.float32) * 2.0 ** -10)
        X[5, :32] = synth.bf16_bits(np.float32(2.0 ** -133) * np.ones(32, np.float32))
    return X


@pytest.mark.parametrize("edges", [False, True])
def test_mxfp4a16_quantiser_bit_exact(gpu, edges):
    M, N, K = 37, 64, 384
    X = _bf16_acts(M, K, 5 + edges, edges)
    B, BS = synth.mxfp4_weights(N, K, 6)
    rc, Y, Q, SX, ok = run_a16(X, B, BS, M, N, K, gpu)
    assert rc == R.RAD_OK and ok
    Qr, SXr = O.quant_act_mxfp8(X)
    assert np.array_equal(SX, SXr), np.argwhere(SX != SXr)[:8]
    assert np.array_equal(Q, Qr), np.argwhere(Q != Qr)[:8]


@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (17, 200, 256), (256, 512, 1024),
                                   (300, 700, 640), (513, 1000, 1152), (64, 2176, 384)])
def test_mxfp4a16_gemm(gpu, M, N, K):
    gu = _gu()
    X = _bf16_acts(M, K, M + N + K)
    B, BS = synth.mxfp4_weights(N, K, M + 3)
    rc, Y, Q, SX, ok = run_a16(X, B, BS, M, N, K, gpu)
    assert rc == R.RAD_OK and ok
    Qr, SXr = O.quant_act_mxfp8(X)
    assert np.array_equal(Q, Qr) and np.array_equal(SX, SXr)
    Yr, Yf, S = O.dot_mx8_mxfp4(Qr, SXr, B, BS, nthreads=16)
    S8 = O.group8_mag("mxfp4a16", Qr, SXr, B, BS, nthreads=16)
    c = gu.compare(Y, Yr, Yf, S, K, S8)
    assert c["sentinel_left"] == 0, c
    assert c["nan_mismatch"] == 0 and c["inf_mismatch"] == 0, c
    assert c["max_viol"] <= 1.0, c
    assert c["row_rel_l2_max"] <= 2.0 ** -8, c


def test_mxfp4a16_short_scratch_refused(gpu):
    M, N, K = 40, 64, 256
    X = _bf16_acts(M, K, 9)
    B, BS = synth.mxfp4_weights(N, K, 10)
    rc, Y, _, _, ok = run_a16(X, B, BS, M, N, K, gpu, scratch_bytes=M * K)
    assert rc == R.RAD_E_UNSUPPORTED and ok
    assert np.all(Y == _gu().Y_SENTINEL)                    # nothing launched
