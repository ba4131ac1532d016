"""GPU parity of the decode rows' fused producer: bf16 activations with no a_scale, quantised
inside the quad GEMV with quant_act_fp8's arithmetic (src/r3d_band.hip:117-153) before the
products (src/r3d_gemm_mxfp4.hip:14-15, src/r3d_gemm_fp8a8.hip:9-15).

Two bars: (1) Y bit-identical to the unfused pair -- the quant_act_fp8 row, then the same
decode row on its codes and scales; (2) Y within the GEMM bar of the oracle's composition
(oracle quant_act_fp8, then the oracle GEMM).  The fused path is the M = 1 decode call, and
M = 2..4 when the engine sets the rows' "fuse" tunable; shapes cover one and several
producer batches per wave (K past 8192), split K, a padded activation view, and special
values (an all-zero group, subnormals, an outlier, an Inf, a NaN).
"""
import numpy as np
import pytest
import torch

import libr3d_amd as R
from libr3d_amd import synth
import oracle as O

pytestmark = pytest.mark.gpu

ROWS = {"mxfp4a8": "gemm_nt_q_mxfp4_decode", "fp8a8": "gemm_nt_q_fp8a8_decode"}
TOL = {"mxfp4a8": 3e-2, "fp8a8": 5e-3}


def _weights(dtype, N, K, rng, rblk):
    if dtype == "mxfp4a8":
        B = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
        BS = rng.integers(115, 140, size=(N, K // 32)).astype(np.uint8)
    else:
        B = synth.random_e4m3_codes((N, K), rng)
        rows = N if rblk == 1 else (N + 127) // 128
        BS = synth.bf16_bits((0.001 + 0.01 * rng.random((rows, K // 128))).astype(np.float32))
    return B, BS


def _run(dtype, x, N, K, B, BS, dev, pitch=None, tunables=None):
    """-> (Y fused, Y unfused, guards ok); x: [M, K] bf16 bits on the host."""
    from tests.gpu_util import Guarded, y_buffer
    M = x.shape[0]
    xp = x if pitch is None else np.pad(x, ((0, 0), (0, pitch - K)))
    gx = Guarded(xp, dev)
    xv = gx.t[:, :K]
    gB, gBS = Guarded(B, dev), Guarded(BS, dev)
    stream = torch.cuda.current_stream().cuda_stream
    gY = y_buffer(M, N, dev)
    ops = R.GemmOperands(xv, None, gB.t, gBS.t, gY.t, dtype=dtype, N=N, K=K, tunables=tunables)
    rc = R.launch_row(ROWS[dtype], ops, stream)
    torch.cuda.synchronize()
    assert rc == R.RAD_OK, rc
    # the unfused pair on the same activations
    q = torch.empty((M, K), dtype=torch.uint8, device=dev)
    s = torch.empty((M, K // 128), dtype=torch.float32, device=dev)
    qa = R.QuantActOperands(xv, q, s, n=K, group=128, M=M, x_dtype="BF16")
    assert R.launch_row("quant_act_fp8_act", qa, stream) == R.RAD_OK
    gY2 = y_buffer(M, N, dev)
    ops2 = R.GemmOperands(q, s, gB.t, gBS.t, gY2.t, dtype=dtype, N=N, K=K, tunables=tunables)
    assert R.launch_row(ROWS[dtype], ops2, stream) == R.RAD_OK
    torch.cuda.synchronize()
    Y = gY.t.cpu().numpy().view(np.uint16)
    Y2 = gY2.t.cpu().numpy().view(np.uint16)
    ok = all(g.guards_intact() for g in (gx, gB, gBS, gY))
    return Y, Y2, ok


def _check(dtype, x, N, K, dev, rblk=1, seed=0, pitch=None, tunables=None):
    from tests import gpu_util as gu
    rng = np.random.default_rng(seed)
    B, BS = _weights(dtype, N, K, rng, rblk)
    Y, Y2, ok = _run(dtype, x, N, K, B, BS, dev, pitch, tunables)
    assert ok, "red zone written"
    assert np.array_equal(Y, Y2), np.argwhere(Y != Y2)[:5]
    qr, sr = O.quant_act_fp8(x, 128)
    if dtype == "mxfp4a8":
        Yr, Yf, S = O.quant_dot_mxfp4a8(qr, sr, B, BS, nthreads=16)
    else:
        Yr, Yf, S = O.quant_dot_fp8a8(qr, sr, B, BS, rblk, nthreads=16)
    S8 = O.group8_mag(dtype, qr, sr, B, BS, rblk, nthreads=16)
    c = gu.compare(Y, Yr, Yf, S, K, S8)
    assert c["sentinel_left"] == 0, c
    assert c["nan_mismatch"] == 0 and c["inf_mismatch"] == 0, c
    assert c["max_viol"] <= 1.0, c
    assert c["rel_l2"] <= TOL[dtype], c
    return Y


def _x(M, K, seed):
    rng = np.random.default_rng(1000 + seed)
    return synth.bf16_bits((rng.standard_normal((M, K), dtype=np.float32) *
                            np.float32(2.0)).astype(np.float32))


@pytest.mark.parametrize("dtype", ["mxfp4a8", "fp8a8"])
@pytest.mark.parametrize("N,K", [(21504, 5376), (5376, 21504), (1000, 4096), (2048, 16384),
                                 (8192, 5376), (64, 256), (100, 128), (3000, 9216)])
def test_fused_decode_shapes(gpu, dtype, N, K):
    _check(dtype, _x(1, K, K + N), N, K, gpu, seed=3 + N)


@pytest.mark.parametrize("rblk", [1, 128])
def test_fused_fp8_row_and_block_scales(gpu, rblk):
    _check("fp8a8", _x(1, 4096, 7), 640, 4096, gpu, rblk=rblk, seed=rblk)


@pytest.mark.parametrize("dtype", ["mxfp4a8", "fp8a8"])
def test_fused_decode_padded_view_and_split(gpu, dtype):
    _check(dtype, _x(1, 2048, 11), 512, 2048, gpu, pitch=2048 + 64)
    _check(dtype, _x(1, 4096, 12), 768, 4096, gpu, tunables=[("splitk", 4)])


@pytest.mark.parametrize("dtype", ["mxfp4a8", "fp8a8"])
def test_fused_decode_special_values(gpu, dtype):
    """An all-zero group (scale 1), a subnormal-only group, a lone outlier; then an Inf (its
    group's scale Inf, its codes NaN) or a NaN (never the group maximum, encoded NaN), each
    of which poisons every output, as in the oracle."""
    K, N = 1024, 384
    x = _x(1, K, 21).copy()
    x[0, :128] = 0
    x[0, 128:256] = synth.bf16_bits(np.full(128, 1e-40, np.float32))
    x[0, 300] = synth.bf16_bits(np.array([3.0e4], np.float32))[0]
    Y = _check(dtype, x, N, K, gpu, seed=5)
    assert not np.isnan(O.bf16_to_f32(Y)).any()
    for pos, bits in ((700, synth.bf16_bits(np.array([np.inf], np.float32))[0]), (900, 0x7FC0)):
        xs = x.copy()
        xs[0, pos] = bits
        Y = _check(dtype, xs, N, K, gpu, seed=5)
        assert np.isnan(O.bf16_to_f32(Y)).all(), pos


@pytest.mark.parametrize("dtype", ["mxfp4a8", "fp8a8"])
@pytest.mark.parametrize("M", [2, 3, 4])
@pytest.mark.parametrize("N,K", [(21504, 5376), (2048, 5376), (5376, 4096), (100, 128),
                                 (3000, 8192)])
def test_fused_decode_rows_on_request(gpu, dtype, M, N, K):
    """The "fuse" tunable: M = 2..4 bf16 rows quantised in the quad GEMV's four activation
    images (one producer batch per wave up to M K = 16384, two beyond), bit-identical to
    the producer row followed by the decode row."""
    _check(dtype, _x(M, K, 31 * M + K), N, K, gpu, seed=M + N, tunables=[("fuse", 1)])


@pytest.mark.parametrize("dtype", ["mxfp4a8", "fp8a8"])
def test_fused_decode_rows_view_split_values(gpu, dtype):
    fuse = [("fuse", 1)]
    _check(dtype, _x(3, 2048, 41), 512, 2048, gpu, pitch=2048 + 64, tunables=fuse)
    _check(dtype, _x(4, 4096, 42), 768, 4096, gpu, tunables=fuse + [("splitk", 4)])
    x = _x(4, 1024, 43).copy()
    x[1, :128] = 0                                                    # an all-zero group
    x[2, 300] = synth.bf16_bits(np.array([3.0e4], np.float32))[0]     # an outlier
    Y = _check(dtype, x, 384, 1024, gpu, seed=9, tunables=fuse)
    assert not np.isnan(O.bf16_to_f32(Y)).any()
    x[3, 700] = 0x7FC0                                                # a NaN poisons row 3 only
    Y = _check(dtype, x, 384, 1024, gpu, seed=9, tunables=fuse)
    Yf = O.bf16_to_f32(Y)
    assert np.isnan(Yf[3]).all() and not np.isnan(Yf[:3]).any()
