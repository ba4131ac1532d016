"""r3d_rad_gemm_nt_q_mxfp4a16_noalloc (run by pytest last): the mxfp4a16 row with its quantiser scratch in a
static device buffer instead of RadArgs::scratch.  Through the C ABI it must give exactly
the bytes of the allocating row on the same operands, on two calls in a row (the second
smaller, over the first call's leftovers), refuse a call whose scratch need passes the
buffer (RAD_E_SHAPE, nothing launched), and leave the device's free memory unchanged."""
import ctypes

import numpy as np
import pytest
import torch

import libr3d_amd as R
from libr3d_amd import synth

A16 = "gemm_nt_q_mxfp4a16"


def _noalloc():
    f = R.lib().r3d_rad_gemm_nt_q_mxfp4a16_noalloc
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.POINTER(R.RadArgs), ctypes.c_void_p]
    return f


def _operands(M, N, K, seed, dev):
    rng = np.random.default_rng(seed)
    X = synth.bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    B, BS = synth.mxfp4_weights(N, K, seed + 1)
    x = torch.from_numpy(X.view(np.int16)).to(dev)
    b, bs = torch.from_numpy(B).to(dev), torch.from_numpy(BS).to(dev)
    return x, b, bs


def _run_both(M, N, K, seed, dev):
    from tests import gpu_util as gu
    x, b, bs = _operands(M, N, K, seed, dev)
    stream = torch.cuda.current_stream().cuda_stream
    y_ref = torch.full((M, N), 0x7777, dtype=torch.int16, device=dev)
    ops = R.GemmOperands(x, None, b, bs, y_ref, dtype="mxfp4a16", N=N, K=K, group=32, M=M)
    scratch = torch.empty(R.row_scratch_bytes(A16, ops), dtype=torch.uint8, device=dev)
    ops.set_scratch(scratch)
    assert R.launch_row(A16, ops, stream) == R.RAD_OK
    gY = gu.y_buffer(M, N, dev)
    ops2 = R.GemmOperands(x, None, b, bs, gY.t, dtype="mxfp4a16", N=N, K=K, group=32, M=M)
    assert _noalloc()(ctypes.byref(ops2.args), ctypes.c_void_p(stream)) == R.RAD_OK
    torch.cuda.synchronize()
    assert gY.guards_intact()
    return y_ref.cpu().numpy(), gY.t.cpu().numpy()


@pytest.mark.gpu
def test_noalloc_matches_allocating_row_twice(gpu):
    for (M, N, K, seed) in [(513, 1000, 1152, 11), (130, 600, 512, 12)]:
        ref, got = _run_both(M, N, K, seed, gpu)
        assert np.array_equal(ref, got), (M, N, K, int(np.sum(ref != got)))
        assert not np.any(got == 0x7777)


@pytest.mark.gpu
def test_noalloc_refuses_past_the_buffer(gpu):
    from tests import gpu_util as gu
    M, K, N = 4096, 4096, 256            # needs 16 MiB + 512 KiB
    x = torch.zeros((M, K), dtype=torch.int16, device=gpu)
    b = torch.zeros((N, K // 2), dtype=torch.uint8, device=gpu)
    bs = torch.full((N, K // 32), 127, dtype=torch.uint8, device=gpu)
    gY = gu.y_buffer(M, N, gpu)
    ops = R.GemmOperands(x, None, b, bs, gY.t, dtype="mxfp4a16", N=N, K=K, group=32, M=M)
    rc = _noalloc()(ctypes.byref(ops.args),
                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert rc == R.RAD_E_SHAPE
    assert np.all(gY.t.cpu().numpy().view(np.uint16) == gu.Y_SENTINEL)   # nothing launched


@pytest.mark.gpu
def test_noalloc_allocates_nothing(gpu):
    """After a first call (which looks the device's buffer up and loads the kernels), calls
    leave the device's free memory (hipMemGetInfo) and torch's allocated bytes unchanged:
    the entry allocates nothing."""
    M, N, K = 513, 1000, 1152
    x, b, bs = _operands(M, N, K, 13, gpu)
    y = torch.empty((M, N), dtype=torch.int16, device=gpu)
    ops = R.GemmOperands(x, None, b, bs, y, dtype="mxfp4a16", N=N, K=K, group=32, M=M)
    f = _noalloc()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert f(ctypes.byref(ops.args), stream) == R.RAD_OK
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    used0 = torch.cuda.memory_allocated()
    for _ in range(3):
        assert f(ctypes.byref(ops.args), stream) == R.RAD_OK
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0 and torch.cuda.memory_allocated() == used0, (free0, free1)
