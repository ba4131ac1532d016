"""GPU parity of the quant_act_fp8 row against the oracle's restatement of the reference
producer (src/r3d_band.hip:117-153; oracle/r3d_oracle.c r3d_ref_quant_act_fp8), through
the C ABI: codes and scales bit-exact, red zones intact, every output written.

Covers bf16 and f32 inputs, the vector path (groups of 8..512 tiling aligned rows: every
group width it instantiates) and the two-element and one-element lane paths (ragged,
even / odd sizes and offsets), a group past n (clamped to n), strided and rank-1 views,
and the special values: NaN (never the group maximum, encoded 0x7F with its sign),
+-Inf (scale Inf, finite codes 0, Inf codes NaN), signed zeros, subnormals, an all-zero
group (scale 1) and a lone non-zero element.
"""
import numpy as np
import pytest
import torch

import libr3d_amd as R
from libr3d_amd import synth
import oracle as O

pytestmark = pytest.mark.gpu

Q_FILL, S_FILL = 0x5A, 0x7FC0DEAD


def _launch(x_dev_view, n, group, M, x_dtype, dev, extra_q=None):
    from tests.gpu_util import Guarded
    g_eff = group if 0 < group <= n else n
    ngrp = (n + g_eff - 1) // g_eff
    gq = Guarded(np.full((M, n), Q_FILL, np.uint8), dev)
    gs = Guarded(np.full((M, ngrp), S_FILL, np.uint32).view(np.float32), dev)
    ops = R.QuantActOperands(x_dev_view, gq.t, gs.t, n=n, group=group, M=M, x_dtype=x_dtype)
    rc = R.launch_row("quant_act_fp8_act", ops, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == R.RAD_OK, rc
    assert gq.guards_intact() and gs.guards_intact(), "red zone written"
    return gq.t.cpu().numpy(), gs.t.cpu().numpy(), g_eff


def _check(x_host, group, dev, x_dtype):
    """x_host: [M, n] uint16 (bf16 bits) or float32, contiguous."""
    from tests.gpu_util import Guarded
    M, n = x_host.shape
    gx = Guarded(x_host, dev)
    q, s, g_eff = _launch(gx.t, n, group, M, x_dtype, dev)
    assert gx.guards_intact()
    qr, sr = O.quant_act_fp8(x_host, g_eff)
    _same_codes(q, qr)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32)), np.argwhere(
        s.view(np.uint32) != sr.view(np.uint32))[:5]


def _same_codes(q, qr):
    """Bit-exact, NaN compared as a class: the sign of a NaN born in the arithmetic (Inf x 0)
    is the machine's default NaN (x86 sets it, the GPU does not); IEEE leaves it open."""
    nan, nanr = (q & 0x7F) == 0x7F, (qr & 0x7F) == 0x7F
    assert np.array_equal(nan, nanr), np.argwhere(nan != nanr)[:5]
    assert np.array_equal(q[~nan], qr[~nanr]), np.argwhere((q != qr) & ~nan)[:5]


def _bf16(a):
    return synth.bf16_bits(np.asarray(a, np.float32))


@pytest.mark.parametrize("M,n,group", [(1, 5376, 128), (4, 5376, 128), (17, 4096, 128),
                                       (3, 200, 128), (2, 256, 32), (5, 384, 64),
                                       (3, 300, 1000), (2, 7, 128), (3, 131, 16),
                                       (2, 1024, 8), (3, 2048, 16), (2, 1024, 256),
                                       (2, 2048, 512), (2048, 5376, 128)])
def test_quant_act_fp8_bf16(gpu, M, n, group):
    rng = np.random.default_rng(M * 7 + n + group)
    x = _bf16(rng.standard_normal((M, n), dtype=np.float32) * np.float32(3.0))
    _check(x, group, gpu, "BF16")


@pytest.mark.parametrize("M,n,group", [(1, 5376, 128), (6, 1000, 128), (3, 129, 128),
                                       (2, 64, 7)])
def test_quant_act_fp8_f32(gpu, M, n, group):
    rng = np.random.default_rng(M + 3 * n + group)
    x = (rng.standard_normal((M, n), dtype=np.float32) *
         np.exp2(rng.integers(-40, 40, size=(M, n))).astype(np.float32)).astype(np.float32)
    _check(x, group, gpu, "F32")


def test_quant_act_fp8_special_values(gpu):
    n = 512
    rows = []
    r = np.zeros(n, np.float32)
    r[5] = np.nan; r[9] = -np.nan; r[10] = 3.0; r[11] = -7.5             # NaN never wins
    rows.append(r.copy())
    r = np.zeros(n, np.float32); r[0] = np.inf; r[1] = -2.0; r[2] = -np.inf  # scale Inf
    rows.append(r.copy())
    rows.append(np.zeros(n, np.float32))                                   # scale 1
    r = np.full(n, -0.0, np.float32); r[200] = 1e-30                       # signed zeros, tiny
    rows.append(r.copy())
    r = np.zeros(n, np.float32); r[300] = -1e38; r[301] = 1e-45            # huge / subnormal
    rows.append(r.copy())
    r = np.full(n, np.nan, np.float32)                                     # all NaN: amax 0
    rows.append(r.copy())
    x32 = np.stack(rows).astype(np.float32)
    _check(x32, 128, gpu, "F32")
    _check(_bf16(x32), 128, gpu, "BF16")
    # bf16 subnormals and the largest finite bf16
    xb = np.zeros((2, 256), np.uint16)
    xb[0, :] = np.arange(256, dtype=np.uint16) | 0x0001                    # subnormal patterns
    xb[1, 3] = 0x7F7F; xb[1, 4] = 0xFF7F; xb[1, 5] = 0x0001
    _check(xb, 128, gpu, "BF16")


def test_quant_act_fp8_views(gpu):
    """A strided [M, n] view into wider rows, a one-element offset (odd base: the
    one-element path), and a rank-1 x of one row."""
    from tests.gpu_util import Guarded
    rng = np.random.default_rng(11)
    M, n, pad = 5, 640, 24
    wide = _bf16(rng.standard_normal((M, n + pad), dtype=np.float32))
    gw = Guarded(wide, gpu)
    q, s, g = _launch(gw.t[:, :n], n, 128, M, "BF16", gpu)
    qr, sr = O.quant_act_fp8(np.ascontiguousarray(wide[:, :n]), 128)
    _same_codes(q, qr)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32))
    flat = _bf16(rng.standard_normal(M * n + 1, dtype=np.float32))
    gf = Guarded(flat, gpu)
    q, s, g = _launch(gf.t[1:].view(M, n), n, 128, M, "BF16", gpu)
    qr, sr = O.quant_act_fp8(flat[1:].reshape(M, n), 128)
    _same_codes(q, qr)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32))
    one = _bf16(rng.standard_normal(n, dtype=np.float32))
    go = Guarded(one, gpu)
    q, s, g = _launch(go.t, n, 128, 1, "BF16", gpu)
    qr, sr = O.quant_act_fp8(one.reshape(1, n), 128)
    _same_codes(q, qr)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32))
