"""GPU parity of rmsnorm_quant_fp8 against the oracle's restatement of the reference kernel
(src/r3d_more.hip:241-330; oracle r3d_ref_rmsnorm_quant_fp8): codes, scales, the normed
bf16 output and the written-back residual bit-exact (NaN codes and NaN bf16 values as a
class), including the sum of squares, whose fold order the kernel reproduces.  Covers
decode and prefill row counts, n from 100 to 30720 (ragged against the 256-lane stride and
the group), both w dtypes, wadd, eps, no / bf16 / f32 output, a group past n, an all-zero
row (rs = 1/sqrt(eps)) and NaN / Inf inputs; red zones around every operand.
"""
import numpy as np
import pytest
import torch

import libr3d_amd as R
from libr3d_amd import synth
import oracle as O

pytestmark = pytest.mark.gpu


def _same_codes(q, qr):
    nan, nanr = (q & 0x7F) == 0x7F, (qr & 0x7F) == 0x7F
    assert np.array_equal(nan, nanr), np.argwhere(nan != nanr)[:5]
    assert np.array_equal(q[~nan], qr[~nanr]), np.argwhere((q != qr) & ~nan)[:5]


def _same_bf16(o, orf):
    nan = ((o & 0x7F80) == 0x7F80) & ((o & 0x7F) != 0)
    nanr = ((orf & 0x7F80) == 0x7F80) & ((orf & 0x7F) != 0)
    assert np.array_equal(nan, nanr), np.argwhere(nan != nanr)[:5]
    assert np.array_equal(o[~nan], orf[~nanr]), np.argwhere((o != orf) & ~nan)[:5]


def _check(x, w, dev, group=128, eps=1e-6, wadd=None, residual=None, out="bf16"):
    from tests.gpu_util import Guarded
    M, n = x.shape
    g_eff = group if 0 < group <= n else n
    ngrp = (n + g_eff - 1) // g_eff
    gx, gw = Guarded(x, dev), Guarded(w, dev)
    gr = Guarded(residual, dev) if residual is not None else None
    gq = Guarded(np.full((M, n), 0x5A, np.uint8), dev)
    gs = Guarded(np.full((M, ngrp), 0x7FC0DEAD, np.uint32).view(np.float32), dev)
    go = None
    if out == "bf16":
        go = Guarded(np.full((M, n), 0x3C3C, np.uint16), dev)
    elif out == "f32":
        go = Guarded(np.full((M, n), 0x3C3C3C3C, np.uint32).view(np.float32), dev)
    ops = R.RmsNormQuantOperands(gx.t, gr.t if gr else None, gw.t, gq.t, gs.t,
                                 go.t if go else None, n=n, eps=eps, group=group, wadd=wadd, M=M,
                                 w_dtype="BF16" if w.dtype == np.uint16 else "F32")
    rc = R.launch_row("rmsnorm_quant_fp8", ops, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == R.RAD_OK, rc
    assert all(g.guards_intact() for g in (gx, gw, gq, gs) + ((gr,) if gr else ()) +
               ((go,) if go else ())), "red zone written"
    qr, sr, orf, rr = O.rmsnorm_quant_fp8(x, w, group=g_eff, eps=eps,
                                          wadd=0.0 if wadd is None else wadd, residual=residual)
    _same_codes(gq.t.cpu().numpy(), qr)
    s = gs.t.cpu().numpy()
    nan_s = np.isnan(s) & np.isnan(sr)
    assert np.array_equal(s.view(np.uint32)[~nan_s], sr.view(np.uint32)[~nan_s])
    if go is not None:
        o = go.t.cpu().numpy()
        o = o.view(np.uint16) if out == "bf16" else (o.view(np.uint32) >> 16).astype(np.uint16)
        _same_bf16(o, orf)
    if gr is not None:
        _same_bf16(gr.t.cpu().numpy().view(np.uint16), rr)


def _x(M, n, seed, scale=2.0):
    rng = np.random.default_rng(seed)
    return synth.bf16_bits((rng.standard_normal((M, n)) * scale).astype(np.float32)), rng


@pytest.mark.parametrize("M,n", [(1, 5376), (4, 5376), (64, 4096), (300, 1024), (2, 30720),
                                 (3, 100), (5, 132), (2, 257)])
@pytest.mark.parametrize("residual", [False, True])
def test_rmsnorm_quant_shapes(gpu, M, n, residual):
    x, rng = _x(M, n, M * 31 + n + residual)
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    r = synth.bf16_bits(rng.standard_normal((M, n)).astype(np.float32)) if residual else None
    _check(x, w, gpu, residual=r)


@pytest.mark.parametrize("out", [None, "f32"])
def test_rmsnorm_quant_params(gpu, out):
    x, rng = _x(4, 2048, 7)
    wb = synth.bf16_bits((0.1 * rng.standard_normal(2048)).astype(np.float32))
    _check(x, wb, gpu, eps=1e-5, wadd=1.0, out=out)            # gemma-style (1 + w)
    _check(x, wb, gpu, group=64, out=out)
    _check(x, wb, gpu, group=5000, out=out)                      # group past n: one group


def test_rmsnorm_quant_special_values(gpu):
    x, rng = _x(4, 1024, 9)
    x[0] = 0                                                     # rs = 1/sqrt(eps), h = 0
    x[1, 10] = 0x7FC0                                            # NaN poisons its row
    x[2, 20] = synth.bf16_bits(np.array([np.inf], np.float32))[0]
    x[3, 30] = synth.bf16_bits(np.array([3.0e38], np.float32))[0]  # square overflows
    w = np.ones(1024, np.float32)
    _check(x, w, gpu)
    r = synth.bf16_bits(rng.standard_normal((4, 1024)).astype(np.float32))
    _check(x, w, gpu, residual=r)
