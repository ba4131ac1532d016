"""GPU parity of the gated rows.

gated_quant_fp8_act: codes, scales and the gated output bit-exact against the oracle's
restatement of the reference producer (src/r3d_band.hip:155-201; oracle
r3d_ref_gated_quant_fp8), NaN codes and NaN bf16 values compared as a class (the sign of a
NaN born of Inf x 0 is the machine's default NaN).  Covers bf16 and f32 inputs, both acts
and the absent one, no / bf16 / f32 gated output, the vector kernel's group widths, the
one-wave path (ragged n, a group that does not tile n, unaligned pitch), strided rows and
special gates (+-0, +-30, +-88, +-100, +-Inf, NaN).

gemm_nt_q_gated_fp8a8: codes, scales and gated output byte-identical to the gemm_nt_q row
the resolver picks at that M followed by gated_quant_fp8_act on its bf16 output, and equal
to the oracle producer on that output; red zones around every operand and the scratch.
"""
import numpy as np
import pytest
import torch

import libr3d_amd as R
from libr3d_amd import synth
import oracle as O

pytestmark = pytest.mark.gpu

Q_FILL, S_FILL, O_FILL = 0x5A, 0x7FC0DEAD, 0x3C


def _same_codes(q, qr):
    nan, nanr = (q & 0x7F) == 0x7F, (qr & 0x7F) == 0x7F
    assert np.array_equal(nan, nanr), np.argwhere(nan != nanr)[:5]
    assert np.array_equal(q[~nan], qr[~nanr]), np.argwhere((q != qr) & ~nan)[:5]


def _same_bf16(o, orf):
    nan = ((o & 0x7F80) == 0x7F80) & ((o & 0x7F) != 0)
    nanr = ((orf & 0x7F80) == 0x7F80) & ((orf & 0x7F) != 0)
    assert np.array_equal(nan, nanr), np.argwhere(nan != nanr)[:5]
    assert np.array_equal(o[~nan], orf[~nanr]), np.argwhere((o != orf) & ~nan)[:5]


def _gates(M, n, rng, special=True, scale=4.0):
    gt = (rng.standard_normal((M, n)) * scale).astype(np.float32)
    if special:
        sp = np.array([0.0, -0.0, 30, -30, 88, -88, 100, -100, np.inf, -np.inf, np.nan],
                      np.float32)
        k = min(sp.size, max(0, n - 5))
        gt[0, 5:5 + k] = sp[:k]
    up = (rng.standard_normal((M, n)) * 3).astype(np.float32)
    return np.concatenate([gt, up], axis=1)


def _run_band(gu_host, n, group, act, out, dev, pitch=None):
    """gu_host: [M, 2n] float32 or bf16 bits; -> (q, s, o bits or None), guards ok."""
    from tests.gpu_util import Guarded
    M = gu_host.shape[0]
    g_eff = group if 0 < group <= n else n
    ngrp = (n + g_eff - 1) // g_eff
    host = gu_host if pitch is None else np.pad(gu_host, ((0, 0), (0, pitch - 2 * n)))
    gx = Guarded(host, dev)
    gq = Guarded(np.full((M, n), Q_FILL, np.uint8), dev)
    gs = Guarded(np.full((M, ngrp), S_FILL, np.uint32).view(np.float32), dev)
    go = None
    if out == "bf16":
        go = Guarded(np.full((M, n), O_FILL, np.uint16), dev)
    elif out == "f32":
        go = Guarded(np.full((M, n), O_FILL, np.uint32).view(np.float32), dev)
    ops = R.GatedQuantOperands(gx.t[:, :2 * n], gq.t, gs.t, go.t if go else None, n=n,
                               group=group, act=act, M=M)
    rc = R.launch_row("gated_quant_fp8_act", ops, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == R.RAD_OK, rc
    ok = all(g.guards_intact() for g in (gx, gq, gs) + ((go,) if go else ()))
    o = None
    if go is not None:
        o = go.t.cpu().numpy()
        o = o.view(np.uint16) if out == "bf16" else (o.view(np.uint32) >> 16).astype(np.uint16)
        if out == "f32":   # the f32 output is the bf16 value widened: low half zero
            assert not (go.t.cpu().numpy().view(np.uint32) & 0xFFFF).any()
    return gq.t.cpu().numpy(), gs.t.cpu().numpy(), o, ok


def _check_band(gu_host, n, group, act, out, dev, pitch=None):
    q, s, o, ok = _run_band(gu_host, n, group, act, out, dev, pitch)
    assert ok, "red zone written"
    g_eff = group if 0 < group <= n else n
    qr, sr, orf = O.gated_quant_fp8(gu_host, n=n, group=g_eff,
                                    act="sigmoid" if act == "sigmoid" else "silu")
    _same_codes(q, qr)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32)), np.argwhere(s != sr)[:5]
    if o is not None:
        _same_bf16(o, orf)


@pytest.mark.parametrize("M,n,group", [(1, 10752, 128), (4, 10752, 128), (64, 1024, 128),
                                       (3, 2048, 8), (2, 2048, 16), (2, 2048, 64),
                                       (2, 4096, 256), (2, 4096, 512), (3, 300, 128),
                                       (2, 1000, 100), (2, 7, 128), (5, 384, 1000)])
@pytest.mark.parametrize("act", ["silu", "sigmoid", None])
def test_gated_quant_bf16(gpu, M, n, group, act):
    rng = np.random.default_rng(M * 11 + n + group)
    gu = synth.bf16_bits(_gates(M, n, rng))
    _check_band(gu, n, group, act, "bf16", gpu)


@pytest.mark.parametrize("out", [None, "f32"])
@pytest.mark.parametrize("M,n,group", [(2, 2048, 128), (3, 300, 128)])
def test_gated_quant_f32_and_outputs(gpu, out, M, n, group):
    rng = np.random.default_rng(5 + n)
    _check_band(_gates(M, n, rng), n, group, "silu", out, gpu)
    _check_band(synth.bf16_bits(_gates(M, n, rng)), n, group, "sigmoid", out, gpu)


@pytest.mark.parametrize("pitch", [2 * 1024 + 64, 2 * 1024 + 4])
def test_gated_quant_strided_rows(gpu, pitch):
    """A padded row pitch: 16-byte multiple (vector kernel) or not (one-wave path)."""
    rng = np.random.default_rng(pitch)
    _check_band(synth.bf16_bits(_gates(3, 1024, rng)), 1024, 128, "silu", "bf16", gpu, pitch)


# ------------------------------------------------------------------ the gated GEMM row
def _gated_case(M, n, K, rblk, seed):
    rng = np.random.default_rng(seed)
    N = 2 * n
    A = synth.random_e4m3_codes((M, K), rng)
    AS = (0.01 + 0.1 * rng.random((M, K // 128))).astype(np.float32)
    B = synth.random_e4m3_codes((N, K), rng)
    rows = N if rblk == 1 else (N + 127) // 128
    BS = synth.bf16_bits((0.001 + 0.01 * rng.random((rows, K // 128))).astype(np.float32))
    return A, AS, B, BS


@pytest.mark.parametrize("M", [1, 3, 16, 17, 64])
@pytest.mark.parametrize("rblk", [1, 128])
@pytest.mark.parametrize("act", ["silu", "sigmoid"])
def test_gated_gemm_is_the_composition(gpu, M, rblk, act):
    from tests.gpu_util import Guarded
    n, K = 1024, 512
    N = 2 * n
    A, AS, B, BS = _gated_case(M, n, K, rblk, M * 7 + rblk)
    gA, gAS, gB, gBS = (Guarded(x, gpu) for x in (A, AS, B, BS))
    gq = Guarded(np.full((M, n), Q_FILL, np.uint8), gpu)
    gs = Guarded(np.full((M, n // 128), S_FILL, np.uint32).view(np.float32), gpu)
    go = Guarded(np.full((M, n), O_FILL, np.uint16), gpu)
    ops = R.GatedGemmOperands(gA.t, gAS.t, gB.t, gBS.t, gq.t, gs.t, go.t, N=N, K=K, act=act,
                              M=M)
    need = R.row_scratch_bytes("gemm_nt_q_gated_fp8a8", ops)
    assert need == 64 * N * 2
    gsc = Guarded(np.zeros(need, np.uint8), gpu)
    ops.set_scratch(gsc.t)
    stream = torch.cuda.current_stream().cuda_stream
    rc = R.launch_row("gemm_nt_q_gated_fp8a8", ops, stream)
    torch.cuda.synchronize()
    assert rc == R.RAD_OK, rc
    assert all(g.guards_intact() for g in (gA, gAS, gB, gBS, gq, gs, go, gsc))
    q, s, o = gq.t.cpu().numpy(), gs.t.cpu().numpy(), go.t.cpu().numpy().view(np.uint16)
    # the two rows it composes
    row = R.resolve("gemm_nt_q", {"dtype": "fp8a8", "M": M, "N": N, "K": K, "group": 128})
    y = torch.empty((M, N), dtype=torch.int16, device=gpu)
    assert R.launch_row(row["name"], R.GemmOperands(gA.t, gAS.t, gB.t, gBS.t, y, dtype="fp8a8",
                                                    N=N, K=K), stream) == R.RAD_OK
    q2 = torch.empty((M, n), dtype=torch.uint8, device=gpu)
    s2 = torch.empty((M, n // 128), dtype=torch.float32, device=gpu)
    o2 = torch.empty((M, n), dtype=torch.int16, device=gpu)
    assert R.launch_row("gated_quant_fp8_act",
                        R.GatedQuantOperands(y, q2, s2, o2, n=n, group=128, act=act, M=M),
                        stream) == R.RAD_OK
    torch.cuda.synchronize()
    assert np.array_equal(q, q2.cpu().numpy())
    assert np.array_equal(s.view(np.uint32), s2.cpu().numpy().view(np.uint32))
    assert np.array_equal(o, o2.cpu().numpy().view(np.uint16))
    # the scratch holds the GEMM's plane, equal to the gemm_nt_q row's y
    plane = gsc.t[:M * N * 2].cpu().numpy().view(np.uint16).reshape(M, N)
    yh = y.cpu().numpy().view(np.uint16)
    assert np.array_equal(plane, yh)
    qr, sr, orf = O.gated_quant_fp8(yh, group=128, act=act)
    _same_codes(q, qr)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32))
    _same_bf16(o, orf)


def test_gated_gemm_c1_shape(gpu):
    """Config 1's gate_up plane shape (N = 21504, K = 5376) at M = 4, no gated output."""
    M, n, K = 4, 10752, 5376
    N = 2 * n
    A, AS, B, BS = _gated_case(M, n, K, 1, 3)
    dev = gpu
    t = lambda x: torch.from_numpy(x.view(np.int16) if x.dtype == np.uint16 else x).to(dev)
    a, as_, b, bs = t(A), t(AS), t(B), t(BS)
    q = torch.empty((M, n), dtype=torch.uint8, device=dev)
    s = torch.empty((M, n // 128), dtype=torch.float32, device=dev)
    ops = R.GatedGemmOperands(a, as_, b, bs, q, s, None, N=N, K=K, act="silu", M=M)
    ops.set_scratch(torch.empty(R.row_scratch_bytes("gemm_nt_q_gated_fp8a8", ops),
                                dtype=torch.uint8, device=dev))
    stream = torch.cuda.current_stream().cuda_stream
    assert R.launch_row("gemm_nt_q_gated_fp8a8", ops, stream) == R.RAD_OK
    y = torch.empty((M, N), dtype=torch.int16, device=dev)
    assert R.launch_row("gemm_nt_q_fp8a8_decode",
                        R.GemmOperands(a, as_, b, bs, y, dtype="fp8a8", N=N, K=K),
                        stream) == R.RAD_OK
    torch.cuda.synchronize()
    qr, sr, _ = O.gated_quant_fp8(y.cpu().numpy().view(np.uint16), group=128, act="silu")
    _same_codes(q.cpu().numpy(), qr)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), sr.view(np.uint32))
