"""GPU parity of the gfx950 gemm_nt_q rows against the CPU oracle, through the C ABI.

Every launch goes through the registered row's launch pointer on guarded operands
(red zones on both sides of every operand, Y poisoned with a sentinel).  A case passes
when: the status is RAD_OK; no red zone was touched; every Y element was written; NaN
classes match; and per element
    |y - y_oracle| <= ulp_bf16 + 2*K*2^-24*S + 2^-10*S8
(S the oracle's magnitude sum; S8 the sum over 8-wide k groups of the largest scaled
product -- the block-scaled MFMA sums each 8 products at a width that truncates bits
below 2^-13 of the group's largest, measured on MI355X; see oracle/r3d_oracle.h).
Whole-tensor rel_l2 must stay inside the reference's own kbench tolerances (3e-2
mxfp4a8, 5e-3 fp8a8; docs/COVERAGE.md:868,1296).  On BASELINE.json's configs' data
(tests/test_gpu_configs.py) the per-row rel_l2 is held to 2^-8 (one bf16 ulp) as well.
The operand law of most cases here is the reference probe's (full-range NaN-free e4m3
codes, tools/probe_m4_entry.cpp:36-40): it maximises cancellation, so it tests the bound,
not the typical error.
"""
import numpy as np
import pytest

import libr3d_amd as R
from libr3d_amd import synth
import oracle as O

pytestmark = pytest.mark.gpu

MX_DEC, MX_TILE = "gemm_nt_q_mxfp4_decode", "gemm_nt_q_mxfp4"
F8_DEC, F8_TILE = "gemm_nt_q_fp8a8_decode", "gemm_nt_q_fp8a8"


def _gu():
    from tests import gpu_util
    return gpu_util


def _mx_case(M, N, K, seed, bs_lo=115, bs_hi=139):
    """The reference probe's operand law (tools/probe_m4_entry.cpp:36-40): NaN-free e4m3
    codes, random nibble bytes, E8M0 in 115..139, a_scale in [0.001, 0.011]."""
    rng = np.random.default_rng(seed)
    A = synth.random_e4m3_codes((M, K), rng)
    AS = (0.001 + 0.01 * rng.random((M, K // 128))).astype(np.float32)
    B = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    BS = rng.integers(bs_lo, bs_hi + 1, size=(N, K // 32)).astype(np.uint8)
    return A, AS, B, BS


def _f8_case(M, N, K, seed, rblk):
    rng = np.random.default_rng(seed)
    A = synth.random_e4m3_codes((M, K), rng)
    AS = (0.001 + 0.01 * rng.random((M, K // 128))).astype(np.float32)
    B = synth.random_e4m3_codes((N, K), rng)
    rows = N if rblk == 1 else (N + 127) // 128
    BS = synth.bf16_bits((0.001 + 0.01 * rng.random((rows, K // 128))).astype(np.float32))
    return A, AS, B, BS


KBENCH_TOL = {"mxfp4a8": 3e-2, "fp8a8": 5e-3}


def _check(row, dtype, A, AS, B, BS, M, N, K, gpu, rblk=1, row_rel_max=None, tunables=None,
           scratch=None):
    gu = _gu()
    rc, Y, guards = gu.run_row(row, dtype, A, AS, B, BS, M, N, K, gpu, tunables=tunables,
                               scratch=scratch)
    assert rc == R.RAD_OK, "row %s refused rc=%d" % (row, rc)
    assert guards, "red zone written"
    if dtype == "mxfp4a8":
        Yr, Yf, S = O.quant_dot_mxfp4a8(A, AS, B, BS, nthreads=16)
    else:
        Yr, Yf, S = O.quant_dot_fp8a8(A, AS, B, BS, rblk, nthreads=16)
    S8 = O.group8_mag(dtype, A, AS, B, BS, rblk, nthreads=16)
    c = gu.compare(Y, Yr, Yf, S, K, S8)
    assert c["sentinel_left"] == 0, c
    assert c["nan_mismatch"] == 0 and c["inf_mismatch"] == 0, c
    assert c["max_viol"] <= 1.0, c
    assert c["rel_l2"] <= KBENCH_TOL[dtype], c
    if row_rel_max is not None:
        assert c["row_rel_l2_max"] <= row_rel_max, c
    return c, Y


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 7, 8, 9, 15, 16])
def test_mxfp4_decode_small(gpu, M):
    A, AS, B, BS = _mx_case(M, 200, 640, 100 + M)
    _check(MX_DEC, "mxfp4a8", A, AS, B, BS, M, 200, 640, gpu)


@pytest.mark.parametrize("N,K", [(16, 128), (17, 256), (1000, 4096), (4096, 1152)])
def test_mxfp4_decode_shapes(gpu, N, K):
    for M in (1, 4):
        A, AS, B, BS = _mx_case(M, N, K, N + K + M)
        _check(MX_DEC, "mxfp4a8", A, AS, B, BS, M, N, K, gpu)


@pytest.mark.parametrize("dtype,M,N", [("fp8a8", 1, 8227), ("fp8a8", 1, 8301),
                                       ("mxfp4a8", 3, 8354), ("mxfp4a8", 3, 8477)])
def test_decode_seven_wave_ragged(gpu, dtype, M, N):
    """Seven-wave quad workgroups (chosen where they even the grid over the CUs) with a last
    workgroup of fewer quads and a partial last quad."""
    K = 1024
    row = MX_DEC if dtype == "mxfp4a8" else F8_DEC
    if dtype == "mxfp4a8":
        A, AS, B, BS = _mx_case(M, N, K, N + M)
    else:
        A, AS, B, BS = _f8_case(M, N, K, N + M, 1)
    _check(row, dtype, A, AS, B, BS, M, N, K, gpu)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 7, 8, 9, 15, 16])
@pytest.mark.parametrize("rblk", [1, 128])
def test_fp8_decode_small(gpu, M, rblk):
    A, AS, B, BS = _f8_case(M, 200, 640, 300 + M, rblk)
    _check(F8_DEC, "fp8a8", A, AS, B, BS, M, 200, 640, gpu, rblk=rblk)


@pytest.mark.parametrize("N,K", [(17, 256), (40, 1152), (1001, 640), (300, 21504)])
@pytest.mark.parametrize("M", [2, 5, 9, 16])
def test_mxfp4_decode_lines_shapes(gpu, N, K, M):
    """The line GEMV (M = 5..16): ragged N, odd group counts (a half-used last line); M = 2
    at K = 21504, whose activation rows are too large for the quad GEMV's staging, runs the
    16-row GEMV."""
    A, AS, B, BS = _mx_case(M, N, K, 7 * N + K + M)
    _check(MX_DEC, "mxfp4a8", A, AS, B, BS, M, N, K, gpu)


@pytest.mark.parametrize("N,K", [(17, 256), (1001, 640), (300, 21504)])
@pytest.mark.parametrize("M", [2, 9, 16])
@pytest.mark.parametrize("rblk", [1, 128])
def test_fp8_decode_lines_shapes(gpu, N, K, M, rblk):
    if rblk == 128 and N <= 128:
        pytest.skip("one 128-row scale block: the grid is ambiguous and the plan refuses it")
    A, AS, B, BS = _f8_case(M, N, K, 5 * N + K + M, rblk)
    _check(F8_DEC, "fp8a8", A, AS, B, BS, M, N, K, gpu, rblk=rblk)


@pytest.mark.parametrize("pad,offset", [(4, 0), (0, 4), (12, 8)])
def test_mxfp4_decode_scale_plane_layouts(gpu, pad, offset):
    """The E8M0 plane as a padded-pitch and/or 4-byte (not 16-byte) aligned view: the decode
    GEMV must stage it row by row instead of as one contiguous run, with the same result."""
    import torch
    gu = _gu()
    M, N, K = 1, 300, 2560
    A, AS, B, BS = _mx_case(M, N, K, 40 + pad + offset)
    wide = np.zeros((N, K // 32 + pad), np.uint8)
    wide[:, :K // 32] = BS
    flat = np.concatenate([np.zeros(offset, np.uint8), wide.reshape(-1)])
    gA, gAS, gB, gW = (gu.Guarded(x, gpu) for x in (A, AS, B, flat))
    bs = gW.t[offset:].view(N, K // 32 + pad)[:, :K // 32]
    gY = gu.y_buffer(M, N, gpu)
    ops = R.GemmOperands(gA.t, gAS.t, gB.t, bs, gY.t, dtype="mxfp4a8", N=N, K=K)
    rc = R.launch_row(MX_DEC, ops, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == R.RAD_OK
    assert all(g.guards_intact() for g in (gA, gAS, gB, gW, gY))
    Y = gY.t.cpu().numpy().view(np.uint16).reshape(M, N)
    Yr, Yf, S = O.quant_dot_mxfp4a8(A, AS, B, BS)
    S8 = O.group8_mag("mxfp4a8", A, AS, B, BS)
    c = gu.compare(Y, Yr, Yf, S, K, S8)
    assert c["sentinel_left"] == 0 and c["max_viol"] <= 1.0, c


@pytest.mark.parametrize("M,N,K", [(1, 1001, 5376), (1, 8227, 1024), (1, 700, 5248),
                                   (4, 777, 2048), (2, 300, 21504)])
def test_fp8_decode_scale_plane_layouts(gpu, M, N, K):
    """fp8a8 decode-row weight scales read through the plane's row pitch and base (the quad
    GEMV; at M = 2, K = 21504 the 16-row GEMV): the same per-row plane as a dense 16-byte
    aligned view and as a padded, 4-byte aligned view must give bit-identical Y (ragged last
    workgroups, even and odd group counts), and the dense one must pass the oracle check."""
    import torch
    gu = _gu()
    A, AS, B, BS = _f8_case(M, N, K, 70 + M + N, 1)
    c, Y_dense = _check(F8_DEC, "fp8a8", A, AS, B, BS, M, N, K, gpu)
    pad, offset = 3, 4
    wide = np.zeros((N, K // 128 + pad), np.uint16)
    wide[:, :K // 128] = BS
    flat = np.concatenate([np.zeros(offset // 2, np.uint16), wide.reshape(-1)])
    gA, gAS, gB, gW = (gu.Guarded(x, gpu) for x in (A, AS, B, flat))
    bs = gW.t[offset // 2:].view(N, K // 128 + pad)[:, :K // 128]
    gY = gu.y_buffer(M, N, gpu)
    ops = R.GemmOperands(gA.t, gAS.t, gB.t, bs, gY.t, dtype="fp8a8", N=N, K=K)
    rc = R.launch_row(F8_DEC, ops, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == R.RAD_OK
    assert all(g.guards_intact() for g in (gA, gAS, gB, gW, gY))
    Y_pad = gY.t.cpu().numpy().view(np.uint16).reshape(M, N)
    assert np.array_equal(Y_pad, Y_dense)


@pytest.mark.parametrize("N,K", [(17, 256), (1001, 4096), (4096, 1152), (6, 21504)])
@pytest.mark.parametrize("rblk", [1, 128])
def test_fp8_decode_shapes(gpu, N, K, rblk):
    """Ragged N (a partial last quad of weight rows), one to 168 groups, both scale grids
    (a 128-row grid needs N > 128 to be told apart from a per-row one)."""
    if rblk == 128 and N <= 128:
        pytest.skip("one block row is a per-row grid")
    for M in (1, 3):
        A, AS, B, BS = _f8_case(M, N, K, N + K + M + rblk, rblk)
        _check(F8_DEC, "fp8a8", A, AS, B, BS, M, N, K, gpu, rblk=rblk)


@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (17, 200, 256), (64, 256, 512),
                                   (130, 300, 384), (256, 512, 1024),
                                   (48, 1000, 4096), (63, 520, 2048),   # skinny: 16-row passes
                                   (32, 21504, 512)])                   # skinny, wide N: prefill
def test_mxfp4_tile(gpu, M, N, K):
    A, AS, B, BS = _mx_case(M, N, K, 7 * M + N)
    _check(MX_TILE, "mxfp4a8", A, AS, B, BS, M, N, K, gpu)


@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (17, 200, 256), (130, 300, 384),
                                   (300, 1000, 1152), (257, 129, 640), (64, 520, 4096),
                                   (40, 1000, 2048), (32, 21504, 512)])
@pytest.mark.parametrize("rblk", [1, 128])
def test_fp8_tile(gpu, M, N, K, rblk):
    A, AS, B, BS = _f8_case(M, N, K, 11 * M + N, rblk)
    _check(F8_TILE, "fp8a8", A, AS, B, BS, M, N, K, gpu, rblk=rblk)


def _geom(desc):
    return dict(kv.split("=") for kv in desc.split() if "=" in kv)


def _split_of(row, dtype, M, N, K):
    """(kc, cst) the row's describe reports with hook-sized scratch, or None unsplit."""
    gu = _gu()
    import torch
    A = np.zeros((M, K), np.uint8)
    AS = np.ones((M, K // 128), np.float32)
    B = np.zeros((N, K // 2 if dtype == "mxfp4a8" else K), np.uint8)
    BS = (np.zeros((N, K // 32), np.uint8) if dtype == "mxfp4a8"
          else np.zeros((N, K // 128), np.uint16))
    ts = [torch.from_numpy(x) for x in (A, AS, B, BS)]
    y = torch.zeros((M, N), dtype=torch.int16)
    ops = R.GemmOperands(*ts, y, dtype=dtype, N=N, K=K)
    need = R.row_scratch_bytes(row, ops)
    if not need:
        return None
    ops.set_scratch(torch.zeros(64, dtype=torch.uint8), need)   # describe reads no memory
    g = dict(kv.split("=") for kv in R.describe(row, ops)[1].split() if "=" in kv)
    assert g["arm"] == "splitk", g
    del gu
    return int(g["kc"]), int(g["cst"])


# split K on the tile rows (M <= 128, narrow N): chunks of equal and unequal length (a
# one-step last chunk at K = 2688), 18 chunks (K = 9216), ragged N (250: partial
# four-column groups, scalar stores), one token, the 128-token bound (the 128 x 128 tile
# past M = 64), config 2's qkv width; token groups wholly past M skip their MFMAs at M = 1,
# 17, 33, 40
SPLIT_SHAPES = [(17, 300, 9216), (40, 1000, 2048), (33, 700, 2688), (100, 250, 1536),
                (1, 64, 1024), (128, 520, 4096), (64, 8192, 1024)]


@pytest.mark.parametrize("M,N,K", SPLIT_SHAPES)
def test_mxfp4_tile_splitk(gpu, M, N, K):
    """The split arm against the oracle at the tile rows' bar, scratch guarded; two calls
    give the same bits (the chunks are summed in one order); without scratch the same
    operands take the unsplit arms and meet the same bar."""
    assert _split_of(MX_TILE, "mxfp4a8", M, N, K) is not None
    A, AS, B, BS = _mx_case(M, N, K, 5 * M + N + K)
    _, Y1 = _check(MX_TILE, "mxfp4a8", A, AS, B, BS, M, N, K, gpu, scratch="hook")
    _, Y2 = _check(MX_TILE, "mxfp4a8", A, AS, B, BS, M, N, K, gpu, scratch="hook")
    assert np.array_equal(Y1, Y2)
    _check(MX_TILE, "mxfp4a8", A, AS, B, BS, M, N, K, gpu)


@pytest.mark.parametrize("M,N,K", SPLIT_SHAPES)
@pytest.mark.parametrize("rblk", [1, 128])
def test_fp8_tile_splitk(gpu, M, N, K, rblk):
    if rblk == 128 and N <= 128:
        pytest.skip("one block row is a per-row grid")
    assert _split_of(F8_TILE, "fp8a8", M, N, K) is not None
    A, AS, B, BS = _f8_case(M, N, K, 3 * M + N + K + rblk, rblk)
    _, Y1 = _check(F8_TILE, "fp8a8", A, AS, B, BS, M, N, K, gpu, rblk=rblk, scratch="hook")
    _, Y2 = _check(F8_TILE, "fp8a8", A, AS, B, BS, M, N, K, gpu, rblk=rblk, scratch="hook")
    assert np.array_equal(Y1, Y2)


# split K on the decode rows (planes of 2^26+ weights past the quad GEMV): 17..64 chunks,
# a short last chunk (K = 25856), ragged M (5, 9) and N (2600: a partial last tile and dead
# rows), an M = 4 shape whose activation rows the quad GEMV cannot stage
DEC_SPLIT_SHAPES = [(16, 2048, 32768), (5, 1024, 65536), (9, 2600, 25856), (4, 3200, 21504)]


@pytest.mark.parametrize("M,N,K", DEC_SPLIT_SHAPES)
def test_mxfp4_decode_splitk(gpu, M, N, K):
    """The decode row's split arm against the oracle at the decode rows' bar, scratch
    guarded; two calls give the same bits; without scratch the GEMV meets the same bar."""
    gu = _gu()
    assert gu.hook_bytes(MX_DEC, "mxfp4a8", M, N, K) > 0
    A, AS, B, BS = _mx_case(M, N, K, 7 * M + N + K)
    _, Y1 = _check(MX_DEC, "mxfp4a8", A, AS, B, BS, M, N, K, gpu, scratch="hook")
    _, Y2 = _check(MX_DEC, "mxfp4a8", A, AS, B, BS, M, N, K, gpu, scratch="hook")
    assert np.array_equal(Y1, Y2)
    _check(MX_DEC, "mxfp4a8", A, AS, B, BS, M, N, K, gpu)


@pytest.mark.parametrize("M,N,K", DEC_SPLIT_SHAPES)
@pytest.mark.parametrize("rblk", [1, 128])
def test_fp8_decode_splitk(gpu, M, N, K, rblk):
    gu = _gu()
    assert gu.hook_bytes(F8_DEC, "fp8a8", M, N, K) > 0
    A, AS, B, BS = _f8_case(M, N, K, 5 * M + N + K + rblk, rblk)
    _, Y1 = _check(F8_DEC, "fp8a8", A, AS, B, BS, M, N, K, gpu, rblk=rblk, scratch="hook")
    _, Y2 = _check(F8_DEC, "fp8a8", A, AS, B, BS, M, N, K, gpu, rblk=rblk, scratch="hook")
    assert np.array_equal(Y1, Y2)


@pytest.mark.parametrize("row,dtype,M,N,K", [
    (MX_DEC, "mxfp4a8", 5, 2048, 32768), (MX_TILE, "mxfp4a8", 40, 1000, 2048),
    (F8_TILE, "fp8a8", 33, 700, 2688), (F8_DEC, "fp8a8", 9, 2048, 32768)])
def test_splitk_padded_views(gpu, row, dtype, M, N, K):
    """The K split on padded-pitch views of the operands (activation, a_scale, scale rows,
    Y, and the e4m3 weight rows; the e2m1 plane must be dense, as the reference's FP4 rule
    requires): the partial planes and their sum follow the pitches, and Y's padding columns
    are never written."""
    import torch
    gu = _gu()
    mx = dtype == "mxfp4a8"
    if mx:
        A, AS, B, BS = _mx_case(M, N, K, 11 * M + N)
    else:
        A, AS, B, BS = _f8_case(M, N, K, 11 * M + N, 1)

    def padded(x, extra):
        w = np.zeros((x.shape[0], x.shape[1] + extra), x.dtype)
        w[:, :x.shape[1]] = x
        return w

    hosts = [padded(A, 128), padded(AS, 4), padded(B, 0 if mx else 64), padded(BS, 8)]
    g = [gu.Guarded(h, gpu) for h in hosts]
    views = [gg.t[:, :x.shape[1]] for gg, x in zip(g, (A, AS, B, BS))]
    gY = gu.Guarded(np.full((M, N + 8), gu.Y_SENTINEL, np.uint16), gpu)
    ops = R.GemmOperands(*views, gY.t[:, :N], dtype=dtype, N=N, K=K)
    need = R.row_scratch_bytes(row, ops)
    assert need > 0
    gS = gu.Guarded(np.zeros(need, np.uint8), gpu, fill=0x5A)
    ops.set_scratch(gS.t, need)
    assert _geom(R.describe(row, ops)[1])["arm"] == "splitk"
    assert R.launch_row(row, ops, torch.cuda.current_stream().cuda_stream) == R.RAD_OK
    torch.cuda.synchronize()
    assert all(gg.guards_intact() for gg in g + [gY, gS])
    Yp = gY.t.cpu().numpy().view(np.uint16).reshape(M, N + 8)
    assert (Yp[:, N:] == gu.Y_SENTINEL).all()
    if mx:
        Yr, Yf, S = O.quant_dot_mxfp4a8(A, AS, B, BS, nthreads=16)
    else:
        Yr, Yf, S = O.quant_dot_fp8a8(A, AS, B, BS, 1, nthreads=16)
    S8 = O.group8_mag(dtype, A, AS, B, BS, 1, nthreads=16)
    c = gu.compare(np.ascontiguousarray(Yp[:, :N]), Yr, Yf, S, K, S8)
    assert c["sentinel_left"] == 0 and c["nan_mismatch"] == 0 and c["max_viol"] <= 1.0, c


@pytest.mark.parametrize("rblk", [1, 128])
def test_fp8_prefill_wide_tile_with_remainder(gpu, rblk):
    """The e4m3 prefill's four-wave 128 x 256 tile over whole rounds of weight rows, and the
    remaining rows as a second launch on the 128 x 128 tile (both scale grids: the second
    launch's weight-scale rows start n1 / rblk rows in)."""
    M, N, K = 512, 16640, 1024
    ops_desc = _f8_desc(M, N, K, rblk)
    assert (ops_desc["waves"], ops_desc["nsplit"]) == ("4", "16384"), ops_desc
    A, AS, B, BS = _f8_case(M, N, K, 77 + rblk, rblk)
    _check(F8_TILE, "fp8a8", A, AS, B, BS, M, N, K, gpu, rblk=rblk)


def _f8_desc(M, N, K, rblk):
    import torch
    rows = N if rblk == 1 else (N + 127) // 128
    ts = [torch.zeros((M, K), dtype=torch.uint8), torch.zeros((M, K // 128), dtype=torch.float32),
          torch.zeros((N, K), dtype=torch.uint8), torch.zeros((rows, K // 128), dtype=torch.int16)]
    ops = R.GemmOperands(*ts, torch.zeros((M, N), dtype=torch.int16), dtype="fp8a8", N=N, K=K)
    return _geom(R.describe(F8_TILE, ops)[1])


def test_splitk_short_scratch_runs_unsplit(gpu):
    """A byte short of the hook's size: the launch takes the unsplit arm, leaves the
    scratch untouched (its poison and red zones intact) and still meets the bar."""
    gu = _gu()
    M, N, K = 40, 1000, 2048
    A, AS, B, BS = _mx_case(M, N, K, 99)
    kc, _ = _split_of(MX_TILE, "mxfp4a8", M, N, K)
    need = kc * M * N * 4
    gA, gAS, gB, gBS = (gu.Guarded(x, gpu) for x in (A, AS, B, BS))
    gY = gu.y_buffer(M, N, gpu)
    gS = gu.Guarded(np.zeros(need - 1, np.uint8), gpu, fill=0x5A)
    import torch
    ops = R.GemmOperands(gA.t, gAS.t, gB.t, gBS.t, gY.t, dtype="mxfp4a8", N=N, K=K)
    ops.set_scratch(gS.t, need - 1)
    assert R.launch_row(MX_TILE, ops, torch.cuda.current_stream().cuda_stream) == R.RAD_OK
    torch.cuda.synchronize()
    assert all(g.guards_intact() for g in (gA, gAS, gB, gBS, gY, gS))
    assert (gS.t.cpu().numpy() == 0x5A).all()
    Y = gY.t.cpu().numpy().view(np.uint16).reshape(M, N)
    Yr, Yf, S = O.quant_dot_mxfp4a8(A, AS, B, BS, nthreads=16)
    c = gu.compare(Y, Yr, Yf, S, K, O.group8_mag("mxfp4a8", A, AS, B, BS, nthreads=16))
    assert c["sentinel_left"] == 0 and c["max_viol"] <= 1.0, c


@pytest.mark.parametrize("row", [MX_DEC, MX_TILE])
def test_mxfp4_dequant_bit_exact(gpu, row):
    """Every (e2m1 code, E8M0 byte) pair through the product path: activation row m is
    one-hot 1.0 at k = m with a_scale 1, weight row n carries the 16 codes at k = 0..15
    and E8M0 byte n on group 0, so Y[m, n] = bf16(e2m1(m) * 2^(n-127)) -- exactly the
    dequantised weight (<= 2 mantissa bits fit bf16).  Compared bit for bit against the
    oracle's dequantisation; byte 0xFF must give NaN."""
    gu = _gu()
    M, N, K = 16, 256, 128
    A = np.zeros((M, K), np.uint8)
    for m in range(M):
        A[m, m] = 0x38                                   # e4m3 1.0
    AS = np.ones((M, 1), np.float32)
    codes = np.arange(16, dtype=np.uint8)
    B = np.zeros((N, K // 2), np.uint8)
    B[:, :8] = (codes[0::2] | (codes[1::2] << 4))[None, :]
    BS = np.full((N, K // 32), 127, np.uint8)
    BS[:, 0] = np.arange(256, dtype=np.uint8)
    rc, Y, guards = gu.run_row(row, "mxfp4a8", A, AS, B, BS, M, N, K, gpu)
    assert rc == R.RAD_OK and guards
    deq = O.mxfp4_dequant(B, BS)[:, :16].T               # [m = code, n]
    got = O.bf16_to_f32(Y)
    got_nan = np.isnan(got)
    ref_nan = np.isnan(deq)
    assert np.array_equal(got_nan, ref_nan)
    assert ref_nan[:, 255].all()
    fin = ~ref_nan
    # value-exact against the dequantised weights (e2m1 * 2^(x-127) is exact in bf16); a
    # sum that starts at +0 returns +0 for code 8 (-0), so zeros compare by value ...
    bad = np.argwhere((got != deq) & fin)
    assert bad.size == 0, "dequant mismatch at %s: got %s want %s" % (
        bad[:5].tolist(), [got[tuple(b)] for b in bad[:5]], [deq[tuple(b)] for b in bad[:5]])
    # ... and bit-exact against the oracle's quant_dot on the same operands
    Yr, _, _ = O.quant_dot_mxfp4a8(A, AS, B, BS)
    assert np.array_equal(Y[fin], Yr[fin])


# bf16 weight scales for the fp8a8 dequant test: powers of two first (e4m3 x 2^e is exact
# in bf16, so the output must equal the dequantised weight itself), then scales whose
# products round, f32-subnormal products, and the two non-finite scales
F8_DEQ_SCALES = [1.0, 2.0 ** -30, 2.0 ** -9, 0.5, 2.0, 2.0 ** 7, 2.0 ** 40, 2.0 ** 100,
                 1.5, -0.75, 3.140625, 448.0, 1.0 / 3.0, 2.0 ** -120, float("nan"), float("inf")]
F8_DEQ_POW2 = 8


@pytest.mark.parametrize("row,mt", [(F8_DEC, 1), (F8_DEC, 4), (F8_DEC, 16), (F8_TILE, 16)])
@pytest.mark.parametrize("rblk", [1, 128])
def test_fp8_dequant_bit_exact(gpu, row, mt, rblk):
    """Every e4m3 weight code (+-0, subnormals, the two NaN codes 0x7F / 0xFF) times each
    bf16 weight scale of F8_DEQ_SCALES through the product path.  Activation row m is
    one-hot e4m3 1.0 at k = m with a_scale 1.  Weight rows come in groups of 32: row j < 16
    of a group carries codes 16 j .. 16 j + 15 at k = 0..15 (a NaN code replaced by 0: any
    NaN code in a row poisons all its outputs, 0 x NaN being NaN), row 16 the code 0x7F
    alone and row 17 0xFF alone at k = 0, the rest zeros; the 128 rows of block b share
    scale b (per-row grid: every row of the block holds it; 128-row grid: one scale row per
    block).  So Y[m, n] = bf16(e4m3(16 j + m) * scale[n // 128]) for j = n % 32 < 16, and
    NaN in every row m for j = 16, 17.  Bit-exact against the oracle's quant_dot for every
    code and scale (NaN as a class); value-exact against the dequantised weight for the
    power-of-two scales.  The decode row runs the quad GEMV at M = 1 and 4 (16 / mt calls,
    activation rows shifted along k) and the line GEMV at 16; the tile row the prefill
    pipeline."""
    gu = _gu()
    K, nsc = 128, len(F8_DEQ_SCALES)
    N = 128 * nsc
    n = np.arange(N)
    j = n % 32
    B = np.zeros((N, K), np.uint8)
    for k in range(16):
        c = (16 * j + k).astype(np.uint8)
        B[:, k] = np.where((j < 16) & ((c & 0x7F) != 0x7F), c, 0)
    B[j == 16, 0] = 0x7F
    B[j == 17, 0] = 0xFF
    sc = synth.bf16_bits(np.array(F8_DEQ_SCALES, np.float32))
    BS = (np.repeat(sc, 128)[:, None] if rblk == 1 else sc[:, None]).astype(np.uint16)
    Y = np.zeros((16, N), np.uint16)
    for c0 in range(0, 16, mt):
        A = np.zeros((mt, K), np.uint8)
        for m in range(mt):
            A[m, c0 + m] = 0x38                              # e4m3 1.0
        AS = np.ones((mt, 1), np.float32)
        rc, Yc, guards = gu.run_row(row, "fp8a8", A, AS, B, BS, mt, N, K, gpu)
        assert rc == R.RAD_OK and guards
        Y[c0:c0 + mt] = Yc
    A = np.zeros((16, K), np.uint8)
    A[np.arange(16), np.arange(16)] = 0x38
    Yr, _, _ = O.quant_dot_fp8a8(A, np.ones((16, 1), np.float32), B, BS, rblk)
    got, ref = O.bf16_to_f32(Y), O.bf16_to_f32(Yr)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.isnan(got[:, (j == 16) | (j == 17)]).all()     # the two NaN codes
    fin = ~np.isnan(ref)
    bad = np.argwhere((Y != Yr) & fin & ~((got == 0) & (ref == 0)))
    assert bad.size == 0, "bits differ at %s: got %s want %s" % (
        bad[:5].tolist(), [hex(Y[tuple(b)]) for b in bad[:5]], [hex(Yr[tuple(b)]) for b in bad[:5]])
    # value-exact against the dequantised weight where the scale is a power of two: all
    # 254 non-NaN codes at each of the F8_DEQ_POW2 scales
    codes = (16 * j[None, :] + np.arange(16)[:, None]).astype(np.uint8)            # [m, n]
    p2 = ((n // 128 < F8_DEQ_POW2) & (j < 16))[None, :] & ((codes & 0x7F) != 0x7F)
    deq = (O.e4m3_to_f32(np.where(p2, codes, 0).astype(np.uint8)).astype(np.float64) *
           np.array(F8_DEQ_SCALES, np.float64)[n // 128][None, :])
    assert len(np.unique(codes[p2])) == 254
    assert np.array_equal(got[p2].astype(np.float64), deq[p2])


@pytest.mark.parametrize("row", [MX_DEC, MX_TILE])
def test_mxfp4_nan_scale_poisons(gpu, row):
    """A 0xFF scale byte poisons its whole output element even when every code in its
    group is zero (oracle: (sub * sa) * NaN with sub = 0)."""
    M, N, K = 4, 64, 256
    A, AS, B, BS = _mx_case(M, N, K, 5)
    B[3, :16] = 0                                        # group 0 of row 3: all zero codes
    BS[3, 0] = 0xFF
    BS[10, 5] = 0xFF
    c, Y = _check(row, "mxfp4a8", A, AS, B, BS, M, N, K, gpu)
    y = O.bf16_to_f32(Y)
    assert np.isnan(y[:, 3]).all() and np.isnan(y[:, 10]).all()
    assert np.isfinite(np.delete(y, [3, 10], axis=1)).all()


def test_decode_m_from_numel_y(gpu):
    """M is numel(y)/N, never the M parameter: an M=99 param with a 3-row y computes 3 rows."""
    gu = _gu()
    M, N, K = 3, 64, 256
    A, AS, B, BS = _mx_case(M, N, K, 9)
    rc, Y, guards = gu.run_row(MX_DEC, "mxfp4a8", A, AS, B, BS, M, N, K, gpu,
                               extra=[("M", 99)])
    assert rc == R.RAD_OK and guards
    Yr, Yf, S = O.quant_dot_mxfp4a8(A, AS, B, BS)
    S8 = O.group8_mag("mxfp4a8", A, AS, B, BS)
    c = gu.compare(Y, Yr, Yf, S, K, S8)
    assert c["max_viol"] <= 1.0 and c["sentinel_left"] == 0


@pytest.mark.parametrize("splitk", [1, 2, 4, 8])
@pytest.mark.parametrize("dtype", ["mxfp4a8", "fp8a8"])
@pytest.mark.parametrize("M", [4, 16])
def test_decode_splitk_deterministic(gpu, splitk, dtype, M):
    """Every chunk count (the decode rows' "splitk" tunable) stays in bound, and repeated
    calls are bit-identical (the LDS fold runs in chunk order)."""
    gu = _gu()
    N, K = 512, 2048
    if dtype == "mxfp4a8":
        A, AS, B, BS = _mx_case(M, N, K, 77)
        row = MX_DEC
    else:
        A, AS, B, BS = _f8_case(M, N, K, 77, 1)
        row = F8_DEC
    tv = [("splitk", splitk)]
    _, y1 = _check(row, dtype, A, AS, B, BS, M, N, K, gpu, tunables=tv)
    rc, y2, guards = gu.run_row(row, dtype, A, AS, B, BS, M, N, K, gpu, tunables=tv)
    assert rc == R.RAD_OK and guards
    assert np.array_equal(y1, y2)


@pytest.mark.parametrize("M,N,K,scratch", [(512, 16640, 1024, None), (300, 1000, 640, None),
                                           (40, 1000, 2048, "hook"), (130, 384, 256, None)])
def test_fp8_block_grid_matches_per_row_grid(gpu, M, N, K, scratch):
    """The tile row on the 128 x 128 block grid folds the weight scale into the token's
    (acc = fma(D, sa * sb, acc)).  With power-of-two a_scales and weight scales every
    product in either order is exact, so it must equal, bit for bit, the per-row grid
    holding the same scales replicated over each block's 128 rows (libref's
    acc + (D * sa) * sb) -- distinct scales per block and K group, so a wrong block, group
    or weight set shows; every tile kind: the four-wave tile with its 128 x 128 remainder,
    the 128 x 128 tile alone, the split K over hook scratch, a partial last block."""
    gu = _gu()
    rng = np.random.default_rng(M + N + K)
    A = synth.random_e4m3_codes((M, K), rng)
    AS = np.exp2(rng.integers(-10, -4, size=(M, K // 128))).astype(np.float32)
    B = synth.random_e4m3_codes((N, K), rng)
    blocks = (N + 127) // 128
    BSb = synth.bf16_bits(np.exp2(rng.integers(-12, -5, size=(blocks, K // 128))).astype(np.float32))
    BSr = np.repeat(BSb, 128, axis=0)[:N].copy()
    rc1, Y1, ok1 = gu.run_row(F8_TILE, "fp8a8", A, AS, B, BSb, M, N, K, gpu, scratch=scratch)
    rc2, Y2, ok2 = gu.run_row(F8_TILE, "fp8a8", A, AS, B, BSr, M, N, K, gpu, scratch=scratch)
    assert rc1 == R.RAD_OK and rc2 == R.RAD_OK and ok1 and ok2
    assert not np.any(Y1 == gu.Y_SENTINEL)
    assert np.array_equal(Y1, Y2), int((Y1 != Y2).sum())
