"""logits_gemm_e4m3 on the GPU, through the row's launch pointer: parity with the oracle
and with the exact float64 sum over ragged and strided shapes, every scale dtype, both
scale row blocks and hand-built scale-plane layouts, passes over many activation rows, the
persistent chunk walk; all 256 codes bit-exact through one-hot activations; red zones round
every operand; the cached header's guard; refusals that need the device header."""
import numpy as np
import pytest
import torch

import libr3d_amd as R
import oracle as O
from libr3d_amd import synth
from tests import gpu_util as gu
from tests import logits_util as LU

pytestmark = pytest.mark.gpu
ROW = "logits_gemm_e4m3"
Y_FILL = np.float32(-7.75e33)            # no output equals it


def kernel_bound(K, S):
    """|y - exact| for the kernel.  Per 256-wide window each of four K slots is two chained
    32-deep MFMAs, each within 66 * 2^-24 of the magnitudes it sums (33 terms, each
    truncated below 2^-23 of the largest; the second's C is the first's result), so within
    132 * 2^-24 of the slot's magnitudes; then one fma per window into the slot's f32
    accumulator, and three adds over the slots.  The product code * x is exact (4 x 8
    significant bits), and code * scale needs none (the scale multiplies the window sum)."""
    nw = (K + 255) // 256
    return (132 + 2 * nw + 4) * 2.0 ** -24 * np.asarray(S, np.float64) + 2.0 ** -126


def custom_blob(codes, sbits, sdt, br, s_pad=0, s_shift=0):
    """A joined head written by hand: the scale plane's rows s_pad elements longer than
    ceil(K / 128), and the plane s_shift bytes past its 256-byte boundary -- layouts the
    library's own join never writes but rad_planes.h admits."""
    N, K = codes.shape
    h = LU.header(N, K, sdt, br)
    esz = 4 if sdt == "f32" else 2
    srows, scols = sbits.shape
    rb = (scols + s_pad) * esz
    c_off = LU.up256(LU.HEADER_BYTES)
    s_off = LU.up256(c_off + N * K) + s_shift
    LU.set_field(h, "row_bytes", rb, 1)
    LU.set_field(h, "offset", s_off, 1)
    LU.set_field(h, "bytes", s_off + srows * rb)
    blob = np.zeros(s_off + srows * rb, np.uint8)
    blob[:LU.HEADER_BYTES] = h
    blob[c_off:c_off + N * K] = codes.reshape(-1)
    plane = np.zeros((srows, scols + s_pad), sbits.dtype)
    plane[:, :scols] = sbits
    if s_pad:                            # NaN in every padding element
        plane[:, scols:] = np.float32(np.nan) if sdt == "f32" else 0x7FC0 if sdt == "bf16" else 0x7E00
    blob[s_off:] = plane.view(np.uint8).reshape(-1)
    return blob


def run(x, codes, sbits, sdt, br, dev, x_pitch=None, y_pitch=None, forget=True, blob=None):
    """Launch the row on guarded device copies; returns (rc, Y [M, N] f32, guards ok)."""
    M, K = x.shape
    N = codes.shape[0]
    xp = x_pitch or K
    xh = np.zeros((M, xp), np.uint16)
    xh[:, :K] = x
    yp = y_pitch or N
    gx = gu.Guarded(xh, dev)
    gw = gu.Guarded(R.join_head(codes, sbits, sdt, br) if blob is None else blob, dev)
    gy = gu.Guarded(np.full((M, yp), Y_FILL, np.float32), dev)
    ops = R.LogitsOperands(gx.t, gw.t, gy.t, n_vocab=N, n_embd=K,
                           shapes={0: [M, K], 2: [M, N]}, strides={0: [xp, 1], 2: [yp, 1]})
    rc = R.launch_row(ROW, ops, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    if forget:
        R.forget_head(gw.t)
    Y = gy.t.cpu().numpy().reshape(M, yp)
    ok = all(g.guards_intact() for g in (gx, gw, gy))
    if yp > N:
        ok = ok and bool(np.all(Y[:, N:] == Y_FILL))        # the row pitch's padding untouched
    return rc, Y[:, :N], ok


def check(Y, x, codes, sbits, sdt, br, case):
    K = x.shape[1]
    Yo, S = O.logits_e4m3(x, codes, sbits, sdt, br, nthreads=O.max_threads())
    ye, se = LU.exact(x, codes, sbits, sdt, br)
    assert not np.any(Y == Y_FILL), "unwritten logits"
    nan = np.isnan(Yo)
    assert np.array_equal(np.isnan(Y), nan), "NaN pattern differs"
    d_or = np.abs(Y.astype(np.float64) - Yo)[~nan]
    d_ex = np.abs(Y.astype(np.float64) - ye)[~nan]
    b_ex = kernel_bound(K, se)[~nan]
    b_or = b_ex + (K + 1) * 2.0 ** -24 * se[~nan]
    assert np.all(d_ex <= b_ex), ("exact", float((d_ex / b_ex).max()))
    assert np.all(d_or <= b_or), ("oracle", float((d_or / b_or).max()))
    yf = np.where(nan, 0, Y).astype(np.float64)
    ref = np.where(nan, 0, ye)
    row_rel = np.sqrt(((yf - ref) ** 2).sum(1) / np.maximum((ref ** 2).sum(1), 1e-300))
    assert row_rel.max() <= 2.0 ** -16, row_rel.max()
    c = {"rel_l2": float(np.sqrt(((yf - ref) ** 2).sum() / max((ref ** 2).sum(), 1e-300))),
         "row_rel_l2_max": float(row_rel.max()), "max_abs": float(d_ex.max()) if d_ex.size else 0.0,
         "max_viol": float((d_or / b_or).max()) if d_or.size else 0.0, "row_rel_l2": row_rel}
    gu.record(case, ROW, list(x.shape) + [codes.shape[0]], c)
    return c


CASES = [  # M, N, K, sdt, br, x_pitch, y_pitch
    (1, 300, 208, "bf16", 1, None, None),        # ragged N, last window 80 wide
    (3, 513, 384, "f16", 128, None, None),       # partial last row block
    (4, 4096, 5376, "bf16", 1, None, None),      # the 27B head's width
    (8, 2000, 1024, "f32", 1, None, None),
    (16, 1000, 640, "bf16", 128, 648, 1003),     # strided x and logits
    (20, 700, 256, "bf16", 1, None, None),       # two passes over x
    (6, 200, 16384, "bf16", 1, None, None),      # 32 KB rows of x: 4 a pass, two passes
    (2, 96, 144, "bf16", 1, None, None),         # two windows, the second 16 wide
    (5, 70000, 256, "bf16", 1, None, None),      # many chunks a wave, 5 rows of x
]


@pytest.mark.parametrize("M,N,K,sdt,br,xp,yp", CASES)
def test_logits_parity(gpu, M, N, K, sdt, br, xp, yp):
    print("logits parity M=%d N=%d K=%d %s br=%d" % (M, N, K, sdt, br), flush=True)
    codes, sbits = LU.head(N, K, M * 7 + N, sdt, br)
    x = synth.bf16_bits(np.random.default_rng(M + K).standard_normal((M, K)).astype(np.float32))
    rc, Y, ok = run(x, codes, sbits, sdt, br, gpu, xp, yp)
    assert rc == R.RAD_OK and ok
    check(Y, x, codes, sbits, sdt, br, "logits_M%d_N%d_K%d_%s_br%d" % (M, N, K, sdt, br))


@pytest.mark.parametrize("sdt,br,pad,shift", [("bf16", 1, 3, 0), ("f16", 1, 0, 2),
                                              ("f32", 1, 1, 4), ("bf16", 128, 5, 6)])
def test_scale_plane_layouts(gpu, sdt, br, pad, shift):
    """Scale rows padded past ceil(K / 128) (the padding holds NaN: read, it would poison the
    logits) and scale planes off 16-byte alignment: the per-chunk scale fetch falls back from
    whole 16-byte units to single elements and must read only the grid."""
    M, N, K = 3, 300, 640
    codes, sbits = LU.head(N, K, 17, sdt, br)
    x = synth.bf16_bits(np.random.default_rng(18).standard_normal((M, K)).astype(np.float32))
    rc, Y, ok = run(x, codes, sbits, sdt, br, gpu, blob=custom_blob(codes, sbits, sdt, br, pad, shift))
    assert rc == R.RAD_OK and ok
    check(Y, x, codes, sbits, sdt, br, "logits_layout_%s_br%d_pad%d_shift%d" % (sdt, br, pad, shift))


@pytest.mark.parametrize("sdt", ["bf16", "f16", "f32"])
def test_every_code_bit_exact(gpu, sdt):
    """Row n holds code n at column 133 (the second window) and zeros elsewhere; x rows are
    one-hot there with 1 and -0.25: every logit is one exact product, so the device's
    dequantised weight f32(e4m3(n) * s) must equal the oracle's bit for bit (NaN codes
    poison their row)."""
    N, K = 256, 256
    codes = np.zeros((N, K), np.uint8)
    codes[:, 133] = np.arange(256)
    s = np.float32(1.3125)
    sbits = {"bf16": synth.bf16_bits(np.full((N, 2), s, np.float32)),
             "f16": np.full((N, 2), s, np.float16).view(np.uint16),
             "f32": np.full((N, 2), s, np.float32)}[sdt]
    x = np.zeros((2, K), np.uint16)
    x[:, 133] = synth.bf16_bits(np.array([1.0, -0.25], np.float32))
    rc, Y, ok = run(x, codes, sbits, sdt, 1, gpu)
    assert rc == R.RAD_OK and ok
    Yo, _ = O.logits_e4m3(x, codes, sbits, sdt, 1)
    nan = np.isnan(Yo)
    assert nan.sum() == 4 and np.array_equal(np.isnan(Y), nan)
    assert np.array_equal(Y[~nan].view(np.uint32), Yo[~nan].view(np.uint32))


def test_nan_code_and_scale_poison_their_rows(gpu):
    M, N, K = 2, 64, 256
    codes, sbits = LU.head(N, K, 3)
    codes[5, 17] = 0x7F                   # NaN code
    codes[9, 200] = 0xFF
    x = synth.bf16_bits(np.random.default_rng(1).standard_normal((M, K)).astype(np.float32))
    rc, Y, ok = run(x, codes, sbits, "bf16", 1, gpu)
    assert rc == R.RAD_OK and ok
    assert np.isnan(Y[:, [5, 9]]).all() and not np.isnan(np.delete(Y, [5, 9], axis=1)).any()
    check(Y, x, codes, sbits, "bf16", 1, "logits_nan_codes")


def test_header_cache_and_guard(gpu):
    """The first launch over a device blob caches its header.  A different head joined at
    the same address (scale rows per 128 instead of per row) without forgetting it: the
    kernel's check of the device header fails and every logit is NaN (never a read past
    the planes); after forget_head the launch reads the new header and is right."""
    M, N, K = 2, 300, 256
    x = synth.bf16_bits(np.random.default_rng(2).standard_normal((M, K)).astype(np.float32))
    c1, s1 = LU.head(N, K, 4, "bf16", 1)
    c2, s2 = LU.head(N, K, 5, "bf16", 128)
    b1, b2 = R.join_head(c1, s1, "bf16", 1), R.join_head(c2, s2, "bf16", 128)
    blob = torch.zeros(max(b1.size, b2.size), dtype=torch.uint8, device=gpu)
    xt = torch.from_numpy(x.view(np.int16)).to(gpu)
    y = torch.empty((M, N), dtype=torch.float32, device=gpu)
    st = torch.cuda.current_stream().cuda_stream

    def launch(b):
        blob[:b.size].copy_(torch.from_numpy(b))
        ops = R.LogitsOperands(xt, blob[:b.size], y, n_vocab=N, n_embd=K)
        rc = R.launch_row(ROW, ops, st)
        torch.cuda.synchronize()
        return rc, y.cpu().numpy().copy()

    try:
        rc, Y = launch(b1)
        assert rc == R.RAD_OK
        check(Y, x, c1, s1, "bf16", 1, "logits_cache_first")
        rc, Y = launch(b2)
        assert rc == R.RAD_OK and np.isnan(Y).all()
        R.forget_head(blob)
        rc, Y = launch(b2)
        assert rc == R.RAD_OK
        check(Y, x, c2, s2, "bf16", 128, "logits_cache_rejoined")
    finally:
        R.forget_head(blob)


def test_device_header_refusals(gpu):
    """Gates that read the device header: no magic -> RAD_E_DTYPE; a head whose codes
    plane is not n_vocab x n_embd -> RAD_E_SHAPE; nothing is written on a refusal."""
    M, N, K = 1, 64, 256
    codes, sbits = LU.head(N, K, 6)
    x = torch.zeros((M, K), dtype=torch.int16, device=gpu)
    y = torch.full((M, N), 3.0, dtype=torch.float32, device=gpu)
    st = torch.cuda.current_stream().cuda_stream
    b = R.join_head(codes, sbits)
    bad = b.copy()
    bad[0] ^= 0xFF
    t = torch.from_numpy(bad).to(gpu)
    assert R.launch_row(ROW, R.LogitsOperands(x, t, y, n_vocab=N, n_embd=K), st) == R.RAD_E_DTYPE
    R.forget_head(t)
    t = torch.from_numpy(b).to(gpu)
    assert R.launch_row(ROW, R.LogitsOperands(x, t, y[:, :32], n_vocab=32, n_embd=K),
                        st) == R.RAD_E_SHAPE
    R.forget_head(t)
    torch.cuda.synchronize()
    assert (y == 3.0).all()
