"""GPU parity of operands at any alignment, against the CPU oracle, through the C ABI.

The reference's rows take their operands at any byte address and pitch: its tile rows read
bytes ("anything odd rides the tile", src/r3d_gemm_fp8a8.hip:985-990,1090-1095) and its
logits row takes n_embd % 4 == 0 with no alignment gate (src/r3d_gemm_logits.hip:166).  An
issue-time refusal is an engine abort (src/r3d_rows.cpp:2197-2215), so here every such
call must run and match the oracle:
  * gemm_nt_q (mxfp4a8 and fp8a8, tile and decode rows; mxfp4a16): A, B or the weight-
    scale plane 1, 4 or 8 bytes off an aligned base, an A row pitch off 16 bytes, Y 2 bytes
    off with a ragged pitch -- the any-alignment GEMM (and mxfp4a16's element-wise
    quantiser), to the same per-element bound as every other arm;
  * logits_gemm_e4m3: n_embd 132 and 260 (off a multiple of 16), x, codes and scale off
    alignment -- the dword walk, to the logits bound.
Every operand sits inside a red-zone buffer whose bytes outside the operand's elements
(the red zones and the pitch gaps) must be unchanged after the launch, and Y starts
poisoned so an unwritten element shows.
"""
import numpy as np
import pytest
import torch

import libr3d_amd as R
from libr3d_amd import synth
import oracle as O
from tests import logits_util as LU

pytestmark = pytest.mark.gpu

GUARD = 512
POISON = 0xA5


class DevView:
    """A 2-D operand placed `off` bytes into a red-zoned device buffer with a row pitch of
    `pitch` elements: the tensor interface the operand builders read (data_ptr, shape,
    stride, element_size, numel)."""

    def __init__(self, host, dev, off=0, pitch=None, poison_body=False):
        host = np.ascontiguousarray(host)
        if host.ndim == 1:
            host = host.reshape(1, -1)
        rows, cols = host.shape
        self.isz = host.itemsize
        self.pitch = pitch or cols
        self.off = off
        span = ((rows - 1) * self.pitch + cols) * self.isz
        img = np.full(GUARD + off + span + GUARD, POISON, np.uint8)
        self.mask = np.zeros(img.size, bool)            # the operand's element bytes
        for r in range(rows):
            b = GUARD + off + r * self.pitch * self.isz
            self.mask[b:b + cols * self.isz] = True
            if not poison_body:
                img[b:b + cols * self.isz] = host[r].view(np.uint8)
        self.img = img
        self.buf = torch.from_numpy(img.copy()).to(dev)
        self.shape = (rows, cols)
        self.dtype = {1: torch.uint8, 2: torch.int16, 4: torch.float32}[self.isz]

    def data_ptr(self):
        return self.buf.data_ptr() + GUARD + self.off

    def stride(self, dim=None):
        s = (self.pitch, 1)
        return s if dim is None else s[dim]

    def element_size(self):
        return self.isz

    def numel(self):
        return self.shape[0] * self.shape[1]

    def read(self):
        raw = self.buf.cpu().numpy()
        rows, cols = self.shape
        out = np.empty((rows, cols * self.isz), np.uint8)
        for r in range(rows):
            b = GUARD + self.off + r * self.pitch * self.isz
            out[r] = raw[b:b + cols * self.isz]
        return raw, out

    def untouched(self, written=False):
        """Bytes outside the operand's elements (all bytes, for an input) are unchanged."""
        raw = self.buf.cpu().numpy()
        keep = ~self.mask if written else np.ones(raw.size, bool)
        return bool(np.array_equal(raw[keep], self.img[keep]))


def _bound_check(Y, Yr, Yf, S, K, S8):
    from tests import gpu_util as gu
    c = gu.compare(Y, Yr, Yf, S, K, S8)
    assert c["sentinel_left"] == 0, c
    assert c["nan_mismatch"] == 0 and c["inf_mismatch"] == 0, c
    assert c["max_viol"] <= 1.0, c
    return c


def _mx_case(M, N, K, seed):
    rng = np.random.default_rng(seed)
    A = synth.random_e4m3_codes((M, K), rng)
    AS = (0.001 + 0.01 * rng.random((M, K // 128))).astype(np.float32)
    B = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    BS = rng.integers(115, 140, size=(N, K // 32)).astype(np.uint8)
    return A, AS, B, BS


def _f8_case(M, N, K, seed, rblk):
    rng = np.random.default_rng(seed)
    A = synth.random_e4m3_codes((M, K), rng)
    AS = (0.001 + 0.01 * rng.random((M, K // 128))).astype(np.float32)
    B = synth.random_e4m3_codes((N, K), rng)
    rows = N if rblk == 1 else (N + 127) // 128
    BS = synth.bf16_bits((0.001 + 0.01 * rng.random((rows, K // 128))).astype(np.float32))
    return A, AS, B, BS


ROWS = [("gemm_nt_q_mxfp4", "mxfp4a8"), ("gemm_nt_q_mxfp4_decode", "mxfp4a8"),
        ("gemm_nt_q_fp8a8", "fp8a8"), ("gemm_nt_q_fp8a8_decode", "fp8a8")]
SHIFTS = [("a", 1), ("a", 4), ("a", 8), ("b", 1), ("b", 4), ("b", 8), ("bs", 1), ("bs", 2),
          ("pitch", 0), ("y", 2)]


@pytest.mark.parametrize("row,dtype", ROWS)
@pytest.mark.parametrize("which,off", SHIFTS)
@pytest.mark.parametrize("M", [1, 3, 16, 40, 130])
def test_gemm_any_alignment(gpu, row, dtype, which, off, M):
    if "decode" in row and M > 16:
        pytest.skip("past the decode band")
    if which == "bs" and dtype == "fp8a8" and off == 1:
        pytest.skip("a bf16 plane on an odd byte is not an element-aligned tensor")
    N, K, rblk = 200, 512, 1
    seed = 1000 * M + 10 * off + len(which)
    if dtype == "mxfp4a8":
        A, AS, B, BS = _mx_case(M, N, K, seed)
    else:
        rblk = 128 if M == 3 else 1
        A, AS, B, BS = _f8_case(M, N, K, seed, rblk)
    sh = lambda w: off if which == w else 0                          # noqa: E731
    vA = DevView(A, gpu, sh("a"), pitch=K + 20 if which == "pitch" else None)
    vAS = DevView(AS, gpu)
    vB = DevView(B, gpu, sh("b"))
    vBS = DevView(BS, gpu, sh("bs"))
    vY = DevView(np.full((M, N), 0xEEEE, np.uint16), gpu, sh("y"),
                 pitch=N + 3 if which == "y" else None)
    ops = R.GemmOperands(vA, vAS, vB, vBS, vY, dtype=dtype, N=N, K=K)
    rc, d = R.describe(row, ops)
    assert rc == R.RAD_OK, d
    if not (which == "y" or (which == "bs" and dtype == "fp8a8")):
        assert d.startswith("arm=any "), d
    print(row, which, off, M, d.split()[0], flush=True)
    rc = R.launch_row(row, ops, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == R.RAD_OK
    for v in (vA, vAS, vB, vBS):
        assert v.untouched(), "an input or its red zone changed"
    assert vY.untouched(written=True), "a byte outside Y's elements was written"
    Y = vY.read()[1].view(np.uint16).reshape(M, N)
    if dtype == "mxfp4a8":
        Yr, Yf, S = O.quant_dot_mxfp4a8(A, AS, B, BS, nthreads=16)
    else:
        Yr, Yf, S = O.quant_dot_fp8a8(A, AS, B, BS, rblk, nthreads=16)
    S8 = O.group8_mag(dtype, A, AS, B, BS, rblk, nthreads=16)
    _bound_check(Y, Yr, Yf, S, K, S8)


@pytest.mark.parametrize("which,off", [("a", 2), ("a", 6), ("pitch", 0), ("b", 1), ("b", 4),
                                       ("bs", 3)])
@pytest.mark.parametrize("M", [5, 70])
def test_mxfp4a16_any_alignment(gpu, which, off, M):
    """The bf16-in row: a misaligned bf16 A runs the element-wise quantiser (its codes and
    scales bit-exact against the oracle's quantiser), a misaligned weight plane the any-
    alignment GEMM."""
    N, K = 200, 384
    rng = np.random.default_rng(M + off)
    X = synth.bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    B, BS = synth.mxfp4_weights(N, K, M + 7)
    sh = lambda w: off if which == w else 0                          # noqa: E731
    vX = DevView(X, gpu, sh("a"), pitch=K + 3 if which == "pitch" else None)
    vB, vBS = DevView(B, gpu, sh("b")), DevView(BS, gpu, sh("bs"))
    vY = DevView(np.full((M, N), 0xEEEE, np.uint16), gpu)
    ops = R.GemmOperands(vX, None, vB, vBS, vY, dtype="mxfp4a16", N=N, K=K, group=32, M=M)
    need = R.row_scratch_bytes("gemm_nt_q_mxfp4a16", ops)
    scr = torch.zeros(need, dtype=torch.uint8, device=gpu)
    ops.set_scratch(scr, need)
    rc = R.launch_row("gemm_nt_q_mxfp4a16", ops, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == R.RAD_OK
    assert all(v.untouched() for v in (vX, vB, vBS)) and vY.untouched(written=True)
    raw = scr.cpu().numpy()
    qb = ((M * K + 255) // 256) * 256
    Qr, SXr = O.quant_act_mxfp8(X)
    assert np.array_equal(raw[:M * K].reshape(M, K), Qr)
    assert np.array_equal(raw[qb:qb + M * (K // 32)].reshape(M, K // 32), SXr)
    Y = vY.read()[1].view(np.uint16).reshape(M, N)
    Yr, Yf, S = O.dot_mx8_mxfp4(Qr, SXr, B, BS, nthreads=16)
    S8 = O.group8_mag("mxfp4a16", Qr, SXr, B, BS, nthreads=16)
    _bound_check(Y, Yr, Yf, S, K, S8)


# ------------------------------------------------------------------ logits_gemm_e4m3
def _logits_run(gpu, M, N, K, sdt, br, x_off=0, x_pitch=None, blob_off=0, s_shift=0):
    """One launch over a head joined at blob_off bytes into its buffer (the scale plane
    s_shift bytes past its rounded offset); (Y f32 [M, N], x bits, codes, scale bits)."""
    codes, sbits = LU.head(N, K, M * 31 + N + K, sdt, br)
    rng = np.random.default_rng(K)
    x = synth.bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    h = LU.header(N, K, sdt, br)
    srows, scols = (N + br - 1) // br, (K + 127) // 128
    esz = 4 if sdt == "f32" else 2
    c_off = LU.up256(LU.HEADER_BYTES)
    s_off = LU.up256(c_off + N * K) + s_shift
    LU.set_field(h, "offset", s_off, 1)
    LU.set_field(h, "bytes", s_off + srows * scols * esz)
    blob = np.zeros(s_off + srows * scols * esz, np.uint8)
    blob[:LU.HEADER_BYTES] = h
    blob[c_off:c_off + N * K] = codes.reshape(-1)
    blob[s_off:] = np.ascontiguousarray(sbits).view(np.uint8).reshape(-1)
    vX = DevView(x, gpu, x_off, pitch=x_pitch)
    vW = DevView(blob, gpu, blob_off)
    vY = DevView(np.full((M, N), np.nan, np.float32), gpu)
    ops = R.LogitsOperands(vX, vW, vY, n_vocab=N, n_embd=K,
                           shapes={1: [blob.size]}, strides={1: [1]})
    rc = R.launch_row("logits_gemm_e4m3", ops, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    R.forget_head(vW.data_ptr())
    assert rc == R.RAD_OK, rc
    assert vX.untouched() and vW.untouched() and vY.untouched(written=True)
    rc2, d = R.describe("logits_gemm_e4m3", ops)     # the header is cached no longer
    assert rc2 == R.RAD_E_UNSUPPORTED and "not host-readable" in d, d
    Y = vY.read()[1].view(np.float32).reshape(M, N)
    return Y, x, codes, sbits


@pytest.mark.parametrize("K,x_off,x_pitch,blob_off,s_shift", [
    (132, 0, None, 0, 0), (260, 0, None, 0, 0),           # n_embd off a multiple of 16
    (256, 2, None, 0, 0), (256, 0, 260, 0, 0),             # x base / pitch off 16 bytes
    (256, 0, None, 4, 0), (256, 0, None, 1, 0),            # codes off 16 bytes, on an odd byte
    (260, 6, 266, 3, 2),                                   # all at once
])
@pytest.mark.parametrize("M", [1, 4, 7])
@pytest.mark.parametrize("sdt,br", [("bf16", 1), ("f16", 128), ("f32", 1)])
def test_logits_any_alignment(gpu, K, x_off, x_pitch, blob_off, s_shift, M, sdt, br):
    if s_shift % (4 if sdt == "f32" else 2) and sdt != "bf16":
        s_shift = 0
    N = 300
    Y, x, codes, sbits = _logits_run(gpu, M, N, K, sdt, br, x_off, x_pitch, blob_off, s_shift)
    Yo, S = O.logits_e4m3(x, codes, sbits, sdt, br)
    ye, se = LU.exact(x, codes, sbits, sdt, br)
    nw = (K + 127) // 128
    # the kernel: (windows + 4 * 66) 2^-24 of the magnitude sum; the oracle K 2^-24
    assert np.all(np.abs(Y - ye) <= (nw + 4 * 66 + 1) * 2.0 ** -24 * se + 1e-30)
    assert np.all(np.abs(Yo - ye) <= (K + 1) * 2.0 ** -24 * se + 1e-30)


def test_logits_describe_device_head(gpu):
    """describe copies nothing from the device: over a device-resident head it answers
    "not host-readable" until a launch has cached the header, then the plan."""
    M, N, K = 2, 64, 256
    codes, sbits = LU.head(N, K, 9)
    blob = R.join_head(codes, sbits)
    w = torch.from_numpy(blob).to(gpu)
    x = torch.zeros((M, K), dtype=torch.int16, device=gpu)
    y = torch.zeros((M, N), dtype=torch.float32, device=gpu)
    ops = R.LogitsOperands(x, w, y, n_vocab=N, n_embd=K)
    R.forget_head(w)
    rc, d = R.describe("logits_gemm_e4m3", ops)
    assert rc == R.RAD_E_UNSUPPORTED and "not host-readable" in d, d
    assert R.launch_row("logits_gemm_e4m3", ops, torch.cuda.current_stream().cuda_stream) == R.RAD_OK
    torch.cuda.synchronize()
    rc, d = R.describe("logits_gemm_e4m3", ops)
    assert rc == R.RAD_OK and d.startswith("arm=logits"), d
    R.forget_head(w)


def test_logits_first_launch_under_capture_refused(gpu):
    """The first launch over a device head reads its header with a copy and a wait, which
    a graph capture cannot hold: under capture it is refused (RAD_E_UNSUPPORTED) and
    nothing is recorded; launched once first, the capture proceeds."""
    M, N, K = 1, 64, 256
    codes, sbits = LU.head(N, K, 10)
    w = torch.from_numpy(R.join_head(codes, sbits)).to(gpu)
    x = torch.zeros((M, K), dtype=torch.int16, device=gpu)
    y = torch.zeros((M, N), dtype=torch.float32, device=gpu)
    ops = R.LogitsOperands(x, w, y, n_vocab=N, n_embd=K)
    R.forget_head(w)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        g.capture_begin()
        rc = R.launch_row("logits_gemm_e4m3", ops, s.cuda_stream)
        g.capture_end()
    assert rc == R.RAD_E_UNSUPPORTED
    torch.cuda.synchronize()
    assert R.launch_row("logits_gemm_e4m3", ops, torch.cuda.current_stream().cuda_stream) == R.RAD_OK
    torch.cuda.synchronize()
    R.forget_head(w)


@pytest.mark.parametrize("N,K,sdt,br", [(300, 260, "bf16", 1), (257, 132, "f16", 128),
                                        (129, 512, "f32", 1)])
def test_logits_over_relayout_blob(gpu, N, K, sdt, br):
    """The row over the blob its own relayout hook wrote from the encoded planes, checked
    against the oracle."""
    M = 4
    codes, sbits = LU.head(N, K, N + K, sdt, br)
    enc = R.head_encoding(sdt, br)
    nb = R.layout_head(enc, ((N, K), "F8E4M3"), (sbits.shape, LU.SDT[sdt]))[2]
    blob = np.zeros(nb, np.uint8)
    assert R.relayout_head(enc, codes, (np.ascontiguousarray(sbits), LU.SDT[sdt]), blob) == R.RAD_OK
    rng = np.random.default_rng(N)
    x = synth.bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    w = torch.from_numpy(blob).to(gpu)
    xt = torch.from_numpy(x.view(np.int16)).to(gpu)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device=gpu)
    ops = R.LogitsOperands(xt, w, y, n_vocab=N, n_embd=K)
    assert R.launch_row("logits_gemm_e4m3", ops, torch.cuda.current_stream().cuda_stream) == R.RAD_OK
    torch.cuda.synchronize()
    R.forget_head(w)
    Y = y.cpu().numpy()
    ye, se = LU.exact(x, codes, sbits, sdt, br)
    nw = (K + 127) // 128
    assert np.all(np.abs(Y - ye) <= (nw + 4 * 66 + 1) * 2.0 ** -24 * se + 1e-30)
