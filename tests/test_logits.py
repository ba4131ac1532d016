"""logits_gemm_e4m3 on the CPU: the joined-planes blob (the library's join / split against
the layout rad_planes.h states, written out independently in tests/logits_util.py), every
gate of the row's plan (through r3d_gfx950_describe, which reads a host header and launches
nothing), and the oracle's logits restatement pinned against float64 sums, all 256 codes,
closed forms and invariants."""
import numpy as np
import pytest

import libr3d_amd as R
import oracle as O
from libr3d_amd import synth
from tests import logits_util as LU

ROW = "logits_gemm_e4m3"


# ------------------------------------------------------------------ the joined blob
@pytest.mark.parametrize("N,K,sdt,br", [(300, 208, "bf16", 1), (257, 128, "f16", 128),
                                        (5, 1040, "f32", 1), (1, 16, "bf16", 128)])
def test_join_layout_and_round_trip(N, K, sdt, br):
    rng = np.random.default_rng(N + K)
    codes = rng.integers(0, 256, (N, K), dtype=np.uint8)
    sshape = ((N + br - 1) // br, (K + 127) // 128)
    scale = (rng.standard_normal(sshape).astype(np.float32) if sdt == "f32"
             else rng.integers(0, 65536, sshape, dtype=np.uint16))
    blob = R.join_head(codes, scale, sdt, br)
    h = LU.header(N, K, sdt, br)
    assert blob.size == R.head_bytes(N, K, sdt, br) == h[24:32].view(np.int64)[0]
    assert np.array_equal(blob[:LU.HEADER_BYTES], h)           # the header, byte for byte
    c_off, s_off = LU.up256(LU.HEADER_BYTES), LU.up256(LU.up256(LU.HEADER_BYTES) + N * K)
    assert np.array_equal(blob[c_off:c_off + N * K].reshape(N, K), codes)
    assert np.array_equal(blob[s_off:].view(scale.dtype).reshape(sshape), scale)
    c2, s2 = R.split_head(blob, N, K, sdt, br)
    assert np.array_equal(c2, codes) and np.array_equal(s2, scale)


def test_join_refusals():
    L = R.lib()
    assert R.head_bytes(10, 128, "bf16", 2) == -R.RAD_E_SHAPE            # br 1 or 128
    assert R.head_bytes(0, 128) == -R.RAD_E_SHAPE
    assert L.r3d_gfx950_logits_head_bytes(10, 128, R.DT["U8"], 1) == -R.RAD_E_DTYPE
    codes = np.zeros((4, 128), np.uint8)
    scale = np.zeros((4, 1), np.uint16)
    dst = np.zeros(R.head_bytes(4, 128) - 1, np.uint8)
    assert L.r3d_gfx950_logits_head_join(codes.ctypes.data, 128, scale.ctypes.data, 2, 4, 128,
                                         R.DT["BF16"], 1, dst.ctypes.data,
                                         dst.size) == R.RAD_E_SHAPE        # dst too small
    bad = R.join_head(codes, scale)
    bad[0] ^= 1                                                           # magic
    assert L.r3d_gfx950_logits_head_split(bad.ctypes.data, bad.size, None, None) == R.RAD_E_DTYPE


# ------------------------------------------------------------------ the plan's gates
class HostT:
    """A host buffer standing in for a device tensor (describe never launches)."""

    def __init__(self, arr, offset=0):
        self.arr, self.offset = arr, offset
        self.shape, self.dtype = arr.shape, arr.dtype

    def data_ptr(self):
        return self.arr.ctypes.data + self.offset

    def numel(self):
        return int(np.prod(self.shape))

    def stride(self):
        return tuple(s // self.arr.itemsize for s in self.arr.strides)


def _aligned(shape, dtype):
    n = int(np.prod(shape)) * np.dtype(dtype).itemsize
    raw = np.zeros(n + 256, np.uint8)
    off = (-raw.ctypes.data) % 256
    return raw[off:off + n].view(dtype).reshape(shape)


def _ops(M=4, N=1000, K=5376, sdt="bf16", br=1, h=None, xdt="BF16", ydt="F32", shapes=None,
         strides=None):
    x = HostT(_aligned((M, K), np.uint16))
    blob = h if h is not None else LU.header(N, K, sdt, br)
    w = HostT(_aligned(blob.shape, np.uint8))
    w.arr[:] = blob
    y = HostT(_aligned((M, N), np.float32))
    ops = R.LogitsOperands(x, w, y, n_vocab=N, n_embd=K, shapes=shapes, strides=strides)
    ops._t[0].dtype, ops._t[2].dtype = R.DT[xdt], R.DT[ydt]
    return ops, (x, w, y)


def _desc(ops):
    rc, d = R.describe(ROW, ops)
    return rc, dict(kv.split("=") for kv in d.split() if "=" in kv) if rc == 0 else d


def test_plan_geometry():
    ops, keep = _ops(M=4, N=262144, K=5376)
    rc, g = _desc(ops)
    assert rc == R.RAD_OK, g
    # 5376 = 42 scale blocks = 21 windows of 256 (a multiple of the 3-window ring); one
    # staged row 21 * 512 + 16 bytes; 8 waves' scale tables of 16 rows x 42 blocks in f32
    xrow = 21 * 512 + 16
    assert g["nwin"] == "42" and g["mt"] == "4" and g["wg_waves"] == "8" and g["depth"] == "2"
    assert g["lds"] == str(4 * xrow + 8 * 16 * 42 * 4) and g["chunks"] == str(262144 // 16)
    assert g["passes"] == "1" and g["blocks"] == "256"          # describe assumes 1 per CU
    ops, keep = _ops(M=1, N=1000, K=5376)
    rc, g = _desc(ops)
    assert rc == R.RAD_OK and g["wg_waves"] == "8" and g["depth"] == "2" and g["mt"] == "1"
    assert g["lds"] == str(xrow + 8 * 16 * 42 * 4)
    ops, keep = _ops(M=16, N=1000, K=5376)
    rc, g = _desc(ops)          # at most 8 rows a pass; 5..8 rows keep one window in flight
    assert rc == R.RAD_OK and g["mt"] == "8" and g["passes"] == "2" and g["depth"] == "1"
    ops, keep = _ops(M=6, N=1000, K=5376)
    rc, g = _desc(ops)
    assert rc == R.RAD_OK and g["mt"] == "6" and g["passes"] == "1" and g["depth"] == "1"
    ops, keep = _ops(M=40, N=1000, K=256)
    rc, g = _desc(ops)
    assert rc == R.RAD_OK and g["mt"] == "8" and g["passes"] == "5" and g["depth"] == "1"
    ops, keep = _ops(M=3, N=50, K=144, sdt="f32", br=128)
    rc, g = _desc(ops)
    assert rc == R.RAD_OK and g["nwin"] == "2" and g["sdt"] == "2" and g["br"] == "128"
    ops, keep = _ops(M=1, N=50, K=16)                 # below the row's n_embd GE 128: the
    assert _desc(ops)[0] == R.RAD_OK                  # constraint is the resolver's, not a gate


def _hdr(N=1000, K=5376, sdt="bf16", br=1, **fields):
    h = LU.header(N, K, sdt, br)
    for key, v in fields.items():
        name, _, ent = key.partition("__")
        LU.set_field(h, name, v, None if not ent else int(ent))
    return h


@pytest.mark.parametrize("case,rc", [
    (dict(ydt="BF16"), R.RAD_E_UNSUPPORTED),                    # logits are f32
    (dict(xdt="F32"), R.RAD_E_UNSUPPORTED),                     # x is bf16
    (dict(K=130, h=LU.header(1000, 130)), R.RAD_E_UNSUPPORTED),  # K % 4 (reference gate)
    (dict(h=_hdr(magic=0)), R.RAD_E_DTYPE),                      # no header
    (dict(h=_hdr(n_planes=3)), R.RAD_E_DTYPE),
    (dict(h=_hdr(n_planes=0)), R.RAD_E_DTYPE),
    (dict(h=_hdr(transform0=1)), R.RAD_E_UNSUPPORTED),
    (dict(h=_hdr(role__1="zero")), R.RAD_E_DTYPE),
    (dict(h=_hdr(dtype__0=4)), R.RAD_E_SHAPE),                   # e5m2 codes
    (dict(h=_hdr(rows__0=999)), R.RAD_E_SHAPE),
    (dict(h=_hdr(block1__0=2)), R.RAD_E_SHAPE),
    (dict(h=_hdr(dtype__1=7)), R.RAD_E_UNSUPPORTED),             # u8 scales
    (dict(h=_hdr(block1__1=64)), R.RAD_E_UNSUPPORTED),
    (dict(h=_hdr(block0__1=2)), R.RAD_E_UNSUPPORTED),
    (dict(h=_hdr(rows__1=999)), R.RAD_E_SHAPE),
    (dict(h=_hdr(cols__1=41)), R.RAD_E_SHAPE),
    (dict(h=_hdr(row_bytes__0=5392)), R.RAD_E_STRIDE),           # codes dense
    (dict(h=_hdr(bytes=1024)), R.RAD_E_SHAPE),                   # scale past the blob
    (dict(h=_hdr(row_bytes__1=82)), R.RAD_E_STRIDE),             # scale rows shorter than 42
    (dict(h=_hdr(offset__0=200000)), R.RAD_E_SHAPE),             # codes past the blob
    (dict(M=1, N=4, K=80000, h=LU.header(4, 80000)), R.RAD_E_UNSUPPORTED),  # a row past LDS
])
def test_plan_refusals(case, rc):
    ops, keep = _ops(**case)
    assert _desc(ops)[0] == rc, (case, _desc(ops))


@pytest.mark.parametrize("case", [
    dict(K=132, N=10, h=LU.header(10, 132)),                     # K % 16: the dword walk
    dict(K=260, N=10, h=LU.header(10, 260), sdt="f16"),
    dict(h=_hdr(offset__0=520)),                                 # codes off 16-byte alignment
    dict(h=_hdr(offset__0=513)),                                 # codes on an odd byte
    dict(N=10, K=256, h=_hdr(N=10, K=256, offset__1=4097, bytes=4097 + 40)),  # scale off 2 B
])
def test_plan_takes_any_alignment(case):
    """Every operand the reference's entry accepts (n_embd a multiple of 4, any alignment,
    src/r3d_gemm_logits.hip:166) is taken: off a multiple of 16 or off alignment, on the
    slower dword walk; aligned multiples of 16 stay on the vector walk."""
    ops, keep = _ops(**case)
    rc, g = _desc(ops)
    assert rc == R.RAD_OK and g["walk"] == "dword", (case, g)
    ops, keep = _ops(M=2, N=10, K=256, h=LU.header(10, 256))
    rc, g = _desc(ops)
    assert rc == R.RAD_OK and g["walk"] == "vector"


def test_reference_style_blob_accepted():
    """A blob written the way the reference's tools write one (tools/bench_skinny.cpp:
    206-220: zeroed, header fields magic / n_planes / transform[0] / bytes, the entries
    right after the header with kind = RAD_PLANE_TILED, planes at rad_planes_round offsets)
    is what the library's join writes, byte for byte, and what its plan accepts."""
    N, K = 300, 256
    h = LU.header(N, K)
    assert h[8:24].view(np.uint32).tolist() == [0, 0, 0, 0]       # transform[], zero
    hb, c_off, s_off, nb = R.head_header(N, K)
    assert np.array_equal(hb, h) and c_off == 256 and s_off == LU.up256(256 + N * K)
    ops, keep = _ops(M=1, N=N, K=K, h=h)
    assert _desc(ops)[0] == R.RAD_OK


# ------------------------------------------------------------------ the layout hooks
def _planes(N, K, sdt, br, rng):
    codes = rng.integers(0, 256, (N, K), dtype=np.uint8)
    sshape = ((N + br - 1) // br, (K + 127) // 128)
    scale = (rng.standard_normal(sshape).astype(np.float32) if sdt == "f32"
             else rng.integers(0, 65536, sshape, dtype=np.uint16))
    return codes, (scale, LU.SDT[sdt])


@pytest.mark.parametrize("N,K,sdt,br", [(300, 208, "bf16", 1), (257, 132, "f16", 128),
                                        (5, 1040, "f32", 1), (129, 128, "bf16", 128)])
def test_hooks_accept_and_round_trip(N, K, sdt, br):
    """The hooks admit the joined e4m3 head: layout answers the canonical rad.planes join and
    its size, relayout writes exactly the bytes the library's join writes, unrelayout reads
    the planes back, and the plan accepts the blob."""
    rng = np.random.default_rng(N * K)
    codes, (scale, sname) = _planes(N, K, sdt, br, rng)
    enc = R.head_encoding(sdt, br)
    geo = ((N, K), "F8E4M3"), (scale.shape, sname)                 # declare time: no data
    rc, tag, nb = R.layout_head(enc, *geo, params=[("n_vocab", N), ("n_embd", K)])
    assert rc == R.RAD_OK and tag == "rad.planes" and nb == R.head_bytes(N, K, sdt, br)
    assert R.relayout_head(enc, *geo, np.zeros(nb, np.uint8)) == R.RAD_E_INVAL   # no data yet
    dst = np.full(nb, 0xAB, np.uint8)
    assert R.relayout_head(enc, codes, (scale, sname), dst) == R.RAD_OK
    assert np.array_equal(dst, R.join_head(codes, scale, sdt, br))
    assert R.relayout_head(enc, codes, (scale, sname), np.zeros(nb - 1, np.uint8)) == R.RAD_E_SHAPE
    c2, s2 = np.zeros_like(codes), np.zeros_like(scale)
    assert R.unrelayout_head(enc, dst, c2, (s2, sname)) == R.RAD_OK
    assert np.array_equal(c2, codes) and np.array_equal(s2, scale)
    bad = dst.copy()
    bad[:4] = 0                                                    # no magic
    assert R.unrelayout_head(enc, bad, c2, (s2, sname)) == R.RAD_E_DTYPE
    ops, keep = _ops(M=1, N=N, K=K, sdt=sdt, br=br, h=dst[:LU.HEADER_BYTES].copy())
    assert _desc(ops)[0] == R.RAD_OK


def _declines():
    N, K = 64, 256
    base = dict(sdt="bf16", br=1, N=N, K=K)
    return [
        (dict(base, enc=dict(scheme="none")), R.RAD_E_DTYPE),
        (dict(base, enc=dict(transform0=1)), R.RAD_E_DTYPE),       # rotated ("givens")
        (dict(base, enc=dict(roles=("scale", "codes"))), R.RAD_E_DTYPE),
        (dict(base, enc=dict(roles=("codes", "zero"))), R.RAD_E_DTYPE),
        (dict(base, enc=dict(code_dtype="F8E5M2")), R.RAD_E_DTYPE),
        (dict(base, enc=dict(code_dtype="I8")), R.RAD_E_DTYPE),    # int8 heads: the host's
        (dict(base, enc=dict(code_block=(1, 2))), R.RAD_E_DTYPE),
        (dict(base, enc=dict(kinds=(1, 0))), R.RAD_E_DTYPE),       # codes not tiled
        (dict(base, enc=dict(kinds=(0, 1))), R.RAD_E_DTYPE),
        (dict(base, enc=dict(n_planes=3)), R.RAD_E_DTYPE),
        (dict(base, sdt="U8"), R.RAD_E_DTYPE),                      # u8 scales
        (dict(base, br=2), R.RAD_E_DTYPE),                          # scale block 2 x 128
        (dict(base, sel=(0, 2)), R.RAD_E_DTYPE),                    # selection past n_planes
        (dict(base, K=130), R.RAD_E_DTYPE),                         # n_embd % 4
        (dict(base, K=80000, N=4), R.RAD_E_DTYPE),                  # a row past the LDS
        (dict(base, srows=63), R.RAD_E_SHAPE),                      # grids disagree
        (dict(base, params=[("n_vocab", 65)]), R.RAD_E_SHAPE),
        (dict(base, operand=0), R.RAD_E_UNSUPPORTED),               # x: stored as it is
        (dict(base, operand=2), R.RAD_E_UNSUPPORTED),
    ]


@pytest.mark.parametrize("case,rc", _declines())
def test_hooks_decline(case, rc):
    """What the reference's hook declines (src/r3d_gemm_logits.hip:233-253), and what this
    row's launch would refuse, declined at declare time instead of refused at issue."""
    N, K, sdt, br = case["N"], case["K"], case["sdt"], case["br"]
    sname = LU.SDT.get(sdt, sdt)
    enc = R.head_encoding(sname if sdt not in LU.SDT else sdt, br, **case.get("enc", {}))
    srows = case.get("srows", (N + max(br, 1) - 1) // max(br, 1))
    geo = ((N, K), "F8E4M3"), ((srows, (K + 127) // 128), sname)
    got = R.layout_head(enc, *geo, operand=case.get("operand", 1), sel=case.get("sel", (0, 1)),
                        params=case.get("params", ()))[0]
    assert got == rc, (case, got)


def test_hooks_decline_a_plain_head():
    """A head without the two-plane encoding (a plain bf16 lm_head: no encoding, or one
    plane) is declined (RAD_E_DTYPE), so it resolves past this row -- the library has no
    bf16 head row declared ahead of it to claim such heads, as the reference's
    logits_gemm_bf16 does (src/r3d_rows.cpp:1570-1585)."""
    import ctypes
    L = R.lib()
    t = (R.RadTensor * 2)()
    t[0].dtype, t[0].rank, t[0].shape[0], t[0].shape[1] = R.DT["BF16"], 2, 64, 256
    out = R.RadLayout()
    assert L.r3d_layout_head(None, 0, 1, None, None, t, 1, ctypes.byref(out)) == R.RAD_E_DTYPE
    enc = R.head_encoding()
    sel = (ctypes.c_int * 2)(0, 1)
    assert L.r3d_layout_head(None, 0, 1, ctypes.byref(enc), sel, t, 1,
                             ctypes.byref(out)) == R.RAD_E_DTYPE


def test_row_registers_the_hooks():
    row = {r["name"]: r for r in R.rows()}["logits_gemm_e4m3"]
    assert row["layout"] and row["relayout"] and row["unrelayout"] and not row["opd_shape"]
    for r in R.rows():                                # no other row declares weight hooks
        if r["name"] != "logits_gemm_e4m3":
            assert not (r["layout"] or r["relayout"] or r["unrelayout"]), r["name"]


def test_plan_shape_and_stride_refusals():
    # numel(logits) not a multiple of n_vocab
    ops, keep = _ops(N=1000, shapes={2: [4, 999]}, strides={2: [999, 1]})
    assert _desc(ops)[0] == R.RAD_E_SHAPE
    # x smaller than M x K
    ops, keep = _ops(shapes={0: [3, 5376]}, strides={0: [5376, 1]})
    assert _desc(ops)[0] == R.RAD_E_SHAPE
    # a last-dimension stride other than 1; a row pitch shorter than the row
    ops, keep = _ops(strides={2: [1000, 2]})
    assert _desc(ops)[0] == R.RAD_E_STRIDE
    ops, keep = _ops(strides={0: [5000, 1]})
    assert _desc(ops)[0] == R.RAD_E_STRIDE
    # x rows 8-element aligned with a longer pitch take the vector walk; a 16-byte
    # misaligned x pitch the dword walk
    ops, keep = _ops(M=2, K=256, N=10, h=LU.header(10, 256), shapes={0: [2, 256]},
                     strides={0: [264, 1]})
    rc, g = _desc(ops)
    assert rc == R.RAD_OK and g["walk"] == "vector"
    ops, keep = _ops(M=2, K=256, N=10, h=LU.header(10, 256), shapes={0: [2, 256]},
                     strides={0: [260, 1]})
    rc, g = _desc(ops)
    assert rc == R.RAD_OK and g["walk"] == "dword"
    # M comes from numel(logits) / n_vocab, not the M parameter
    x = HostT(_aligned((6, 256), np.uint16))
    w = HostT(_aligned((LU.HEADER_BYTES,), np.uint8))
    w.arr[:] = LU.header(10, 256)
    y = HostT(_aligned((6, 10), np.float32))
    ops = R.LogitsOperands(x, w, y, n_vocab=10, n_embd=256, M=1)
    rc, g = _desc(ops)
    assert rc == R.RAD_OK and g["M"] == "6"


def test_launch_refuses_without_gfx950():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    ops, keep = _ops(M=1, N=10, K=256, h=LU.header(10, 256))
    assert R.launch_row(ROW, ops, 0) == R.RAD_E_UNSUPPORTED


# ------------------------------------------------------------------ the oracle, pinned
def test_f16_decode_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    got = O.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("sdt,br", [("bf16", 1), ("f16", 128), ("f32", 1), ("bf16", 128)])
def test_oracle_against_float64(sdt, br):
    """Bound: the oracle's f32 chain is within K * 2^-24 of the magnitude sum of the exact
    float64 value; the scales swing over 2^-8 .. 2^8 across blocks and rows, so a scale
    taken from the wrong block or row misses by far more."""
    rng = np.random.default_rng(7)
    M, N, K = 3, 260, 400
    codes, _ = LU.head(N, K, 3, sdt, br)
    sshape = ((N + br - 1) // br, (K + 127) // 128)
    sv = np.ldexp(1.0, rng.integers(-8, 9, sshape)) * rng.uniform(1, 2, sshape)
    sbits = (synth.bf16_bits(sv.astype(np.float32)) if sdt == "bf16" else
             sv.astype(np.float16).view(np.uint16) if sdt == "f16" else sv.astype(np.float32))
    x = synth.bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    Y, S = O.logits_e4m3(x, codes, sbits, sdt, br)
    ye, se = LU.exact(x, codes, sbits, sdt, br)
    assert np.all(np.abs(Y - ye) <= (K + 1) * 2.0 ** -24 * se + 1e-30)
    assert np.allclose(S, se, rtol=K * 2.0 ** -23)
    # the same scales transposed within each row block would not pass
    if sshape[0] >= 3 and sshape[1] >= 3:
        bad = sbits.copy()
        bad[:, [0, 1]] = bad[:, [1, 0]]
        yb, _ = LU.exact(x, codes, bad, sdt, br)
        assert np.any(np.abs(Y - yb) > (K + 1) * 2.0 ** -24 * se)


@pytest.mark.parametrize("sdt", ["bf16", "f16", "f32"])
def test_oracle_every_code_one_hot(sdt):
    """Row n carries code n at column 5 and zeros elsewhere, x is one-hot at column 5: the
    single product is exact, so y[n] = f32(e4m3(n) * s) -- against torch's float8_e4m3fn
    decode (a library, not this oracle), NaN codes poisoning their row."""
    N, K = 256, 256
    codes = np.zeros((N, K), np.uint8)
    codes[:, 5] = np.arange(256)
    s = np.float32(1.3125)
    sbits = {"bf16": synth.bf16_bits(np.full((N, 2), s, np.float32)),
             "f16": np.full((N, 2), s, np.float16).view(np.uint16),
             "f32": np.full((N, 2), s, np.float32)}[sdt]
    x = np.zeros((2, K), np.uint16)
    x[0, 5] = synth.bf16_bits(np.array([1.0], np.float32))[0]
    x[1, 5] = synth.bf16_bits(np.array([-0.25], np.float32))[0]
    Y, _ = O.logits_e4m3(x, codes, sbits, sdt, 1)
    dec = LU.e4m3_values(np.arange(256, dtype=np.uint8))
    ref = np.stack([(dec * s).astype(np.float32), (dec * s * np.float32(-0.25)).astype(np.float32)])
    ref = ref + np.float32(0.0)           # the accumulator starts at +0: -0 + +0 = +0
    nan = np.isnan(ref)
    assert nan.sum() == 4 and np.array_equal(np.isnan(Y), nan)
    assert np.array_equal(Y[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_oracle_row_block_scale_equals_expanded_grid():
    """br = 128 is the per-row grid with each scale repeated over its 128 rows, bit for bit;
    permuting head rows (with their per-row scales) permutes the logits, bit for bit."""
    rng = np.random.default_rng(11)
    M, N, K = 2, 300, 256
    codes, sb = LU.head(N, K, 5, "bf16", 128)
    x = synth.bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    Y128, _ = O.logits_e4m3(x, codes, sb, "bf16", 128)
    Y1, _ = O.logits_e4m3(x, codes, np.repeat(sb, 128, axis=0)[:N], "bf16", 1)
    assert np.array_equal(Y128.view(np.uint32), Y1.view(np.uint32))
    perm = rng.permutation(N)
    Yp, _ = O.logits_e4m3(x, codes[perm], np.repeat(sb, 128, axis=0)[:N][perm], "bf16", 1)
    assert np.array_equal(Yp.view(np.uint32), Y1[:, perm].view(np.uint32))
