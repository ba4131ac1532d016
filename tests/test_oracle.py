"""Pins the CPU oracle (oracle/r3d_oracle.c) against independent references: torch's
float8/bfloat16 codecs (a library, not the reference), closed forms, float64 brute force,
and invariants that a dropped term, a wrong index or a transposed operand would break.
No reference-held vectors exist for this path (the kbench packs are off-repo), so these
checks are what pins it."""
import math

import numpy as np
import pytest
import torch

import oracle as O
from libr3d_amd import synth


def _f32(bits):
    return np.array(bits, np.uint32).view(np.float32)


# ------------------------------------------------------------------ codecs
def test_e4m3_decode_exhaustive_vs_torch():
    codes = np.arange(256, dtype=np.uint8)
    got = O.e4m3_to_f32(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert nan.sum() == 2 and nan[0x7F] and nan[0xFF]           # S1111111 only
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))  # incl. -0
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9


def test_e2m1_decode_closed_form():
    for n in range(16):
        e, m, s = (n >> 1) & 3, n & 1, -1.0 if n & 8 else 1.0
        want = s * (m * 0.5 if e == 0 else (1 + m / 2) * 2.0 ** (e - 1))
        assert O.e2m1_to_f32([n])[0] == want, n


def test_e8m0_decode_all_bytes():
    x = np.arange(256, dtype=np.uint8)
    got = O.e8m0_to_f32(x)
    assert np.isnan(got[255]) and not np.isnan(got[:255]).any()
    for v in range(255):
        assert got[v] == np.float32(math.ldexp(1.0, v - 127)), v
    assert got[0] == np.float32(2.0 ** -127) and got[0] > 0      # f32 subnormal kept
    if hasattr(torch, "float8_e8m0fnu"):
        ref = torch.from_numpy(x).view(torch.float8_e8m0fnu).to(torch.float32).numpy()
        assert np.array_equal(np.isnan(ref), np.isnan(got))
        fin = ~np.isnan(ref)
        assert np.array_equal(ref[fin], got[fin])


def _e4m3_table():
    codes = np.arange(0x7F, dtype=np.uint8)                      # +0 .. 448
    return codes, O.e4m3_to_f32(codes).astype(np.float64)


def _nearest_even_code(x):
    """Independent encoder: nearest value in the decoded positive table, ties to the even
    code, saturating at 448, sign applied by the sign bit."""
    codes, vals = _e4m3_table()
    s = 0x80 if math.copysign(1.0, x) < 0 else 0
    a = abs(x)
    if a >= 448.0:
        return s | 0x7E
    i = int(np.searchsorted(vals, a))
    if i < len(vals) and vals[i] == a:
        return s | int(codes[i])
    lo, hi = i - 1, i
    dlo, dhi = a - vals[lo], vals[hi] - a
    if dlo < dhi:
        return s | int(codes[lo])
    if dhi < dlo:
        return s | int(codes[hi])
    return s | int(codes[lo] if codes[lo] % 2 == 0 else codes[hi])


def test_e4m3_encode_ties_and_midpoints():
    codes, vals = _e4m3_table()
    pts = [0.0, -0.0, 2.0 ** -12, 2.0 ** -11, 2.0 ** -10, 2.0 ** -10 * 1.0000001, 447.9, 448.0,
           460.0, 464.0, 1e6, -1e6]
    mids = list((vals[1:] + vals[:-1]) / 2)
    near = []
    for m in mids:
        f = np.float32(m)
        near += [float(np.nextafter(f, np.float32(0))), float(f), float(np.nextafter(f, np.float32(1e9)))]
    xs = np.array(pts + mids + near + [-v for v in mids + near], np.float32)
    got = O.f32_to_e4m3(xs)
    want = np.array([_nearest_even_code(float(x)) for x in xs], np.uint8)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(xs[i]), hex(got[i]), hex(want[i])) for i in bad[:8]]


def test_e4m3_encode_vs_torch_in_range():
    rng = np.random.default_rng(5)
    exps = rng.integers(-14, 9, size=400000)
    x = (rng.random(400000) + 1.0) * np.exp2(exps.astype(np.float64))
    x = (x * rng.choice([-1.0, 1.0], size=x.size)).astype(np.float32)
    x = np.clip(x, -448.0, 448.0).astype(np.float32)
    got = O.f32_to_e4m3(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    mism = np.nonzero(got != ref)[0]
    assert mism.size == 0, [(float(x[i]), hex(got[i]), hex(ref[i])) for i in mism[:8]]


def test_e4m3_encode_saturation_and_nan():
    got = O.f32_to_e4m3(np.array([448.0, 449.0, 1e30, np.inf, -np.inf, -500.0, np.nan, -np.nan],
                                 np.float32))
    assert list(got[:6]) == [0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE]
    assert (got[6] & 0x7F) == 0x7F and (got[7] & 0x7F) == 0x7F


def test_bf16_rne_vs_torch():
    rng = np.random.default_rng(6)
    bits = rng.integers(0, 2 ** 32, size=300000, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x3F808000, 0x3F818000,
                        0x7F7FFFFF, 0x00000001, 0x00008000, 0x00018000], np.uint32)
    bits = np.concatenate([bits, special])
    x = bits.view(np.float32)
    got = O.f32_to_bf16(x)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert (((got[nan] & 0x7F80) == 0x7F80) & ((got[nan] & 0x7F) != 0)).all()   # NaN class


def test_grid_block_closed_forms():
    for K in (128, 640, 4096, 5376, 21504):
        assert O.grid_block(K, K // 32) == 32
        assert O.grid_block(K, K // 128) == 128
        assert O.grid_block(K, 1) == K
    assert O.grid_block(100, 4) == 32     # ceil(100/32) == 4: the power of two wins
    assert O.grid_block(96, 4) == 24      # no power of two gives 4 blocks of 96


# ------------------------------------------------------------------ quant_act_fp8
def test_quant_act_fp8_invariants():
    rng = np.random.default_rng(7)
    x = synth.bf16_bits(rng.standard_normal((6, 700)).astype(np.float32) * 3)
    x[2, 128:256] = 0                                      # an all-zero group
    x[3, 5] = 0x7FC0                                       # a NaN input
    q, sc = O.quant_act_fp8(x, 128)
    xf = synth.bits_to_f32(x)
    assert sc.shape == (6, 6)
    assert sc[2, 1] == 1.0 and (q[2, 128:256] == 0).all()
    assert (q[3, 5] & 0x7F) == 0x7F
    for m in range(6):
        for g in range(6):
            seg = xf[m, g * 128:(g + 1) * 128]
            fin = seg[~np.isnan(seg)]
            amax = np.max(np.abs(fin)) if fin.size else 0
            if amax == 0:
                continue
            assert sc[m, g] == np.float32(np.float32(amax) * np.float32(1.0 / 448.0))
            codes = q[m, g * 128:(g + 1) * 128]
            i = int(np.argmax(np.where(np.isnan(seg), -1, np.abs(seg))))
            assert (codes[i] & 0x7F) == 0x7E                # the amax element encodes to 448
            dq = O.e4m3_to_f32(codes).astype(np.float64) * sc[m, g]
            ok = ~np.isnan(seg)
            rel = np.abs(dq[ok] - seg[ok]) / np.maximum(np.abs(seg[ok]), 1e-30)
            tiny = np.abs(seg[ok]) < sc[m, g] * 2.0 ** -6      # subnormal range: abs bound
            assert (rel[~tiny] <= 2.0 ** -4 + 1e-6).all()
            assert (np.abs(dq[ok] - seg[ok])[tiny] <= sc[m, g] * 2.0 ** -10 + 1e-30).all()


def test_quant_act_fp8_matches_numpy_float32_steps():
    """The reference's step order (src/r3d_band.hip:117-153) evaluated with numpy float32
    arithmetic and torch's RNE encoder (in range after the clamp)."""
    rng = np.random.default_rng(8)
    x = synth.bf16_bits((rng.standard_normal((5, 384)) * 10).astype(np.float32))
    q, sc = O.quant_act_fp8(x, 128)
    q2, sc2 = synth.quant_act_groups(x, 128)
    assert np.array_equal(sc, sc2)
    assert np.array_equal(q, q2)


# ------------------------------------------------------------------ gated_quant_fp8
def _same_nan_class(a, b):
    na, nb = (a & 0x7F80) == 0x7F80, (b & 0x7F80) == 0x7F80   # bf16 Inf/NaN exponent
    nan_a, nan_b = na & ((a & 0x7F) != 0), nb & ((b & 0x7F) != 0)
    assert np.array_equal(nan_a, nan_b)
    assert np.array_equal(a[~nan_a], b[~nan_b])


def test_gated_quant_fp8_closed_forms():
    """sigmoid(0) = 1/2 exactly, so act=sigmoid with a zero gate gives h = up/2; a gate of
    30 has sigmoid 1 in f32 (exp(-30) is below half an ulp of 1), so silu gives
    h = bf16(30 * up).  Both must equal quant_act_fp8 of that h, with gate/up taken from
    the right halves."""
    rng = np.random.default_rng(77)
    M, n = 3, 512
    up = synth.bf16_bits((rng.standard_normal((M, n)) * 2).astype(np.float32))
    upf = O.bf16_to_f32(up)
    gu = np.concatenate([np.zeros((M, n), np.uint16), up], axis=1)
    q, s, o = O.gated_quant_fp8(gu, group=128, act="sigmoid")
    half = synth.bf16_bits(upf * np.float32(0.5))
    assert np.array_equal(o, half)
    qr, sr = O.quant_act_fp8(half, 128)
    assert np.array_equal(q, qr) and np.array_equal(s.view(np.uint32), sr.view(np.uint32))
    # silu with a zero gate is exactly zero: every group all-zero, scale 1, code 0
    q, s, o = O.gated_quant_fp8(gu, group=128, act="silu")
    assert not o.any() or set(np.unique(o & 0x7FFF)) == {0}
    assert (s == 1.0).all() and not (q & 0x7F).any()
    g30 = synth.bf16_bits(np.full((M, n), 30.0, np.float32))
    q, s, o = O.gated_quant_fp8(np.concatenate([g30, up], axis=1), group=64, act="silu")
    h = synth.bf16_bits(np.float32(30.0) * upf)
    assert np.array_equal(o, h)
    qr, sr = O.quant_act_fp8(h, 64)
    assert np.array_equal(q, qr) and np.array_equal(s, sr)
    # swapped halves (gate = up values, up = 30) differ: the order is pinned
    q2, _, o2 = O.gated_quant_fp8(np.concatenate([up, g30], axis=1), group=64, act="silu")
    assert not np.array_equal(o2, o)


@pytest.mark.parametrize("act", ["silu", "sigmoid"])
@pytest.mark.parametrize("f32_in", [False, True])
def test_gated_quant_fp8_numpy_eval(act, f32_in):
    """numpy evaluation of the gated step (exp in float64, narrowed to float32, then float32
    arithmetic and torch's RNE bf16), on random gates and the special ones (+-0, +-30,
    +-88, +-100, +-inf, NaN), then quant_act_fp8 on the result."""
    rng = np.random.default_rng(91 if f32_in else 90)
    M, n = 4, 384
    gt = (rng.standard_normal((M, n)) * 4).astype(np.float32)
    sp = np.array([0.0, -0.0, 30, -30, 88, -88, 100, -100, np.inf, -np.inf, np.nan],
                  np.float32)
    gt[0, :sp.size] = sp
    upf = (rng.standard_normal((M, n)) * 3).astype(np.float32)
    if f32_in:
        gu = np.concatenate([gt, upf], axis=1)
        gtf, uf = gt, upf
    else:
        gu = synth.bf16_bits(np.concatenate([gt, upf], axis=1))
        gtf, uf = O.bf16_to_f32(gu[:, :n]), O.bf16_to_f32(gu[:, n:])
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(-gtf.astype(np.float64)).astype(np.float32)
        sg = np.float32(1.0) / (np.float32(1.0) + e)
        t = gtf * sg if act == "silu" else sg
        h = synth.bf16_bits((t * uf).astype(np.float32))
    q, s, o = O.gated_quant_fp8(gu, group=128, act=act)
    _same_nan_class(o, h)
    qr, sr = O.quant_act_fp8(o, 128)
    assert np.array_equal(q, qr) and np.array_equal(s.view(np.uint32), sr.view(np.uint32))


# ------------------------------------------------------------------ rmsnorm_quant_fp8
@pytest.mark.parametrize("w_bf16", [False, True])
@pytest.mark.parametrize("n", [5376, 300, 30720])
def test_rmsnorm_quant_fp8_exact_sums(n, w_bf16):
    """Integer-valued rows in [-8, 8]: every square and partial sum is exact in f32, so the
    sum (hence rs) is the same in any order; the oracle must then equal a numpy float32
    evaluation of rs = 1/sqrt(ss/n + eps), h = bf16((x * rs) * (w + wadd)), and the
    quantiser over h."""
    rng = np.random.default_rng(n + w_bf16)
    M = 3
    xf = rng.integers(-8, 9, size=(M, n)).astype(np.float32)
    x = synth.bf16_bits(xf)
    wf = (1.0 + 0.25 * rng.standard_normal(n)).astype(np.float32)
    w = synth.bf16_bits(wf) if w_bf16 else wf
    wv = (O.bf16_to_f32(w) if w_bf16 else wf).astype(np.float32)
    eps, wadd = np.float32(1e-6), np.float32(0.5)
    q, s, out, _ = O.rmsnorm_quant_fp8(x, w, group=128, eps=float(eps), wadd=float(wadd))
    ss = (xf.astype(np.float64) ** 2).sum(axis=1).astype(np.float32)   # exact
    rs = np.float32(1.0) / np.sqrt(ss / np.float32(n) + eps, dtype=np.float32)
    h = synth.bf16_bits((xf * rs[:, None]).astype(np.float32) * (wv + wadd))
    assert np.array_equal(out, h)
    qr, sr = O.quant_act_fp8(h, 128)
    assert np.array_equal(q, qr) and np.array_equal(s, sr)


def test_rmsnorm_quant_fp8_residual_and_closed_form():
    rng = np.random.default_rng(4)
    M, n = 2, 1024
    x = synth.bf16_bits(rng.standard_normal((M, n)).astype(np.float32))
    r0 = synth.bf16_bits(rng.standard_normal((M, n)).astype(np.float32))
    w = synth.bf16_bits(np.ones(n, np.float32))
    q, s, out, r1 = O.rmsnorm_quant_fp8(x, w, residual=r0)
    assert np.array_equal(r1, synth.bf16_bits(O.bf16_to_f32(r0) + O.bf16_to_f32(x)))
    q2, s2, out2, _ = O.rmsnorm_quant_fp8(r1, w)        # the plain form on the written sum
    assert np.array_equal(q, q2) and np.array_equal(s, s2) and np.array_equal(out, out2)
    # a constant row c = 2: ss = 4n exactly, rs = 1/sqrt(4 + eps) -> h = bf16(2 * rs)
    xc = synth.bf16_bits(np.full((1, n), 2.0, np.float32))
    _, _, oc, _ = O.rmsnorm_quant_fp8(xc, w, eps=0.0)
    assert (O.bf16_to_f32(oc) == 1.0).all()


# ------------------------------------------------------------------ quant_dot
def _mx(M, N, K, seed, lo=115, hi=139):
    rng = np.random.default_rng(seed)
    A = synth.random_e4m3_codes((M, K), rng)
    AS = (0.001 + 0.01 * rng.random((M, K // 128))).astype(np.float32)
    B = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    BS = rng.integers(lo, hi + 1, size=(N, K // 32)).astype(np.uint8)
    return A, AS, B, BS


def _exact_mx(A, AS, B, BS):
    a = O.e4m3_to_f32(A).astype(np.float64)
    w = O.mxfp4_dequant(B, BS).astype(np.float64)
    K = a.shape[1]
    sa = np.repeat(AS.astype(np.float64), 128, axis=1)[:, :K]
    return (a * sa) @ w.T


def test_quant_dot_mxfp4a8_f64_brute_force():
    A, AS, B, BS = _mx(5, 40, 384, 1)
    Y, Yf, S = O.quant_dot_mxfp4a8(A, AS, B, BS)
    ex = _exact_mx(A, AS, B, BS)
    # the oracle's own f32 error vs exact is within K * 2^-24 * S
    assert (np.abs(Yf - ex) <= 384 * 2.0 ** -24 * S.astype(np.float64) + 1e-30).all()
    assert np.array_equal(Y, O.f32_to_bf16(Yf))
    assert (S >= np.abs(ex) * (1 - 1e-6)).all()


def test_quant_dot_mxfp4a8_single_nonzero_closed_form():
    M, N, K = 2, 3, 256
    A = np.zeros((M, K), np.uint8)
    AS = np.full((M, K // 128), 0.5, np.float32)
    B = np.zeros((N, K // 2), np.uint8)
    BS = np.full((N, K // 32), 127, np.uint8)
    A[1, 201] = 0x44                       # e4m3 3.0 (e=8, m=4: 1.5 * 2)
    B[2, 100] = 0x50                       # k = 201 -> high nibble of byte 100: code 5 = 3.0
    BS[2, 201 // 32] = 130                 # 2^3
    AS[1, 201 // 128] = 0.25
    Y, Yf, _ = O.quant_dot_mxfp4a8(A, AS, B, BS)
    assert Yf[1, 2] == 3.0 * 3.0 * 0.25 * 8.0
    assert (np.delete(Yf.ravel(), 1 * N + 2) == 0).all()


def test_quant_dot_single_group_forms():
    """K = 32 (one weight block) and K = 128 (one activation group): the flush is one
    (sub * sa) * sb with sub the ascending f32 sum."""
    rng = np.random.default_rng(3)
    A, AS, B, BS = _mx(3, 4, 128, 2)
    Y, Yf, _ = O.quant_dot_mxfp4a8(A, AS, B, BS)
    a = O.e4m3_to_f32(A)
    w = O.mxfp4_dequant(B, np.full_like(BS, 127))
    for m in range(3):
        for n in range(4):
            acc = np.float32(0)
            for g in range(4):
                sub = np.float32(0)
                for k in range(32 * g, 32 * g + 32):
                    sub = np.float32(sub + np.float32(a[m, k] * w[n, k]))
                acc = np.float32(acc + np.float32(np.float32(sub * AS[m, 0]) *
                                                  np.float32(O.e8m0_to_f32([BS[n, g]])[0])))
            assert Yf[m, n] == acc


def test_quant_dot_power_of_two_scale_exactness():
    A, AS, B, BS = _mx(3, 16, 256, 4)
    _, Yf1, _ = O.quant_dot_mxfp4a8(A, AS, B, BS)
    _, Yf2, _ = O.quant_dot_mxfp4a8(A, AS * 4, B, BS)
    _, Yf3, _ = O.quant_dot_mxfp4a8(A, AS, B, (BS - 1).astype(np.uint8))
    assert np.array_equal(Yf2, Yf1 * 4)
    assert np.array_equal(Yf3, Yf1 / 2)


def test_quant_dot_nan_scale_poisons_even_zero_codes():
    A, AS, B, BS = _mx(2, 8, 128, 5)
    B[4, :16] = 0
    BS[4, 0] = 0xFF
    Y, Yf, _ = O.quant_dot_mxfp4a8(A, AS, B, BS)
    assert np.isnan(Yf[:, 4]).all()
    assert np.isfinite(np.delete(Yf, 4, axis=1)).all()


def test_quant_dot_permutation_equivariance():
    A, AS, B, BS = _mx(4, 24, 256, 6)
    _, Yf, _ = O.quant_dot_mxfp4a8(A, AS, B, BS)
    pm, pn = np.random.default_rng(1).permutation(4), np.random.default_rng(2).permutation(24)
    _, Yp, _ = O.quant_dot_mxfp4a8(A[pm], AS[pm], B[pn], BS[pn])
    assert np.array_equal(Yp, Yf[pm][:, pn])


def test_quant_dot_nibble_order():
    """Low nibble = even k: swapping the nibbles of every byte must change the result
    unless the activation is symmetric between k and k+1."""
    M, N, K = 1, 1, 128
    A = np.zeros((M, K), np.uint8)
    A[0, 0] = 0x38                                        # only k = 0 active
    AS = np.ones((M, 1), np.float32)
    B = np.zeros((N, K // 2), np.uint8)
    B[0, 0] = 0x70                                        # k=0 -> code 0, k=1 -> code 7 (6.0)
    BS = np.full((N, K // 32), 127, np.uint8)
    _, Yf, _ = O.quant_dot_mxfp4a8(A, AS, B, BS)
    assert Yf[0, 0] == 0.0
    B[0, 0] = 0x07
    _, Yf, _ = O.quant_dot_mxfp4a8(A, AS, B, BS)
    assert Yf[0, 0] == 6.0


@pytest.mark.parametrize("rblk", [1, 128])
def test_quant_dot_fp8a8_brute_force_and_order(rblk):
    rng = np.random.default_rng(9)
    M, N, K = 3, 200, 384
    A = synth.random_e4m3_codes((M, K), rng)
    AS = (0.001 + 0.01 * rng.random((M, K // 128))).astype(np.float32)
    B = synth.random_e4m3_codes((N, K), rng)
    rows = N if rblk == 1 else (N + 127) // 128
    BS = synth.bf16_bits((0.001 + 0.01 * rng.random((rows, K // 128))).astype(np.float32))
    Y, Yf, S = O.quant_dot_fp8a8(A, AS, B, BS, rblk)
    a = O.e4m3_to_f32(A).astype(np.float64)
    b = O.e4m3_to_f32(B).astype(np.float64)
    sb = synth.bits_to_f32(BS).astype(np.float64)
    sbf = np.repeat(sb, 128, axis=1)[:, :K]
    if rblk == 128:
        sbf = np.repeat(sbf, 128, axis=0)[:N]
    ex = (a * np.repeat(AS.astype(np.float64), 128, axis=1)) @ (b * sbf).T
    assert (np.abs(Yf - ex) <= 2 * K * 2.0 ** -24 * S.astype(np.float64) + 1e-30).all()
    # one group, explicit (sub * sa) * sb order
    sub = np.float32(0)
    for k in range(128):
        sub = np.float32(sub + np.float32(a[0, k] * b[7, k]))
    acc = np.float32(np.float32(sub * AS[0, 0]) * np.float32(sb[7 // rblk, 0]))
    _, Yf1, _ = O.quant_dot_fp8a8(A[:1, :128], AS[:1, :1], B[:, :128], BS[:, :1], rblk)
    assert Yf1[0, 7] == acc


# ------------------------------------------------------------------ mxfp8 quantiser
def test_quant_act_mxfp8_invariants():
    rng = np.random.default_rng(10)
    x = synth.bf16_bits((rng.standard_normal((3, 256)) * np.exp2(rng.integers(-20, 20, (3, 1)))).astype(np.float32))
    x[1, 32:64] = 0
    q, sx = O.quant_act_mxfp8(x)
    xf = synth.bits_to_f32(x).astype(np.float64)
    assert sx[1, 1] == 127 and (q[1, 32:64] == 0).all()
    for m in range(3):
        for g in range(8):
            seg = xf[m, 32 * g:32 * g + 32]
            if not seg.any():
                continue
            e = int(sx[m, g]) - 127
            amax = np.abs(seg).max()
            assert amax * 2.0 ** -e <= 448.0 and amax * 2.0 ** -(e - 1) > 448.0   # least e
            dq = O.e4m3_to_f32(q[m, 32 * g:32 * g + 32]).astype(np.float64) * 2.0 ** e
            big = np.abs(seg) >= 2.0 ** (e - 6)
            assert (np.abs(dq - seg)[big] <= np.abs(seg)[big] * 2.0 ** -4).all()


def test_dot_mx8_mxfp4_brute_force():
    rng = np.random.default_rng(11)
    x = synth.bf16_bits(rng.standard_normal((2, 256)).astype(np.float32))
    q, sx = O.quant_act_mxfp8(x)
    B, BS = synth.mxfp4_weights(24, 256, 12)
    Y, Yf, S = O.dot_mx8_mxfp4(q, sx, B, BS)
    a = O.e4m3_to_f32(q).astype(np.float64) * np.repeat(np.exp2(sx.astype(np.float64) - 127), 32, axis=1)
    ex = a @ O.mxfp4_dequant(B, BS).astype(np.float64).T
    assert (np.abs(Yf - ex) <= 2 * 256 * 2.0 ** -24 * S.astype(np.float64) + 1e-30).all()


def test_group8_mag_bounds():
    A, AS, B, BS = _mx(2, 16, 256, 13)
    _, _, S = O.quant_dot_mxfp4a8(A, AS, B, BS)
    S8 = O.group8_mag("mxfp4a8", A, AS, B, BS)
    assert (S8 <= S * (1 + 1e-5)).all() and (S8 >= S / 8 * (1 - 1e-5)).all()


@pytest.mark.parametrize("enc", ["mxfp4a8", "fp8a8"])
def test_group8_mag_is_sum_of_group_maxima(enc):
    """S8 is the sum over 8-wide k groups of each group's LARGEST scaled product: products
    {1, 2, 3} in group 0 and {4} in group 1 give S8 = 3 + 4 = 7 -- a sum inside the groups
    would give 10, a maximum over all k 4, a missing scale or a wrong group width
    something else.  The scales (a_scale 2, weight scale 2^-1) multiply every product."""
    K = 128
    A = np.zeros((1, K), np.uint8)
    A[0, [0, 1, 2, 8]] = 0x38                                   # e4m3 1.0
    AS = np.full((1, 1), 2.0, np.float32)
    if enc == "mxfp4a8":
        w = np.zeros(K, np.uint8)
        w[[0, 1, 2, 8]] = [2, 4, 5, 6]                          # e2m1 1, 2, 3, 4
        B = (w[0::2] | (w[1::2] << 4)).astype(np.uint8)[None, :]
        BS = np.full((1, K // 32), 126, np.uint8)               # 2^-1
    else:
        B = np.zeros((1, K), np.uint8)
        B[0, [0, 1, 2, 8]] = [0x38, 0x40, 0x44, 0x48]           # e4m3 1, 2, 3, 4
        BS = synth.bf16_bits(np.full((1, 1), 0.5, np.float32))
    S8 = O.group8_mag(enc, A, AS, B, BS)
    assert S8[0, 0] == np.float32(7.0), S8
    if enc == "mxfp4a8":
        _, _, S = O.quant_dot_mxfp4a8(A, AS, B, BS)
    else:
        _, _, S = O.quant_dot_fp8a8(A, AS, B, BS, 1)
    assert S[0, 0] == np.float32(10.0), S
