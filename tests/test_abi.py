"""The C-ABI boundary on the CPU: exports, plugin identity, the gemm_nt_q schema, the row
table and its resolver behaviour, the registration-time kill switches, and every plan
refusal and geometry choice (through r3d_gfx950_describe, which launches nothing and
touches no device memory)."""
import ctypes
import json
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import libr3d_amd as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_every_declared_symbol_is_exported():
    L = R.lib()
    names = []
    for h in ("r3d_gfx950.h",):
        txt = open(os.path.join(ROOT, "include", h)).read()
        names += re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(\w+)\s*\([^;]*\);", txt, re.M)
    assert len(names) >= 10, names
    for n in names:
        assert hasattr(L, n), n


def test_plugin_identity_and_schema():
    L = R.lib()
    assert L.rad_plugin_abi_version() == 26
    info = L.rad_plugin_info().contents
    assert info.targets == b"gfx950" and info.kind == 1
    sch = R.schemas()
    assert [s["op"] for s in sch] == ["gemm_nt_q", "quant_act_fp8", "gemm_nt_q_gated",
                                      "gated_quant_fp8", "rmsnorm_quant_fp8", "logits_gemm"]
    lg = sch[5]                             # src/r3d_rows.cpp:235-245, verbatim
    assert [(p[0], p[1], p[2]) for p in lg["params"]] == [
        ("M", 0, 0), ("n_vocab", 0, 0), ("n_embd", 0, 0), ("dtype", 1, 0)]
    assert [(o[0], o[1], o[2]) for o in lg["operands"]] == [
        ("x", 0, 0), ("lm_head", 3, 0), ("logits", 1, 0)]
    rq = sch[4]                             # src/r3d_rows.cpp:701-716, verbatim
    assert [(p[0], p[1], p[2]) for p in rq["params"]] == [
        ("M", 0, 0), ("n", 0, 0), ("eps", 2, 0), ("group", 0, 0), ("dtype", 1, 0), ("wadd", 2, 1)]
    assert [(o[0], o[1], o[2]) for o in rq["operands"]] == [
        ("x", 0, 0), ("residual", 2, 1), ("w", 3, 0), ("q", 1, 0), ("scale", 1, 0),
        ("out_bf16", 1, 1)]
    gg, gq = sch[2], sch[3]                 # src/r3d_rows.cpp:215-230 and :626-637, verbatim
    assert [(p[0], p[2]) for p in gg["params"]] == [("M", 0), ("N", 0), ("K", 0), ("group", 0),
                                                    ("dtype", 0), ("act", 0)]
    assert [(o[0], o[1], o[2]) for o in gg["operands"]] == [
        ("a", 0, 0), ("a_scale", 0, 0), ("b", 3, 0), ("b_scale", 3, 0), ("q", 1, 0),
        ("scale", 1, 0), ("out_bf16", 1, 1)]
    assert [(p[0], p[2]) for p in gq["params"]] == [("M", 0), ("n", 0), ("group", 0),
                                                    ("dtype", 0), ("act", 1)]
    assert [(o[0], o[1], o[2]) for o in gq["operands"]] == [
        ("gate_up", 0, 0), ("q", 1, 0), ("scale", 1, 0), ("out_bf16", 1, 1)]
    q = sch[1]                              # src/r3d_rows.cpp:615-625, verbatim
    assert [(p[0], p[2]) for p in q["params"]] == [("M", 0), ("n", 0), ("group", 0), ("dtype", 0)]
    assert [(o[0], o[1], o[2]) for o in q["operands"]] == [("x", 0, 0), ("q", 1, 0), ("scale", 1, 0)]
    s = sch[0]
    assert [p[0] for p in s["params"]] == ["M", "N", "K", "group", "dtype", "pb1", "pb2", "split_n"]
    assert [p[2] for p in s["params"]] == [0, 0, 0, 0, 0, 1, 1, 1]          # required / optional
    assert [(o[0], o[2]) for o in s["operands"]] == [
        ("a", 0), ("a_scale", 1), ("b", 0), ("b_scale", 0), ("y", 0), ("a_sum", 1), ("b_ref", 1)]
    assert [o[1] for o in s["operands"]] == [0, 0, 3, 3, 1, 0, 3]            # IN/WEIGHT/OUT


def test_rows_and_resolver():
    rows = {r["name"]: r for r in R.rows()}
    assert set(rows) == {"gemm_nt_q_mxfp4", "gemm_nt_q_mxfp4_decode", "gemm_nt_q_fp8a8",
                         "gemm_nt_q_fp8a8_decode", "gemm_nt_q_mxfp4a16", "quant_act_fp8_act",
                         "gated_quant_fp8_act", "gemm_nt_q_gated_fp8a8", "rmsnorm_quant_fp8",
                         "logits_gemm_e4m3"}
    lg = lambda **kw: (R.resolve("logits_gemm", kw) or {}).get("name")
    assert lg(M=4, n_vocab=262144, n_embd=5376, dtype="bf16") == "logits_gemm_e4m3"
    assert lg(M=4, n_vocab=262144, n_embd=64, dtype="bf16") is None          # n_embd GE 128
    assert lg(M=4, n_vocab=262144, n_embd=5376, dtype="f16") is None
    assert lg(M=4, n_vocab=0, n_embd=5376, dtype="bf16") is None
    assert rows["logits_gemm_e4m3"]["priority"] == 1000 and not rows["logits_gemm_e4m3"]["scratch"]
    rq = lambda **kw: (R.resolve("rmsnorm_quant_fp8", kw) or {}).get("name")
    assert rq(M=4, n=5376, eps=1e-6, group=128, dtype="bf16") == "rmsnorm_quant_fp8"
    assert rq(M=4, n=5378, eps=1e-6, group=128, dtype="bf16") is None      # n DIV 4
    assert rq(M=4, n=5376, eps=1e-6, group=64, dtype="bf16") is None
    gq = lambda **kw: (R.resolve("gated_quant_fp8", kw) or {}).get("name")
    assert gq(M=1, n=10752, group=128, dtype="bf16") == "gated_quant_fp8_act"
    assert gq(M=1, n=10752, group=128, dtype="f16") is None
    gg = lambda **kw: (R.resolve("gemm_nt_q_gated", kw) or {}).get("name")
    ok = dict(dtype="fp8a8", M=64, N=21504, K=5376, group=128, act="silu")
    assert gg(**ok) == "gemm_nt_q_gated_fp8a8"
    assert gg(**dict(ok, act="sigmoid")) == "gemm_nt_q_gated_fp8a8"
    assert gg(**dict(ok, M=65)) is None and gg(**dict(ok, act="gelu")) is None
    assert gg(**dict(ok, K=5377)) is None and gg(**dict(ok, dtype="mxfp4a8")) is None
    assert rows["gemm_nt_q_gated_fp8a8"]["scratch"]
    qa = lambda **kw: R.resolve("quant_act_fp8", kw)["name"] if R.resolve("quant_act_fp8", kw) else None
    assert qa(M=4, n=5376, group=128, dtype="bf16") == "quant_act_fp8_act"
    assert qa(M=4, n=5376, group=128, dtype="f32") == "quant_act_fp8_act"
    assert qa(M=4, n=5376, group=128, dtype="f16") is None
    assert qa(M=4, n=0, group=128, dtype="bf16") is None
    assert rows["gemm_nt_q_mxfp4_decode"]["priority"] == 1100
    assert rows["gemm_nt_q_mxfp4"]["priority"] == 1000
    q = lambda **kw: R.resolve("gemm_nt_q", kw)["name"] if R.resolve("gemm_nt_q", kw) else None
    assert q(dtype="mxfp4a8", M=1, K=4096, N=4096, group=32) == "gemm_nt_q_mxfp4_decode"
    assert q(dtype="mxfp4a8", M=16, K=4096, N=4096, group=32) == "gemm_nt_q_mxfp4_decode"
    assert q(dtype="mxfp4a8", M=17, K=4096, N=4096, group=32) == "gemm_nt_q_mxfp4"
    assert q(dtype="mxfp4a8", M=1, K=4160, N=4096, group=32) is None        # ragged K -> host
    assert q(dtype="fp8a8", M=4, K=5376, N=21504, group=128) == "gemm_nt_q_fp8a8_decode"
    assert q(dtype="fp8a8", M=2048, K=5376, N=21504, group=128) == "gemm_nt_q_fp8a8"
    assert q(dtype="fp8a8", M=4, K=5376, N=21504, group=64) is None
    assert q(dtype="w2a8", M=1, K=5376, N=16, group=128) is None
    # a constraint on an absent key never holds: without M only the decode row drops out
    assert q(dtype="mxfp4a8", K=4096, N=4096, group=32) == "gemm_nt_q_mxfp4"
    assert q(dtype="fp8a8", M=4, K=5376, N=21504) is None                   # no group key


_ROWS_SCRIPT = r"""
import json, sys
sys.path.insert(0, %r)
import libr3d_amd as R
print(json.dumps(sorted(r["name"] for r in R.rows())))
"""


A16 = "gemm_nt_q_mxfp4a16"


QA = "quant_act_fp8_act"
GQ = "gated_quant_fp8_act"
GG = "gemm_nt_q_gated_fp8a8"
RQ = "rmsnorm_quant_fp8"
LG = "logits_gemm_e4m3"


@pytest.mark.parametrize("env,expect", [
    ({}, [GQ, "gemm_nt_q_fp8a8", "gemm_nt_q_fp8a8_decode", GG, "gemm_nt_q_mxfp4",
          "gemm_nt_q_mxfp4_decode", A16, LG, QA, RQ]),
    ({"R3D_NO_MXFP4": "1"}, [GQ, "gemm_nt_q_fp8a8", "gemm_nt_q_fp8a8_decode", GG, LG, QA, RQ]),
    ({"R3D_NO_FP4_DEC": "1"}, [GQ, "gemm_nt_q_fp8a8", "gemm_nt_q_fp8a8_decode", GG,
                               "gemm_nt_q_mxfp4", A16, LG, QA, RQ]),
    ({"R3D_NO_FP8A8": "1"}, [GQ, "gemm_nt_q_mxfp4", "gemm_nt_q_mxfp4_decode", A16, LG, QA, RQ]),
    ({"R3D_NO_FP8_DEC": "1"}, [GQ, "gemm_nt_q_fp8a8", GG, "gemm_nt_q_mxfp4",
                               "gemm_nt_q_mxfp4_decode", A16, LG, QA, RQ]),
    ({"R3D_NO_FP8_DEC": "", "R3D_NO_FP4_DEC": "0"}, [GQ, "gemm_nt_q_fp8a8", GG,
                                                     "gemm_nt_q_mxfp4", A16, LG, QA, RQ]),
    ({"R3D_MXFP4_Q8X": "0"}, [GQ, "gemm_nt_q_fp8a8", "gemm_nt_q_fp8a8_decode", GG,
                              "gemm_nt_q_mxfp4", "gemm_nt_q_mxfp4_decode", A16, LG, QA, RQ]),
    ({"R3D_NO_MXFP4": "1", "R3D_NO_FP8A8": "1"}, [GQ, LG, QA, RQ]),
])
def test_kill_switch_matrix(env, expect):
    """Presence-tested levers hide rows at registration (the value does not matter: an
    empty or "0" value still counts as set); R3D_MXFP4_Q8X is inert here; the band row has
    no lever."""
    e = {k: v for k, v in os.environ.items() if not k.startswith("R3D_")}
    e.update(env)
    out = subprocess.run([sys.executable, "-c", _ROWS_SCRIPT % ROOT], env=e, capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert json.loads(out.stdout.strip().splitlines()[-1]) == expect


# ------------------------------------------------------------------ plans (host only)
class FakeT:
    """Host numpy buffer standing in for a device tensor: describe() never dereferences."""

    def __init__(self, arr, offset=0):
        self.arr = arr
        self.offset = offset
        self.shape = arr.shape
        self.dtype = arr.dtype

    def data_ptr(self):
        return self.arr.ctypes.data + self.offset

    def stride(self, dim=None):
        st = tuple(s // self.arr.itemsize for s in self.arr.strides)
        return st if dim is None else st[dim]

    def numel(self):
        return self.arr.size

    def element_size(self):
        return self.arr.itemsize


def _aligned(shape, dtype):
    n = int(np.prod(shape)) * np.dtype(dtype).itemsize
    raw = np.zeros(n + 256, np.uint8)
    off = (-raw.ctypes.data) % 256
    return raw[off:off + n].view(dtype).reshape(shape)


def _mx_ops(M=1, N=64, K=256, **kw):
    a = FakeT(_aligned((M, K), np.uint8))
    s = FakeT(_aligned((M, K // 128), np.float32))
    b = FakeT(_aligned((N, K // 2), np.uint8))
    bs = FakeT(_aligned((N, K // 32), np.uint8))
    y = FakeT(_aligned((M, N), np.uint16))
    kw.setdefault("dtype", "mxfp4a8")
    return R.GemmOperands(a, s, b, bs, y, N=N, K=K, **kw), (a, s, b, bs, y)


def _f8_ops(M=1, N=256, K=256, rblk=1, **kw):
    a = FakeT(_aligned((M, K), np.uint8))
    s = FakeT(_aligned((M, K // 128), np.float32))
    b = FakeT(_aligned((N, K), np.uint8))
    rows = N if rblk == 1 else (N + 127) // 128
    bs = FakeT(_aligned((rows, K // 128), np.uint16))
    y = FakeT(_aligned((M, N), np.uint16))
    kw.setdefault("dtype", "fp8a8")
    return R.GemmOperands(a, s, b, bs, y, N=N, K=K, **kw), (a, s, b, bs, y)


def _geom(desc):
    return dict(kv.split("=") for kv in desc.split() if "=" in kv)


def test_plan_accepts_and_derives_m_from_y():
    ops, _ = _mx_ops(M=3, extra_params=[("M", 99)])
    rc, d = R.describe("gemm_nt_q_mxfp4_decode", ops)
    assert rc == R.RAD_OK, d
    g = _geom(d)
    assert g["M"] == "3" and g["mt"] == "4"              # M = numel(y)/N; MT rounds up


@pytest.mark.parametrize("M,mt", [(1, "1"), (2, "4"), (4, "4"), (5, "8"), (8, "8"), (9, "16"),
                                  (16, "16")])
def test_mt_ladder_rounds_up(M, mt):
    ops, _ = _mx_ops(M=M)
    rc, d = R.describe("gemm_nt_q_mxfp4_decode", ops)
    assert rc == R.RAD_OK and _geom(d)["mt"] == mt


def test_decode_band_bound_and_tile_any_m():
    """The decode rows stop at M = 16; the tile rows take any M: the skinny band (17..64)
    on a narrow N runs 16-row decode-GEMV passes while passes x min(tiles, 256) < 300, the
    rest the prefill pipeline."""
    ops, _ = _mx_ops(M=17)
    assert R.describe("gemm_nt_q_mxfp4_decode", ops)[0] == R.RAD_E_UNSUPPORTED
    for mk, row in ((_mx_ops, "gemm_nt_q_mxfp4"), (_f8_ops, "gemm_nt_q_fp8a8")):
        for M, N, K, arm, passes in [(17, 64, 256, "skinny", "2"), (64, 5376, 21504, "skinny", "4"),
                                     (48, 8192, 5376, "skinny", "3"),
                                     (64, 8192, 5376, "skinny", "4"),
                                     (17, 21504, 5376, "prefill", None),
                                     (32, 21504, 5376, "prefill", None),
                                     (65, 5376, 21504, "prefill", None)]:
            rc, d = R.describe(row, mk(M=M, N=N, K=K)[0])
            g = _geom(d)
            assert rc == R.RAD_OK and g["arm"] == arm and g.get("passes") == passes, (M, N, d)


def _splitk(N, K, bn=128, units=256, min_steps=4):
    """kc, cst of the tile rows' K split, from its stated rule: units aim at one per CU
    over ceil(N / bn) tiles, at least min_steps K steps a chunk, no empty chunk."""
    tiles, steps = -(-N // bn), K // 128
    kc = min(units // tiles, steps // min_steps)
    if kc < 2:
        return 0, 0
    cst = -(-steps // kc)
    kc = -(-steps // cst)
    return (kc, cst) if kc >= 2 else (0, 0)


def _wide_split(N, K, M, mx, units=256, min_steps=4):
    """kc, cst of the skinny-band GEMV's K split (M <= 64), from its stated rule: units aim
    at one per CU over ceil(N / 256) tiles with at least min_steps groups a chunk; a chunk is
    a whole number of 128-byte lines (2 groups at e2m1) and fits the LDS budget with its
    ceil(M / 16) x 16 staged activation rows."""
    G = 2 if mx else 1
    steps, ntiles = K // 128, -(-N // 256)
    kc0 = min(units // ntiles, steps // min_steps)
    if kc0 < 2:
        return 0, 0
    cg = -(-steps // kc0)
    cg = -(-cg // G) * G
    ntg = -(-M // 16)
    lds = lambda c: c * ntg * 2048 + c * 256 + 8 * (-(-(32 * c * 4) // 256) * 256)
    while cg > G and lds(cg) > 152 * 1024:
        cg -= G
    kc = -(-steps // cg)
    return (kc, cg) if kc >= 2 else (0, 0)


def test_tile_splitk_hook_and_arm():
    """The tile rows' scratch hook sizes split K's f32 partial planes (kc * M * N * 4) up to
    M = 128 on a narrow N and returns 0 elsewhere; with that scratch the launch describes
    the split arm, with less (or misaligned) the unsplit arms it had before."""
    rows = {r["name"]: r for r in R.rows()}
    assert rows["gemm_nt_q_mxfp4"]["scratch"] and rows["gemm_nt_q_fp8a8"]["scratch"]
    # up to M = 64 the skinny-band GEMV over 256-row tiles, else the 128 x 128 tile.  Config 2
    # at M = 64: down 21 tiles x 12 chunks of 14 groups, qkv 32 x 7 of 6, gate_up 84 x 3 of
    # 14 (both encodings); past M = 64 down splits 42 x 6 of 28 and gate_up's 168 tiles fill
    # the chip unsplit; M past 128 and one-chunk K never split
    assert _wide_split(5376, 21504, 64, True) == (12, 14) == _wide_split(5376, 21504, 64, False)
    assert _wide_split(8192, 5376, 64, True) == (7, 6)
    assert _wide_split(21504, 5376, 64, False) == (3, 14)
    assert _splitk(5376, 21504) == (6, 28)
    assert _splitk(21504, 5376) == (0, 0) and _splitk(1000, 384) == (0, 0)
    for mk, row in ((_mx_ops, "gemm_nt_q_mxfp4"), (_f8_ops, "gemm_nt_q_fp8a8")):
        for M, N, K in [(64, 5376, 21504), (17, 8192, 5376), (32, 8192, 5376), (17, 5376, 21504),
                        (40, 1000, 2048), (128, 300, 1024), (17, 300, 9216), (17, 300, 2048),
                        (1, 64, 512), (129, 5376, 21504), (64, 21504, 5376), (64, 1000, 384),
                        (65, 5376, 21504), (100, 21504, 5376)]:
            ops, keep = mk(M=M, N=N, K=K)
            mx = row == "gemm_nt_q_mxfp4"
            if M <= 64:
                kc, cst = _wide_split(N, K, M, mx)
            else:
                kc, cst = _splitk(N, K, 128) if M <= 128 else (0, 0)
            need = kc * M * N * 4
            assert R.row_scratch_bytes(row, ops) == need, (row, M, N, K)
            base = _geom(R.describe(row, ops)[1])["arm"]
            assert base in ("skinny", "prefill")
            if not need:
                continue
            sc = FakeT(_aligned((64,), np.uint8))
            ops.set_scratch(sc, need)
            rc, d = R.describe(row, ops)
            g = _geom(d)
            assert rc == R.RAD_OK and g["arm"] == "splitk", d
            assert (g["kc"], g["cst"], g["partials"]) == (str(kc), str(cst), str(need)), d
            if M <= 64:
                assert (g["kernel"], g["bn"], g["ntg"]) == ("wide", "256", str(-(-M // 16))), d
            else:
                assert (g["kernel"], g["bn"], g["bm"]) == ("tile", "128", "128"), d
            ops.set_scratch(sc, need - 1)                      # short: the unsplit arm
            assert _geom(R.describe(row, ops)[1])["arm"] == base
            ops.set_scratch(FakeT(sc.arr, offset=8), need)     # misaligned: the unsplit arm
            assert _geom(R.describe(row, ops)[1])["arm"] == base
    # without y the hook sizes at the M parameter, without either at M = 128
    _, (a, s, b, bs, _y) = _mx_ops(M=64, N=5376, K=21504)
    for extra, M in ((None, 128), ([("M", 17)], 17)):
        ops = R.GemmOperands(a, s, b, bs, None, dtype="mxfp4a8", N=5376, K=21504,
                             extra_params=extra)
        assert R.row_scratch_bytes("gemm_nt_q_mxfp4", ops) == (6 if M > 64 else 12) * M * 5376 * 4


def test_decode_split_hook_and_arm():
    """The decode rows' scratch hook sizes the skinny-band GEMV's K split (kc * M * N * 4)
    where the quad GEMV does not take the launch and the plane holds at least 2^26 weights,
    with no pinned split; with that scratch the launch describes the split, with less, a
    misaligned one or a pinned split the GEMV it had before."""
    rows = {r["name"]: r for r in R.rows()}
    assert rows["gemm_nt_q_mxfp4_decode"]["scratch"] and rows["gemm_nt_q_fp8a8_decode"]["scratch"]
    for mk, row in ((_mx_ops, "gemm_nt_q_mxfp4_decode"), (_f8_ops, "gemm_nt_q_fp8a8_decode")):
        mx = row == "gemm_nt_q_mxfp4_decode"
        # config 2's gate_up / down / qkv at M = 16, 4 and 1, and both sides of 2^26 weights
        for M, N, K, split in [(16, 21504, 5376, True), (16, 5376, 21504, True),
                               (16, 8192, 5376, False), (8, 5376, 21504, True),
                               (4, 5376, 21504, True), (4, 21504, 5376, False),
                               (1, 5376, 21504, False), (5, 2048, 32768, True),
                               (5, 2048, 32512, False)]:
            ops, keep = mk(M=M, N=N, K=K)
            base = _geom(R.describe(row, ops)[1])
            assert base["arm"] == "decode"
            assert split == (base["kernel"] != "quad" and N * K >= 1 << 26), (row, M, N, K)
            kc, cst = _wide_split(N, K, M, mx) if split else (0, 0)
            need = kc * M * N * 4
            assert R.row_scratch_bytes(row, ops) == need, (row, M, N, K)
            if not need:
                continue
            sc = FakeT(_aligned((64,), np.uint8))
            ops.set_scratch(sc, need)
            rc, d = R.describe(row, ops)
            g = _geom(d)
            assert rc == R.RAD_OK and g["arm"] == "splitk" and g["kernel"] == "wide", d
            assert (g["kc"], g["cst"], g["partials"]) == (str(kc), str(cst), str(need)), d
            ops.set_scratch(sc, need - 1)                      # short: the GEMV
            assert _geom(R.describe(row, ops)[1])["kernel"] == base["kernel"]
            ops.set_scratch(FakeT(sc.arr, offset=8), need)     # misaligned: the GEMV
            assert _geom(R.describe(row, ops)[1])["kernel"] == base["kernel"]
            del ops, keep
    # a pinned split keeps the GEMV and asks for no scratch
    ops, _ = _mx_ops(M=16, N=5376, K=21504, tunables=[("splitk", 2)])
    assert R.row_scratch_bytes("gemm_nt_q_mxfp4_decode", ops) == 0
    # without y the hook sizes at the M parameter, without either at M = 16
    _, (a, s, b, bs, _y) = _mx_ops(M=16, N=5376, K=21504)
    for extra, M in ((None, 16), ([("M", 8)], 8)):
        ops = R.GemmOperands(a, s, b, bs, None, dtype="mxfp4a8", N=5376, K=21504,
                             extra_params=extra)
        assert R.row_scratch_bytes("gemm_nt_q_mxfp4_decode", ops) == 12 * M * 5376 * 4


def test_decode_geometry_policy():
    """M <= 4 runs the quad GEMV, split in K until ~2048 waves (>= 16 groups per chunk),
    while its workgroup LDS (whole-K activation rows) stays <= 48 KB, else the 16-row GEMV;
    M = 5..16 runs the line GEMV (two 16-row tiles per wave), split until ~4096 waves (>= 4
    lines per chunk); a pinned split of 8 runs the 16-row GEMV."""
    for (M, N, K, kern, chunks) in [(1, 21504, 5376, "quad", "1"), (1, 5376, 21504, "quad", "2"),
                                    (1, 4096, 4096, "quad", "2"), (1, 1000, 4096, "quad", "4"),
                                    (1, 64, 256, "quad", "1"), (4, 8192, 5376, "quad", "1"),
                                    (4, 5376, 21504, "tile16", "2"), (16, 21504, 5376, "lines", "4"),
                                    (16, 5376, 21504, "lines", "4"), (8, 8192, 5376, "lines", "4"),
                                    (16, 64, 256, "lines", "1"), (16, 64, 2048, "lines", "2")]:
        ops, _ = _mx_ops(M=M, N=N, K=K)
        rc, d = R.describe("gemm_nt_q_mxfp4_decode", ops)
        assert rc == R.RAD_OK, d
        g = _geom(d)
        assert g["kernel"] == kern and g["chunks"] == chunks, (M, N, K, d)
    # waves per quad workgroup: 8 at MT = 4 and for fp8a8 at MT = 1 without a K split
    # (seven when that evens the workgroups over 256 CUs without a K split; the ragged
    # shapes the GPU tests run at seven waves)
    for (mk, row, M, N) in [(_f8_ops, "gemm_nt_q_fp8a8_decode", 1, 8227),
                            (_mx_ops, "gemm_nt_q_mxfp4_decode", 3, 8354)]:
        assert _geom(R.describe(row, mk(M=M, N=N, K=1024)[0])[1])["waves"] == "7"
    for (mk, M, N, K, wv) in [(_mx_ops, 1, 21504, 5376, "7"), (_mx_ops, 1, 8192, 5376, "4"),
                              (_mx_ops, 1, 5376, 21504, "4"), (_mx_ops, 4, 21504, 5376, "7"),
                              (_f8_ops, 1, 21504, 5376, "7"), (_f8_ops, 1, 16384, 5376, "8"),
                              (_f8_ops, 1, 4096, 4096, "4"), (_f8_ops, 3, 2048, 5376, "8")]:
        ops, _ = mk(M=M, N=N, K=K)
        rc, d = R.describe("gemm_nt_q_mxfp4_decode" if mk is _mx_ops else
                           "gemm_nt_q_fp8a8_decode", ops)
        assert rc == R.RAD_OK and _geom(d)["waves"] == wv, (M, N, K, d)
    # long K: the policy's seven / eight waves would overflow the 48 KB staging, four fit
    # (mxfp4a8 N=21504 K=26624..30720 and fp8a8 at 70B-class down shapes)
    for (mk, M, N, K) in [(_mx_ops, 1, 21504, 26624), (_mx_ops, 1, 21504, 28672),
                          (_mx_ops, 1, 21504, 30720), (_f8_ops, 1, 8192, 28672),
                          (_f8_ops, 1, 16384, 24576)]:
        ops, _ = mk(M=M, N=N, K=K)
        rc, d = R.describe("gemm_nt_q_mxfp4_decode" if mk is _mx_ops else
                           "gemm_nt_q_fp8a8_decode", ops)
        g = _geom(d)
        assert rc == R.RAD_OK and g["kernel"] == "quad" and g["waves"] == "4", (M, N, K, d)
        assert int(g["lds"]) <= 48 * 1024, d
    ops, _ = _mx_ops(M=1, N=21504, K=5376, tunables=[("splitk", 2)])
    g = _geom(R.describe("gemm_nt_q_mxfp4_decode", ops)[1])
    assert g["kernel"] == "quad" and g["chunks"] == "2"
    ops, _ = _mx_ops(M=1, N=21504, K=5376, tunables=[("splitk", 8)])
    g = _geom(R.describe("gemm_nt_q_mxfp4_decode", ops)[1])
    assert g["kernel"] == "tile16" and g["chunks"] == "8"


@pytest.mark.parametrize("case,rc", [
    ("dtype", R.RAD_E_UNSUPPORTED), ("a_sum", R.RAD_E_UNSUPPORTED), ("pb1", R.RAD_E_UNSUPPORTED),
    ("k_ragged", R.RAD_E_UNSUPPORTED), ("a_misaligned", R.RAD_OK),
    ("no_n", R.RAD_E_SHAPE), ("y_ragged", R.RAD_E_SHAPE), ("bs_grid", R.RAD_E_UNSUPPORTED),
    ("y_dtype", R.RAD_E_UNSUPPORTED), ("b_ref_ok", R.RAD_OK), ("a_small", R.RAD_E_SHAPE),
])
def test_mxfp4_plan_refusals(case, rc):
    M, N, K = 2, 64, 256
    kw = {}
    if case == "dtype":
        kw["dtype"] = "fp8a8"
    if case == "pb1":
        kw["extra_params"] = [("pb1", 2)]
    a = FakeT(_aligned((M, K), np.uint8))
    s = FakeT(_aligned((M, K // 128), np.float32))
    b = FakeT(_aligned((N, K // 2), np.uint8))
    bs = FakeT(_aligned((N, K // 32), np.uint8))
    y = FakeT(_aligned((M, N), np.uint16))
    extra = {}
    if case == "a_sum":
        extra["a_sum"] = FakeT(_aligned((M, 2), np.float32))
    if case == "b_ref_ok":
        extra["b_ref"] = FakeT(_aligned((N, 2), np.uint16))
    if case == "a_misaligned":
        a = FakeT(_aligned((M, K + 16), np.uint8), offset=4)
    if case == "bs_grid":
        bs = FakeT(_aligned((N, K // 64), np.uint8))
    if case == "a_small":
        a = FakeT(_aligned((1, K), np.uint8))
    Kp = K + 64 if case == "k_ragged" else K
    if case == "k_ragged":
        a = FakeT(_aligned((M, Kp), np.uint8))
        b = FakeT(_aligned((N, Kp // 2), np.uint8))
        bs = FakeT(_aligned((N, (Kp + 31) // 32), np.uint8))
        s = FakeT(_aligned((M, (Kp + 127) // 128), np.float32))
    ops = R.GemmOperands(a, s, b, bs, y, dtype=kw.get("dtype", "mxfp4a8"), N=N, K=Kp,
                         extra_params=kw.get("extra_params"), **extra)
    if case == "no_n":
        ops._p[1].key = b"Nx"
    if case == "y_ragged":
        ops._t[4].shape[1] = N - 1
    if case == "y_dtype":
        ops._t[4].dtype = R.DT["F32"]
    got, d = R.describe("gemm_nt_q_mxfp4_decode", ops)
    assert got == rc, (case, d)
    if case == "a_misaligned":              # taken, on the any-alignment arm
        assert d.startswith("arm=any "), d


@pytest.mark.parametrize("case,rc", [
    ("ok_row", R.RAD_OK), ("ok_block", R.RAD_OK), ("b_ref", R.RAD_E_UNSUPPORTED),
    ("group64", R.RAD_E_SHAPE), ("bs_dtype", R.RAD_E_UNSUPPORTED), ("inner_stride", R.RAD_E_STRIDE),
])
def test_fp8_plan_refusals(case, rc):
    rblk = 128 if case == "ok_block" else 1
    extra = {}
    if case == "b_ref":
        extra["b_ref"] = FakeT(_aligned((256, 2), np.uint16))
    ops, (a, s, b, bs, y) = _f8_ops(rblk=rblk, group=64 if case == "group64" else None, **extra)
    if case == "bs_dtype":
        ops._t[3].dtype = R.DT["F32"]
    if case == "inner_stride":
        ops._t[2].stride[1] = 2
    got, d = R.describe("gemm_nt_q_fp8a8_decode", ops)
    assert got == rc, (case, d)
    if rc == R.RAD_OK:
        assert _geom(d)["rblk"] == str(rblk)


def _xq_ops(dtype, M, N, K, pitch=None, rblk=1, a_dt=np.uint16, **kw):
    """Decode operands with bf16 activations and no a_scale (the fused producer)."""
    a = FakeT(_aligned((M, pitch or K), a_dt))
    if pitch:
        a.shape, a.arr = (M, K), a.arr
        a.stride = lambda dim=None, p=pitch: (p, 1) if dim is None else (p, 1)[dim]
    if dtype == "mxfp4a8":
        b = FakeT(_aligned((N, K // 2), np.uint8))
        bs = FakeT(_aligned((N, K // 32), np.uint8))
    else:
        b = FakeT(_aligned((N, K), np.uint8))
        bs = FakeT(_aligned((N if rblk == 1 else (N + 127) // 128, K // 128), np.uint16))
    y = FakeT(_aligned((M, N), np.uint16))
    return R.GemmOperands(a, None, b, bs, y, dtype=dtype, N=N, K=K, **kw)


@pytest.mark.parametrize("dtype,row", [("mxfp4a8", "gemm_nt_q_mxfp4_decode"),
                                       ("fp8a8", "gemm_nt_q_fp8a8_decode")])
def test_fused_producer_plan(dtype, row):
    """bf16 activations without a_scale: accepted by the decode row at M = 1 (the quad GEMV
    quantises the row in its LDS staging), refused everywhere else so the engine runs the
    producer first."""
    for M, N, K in [(1, 21504, 5376), (1, 64, 256), (1, 5376, 21504), (1, 2048, 16384)]:
        rc, d = R.describe(row, _xq_ops(dtype, M, N, K))
        assert rc == R.RAD_OK, (M, N, K, d)
        g = _geom(d)
        assert g["kernel"] == "quad" and g["xq"] == "1" and g["waves"] == "8", d
    # long K (70B-class down projections): eight waves' staging would pass 48 KB, four fit;
    # the fused producer still runs.  From K = 31744 on even four waves do not fit (refused).
    for N, K in [(8192, 24576), (8192, 28672)]:
        rc, d = R.describe(row, _xq_ops(dtype, 1, N, K))
        g = _geom(d)
        assert rc == R.RAD_OK and g["kernel"] == "quad" and g["waves"] == "4", (N, K, d)
    if dtype == "fp8a8":
        rc, d = R.describe(row, _xq_ops(dtype, 1, 512, 1024, rblk=128))
        assert rc == R.RAD_OK and _geom(d)["rblk"] == "128", d
    rc, d = R.describe(row, _xq_ops(dtype, 1, 256, 512, pitch=512 + 64))
    assert rc == R.RAD_OK, d
    refused = [
        _xq_ops(dtype, 4, 5376, 5376),                        # M > 1
        _xq_ops(dtype, 2, 64, 256),
        _xq_ops(dtype, 8, 512, 1024),
        _xq_ops(dtype, 1, 512, 1024, tunables=[("splitk", 8)]),
        _xq_ops(dtype, 1, 256, 512, pitch=512 + 4),           # pitch not 16 bytes
        _xq_ops(dtype, 1, 256, 512, a_dt=np.float32),         # f32 activations
    ]
    for ops in refused:
        assert R.describe(row, ops)[0] == R.RAD_E_UNSUPPORTED
    tile = "gemm_nt_q_mxfp4" if dtype == "mxfp4a8" else "gemm_nt_q_fp8a8"
    assert R.describe(tile, _xq_ops(dtype, 64, 512, 1024))[0] == R.RAD_E_UNSUPPORTED


@pytest.mark.parametrize("dtype,row", [("mxfp4a8", "gemm_nt_q_mxfp4_decode"),
                                       ("fp8a8", "gemm_nt_q_fp8a8_decode")])
def test_fused_producer_beyond_one_row_on_request(dtype, row):
    """The "fuse" tunable extends the fused producer to M = 2..4 (the quad GEMV's four
    activation images), and only there: M = 5.. stays refused, as do shapes whose four
    whole-K rows the workgroup cannot stage (K = 21504), and "fuse" = 0 is the default."""
    fuse = [("fuse", 1)]
    for M, N, K in [(2, 64, 256), (3, 5376, 4096), (4, 21504, 5376), (4, 2048, 5376)]:
        rc, d = R.describe(row, _xq_ops(dtype, M, N, K, tunables=fuse))
        assert rc == R.RAD_OK, (M, N, K, d)
        g = _geom(d)
        assert g["kernel"] == "quad" and g["xq"] == "1" and g["mt"] == "4", d
        assert R.describe(row, _xq_ops(dtype, M, N, K, tunables=[("fuse", 0)]))[0] == \
            R.RAD_E_UNSUPPORTED
    for ops in (_xq_ops(dtype, 5, 512, 1024, tunables=fuse),
                _xq_ops(dtype, 16, 512, 1024, tunables=fuse),
                _xq_ops(dtype, 4, 5376, 21504, tunables=fuse)):
        assert R.describe(row, ops)[0] == R.RAD_E_UNSUPPORTED
    names = [t for r in R.rows() if r["name"] == row for t in r.get("tunables", [])]
    assert names == ["splitk", "fuse"], names


_QWV_SCRIPT = r"""
import sys
sys.path.insert(0, %r)
sys.path.insert(0, %r)
import test_abi as T
import libr3d_amd as R
for mk, row, M, N, K in [(T._mx_ops, "gemm_nt_q_mxfp4_decode", 1, 5376, 21504),
                         (T._mx_ops, "gemm_nt_q_mxfp4_decode", 1, 21504, 5376),
                         (T._f8_ops, "gemm_nt_q_fp8a8_decode", 1, 5376, 21504)]:
    print(R.describe(row, mk(M=M, N=N, K=K)[0])[1])
for dt, row in (("mxfp4a8", "gemm_nt_q_mxfp4_decode"), ("fp8a8", "gemm_nt_q_fp8a8_decode")):
    print(R.describe(row, T._xq_ops(dt, 1, 21504, 5376))[1])
"""


def test_seven_wave_lever_only_where_it_launches():
    """R3D_GFX950_QWV=7 is honoured without a K split and without the fused producer; with
    either, the policy decides (the seven-wave kernel has no split or fused form, so
    describe never reports a geometry the launch would refuse)."""
    e = {k: v for k, v in os.environ.items() if not k.startswith("R3D_")}
    e["R3D_GFX950_QWV"] = "7"
    out = subprocess.run([sys.executable, "-c", _QWV_SCRIPT % (ROOT, os.path.join(ROOT, "tests"))],
                         env=e, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    got = [_geom(l) for l in out.stdout.strip().splitlines()[-5:]]
    assert (got[0]["chunks"], got[0]["waves"]) == ("2", "4"), got[0]
    assert (got[1]["chunks"], got[1]["waves"]) == ("1", "7"), got[1]
    assert (got[2]["chunks"], got[2]["waves"]) == ("2", "4"), got[2]
    assert got[3]["xq"] == "1" and got[3]["waves"] == "8", got[3]
    assert got[4]["xq"] == "1" and got[4]["waves"] == "8", got[4]


def test_entries_refuse_without_gfx950():
    """On a host without a gfx950 device a valid plan stops at the chip gate: the entry
    returns RAD_E_UNSUPPORTED and launches nothing."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    ops, _ = _mx_ops(M=1)
    assert R.launch_row("gemm_nt_q_mxfp4_decode", ops, 0) == R.RAD_E_UNSUPPORTED


# ------------------------------------------------------------------ prefill plans
def _a16_ops(M=64, N=256, K=256, scratch=True, with_as=False, **kw):
    a = FakeT(_aligned((M, K), np.uint16))
    s = FakeT(_aligned((M, K // 128), np.float32)) if with_as else None
    b = FakeT(_aligned((N, K // 2), np.uint8))
    bs = FakeT(_aligned((N, K // 32), np.uint8))
    y = FakeT(_aligned((M, N), np.uint16))
    kw.setdefault("extra_params", [("M", M)])
    ops = R.GemmOperands(a, s, b, bs, y, dtype="mxfp4a16", N=N, K=K, group=32, **kw)
    need = ((M * K + 255) // 256) * 256 + M * (K // 32)
    sc = FakeT(_aligned((need + 64,), np.uint8))
    if scratch:
        ops.set_scratch(sc, need if scratch is True else scratch)
    return ops, (a, s, b, bs, y, sc), need


def test_prefill_tile_choice_fills_the_last_round():
    # config 3: 96 x 8 = 768 tiles of 224 x 256 -- exactly three rounds of 256 CUs
    ops, keep, need = _a16_ops(M=2048, N=21504, K=5376)
    rc, d = R.describe("gemm_nt_q_mxfp4a16", ops)
    assert rc == R.RAD_OK, d
    g = _geom(d)
    assert (g["arm"], g["bn"], g["bm"], g["tiles"], g["steps"]) == ("prefill", "224", "256", "768", "42")
    assert int(g["lds"]) <= 160 * 1024
    # the f32-a_scale mode takes the same tile at config 3, 128-token tiles up to 128
    # tokens; e4m3 weights run 128 x 256 on four waves past 128 tokens, 128 x 128 up to it
    ops, _ = _mx_ops(M=2048, N=21504, K=5376)
    g = _geom(R.describe("gemm_nt_q_mxfp4", ops)[1])
    assert (g["bn"], g["bm"], g["tiles"]) == ("224", "256", "768")
    ops, _ = _mx_ops(M=64, N=21504, K=5376)
    g = _geom(R.describe("gemm_nt_q_mxfp4", ops)[1])
    assert (g["bn"], g["bm"]) == ("128", "128")
    ops, _ = _f8_ops(M=2048, N=21504, K=5376)
    g = _geom(R.describe("gemm_nt_q_fp8a8", ops)[1])
    assert (g["arm"], g["bn"], g["bm"], g["waves"], g["tiles"]) == ("prefill", "128", "256", "4", "1344")
    assert int(g["lds"]) <= 160 * 1024
    ops, _ = _f8_ops(M=128, N=21504, K=5376)
    g = _geom(R.describe("gemm_nt_q_fp8a8", ops)[1])
    assert (g["arm"], g["bn"], g["bm"], g["waves"]) == ("prefill", "128", "128", "8")
    # the wider tile only where its rounds (1.71x as long) cost less: one round of either
    # at M = 256, N = 4096
    ops, _ = _f8_ops(M=256, N=4096, K=1024)
    g = _geom(R.describe("gemm_nt_q_fp8a8", ops)[1])
    assert (g["bn"], g["bm"], g["waves"]) == ("128", "128", "8")
    # at M = 512, N = 21504: 3 rounds of 128 x 128, against one round of 128 x 256 over the
    # first 16384 weight rows and one of 128 x 128 over the rest (1.71 + 1)
    ops, _ = _f8_ops(M=512, N=21504, K=5376)
    g = _geom(R.describe("gemm_nt_q_fp8a8", ops)[1])
    assert (g["bn"], g["bm"], g["waves"], g["nsplit"]) == ("128", "256", "4", "16384")
    # config 3's 1344 four-wave tiles are 5.25 rounds: the first 20480 weight rows run as 5
    # whole rounds, the last 1024 as one launch of 128 x 128 tiles (5 x 1.71 + 1 < 6 x 1.71)
    ops, _ = _f8_ops(M=2048, N=21504, K=5376)
    assert _geom(R.describe("gemm_nt_q_fp8a8", ops)[1])["nsplit"] == "20480"
    # the remainder launch can make the four-wave tile pay where it alone would not:
    # 260 tiles at M = 512, N = 16640 are 1 round + 4 tiles
    ops, _ = _f8_ops(M=512, N=16640, K=1024)
    g = _geom(R.describe("gemm_nt_q_fp8a8", ops)[1])
    assert (g["waves"], g["nsplit"]) == ("4", "16384"), g
    ops, _ = _f8_ops(M=512, N=16384, K=1024)                  # 256 tiles: one whole round
    g = _geom(R.describe("gemm_nt_q_fp8a8", ops)[1])
    assert (g["waves"], g["nsplit"]) == ("4", "0"), g
    # few tiles: the narrowest tile spreads the work over more CUs
    ops, _ = _mx_ops(M=256, N=4096, K=1024)
    g = _geom(R.describe("gemm_nt_q_mxfp4", ops)[1])
    assert g["bn"] == "128", g


def test_a16_scratch_hook_and_refusals():
    ops, keep, need = _a16_ops()
    assert R.row_scratch_bytes("gemm_nt_q_mxfp4a16", ops) == need
    assert R.describe("gemm_nt_q_mxfp4a16", ops)[0] == R.RAD_OK
    ops, keep, need = _a16_ops(scratch=False)
    assert R.describe("gemm_nt_q_mxfp4a16", ops)[0] == R.RAD_E_UNSUPPORTED
    ops, keep, need = _a16_ops(scratch=need - 1)
    assert R.describe("gemm_nt_q_mxfp4a16", ops)[0] == R.RAD_E_UNSUPPORTED
    ops, keep, need = _a16_ops(with_as=True)               # a_scale has no meaning here
    assert R.describe("gemm_nt_q_mxfp4a16", ops)[0] == R.RAD_E_UNSUPPORTED
    ops, keep, need = _a16_ops(K=320)                      # whole 128-wide steps only
    assert R.describe("gemm_nt_q_mxfp4a16", ops)[0] != R.RAD_OK
    # the a8 row refuses bf16 activations and the a16 row refuses e4m3 ones
    ops, keep, need = _a16_ops()
    ops.dtype = "mxfp4a8"
    ops2, _ = _mx_ops(M=64, N=256, K=256)
    ops2.set_scratch(keep[5], need)
    assert R.describe("gemm_nt_q_mxfp4a16", ops2)[0] == R.RAD_E_UNSUPPORTED
    # no M parameter: the hook has nothing to size
    ops, keep, need = _a16_ops(extra_params=[])
    assert R.row_scratch_bytes("gemm_nt_q_mxfp4a16", ops) == 0


def test_resolver_routes_a16_to_its_row():
    r = R.resolve("gemm_nt_q", {"dtype": "mxfp4a16", "M": 2048, "N": 21504, "K": 5376, "group": 32})
    assert r["name"] == "gemm_nt_q_mxfp4a16"
    assert R.resolve("gemm_nt_q", {"dtype": "mxfp4a16", "M": 4, "N": 64, "K": 320, "group": 32}) is None


# ------------------------------------------------------------------ quant_act_fp8 plan
def _qa(x, q, s, **kw):
    return R.QuantActOperands(FakeT(x), FakeT(q) if q is not None else None,
                              FakeT(s) if s is not None else None, **kw)


@pytest.mark.parametrize("case,rc", [
    ("ok", R.RAD_OK), ("no_scale", R.RAD_E_INVAL), ("x_f16", R.RAD_E_DTYPE),
    ("q_u8", R.RAD_E_DTYPE), ("n0", R.RAD_E_SHAPE), ("rows", R.RAD_E_SHAPE),
    ("q_short", R.RAD_E_SHAPE), ("x_col_stride", R.RAD_E_STRIDE),
])
def test_quant_act_plan_refusals(case, rc):
    """The reference's gates and codes (src/r3d_band.hip:463-481), on the host."""
    M, n = 4, 256
    x = _aligned((M, n), np.uint16)
    q = _aligned((M, n), np.uint8)
    s = _aligned((M, 2), np.float32)
    kw = dict(n=n, group=128, M=M, x_dtype="BF16")
    if case == "no_scale":
        ops = _qa(x, q, None, **kw)
    else:
        ops = _qa(x, q, s, **kw)
        if case == "x_f16":
            ops._t[0].dtype = R.DT["F16"]
        elif case == "q_u8":
            ops._t[1].dtype = R.DT["U8"]
        elif case == "n0":
            ops._p[0].ival = 0
        elif case == "rows":
            ops._t[0].shape[0] = 70000                      # rows above 65535
            ops._t[1].shape[0] = 70000
        elif case == "q_short":
            ops._t[1].shape[0] = 3
        elif case == "x_col_stride":
            ops._t[0].stride[1] = 2
    got, d = R.describe("quant_act_fp8_act", ops)
    assert got == rc, d


def test_quant_act_plan_walk():
    """Group clamp, ragged groups and the band row walk (src/r3d_band.hip:419-449): a
    wider-row view pitches by its row stride, a rank-1 x is one row (pitch 0), a view
    whose shape[1] differs from n reads flat."""
    x = _aligned((3, 300), np.float32)
    q = _aligned((3, 300), np.uint8)
    s = _aligned((3, 3), np.float32)
    g = _geom(R.describe("quant_act_fp8_act", _qa(x, q, s, n=300, group=128, M=3))[1])
    assert (g["x"], g["rows"], g["group"], g["ngrp"], g["x_pitch"]) == ("f32", "3", "128", "3", "300")
    g = _geom(R.describe("quant_act_fp8_act", _qa(x, q, s, n=300, group=1000, M=3))[1])
    assert (g["group"], g["ngrp"]) == ("300", "1")
    g = _geom(R.describe("quant_act_fp8_act", _qa(x, q, s, n=300, group=0, M=3))[1])
    assert g["group"] == "300"
    wide = _aligned((3, 320), np.uint16)
    ops = R.QuantActOperands(FakeT(wide), FakeT(q), FakeT(s), n=300, group=128, M=3,
                             x_dtype="BF16", shapes={0: (3, 300)}, strides={0: (320, 1)})
    g = _geom(R.describe("quant_act_fp8_act", ops)[1])
    assert (g["x"], g["x_pitch"], g["q_pitch"]) == ("bf16", "320", "300")
    one = _aligned((300,), np.uint16)
    ops = R.QuantActOperands(FakeT(one), FakeT(q), FakeT(s), n=300, group=128, M=1, x_dtype="BF16")
    g = _geom(R.describe("quant_act_fp8_act", ops)[1])
    assert (g["rows"], g["x_pitch"]) == ("1", "0")
    ops = R.QuantActOperands(FakeT(wide), FakeT(q), FakeT(s), n=300, group=128, M=3,
                             x_dtype="BF16", shapes={0: (3, 320)}, strides={0: (320, 1)})
    g = _geom(R.describe("quant_act_fp8_act", ops)[1])
    assert g["x_pitch"] == "300"                              # shape[1] != n: flat walk


# ------------------------------------------------------------------ gated rows (host only)
def _gated_ops(M=4, n=1024, K=512, rblk=128, out=True, scratch=True, act="silu", **kw):
    N = 2 * n
    a = FakeT(_aligned((M, K), np.uint8))
    s = FakeT(_aligned((M, K // 128), np.float32))
    b = FakeT(_aligned((N, K), np.uint8))
    bs = FakeT(_aligned((N if rblk == 1 else (N + 127) // 128, K // 128), np.uint16))
    q = FakeT(_aligned((M, n), np.uint8))
    sc = FakeT(_aligned((M, n // 128), np.float32))
    ob = FakeT(_aligned((M, n), np.uint16)) if out else None
    ops = R.GatedGemmOperands(a, s, b, bs, q, sc, ob, N=N, K=K, act=act, **kw)
    need = R.lib().r3d_rad_gemm_nt_q_gated_fp8_scratch(ctypes.byref(ops.args))
    assert need == 64 * N * 2
    if scratch:
        buf = FakeT(_aligned((need,), np.uint8))
        ops.set_scratch(buf, need if scratch is True else scratch)
        ops._buf = buf
    return ops


def test_gated_gemm_plan_and_refusals():
    """The gated row's gates (src/r3d_gemm_fp8a8.hip:1166-1219): GEMM arm by M (decode GEMV
    to 16, the prefill pipeline above), act required, N even, M from numel(q)/n, scratch
    at least M*N*2 bytes."""
    G = "gemm_nt_q_gated_fp8a8"
    for M, arm in ((1, "decode"), (16, "decode"), (17, "prefill"), (64, "prefill")):
        rc, d = R.describe(G, _gated_ops(M=M))
        assert rc == R.RAD_OK, d
        g = _geom(d)
        assert g["gemm"] == arm and g["M"] == str(M) and g["n"] == "1024" and g["ob"] == "bf16", d
    rc, d = R.describe(G, _gated_ops(M=2, rblk=1, out=False, act="sigmoid"))
    assert rc == R.RAD_OK and _geom(d)["act"] == "sigmoid" and _geom(d)["ob"] == "none", d
    assert R.describe(G, _gated_ops(act=None))[0] == R.RAD_E_UNSUPPORTED
    assert R.describe(G, _gated_ops(act="gelu"))[0] == R.RAD_E_UNSUPPORTED
    assert R.describe(G, _gated_ops(scratch=False))[0] == R.RAD_E_UNSUPPORTED
    assert R.describe(G, _gated_ops(M=4, scratch=4 * 2048 * 2 - 2))[0] == R.RAD_E_UNSUPPORTED
    assert R.describe(G, _gated_ops(M=4, scratch=4 * 2048 * 2))[0] == R.RAD_OK
    ops = _gated_ops()
    ops._p[0].ival = 2047                                   # N odd
    assert R.describe(G, ops)[0] == R.RAD_E_SHAPE
    ops = _gated_ops()
    ops._t[4].shape[1] = 1000                               # numel(q) not a multiple of n
    assert R.describe(G, ops)[0] == R.RAD_E_SHAPE
    ops = _gated_ops()
    ops._t[1].data = None                                   # a_scale absent
    assert R.describe(G, ops)[0] == R.RAD_E_UNSUPPORTED


def _gq_ops(M=3, n=512, group=128, gu_dt=np.uint16, out_dt=np.uint16, act=None, pitch=None):
    gu = FakeT(_aligned((M, pitch or 2 * n), gu_dt))
    if pitch:
        gu.shape = (M, 2 * n)
        gu.stride = lambda dim=None, p=pitch: (p, 1) if dim is None else (p, 1)[dim]
    q = FakeT(_aligned((M, n), np.uint8))
    sc = FakeT(_aligned((M, (n + group - 1) // group), np.float32))
    ob = FakeT(_aligned((M, n), out_dt)) if out_dt is not None else None
    return R.GatedQuantOperands(gu, q, sc, ob, n=n, group=group, act=act, M=M)


def test_gated_quant_plan_and_refusals():
    G = "gated_quant_fp8_act"
    rc, d = R.describe(G, _gq_ops())
    g = _geom(d)
    assert rc == R.RAD_OK and g["act"] == "silu" and g["ob"] == "bf16" and g["gu_pitch"] == "1024", d
    g = _geom(R.describe(G, _gq_ops(act="sigmoid", gu_dt=np.float32, out_dt=np.float32))[1])
    assert g["act"] == "sigmoid" and g["gate_up"] == "f32" and g["ob"] == "f32"
    g = _geom(R.describe(G, _gq_ops(act="tanh", out_dt=None))[1])   # any other act: silu
    assert g["act"] == "silu" and g["ob"] == "none"
    g = _geom(R.describe(G, _gq_ops(n=300, group=1000))[1])          # group clamps to n
    assert g["group"] == "300" and g["ngrp"] == "1"
    g = _geom(R.describe(G, _gq_ops(pitch=1100))[1])
    assert g["gu_pitch"] == "1100"
    ops = _gq_ops()
    ops._t[0].dtype = R.DT["F8E4M3"]
    assert R.describe(G, ops)[0] == R.RAD_E_DTYPE
    ops = _gq_ops()
    ops._t[3].dtype = R.DT["F8E4M3"]                        # out_bf16 not f32/bf16
    assert R.describe(G, ops)[0] == R.RAD_E_DTYPE
    ops = _gq_ops()
    ops._t[1].data = None
    assert R.describe(G, ops)[0] == R.RAD_E_INVAL
    ops = _gq_ops()
    ops._t[2].shape[1] = 3                                   # too few scales
    assert R.describe(G, ops)[0] == R.RAD_E_SHAPE


def _rms_ops(M=3, n=512, group=128, res=True, out=True, w_dt=np.float32, **kw):
    x = FakeT(_aligned((M, n), np.uint16))
    r = FakeT(_aligned((M, n), np.uint16)) if res else None
    w = FakeT(_aligned((n,), w_dt))
    q = FakeT(_aligned((M, n), np.uint8))
    sc = FakeT(_aligned((M, (n + group - 1) // group), np.float32))
    ob = FakeT(_aligned((M, n), np.uint16)) if out else None
    return R.RmsNormQuantOperands(x, r, w, q, sc, ob, n=n, group=group, M=M, **kw)


def test_rmsnorm_quant_plan_and_refusals():
    """src/r3d_more.hip:482-521's gates: bf16 x (and residual), f32/bf16 w of rank 1, n at
    most 30720, group clamped, eps / wadd from F64 params."""
    G = "rmsnorm_quant_fp8"
    rc, d = R.describe(G, _rms_ops(eps=1e-5, wadd=1.0))
    g = _geom(d)
    assert rc == R.RAD_OK and g["residual"] == "1" and g["ob"] == "bf16" and g["w"] == "f32", d
    assert float(g["eps"]) == np.float32(1e-5) and float(g["wadd"]) == 1.0
    g = _geom(R.describe(G, _rms_ops(res=False, out=False, w_dt=np.uint16))[1])
    assert g["residual"] == "0" and g["ob"] == "none" and g["w"] == "bf16" and float(g["eps"]) == np.float32(1e-6)
    g = _geom(R.describe(G, _rms_ops(n=300, group=1000))[1])
    assert g["group"] == "300" and g["ngrp"] == "1"
    assert R.describe(G, _rms_ops(n=30720))[0] == R.RAD_OK
    assert R.describe(G, _rms_ops(n=30724))[0] == R.RAD_E_SHAPE
    ops = _rms_ops()
    ops._t[0].dtype = R.DT["F32"]
    assert R.describe(G, ops)[0] == R.RAD_E_DTYPE                        # x must be bf16
    ops = _rms_ops()
    ops._t[1].dtype = R.DT["F32"]
    assert R.describe(G, ops)[0] == R.RAD_E_DTYPE                        # residual bf16
    ops = _rms_ops()
    ops._t[2].rank = 2
    ops._t[2].shape[0], ops._t[2].shape[1] = 1, 512
    ops._t[2].stride[0], ops._t[2].stride[1] = 512, 1
    assert R.describe(G, ops)[0] == R.RAD_E_STRIDE                       # w rank 1
    ops = _rms_ops()
    ops._t[3].data = None
    assert R.describe(G, ops)[0] == R.RAD_E_INVAL
    ops = _rms_ops()
    ops.args.n_t = 4
    assert R.describe(G, ops)[0] == R.RAD_E_INVAL                        # n_t < 5


def _shift(t, off, extra_cols=0):
    """The same tensor viewed `off` bytes past an aligned base (its own storage widened so
    the view stays inside it)."""
    rows, cols = t.arr.shape if t.arr.ndim == 2 else (1, t.arr.shape[0])
    pitch = cols + extra_cols
    base = _aligned((rows * pitch + 16,), t.arr.dtype)
    v = FakeT(base, offset=off)
    v.shape = t.shape
    v.stride = lambda dim=None, p=pitch: (p, 1) if dim is None else (p, 1)[dim]
    return v


@pytest.mark.parametrize("row,dtype", [("gemm_nt_q_mxfp4", "mxfp4a8"),
                                       ("gemm_nt_q_mxfp4_decode", "mxfp4a8"),
                                       ("gemm_nt_q_fp8a8", "fp8a8"),
                                       ("gemm_nt_q_fp8a8_decode", "fp8a8")])
@pytest.mark.parametrize("which,off", [("a", 1), ("a", 4), ("a", 8), ("b", 1), ("b", 4),
                                       ("b", 8), ("bs", 1), ("bs", 2), ("pitch", 0)])
@pytest.mark.parametrize("M", [1, 4, 40, 300])
def test_any_alignment_taken(row, dtype, which, off, M):
    """Operands the reference's rows accept at any alignment (src/r3d_gemm_fp8a8.hip:985-990,
    1090-1095) are taken, never refused at issue time: A, B or the weight-scale plane at
    1-, 4- or 8-byte offsets, or an A row pitch off 16 bytes, go to the any-alignment arm."""
    if "decode" in row and M > 16:
        pytest.skip("past the decode band")
    N, K = 200, 512
    mk = _mx_ops if dtype == "mxfp4a8" else _f8_ops
    ops, (a, s, b, bs, y) = mk(M=M, N=N, K=K)
    if which == "bs" and dtype == "fp8a8" and off == 1:
        pytest.skip("a bf16 plane on an odd byte: not an element-aligned tensor")
    if which == "a":
        a = _shift(a, off)
    elif which == "b":
        b = _shift(b, off)
    elif which == "bs":
        bs = _shift(bs, off)
    elif which == "pitch":
        a = _shift(a, 0, extra_cols=4)             # row pitch K + 20: off 16 bytes
    ops = R.GemmOperands(a, s, b, bs, y, dtype=dtype, N=N, K=K)
    rc, d = R.describe(row, ops)
    assert rc == R.RAD_OK, (row, which, off, d)
    if which == "bs" and dtype == "fp8a8":
        return                  # bf16 row scales are read by the element: the fast arms
    assert d.startswith("arm=any "), (row, which, off, d)
    g = _geom(d)
    assert g["tm"] == ("1" if M <= 16 else "2") and g["grid"] == "2x%d" % (
        (M + 15) // 16 if M <= 16 else (M + 31) // 32), d


def test_any_alignment_mxfp4a16_and_fused():
    """The bf16-in row: a misaligned bf16 A takes the element-wise quantiser, a misaligned
    weight plane the any-alignment GEMM; the decode rows' fused bf16 producer (no
    counterpart in the reference, whose rows take e4m3 A only) still needs aligned rows."""
    M, N, K = 64, 256, 512
    a = FakeT(_aligned((M, K), np.uint16))
    b = FakeT(_aligned((N, K // 2), np.uint8))
    bs = FakeT(_aligned((N, K // 32), np.uint8))
    y = FakeT(_aligned((M, N), np.uint16))
    need = R.lib().r3d_rad_gemm_nt_q_mxfp4a16_scratch
    for av, bv, quant, arm in [(a, b, "vector", "prefill"), (_shift(a, 2), b, "elementwise", "prefill"),
                               (a, _shift(b, 1), "vector", "any"),
                               (_shift(a, 0, extra_cols=4), _shift(b, 4), "elementwise", "any")]:
        ops = R.GemmOperands(av, None, bv, bs, y, dtype="mxfp4a16", N=N, K=K, M=M)
        sc = FakeT(_aligned((M * K + M * K // 32 + 256,), np.uint8))
        ops.set_scratch(sc, sc.arr.size)
        rc, d = R.describe("gemm_nt_q_mxfp4a16", ops)
        assert rc == R.RAD_OK and d.startswith("arm=%s " % arm), d
        if quant:
            assert _geom(d)["quant"] == quant, d
    for dtype, row in [("mxfp4a8", "gemm_nt_q_mxfp4_decode"), ("fp8a8", "gemm_nt_q_fp8a8_decode")]:
        ops = _xq_ops(dtype, 1, 256, 512)
        ops._t[0].data = ops._t[0].data + 2
        rc, d = R.describe(row, ops)
        assert rc == R.RAD_E_UNSUPPORTED, d


def _set_param(ops, key, val):
    for i in range(ops.args.n_p):
        if ops.args.p[i].key == key.encode():
            ops.args.p[i].ival = val
            return
    raise KeyError(key)


def test_malformed_operands_refused():
    """Operand metadata no engine would send -- a rank past RAD_MAX_RANK, extents whose
    product leaves int64, negative or absurd row pitches, a band row width past int32 --
    is refused with a status instead of being turned into addresses (found by fuzzing the
    plans under the host address and undefined-behaviour sanitizers)."""
    rows = ["gemm_nt_q_mxfp4", "gemm_nt_q_mxfp4_decode", "gemm_nt_q_fp8a8", "gemm_nt_q_fp8a8_decode"]
    for row in rows:
        mk = _mx_ops if "mxfp4" in row else _f8_ops
        ops, keep = mk(M=4, N=256, K=256)
        assert R.describe(row, ops)[0] == R.RAD_OK
        ops._t[0].rank = 9                                  # A: past RAD_MAX_RANK -> absent
        assert R.describe(row, ops)[0] != R.RAD_OK
        ops, keep = mk(M=4, N=256, K=256)
        ops._t[0].shape[0] = 1 << 62                        # numel past int64
        assert R.describe(row, ops)[0] == R.RAD_E_SHAPE
        ops, keep = mk(M=4, N=256, K=256)
        ops._t[0].stride[0] = -(1 << 62)                    # a negative row pitch
        assert R.describe(row, ops)[0] == R.RAD_E_STRIDE
        ops, keep = mk(M=4, N=256, K=256)
        ops._t[4].stride[0] = 1 << 50                       # Y rows past any allocation
        assert R.describe(row, ops)[0] == R.RAD_E_STRIDE
    ops = _gq_ops()
    _set_param(ops, "n", 1 << 62)                           # 2n past int64
    assert R.describe("gated_quant_fp8_act", ops)[0] == R.RAD_E_SHAPE
