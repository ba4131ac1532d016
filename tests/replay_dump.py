"""Offline replay of R3D_DUMP captures (libr3d_amd/csrc/r3d_dump.cpp): the counterpart of
the reference's tools/replay_dump.cpp, checked against this repository's CPU oracle.

    python tests/replay_dump.py <capture dir or a directory of them>... [--device]

Each capture (<seq>_<row>/manifest.tsv, pre.bin, post.bin) is rebuilt into host arrays
through the recorded shapes and strides, the oracle computes the row's outputs from the
PRE state, and those are compared with the POST state the GPU wrote:
  quant_act_fp8 / gated_quant_fp8 / rmsnorm_quant_fp8   bit for bit (NaN as a class)
  gemm_nt_q (mxfp4a8, fp8a8, bf16-in decode, mxfp4a16)   within the GEMM parity bound
      |y - y_oracle| <= ulp_bf16 + 2K 2^-24 S + 2^-10 S8, NaN classes equal; the
      mxfp4a16 row's quantised activations in the scratch bit for bit
  gemm_nt_q_gated (fp8a8)                                the gate_up plane in the scratch
      within the GEMM bound, the codes, scales and gated output bit for bit from it
  logits_gemm_e4m3                                       the planes out of the captured
      joined head, the logits within the row's bound (its MFMA sums and the oracle's
      f32 chain: (140 + 2 ceil(K/256) + K) 2^-24 S), NaN classes equal
--device re-launches each capture through libr3d_gfx950.so on a GPU instead (operands
rebuilt from PRE at the same offsets, the same parameters, tunables and scratch size) and
requires the outputs to equal POST byte for byte: the kernels are deterministic.

Test infrastructure: it loads the oracle as the checker, never the product.  Exit status
0 when every capture agrees.
"""
import argparse
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

DT_NAMES = ["F32", "BF16", "F16", "F8E4M3", "F8E5M2", "FP4E2M1", "E8M0", "U8", "I8", "I16",
            "I32", "U32", "I64", "BOOL"]
DT = {n: i for i, n in enumerate(DT_NAMES)}
ESZ = {DT["F32"]: 4, DT["I32"]: 4, DT["U32"]: 4, DT["I64"]: 8, DT["BF16"]: 2, DT["F16"]: 2,
       DT["I16"]: 2}
NP = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}


class Capture:
    def __init__(self, d):
        self.dir = d
        self.params, self.tensors, self.tunables = {}, [], []
        self.scratch = None                      # (scratch_bytes, captured, truncated)
        for line in open(os.path.join(d, "manifest.tsv")):
            f = line.rstrip("\n").split("\t")
            if f[0] == "H":
                self.row, self.rc, self.n_t, self.n_p = f[1], int(f[2]), int(f[3]), int(f[4])
            elif f[0] == "P":
                kind, key = int(f[1]), f[2]
                self.params[key] = (kind, int(f[3]), int(f[4]), None if f[5] == "-" else f[5],
                                    float(f[6]))
            elif f[0] == "T":
                dt, rank = int(f[2]), int(f[3])
                shape = [int(x) for x in f[4:4 + rank]]
                stride = [int(x) for x in f[4 + rank:4 + 2 * rank]]
                nb, trunc, null = int(f[4 + 2 * rank]), int(f[5 + 2 * rank]), int(f[6 + 2 * rank])
                self.tensors.append(dict(dt=dt, rank=rank, shape=shape, stride=stride, bytes=nb,
                                         trunc=trunc, null=null))
            elif f[0] == "V":
                self.tunables.append((f[1], int(f[2])))
            elif f[0] == "X":
                self.scratch = (int(f[1]), int(f[2]), int(f[3]))
        self.pre = self._spans("pre.bin")
        self.post = self._spans("post.bin") if self.rc == 0 else None

    def _spans(self, name):
        raw = np.fromfile(os.path.join(self.dir, name), np.uint8)
        out, off = [], 0
        for t in self.tensors:
            out.append(raw[off:off + t["bytes"]])
            off += t["bytes"]
        if self.scratch:
            out.append(raw[off:off + self.scratch[1]])
            off += self.scratch[1]
        assert off == raw.size, "%s: %d bytes, manifest says %d" % (name, raw.size, off)
        return out

    def geti(self, key, default=None):
        p = self.params.get(key)
        return p[1] if p and p[0] == 0 else default

    def gets(self, key, default=None):
        p = self.params.get(key)
        return p[3] if p and p[0] == 1 else default

    def getf(self, key, default=None):
        p = self.params.get(key)
        return p[4] if p and p[0] == 2 else default

    def present(self, i):
        return i < len(self.tensors) and not self.tensors[i]["null"]

    def truncated(self):
        return any(t["trunc"] for t in self.tensors) or (self.scratch and self.scratch[2])


def row_stride(t, cols):
    """libref's row_stride (src/r3d_gemm_mxfp4.hip:86-95), in elements."""
    if t["rank"] < 2:
        return cols
    span = 1
    for i in range(t["rank"] - 1, -1, -1):
        span *= t["shape"][i]
        if span == cols:
            return t["stride"][i - 1] if i > 0 else cols
        if span > cols:
            break
    return t["stride"][t["rank"] - 2]


def band_pitch(t, cols):
    """The band rows' operand walk (src/r3d_band.hip:419-449), in elements."""
    if t["rank"] == 1:
        return 0
    if t["rank"] == 2:
        return t["stride"][0] if t["shape"][1] == cols else cols
    return cols


def rows_of(span, t, rows, cols, pitch, esz=None):
    """[rows, cols] elements of a span whose rows start `pitch` elements apart (unit inner
    stride); FP4 spans are read as packed bytes [rows, cols / 2]."""
    if t["dt"] == DT["FP4E2M1"]:
        b = np.asarray(span, np.uint8)
        return np.stack([b[(r * pitch) // 2:(r * pitch) // 2 + cols // 2] for r in range(rows)])
    e = esz or ESZ.get(t["dt"], 1)
    v = np.asarray(span, np.uint8).view(NP[e])
    return np.stack([v[r * pitch:r * pitch + cols] for r in range(rows)]).copy()


def f32(a):
    return np.asarray(a).view(np.float32)


def numel(t):
    n = 1
    for s in t["shape"]:
        n *= s
    return n


# ------------------------------------------------------------------ oracle checks
def check_gemm(c, O, gu):
    dtype = c.gets("dtype")
    N, K = c.geti("N"), c.geti("K")
    tY = c.tensors[4]
    M = numel(tY) // N
    A_t = c.tensors[0]
    ypitch = row_stride(tY, N)
    Y = rows_of(c.post[4], tY, M, N, ypitch, 2)
    notes = []
    if dtype == "mxfp4a16":
        X = rows_of(c.pre[0], A_t, M, K, row_stride(A_t, K), 2)
        Q, SX = O.quant_act_mxfp8(X)
        if c.scratch:
            sc = np.asarray(c.post[-1], np.uint8)
            qb = ((M * K + 255) // 256) * 256
            if not (np.array_equal(sc[:M * K].reshape(M, K), Q) and
                    np.array_equal(sc[qb:qb + M * (K // 32)].reshape(M, K // 32), SX)):
                return False, "quantised activations in the scratch differ from the oracle's"
            notes.append("scratch codes and scales bit-exact")
        B = rows_of(c.pre[2], c.tensors[2], N, K, row_stride(c.tensors[2], K))
        BS = rows_of(c.pre[3], c.tensors[3], N, K // 32, row_stride(c.tensors[3], K // 32))
        Yr, Yf, S = O.dot_mx8_mxfp4(Q, SX, B, BS, nthreads=8)
        S8 = O.group8_mag("mxfp4a16", Q, SX, B, BS, nthreads=8)
    else:
        mx = dtype == "mxfp4a8"
        if c.present(1):
            A = rows_of(c.pre[0], A_t, M, K, row_stride(A_t, K), 1)
            AS = f32(rows_of(c.pre[1], c.tensors[1], M, K // 128,
                             row_stride(c.tensors[1], K // 128), 4))
        else:                                        # the decode rows' fused producer
            X = rows_of(c.pre[0], A_t, M, K, row_stride(A_t, K), 2)
            A, AS = O.quant_act_fp8(X, 128)
            notes.append("bf16 activations quantised by the oracle's quant_act_fp8")
        B = rows_of(c.pre[2], c.tensors[2], N, K if mx else K, row_stride(c.tensors[2], K), 1)
        tBS = c.tensors[3]
        if mx:
            BS = rows_of(c.pre[3], tBS, N, K // 32, row_stride(tBS, K // 32), 1)
            Yr, Yf, S = O.quant_dot_mxfp4a8(A, AS, B, BS, nthreads=8)
            S8 = O.group8_mag("mxfp4a8", A, AS, B, BS, nthreads=8)
        else:
            srows = tBS["shape"][0]
            rblk = 1 if srows >= N else 128
            BS = rows_of(c.pre[3], tBS, srows, K // 128, row_stride(tBS, K // 128), 2)
            Yr, Yf, S = O.quant_dot_fp8a8(A, AS, B, BS, rblk, nthreads=8)
            S8 = O.group8_mag("fp8a8", A, AS, B, BS, rblk, nthreads=8)
    cmp = gu.compare(Y, Yr, Yf, S, K, S8)
    ok = cmp["max_viol"] <= 1.0 and cmp["nan_mismatch"] == 0 and cmp["inf_mismatch"] == 0
    notes.append("M=%d N=%d K=%d bound use %.3f, rel_l2 %.2e" % (M, N, K, cmp["max_viol"],
                                                                 cmp["rel_l2"]))
    return ok, "; ".join(notes)


def _eq_codes(a, b):
    """e4m3 codes equal, NaN codes (S1111111) as a class"""
    a, b = np.asarray(a, np.uint8), np.asarray(b, np.uint8)
    nan = ((a & 0x7F) == 0x7F) & ((b & 0x7F) == 0x7F)
    return bool(np.all((a == b) | nan))


def _eq_f32(a, b):
    a, b = f32(np.ascontiguousarray(a)), f32(np.ascontiguousarray(b))
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


def _eq_bf16(a, b):
    a, b = np.asarray(a, np.uint16), np.asarray(b, np.uint16)
    nan = ((a & 0x7FFF) > 0x7F80) & ((b & 0x7FFF) > 0x7F80)
    return bool(np.all((a == b) | nan))


def check_quant(c, O):
    tx, tq, ts = c.tensors[0], c.tensors[1], c.tensors[2]
    n = c.geti("n", tx["shape"][1] if tx["rank"] >= 2 else 0)
    rows = numel(tx) // n
    g = c.geti("group", n)
    g = n if (g is None or g <= 0 or g > n) else g
    ng = (n + g - 1) // g
    bf = tx["dt"] == DT["BF16"]
    X = rows_of(c.pre[0], tx, rows, n, band_pitch(tx, n), 2 if bf else 4)
    if not bf:
        X = f32(X)
    q, sc = O.quant_act_fp8(X, g)
    Q = rows_of(c.post[1], tq, rows, n, band_pitch(tq, n), 1)
    S = rows_of(c.post[2], ts, rows, ng, band_pitch(ts, ng), 4)
    ok = _eq_codes(Q, q) and _eq_f32(S, sc)
    return ok, "rows=%d n=%d group=%d codes and scales %s" % (rows, n, g, "bit-exact" if ok else "DIFFER")


def check_gated_plane(c, O, GU, n, g, act, q_i, s_i, o_i, rows):
    ng = (n + g - 1) // g
    q, sc, out = O.gated_quant_fp8(GU, n, g, act)
    tq, ts = c.tensors[q_i], c.tensors[s_i]
    ok = _eq_codes(rows_of(c.post[q_i], tq, rows, n, band_pitch(tq, n), 1), q)
    ok = ok and _eq_f32(rows_of(c.post[s_i], ts, rows, ng, band_pitch(ts, ng), 4), sc)
    if o_i is not None and c.present(o_i):
        to = c.tensors[o_i]
        got = rows_of(c.post[o_i], to, rows, n, band_pitch(to, n), 2 if to["dt"] == DT["BF16"] else 4)
        if to["dt"] == DT["BF16"]:
            ok = ok and _eq_bf16(got, out)
        else:
            ok = ok and _eq_f32(got, (out.astype(np.uint32) << 16).view(np.float32))
    return ok


def check_gated(c, O):
    tg = c.tensors[0]
    n = c.geti("n", tg["shape"][1] // 2 if tg["rank"] >= 2 else 0)
    rows = numel(tg) // (2 * n)
    g = c.geti("group", n)
    g = n if (g is None or g <= 0 or g > n) else g
    bf = tg["dt"] == DT["BF16"]
    GU = rows_of(c.pre[0], tg, rows, 2 * n, band_pitch(tg, 2 * n), 2 if bf else 4)
    if not bf:
        GU = f32(GU)
    act = "sigmoid" if c.gets("act") == "sigmoid" else "silu"
    ok = check_gated_plane(c, O, GU, n, g, act, 1, 2, 3, rows)
    return ok, "rows=%d n=%d group=%d act=%s outputs %s" % (rows, n, g, act, "bit-exact" if ok else "DIFFER")


def check_rms(c, O):
    tx, tw = c.tensors[0], c.tensors[2]
    n = c.geti("n", tw["shape"][-1])
    rows = numel(tx) // n
    g = c.geti("group", 0)
    g = n if (g is None or g <= 0 or g > n) else g
    ng = (n + g - 1) // g
    X = rows_of(c.pre[0], tx, rows, n, band_pitch(tx, n), 2)
    wbf = tw["dt"] == DT["BF16"]
    W = np.asarray(c.pre[2], np.uint8).view(np.uint16 if wbf else np.float32)[:n]
    res = None
    if c.present(1):
        res = rows_of(c.pre[1], c.tensors[1], rows, n, band_pitch(c.tensors[1], n), 2)
    q, sc, out, res2 = O.rmsnorm_quant_fp8(X, W, g, np.float32(c.getf("eps", 1e-6)),
                                           np.float32(c.getf("wadd", 0.0)), res)
    tq, ts = c.tensors[3], c.tensors[4]
    ok = _eq_codes(rows_of(c.post[3], tq, rows, n, band_pitch(tq, n), 1), q)
    ok = ok and _eq_f32(rows_of(c.post[4], ts, rows, ng, band_pitch(ts, ng), 4), sc)
    if c.present(5):
        to = c.tensors[5]
        got = rows_of(c.post[5], to, rows, n, band_pitch(to, n), 2 if to["dt"] == DT["BF16"] else 4)
        ok = ok and (_eq_bf16(got, out) if to["dt"] == DT["BF16"]
                     else _eq_f32(got, (out.astype(np.uint32) << 16).view(np.float32)))
    if res is not None:
        ok = ok and _eq_bf16(rows_of(c.post[1], c.tensors[1], rows, n, band_pitch(c.tensors[1], n), 2), res2)
    return ok, "rows=%d n=%d group=%d outputs %s" % (rows, n, g, "bit-exact" if ok else "DIFFER")


def check_gemm_gated(c, O, gu):
    N, K = c.geti("N"), c.geti("K")
    n = N // 2
    tq = c.tensors[4]
    M = numel(tq) // n
    A = rows_of(c.pre[0], c.tensors[0], M, K, row_stride(c.tensors[0], K), 1)
    AS = f32(rows_of(c.pre[1], c.tensors[1], M, K // 128, row_stride(c.tensors[1], K // 128), 4))
    B = rows_of(c.pre[2], c.tensors[2], N, K, row_stride(c.tensors[2], K), 1)
    tBS = c.tensors[3]
    srows = tBS["shape"][0]
    rblk = 1 if srows >= N else 128
    BS = rows_of(c.pre[3], tBS, srows, K // 128, row_stride(tBS, K // 128), 2)
    plane = np.asarray(c.post[-1], np.uint8)[:M * N * 2].view(np.uint16).reshape(M, N)
    Yr, Yf, S = O.quant_dot_fp8a8(A, AS, B, BS, rblk, nthreads=8)
    S8 = O.group8_mag("fp8a8", A, AS, B, BS, rblk, nthreads=8)
    cmp = gu.compare(plane, Yr, Yf, S, K, S8)
    ok = cmp["max_viol"] <= 1.0 and cmp["nan_mismatch"] == 0
    g = c.geti("group", n)
    g = n if (g is None or g <= 0 or g > n) else g
    act = "sigmoid" if c.gets("act") == "sigmoid" else "silu"
    ok2 = check_gated_plane(c, O, plane, n, g, act, 4, 5, 6, M)
    return ok and ok2, "M=%d N=%d K=%d plane bound use %.3f; gated outputs from it %s" % (
        M, N, K, cmp["max_viol"], "bit-exact" if ok2 else "DIFFER")


def head_planes(blob):
    """(codes [N, K] uint8, scale grid (uint16 bits or float32), scale dtype name, rows per
    scale row) out of a joined head (include/rad_planes.h's layout)."""
    b = np.asarray(blob, np.uint8)
    u32 = b[:24].view(np.uint32)        # magic, n_planes, transform[4]; then bytes (i64)
    if u32[0] != 0x534E4C50 or not 1 <= u32[1] <= 4:
        raise ValueError("no joined-planes header")
    ents = {}
    for i in range(int(u32[1])):        # the entries follow the 32-byte header
        e = b[32 + 72 * i: 32 + 72 * (i + 1)]
        role = bytes(e[:16]).split(b"\0")[0].decode()
        dt = int(e[16:20].view(np.uint32)[0])
        blk0, blk1, rows, cols, rb, off = (int(v) for v in e[24:72].view(np.int64))
        ents[role] = (dt, blk0, rows, cols, rb, off)
    dt, _, rows, cols, rb, off = ents["codes"]
    codes = b[off:off + rows * rb].reshape(rows, rb)[:, :cols].copy()
    dt, br, srows, scols, rb, off = ents["scale"]
    sdt = {DT["BF16"]: "bf16", DT["F16"]: "f16", DT["F32"]: "f32"}[dt]
    e = 4 if sdt == "f32" else 2
    grid = b[off:off + srows * rb].view(np.float32 if e == 4 else np.uint16).reshape(srows, rb // e)
    return codes, grid[:, :scols].copy(), sdt, br


def check_logits(c, O):
    N, K = c.geti("n_vocab"), c.geti("n_embd")
    tx, ty = c.tensors[0], c.tensors[2]
    M = numel(ty) // N
    X = rows_of(c.pre[0], tx, M, K, row_stride(tx, K), 2)
    codes, grid, sdt, br = head_planes(c.pre[1])
    Y = f32(rows_of(c.post[2], ty, M, N, row_stride(ty, N), 4)).astype(np.float64)
    Yo, S = O.logits_e4m3(X, codes, grid, sdt, br, nthreads=8)
    nan = np.isnan(Yo)
    if not np.array_equal(np.isnan(Y), nan):
        return False, "NaN pattern differs"
    bound = (140 + 2 * ((K + 255) // 256) + K) * 2.0 ** -24 * S.astype(np.float64) + 2.0 ** -126
    viol = (np.abs(Y - Yo) / bound)[~nan]
    use = float(viol.max()) if viol.size else 0.0
    return use <= 1.0, "M=%d N=%d K=%d %s scales, %d rows a scale row; bound use %.3f" % (
        M, N, K, sdt, br, use)


def replay_oracle(c):
    import oracle as O
    from tests import gpu_util as gu       # the comparison helpers (numpy only here)
    if c.row.startswith("gemm_nt_q_gated"):
        return check_gemm_gated(c, O, gu)
    if c.row.startswith("gemm_nt_q"):
        return check_gemm(c, O, gu)
    if c.row.startswith("quant_act_fp8"):
        return check_quant(c, O)
    if c.row.startswith("gated_quant_fp8"):
        return check_gated(c, O)
    if c.row.startswith("rmsnorm_quant_fp8"):
        return check_rms(c, O)
    if c.row.startswith("logits_gemm"):
        return check_logits(c, O)
    return False, "no oracle for row %s" % c.row


def replay_device(c):
    """Re-launch the capture through the library on cuda:0; outputs must equal POST."""
    import ctypes
    import torch
    import libr3d_amd as R
    dev = torch.device("cuda:0")
    bufs, t = [], (R.RadTensor * len(c.tensors))()
    for i, (tt, span) in enumerate(zip(c.tensors, c.pre)):
        if tt["null"]:
            t[i].data, t[i].rank = None, 0
            bufs.append(None)
            continue
        b = torch.from_numpy(np.ascontiguousarray(span)).to(dev)
        bufs.append(b)
        t[i].data, t[i].dtype, t[i].rank = b.data_ptr(), tt["dt"], tt["rank"]
        for r in range(tt["rank"]):
            t[i].shape[r], t[i].stride[r] = tt["shape"][r], tt["stride"][r]
    keep, p = [], (R.RadParam * max(1, len(c.params)))()
    for i, (k, (kind, iv, ih, sv, dv)) in enumerate(c.params.items()):
        kb = k.encode()
        keep.append(kb)
        p[i].kind, p[i].key, p[i].ival, p[i].ihi, p[i].dval = kind, kb, iv, ih, dv
        if sv is not None:
            vb = sv.encode()
            keep.append(vb)
            p[i].sval = vb
    tv = (R.RadTunableValue * max(1, len(c.tunables)))()
    for i, (k, v) in enumerate(c.tunables):
        kb = k.encode()
        keep.append(kb)
        tv[i].name, tv[i].value = kb, v
    scratch = None
    if c.scratch:
        scratch = torch.from_numpy(np.ascontiguousarray(c.pre[-1])).to(dev) if c.scratch[1] \
            else torch.zeros(c.scratch[0], dtype=torch.uint8, device=dev)
    args = R.RadArgs(ctypes.cast(t, ctypes.POINTER(R.RadTensor)), len(c.tensors),
                     ctypes.cast(p, ctypes.POINTER(R.RadParam)), len(c.params),
                     ctypes.cast(tv, ctypes.POINTER(R.RadTunableValue)), len(c.tunables),
                     scratch.data_ptr() if scratch is not None else None,
                     c.scratch[0] if c.scratch else 0, 0)
    fn = R.row_launcher(c.row)

    class _Ops:
        pass
    ops = _Ops()
    ops.args = args
    rc = fn(ops, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    if c.row.startswith("logits_gemm") and bufs[1] is not None:
        R.forget_head(bufs[1])          # the next capture's head may land at this address
    if rc != c.rc:
        return False, "status %d, the capture recorded %d" % (rc, c.rc)
    if c.post is None:
        return True, "refused again (status %d)" % rc
    diff = [i for i, b in enumerate(bufs)
            if b is not None and not np.array_equal(b.cpu().numpy(), c.post[i])]
    if diff:
        return False, "operands %s differ from the captured post state" % diff
    return True, "every operand byte-identical to the capture"


def captures(paths):
    out = []
    for p in paths:
        if os.path.exists(os.path.join(p, "manifest.tsv")):
            out.append(p)
        elif os.path.isdir(p):
            out += sorted(os.path.join(p, d) for d in os.listdir(p)
                          if os.path.exists(os.path.join(p, d, "manifest.tsv")))
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("paths", nargs="+")
    ap.add_argument("--device", action="store_true", help="re-launch on the GPU instead")
    args = ap.parse_args(argv)
    caps = captures(args.paths)
    bad = 0
    for d in caps:
        c = Capture(d)
        if c.post is None and not args.device:
            print("%s  %s: refused (status %d), nothing to compare" % (os.path.basename(d), c.row, c.rc))
            continue
        if c.truncated() and not args.device:
            print("%s  %s: an operand was cut at R3D_DUMP_CAP, not replayed" % (os.path.basename(d), c.row))
            continue
        ok, msg = replay_device(c) if args.device else replay_oracle(c)
        bad += not ok
        print("%s  %s: %s -- %s" % (os.path.basename(d), c.row, "EXACT" if ok else "DIVERGENT", msg))
    print("%d capture(s), %d divergent" % (len(caps), bad))
    return 1 if bad or not caps else 0


if __name__ == "__main__":
    sys.exit(main())
