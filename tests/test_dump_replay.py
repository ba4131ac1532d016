"""The R3D_DUMP replay checker (tests/replay_dump.py) on the CPU: captures written here in
the library's format (r3d_dump.cpp) with the oracle's own outputs as the post state must
replay EXACT, and the same captures with one output byte changed must replay DIVERGENT --
so the checker reads the format, rebuilds strided views and compares what it should."""
import os

import numpy as np
import pytest

import oracle as O
from libr3d_amd import synth
from tests import replay_dump as RD

DT = RD.DT


def write_capture(d, row, params, tensors, pre, post, scratch=None, rc=0):
    """tensors: [(dtype name, shape, stride) or None]; pre/post: per-operand byte arrays
    (+ the scratch span last when scratch = (bytes, captured))."""
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "manifest.tsv"), "w") as f:
        f.write("H\t%s\t%d\t%d\t%d\n" % (row, rc, len(tensors), len(params)))
        for k, v in params:
            if isinstance(v, str):
                f.write("P\t1\t%s\t0\t0\t%s\t0\n" % (k, v))
            elif isinstance(v, float):
                f.write("P\t2\t%s\t0\t0\t-\t%.17g\n" % (k, v))
            else:
                f.write("P\t0\t%s\t%d\t0\t-\t0\n" % (k, v))
        for i, t in enumerate(tensors):
            if t is None:
                f.write("T\t%d\t0\t0\t0\t0\t1\t0x0\n" % i)
                continue
            name, shape, stride = t
            f.write("T\t%d\t%d\t%d\t%s\t%s\t%d\t0\t0\t0x1000\n" % (
                i, DT[name], len(shape), "\t".join(map(str, shape)), "\t".join(map(str, stride)),
                pre[i].size))
        if scratch:
            f.write("X\t%d\t%d\t0\n" % scratch)
    for name, spans in (("pre.bin", pre), ("post.bin", post)):
        with open(os.path.join(d, name), "wb") as g:
            for s in spans:
                if s is not None:
                    g.write(np.ascontiguousarray(s).view(np.uint8).tobytes())


def b(x):
    return np.ascontiguousarray(x).view(np.uint8).reshape(-1)


def _flip(x):
    y = b(x).copy()
    y[0] ^= 0x01
    return y


def test_quant_act_capture_replays_exact(tmp_path):
    rng = np.random.default_rng(1)
    rows, n, g = 3, 256, 128
    x = synth.bf16_bits(rng.standard_normal((rows, n)).astype(np.float32))
    q, sc = O.quant_act_fp8(x, g)
    ten = [("BF16", [rows, n], [n, 1]), ("F8E4M3", [rows, n], [n, 1]), ("F32", [rows, 2], [2, 1])]
    pre = [b(x), np.zeros(rows * n, np.uint8), np.zeros(rows * 2 * 4, np.uint8)]
    params = [("M", rows), ("n", n), ("group", g), ("dtype", "bf16")]
    write_capture(tmp_path / "0000_quant_act_fp8_act", "quant_act_fp8_act", params, ten, pre,
                  [b(x), b(q), b(sc)])
    write_capture(tmp_path / "0001_quant_act_fp8_act", "quant_act_fp8_act", params, ten, pre,
                  [b(x), _flip(q), b(sc)])
    caps = RD.captures([str(tmp_path)])
    assert [RD.replay_oracle(RD.Capture(c))[0] for c in caps] == [True, False]
    assert RD.main([str(tmp_path / "0000_quant_act_fp8_act")]) == 0
    assert RD.main([str(tmp_path)]) == 1


@pytest.mark.parametrize("pad", [0, 64])
def test_mxfp4_gemm_capture_replays_within_bound(tmp_path, pad):
    """A padded activation view (row pitch K + pad) is rebuilt through its stride."""
    rng = np.random.default_rng(2)
    M, N, K = 2, 40, 256
    _, A, AS = synth.activations(M, K, 3)
    B, BS = synth.mxfp4_weights(N, K, 4)
    Yr, _, _ = O.quant_dot_mxfp4a8(A, AS, B, BS)
    Ap = np.zeros((M, K + pad), np.uint8)
    Ap[:, :K] = A
    a_span = b(Ap)[:(M - 1) * (K + pad) + K]
    ten = [("F8E4M3", [M, K], [K + pad, 1]), ("F32", [M, 2], [2, 1]), ("FP4E2M1", [N, K], [K, 1]),
           ("E8M0", [N, K // 32], [K // 32, 1]), ("BF16", [M, N], [N, 1]), None, None]
    pre = [a_span, b(AS), b(B), b(BS), np.zeros(M * N * 2, np.uint8), None, None]
    params = [("dtype", "mxfp4a8"), ("N", N), ("K", K), ("group", 32)]
    write_capture(tmp_path / "0000_gemm_nt_q_mxfp4_decode", "gemm_nt_q_mxfp4_decode", params, ten,
                  pre, [a_span, b(AS), b(B), b(BS), b(Yr), None, None])
    bad = Yr.copy()
    bad[1, 7] ^= 0x0400                                   # far outside the bound
    write_capture(tmp_path / "0001_gemm_nt_q_mxfp4_decode", "gemm_nt_q_mxfp4_decode", params, ten,
                  pre, [a_span, b(AS), b(B), b(BS), b(bad), None, None])
    res = [RD.replay_oracle(RD.Capture(c)) for c in RD.captures([str(tmp_path)])]
    assert res[0][0] and not res[1][0], res


def test_rmsnorm_capture_with_residual_replays_exact(tmp_path):
    rng = np.random.default_rng(5)
    rows, n = 2, 256
    x = synth.bf16_bits(rng.standard_normal((rows, n)).astype(np.float32))
    r = synth.bf16_bits(rng.standard_normal((rows, n)).astype(np.float32))
    w = rng.standard_normal(n).astype(np.float32)
    q, sc, out, r2 = O.rmsnorm_quant_fp8(x, w, 128, np.float32(1e-6), np.float32(0.0), r)
    ten = [("BF16", [rows, n], [n, 1]), ("BF16", [rows, n], [n, 1]), ("F32", [n], [1]),
           ("F8E4M3", [rows, n], [n, 1]), ("F32", [rows, 2], [2, 1]), ("BF16", [rows, n], [n, 1])]
    pre = [b(x), b(r), b(w), np.zeros(rows * n, np.uint8), np.zeros(rows * 8, np.uint8),
           np.zeros(rows * n * 2, np.uint8)]
    params = [("n", n), ("eps", 1e-6), ("group", 128), ("dtype", "bf16")]
    write_capture(tmp_path / "0000_rmsnorm_quant_fp8", "rmsnorm_quant_fp8", params, ten, pre,
                  [b(x), b(r2), b(w), b(q), b(sc), b(out)])
    ok, msg = RD.replay_oracle(RD.Capture(str(tmp_path / "0000_rmsnorm_quant_fp8")))
    assert ok, msg


@pytest.mark.parametrize("sdt,br", [("bf16", 1), ("f32", 128)])
def test_logits_capture_replays_within_bound(tmp_path, sdt, br):
    """The joined head travels as one U8 operand: the checker takes its planes out of the
    captured blob (tests/logits_util.py's layout), and a logit moved far outside the bound
    replays DIVERGENT."""
    from tests import logits_util as LU
    import libr3d_amd as R
    rng = np.random.default_rng(9)
    M, N, K = 2, 40, 384
    codes, sb = LU.head(N, K, 10, sdt, br)
    blob = R.join_head(codes, sb, sdt, br)
    x = synth.bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    Y, _ = O.logits_e4m3(x, codes, sb, sdt, br)
    ten = [("BF16", [M, K], [K, 1]), ("U8", [blob.size], [1]), ("F32", [M, N], [N, 1])]
    pre = [b(x), blob, np.zeros(M * N * 4, np.uint8)]
    params = [("M", M), ("n_vocab", N), ("n_embd", K), ("dtype", "bf16")]
    write_capture(tmp_path / "0000_logits_gemm_e4m3", "logits_gemm_e4m3", params, ten, pre,
                  [b(x), blob, b(Y)])
    bad = Y.copy()
    bad[1, 3] = bad[1, 3] * 1.01 + 1.0
    write_capture(tmp_path / "0001_logits_gemm_e4m3", "logits_gemm_e4m3", params, ten, pre,
                  [b(x), blob, b(bad)])
    res = [RD.replay_oracle(RD.Capture(c)) for c in RD.captures([str(tmp_path)])]
    assert res[0][0] and not res[1][0], res
