"""Writes the golden fixtures in this directory from the CPU oracle (oracle/).

    python tests/golden/make_golden.py

No reference-held vectors exist for this path (radiance's kbench packs live off-repo), so
the fixtures are the oracle's own outputs on small seeded cases that exercise the edges:
NaN (0xFF) and 0x00 E8M0 scales, e4m3 subnormals, ragged N, M across the decode band,
both fp8a8 scale grids.  Each .npz holds inputs and expected outputs (bf16 bits and the
f32 accumulator, plus the magnitude sums the parity bound uses); a_edited marks cases whose
activation codes were overwritten after quant_act_fp8.  numpy.savez_compressed, no pickle.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O                     # noqa: E402
from libr3d_amd import synth          # noqa: E402


def mx_case(name, M, N, K, seed, edges=False):
    rng = np.random.default_rng(seed)
    x = synth.bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    A, AS = O.quant_act_fp8(x, 128)
    B = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    BS = (127 + rng.integers(-8, 1, size=(N, K // 32))).astype(np.uint8)
    if edges:
        A[0, :8] = [0x01, 0x02, 0x03, 0x04, 0x05, 0x06, 0x07, 0x81]   # subnormals
        BS[1, 0] = 0xFF                                               # NaN scale
        BS[2, 1] = 0x00                                               # 2^-127
        B[3, :] = 0                                                   # all-zero row
    Y, Yf, S = O.quant_dot_mxfp4a8(A, AS, B, BS)
    S8 = O.group8_mag("mxfp4a8", A, AS, B, BS)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), dtype="mxfp4a8", x=x, A=A, AS=AS,
                        B=B, BS=BS, Y=Y, Yf=Yf, S=S, S8=S8, rblk=1, a_edited=edges)


def f8_case(name, M, N, K, seed, rblk):
    rng = np.random.default_rng(seed)
    x = synth.bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    A, AS = O.quant_act_fp8(x, 128)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    rows = N if rblk == 1 else (N + 127) // 128
    sc = np.empty((rows, K // 128), np.float32)
    B = np.empty((N, K), np.uint8)
    for r in range(rows):
        blk = W[r * rblk:(r + 1) * rblk] if rblk > 1 else W[r:r + 1]
        for g in range(K // 128):
            amax = float(np.abs(blk[:, g * 128:(g + 1) * 128]).max())
            sc[r, g] = synth.bits_to_f32(synth.bf16_bits(np.array([amax / 448.0], np.float32)))[0]
    BS = synth.bf16_bits(sc)
    for n in range(N):
        srow = n // rblk
        B[n] = O.f32_to_e4m3(W[n] / np.repeat(sc[srow], 128))
    Y, Yf, S = O.quant_dot_fp8a8(A, AS, B, BS, rblk)
    S8 = O.group8_mag("fp8a8", A, AS, B, BS, rblk)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), dtype="fp8a8", x=x, A=A, AS=AS,
                        B=B, BS=BS, Y=Y, Yf=Yf, S=S, S8=S8, rblk=rblk, a_edited=False)


def main():
    mx_case("mxfp4a8_m1_k512_n48_edges", 1, 48, 512, 101, edges=True)
    mx_case("mxfp4a8_m4_k256_n40", 4, 40, 256, 102, edges=True)
    mx_case("mxfp4a8_m16_k384_n33", 16, 33, 384, 103)
    mx_case("mxfp4a8_m24_k256_n130", 24, 130, 256, 104)
    f8_case("fp8a8_m1_k384_n70_row", 1, 70, 384, 201, 1)
    f8_case("fp8a8_m5_k256_n200_block", 5, 200, 256, 202, 128)
    f8_case("fp8a8_m20_k256_n130_row", 20, 130, 256, 203, 1)


if __name__ == "__main__":
    main()
