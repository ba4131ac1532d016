"""Seeded fuzz of every row's host side on the CPU: describe, the entries (on a machine without a
GPU only, where they stop at the gfx950 gate after the plan) and the scratch hooks, over
operand metadata mutated the ways a broken caller could (ranks, extents, strides, dtypes,
missing tensors, operand counts, integer parameters), and describe over logits blob
headers with mutated bytes.  Every call must return a status; none may crash.  Built with
`-Xarch_host -fsanitize=address,undefined` (and the sanitizer runtime preloaded) the same
loops also check every host read and every integer operation the plans make."""
import ctypes
import random
import struct

import numpy as np
import pytest

import libr3d_amd as R
from tests.test_abi import FakeT, _aligned, _f8_ops, _mx_ops
from tests import test_logits as TL
from tests import logits_util as LU

VALS = [0, 1, 2, 3, 4, 7, 8, 15, 16, 17, 31, 32, 64, 127, 128, 129, 255, 256, 1000, 4096, 5376,
        -1, -128, 1 << 20, 1 << 31, 1 << 40, 1 << 62, -(1 << 62)]
GEMM = ["r3d_rad_gemm_nt_q", "r3d_rad_gemm_nt_q_fp8", "r3d_rad_gemm_nt_q_mxfp4_decode",
        "r3d_rad_gemm_nt_q_fp8_decode", "r3d_rad_gemm_nt_q_mxfp4a16", "r3d_rad_gemm_nt_q_gated_fp8"]
GEMM_ONLY = ["r3d_rad_gemm_nt_q_mxfp4a16_noalloc"]          # entries without a scratch hook
BAND = {"quant": ("r3d_rad_quant_act_fp8", "quant_act_fp8_act"),
        "gated": ("r3d_rad_gated_quant_fp8", "gated_quant_fp8_act"),
        "rms": ("r3d_rad_rmsnorm_quant_fp8", "rmsnorm_quant_fp8"),
        "logits": ("r3d_rad_logits_gemm_e4m3", "logits_gemm_e4m3")}
CODES = set(range(7))


def _fn(name, hook=False):
    f = getattr(R.lib(), name)
    f.argtypes = [ctypes.c_void_p] if hook else [ctypes.c_void_p, ctypes.c_void_p]
    f.restype = ctypes.c_int64 if hook else ctypes.c_int
    return f


def _host(shape, dt):
    return FakeT(_aligned(shape, dt))


def _build(kind, rng, M, n, K, N):
    if kind == "gemm":
        if rng.random() < 0.5:
            return _mx_ops(M=M, N=N, K=K, dtype=rng.choice(["mxfp4a8", "mxfp4a16"]))
        return _f8_ops(M=M, N=N, K=K)
    if kind == "quant":
        keep = (_host((M, n), np.uint16), _host((M, n), np.uint8),
                _host((M, (n + 127) // 128), np.float32))
        return R.QuantActOperands(*keep, n=n, group=128, M=M, x_dtype="BF16"), keep
    if kind == "gated":
        keep = (_host((M, 2 * n), np.uint16), _host((M, n), np.uint8),
                _host((M, (n + 127) // 128), np.float32))
        return R.GatedQuantOperands(*keep, n=n, M=M), keep
    if kind == "rms":
        keep = (_host((M, n), np.uint16), _host((M, n), np.uint16), _host((n,), np.uint16),
                _host((M, n), np.uint8), _host((M, (n + 127) // 128), np.float32),
                _host((M, n), np.uint16))
        return R.RmsNormQuantOperands(*keep, n=n, M=M), keep
    return TL._ops(M=M, N=N, K=K)


def _mutate(args, rng):
    for _ in range(rng.randint(0, 4)):
        if args.n_t <= 0:
            return
        t = args.t[rng.randrange(args.n_t)]
        f = rng.choice(["rank", "shape", "stride", "dtype", "null", "param", "nt"])
        if f == "rank":
            t.rank = rng.choice([0, 1, 2, 3, 4, 8, 9, 100, 0xFFFFFFFF])
        elif f == "shape":
            t.shape[rng.randrange(8)] = rng.choice(VALS)
        elif f == "stride":
            t.stride[rng.randrange(8)] = rng.choice(VALS)
        elif f == "dtype":
            t.dtype = rng.choice(list(range(17)) + [0xFFFF])
        elif f == "null":
            t.data = None
        elif f == "nt":
            args.n_t = rng.choice([0, 1, args.n_t])
        elif args.n_p > 0:
            p = args.p[rng.randrange(args.n_p)]
            if p.kind == R.RAD_P_INT:
                p.ival = rng.choice(VALS)


def _no_gpu():
    """The entries run only where no GPU is present: there they stop at the gfx950 gate,
    while on a GPU a plan that accepts these host buffers would launch on them."""
    import torch
    return not torch.cuda.is_available()


@pytest.mark.parametrize("seed", [1, 2])
def test_plans_survive_mutated_operands(seed):
    rng = random.Random(seed)
    call_entries = _no_gpu()
    buf = ctypes.create_string_buffer(512)
    gemm_rows = [r["name"] for r in R.rows() if "gemm_nt_q" in r["name"]]
    ents = [_fn(n) for n in GEMM + GEMM_ONLY]
    hooks = [_fn(n + "_scratch", hook=True) for n in GEMM]
    band = {k: _fn(v[0]) for k, v in BAND.items()}
    for _ in range(600):
        kind = rng.choice(["gemm", "quant", "gated", "rms", "logits"])
        ops, keep = _build(kind, rng, rng.choice([1, 2, 4, 5, 16, 17, 64]),
                           rng.choice([4, 128, 130, 256, 1000]), rng.choice([128, 256, 384]),
                           rng.choice([1, 16, 17, 130, 256]))
        _mutate(ops.args, rng)
        a = ctypes.byref(ops.args)
        if kind == "gemm":
            for name in gemm_rows:
                assert R.lib().r3d_gfx950_describe(name.encode(), a, buf, 512) in CODES
            for f in ents if call_entries else []:
                assert f(a, None) in CODES
            for h in hooks:
                assert h(a) >= 0
        else:
            assert R.lib().r3d_gfx950_describe(BAND[kind][1].encode(), a, buf, 512) in CODES
            if call_entries:
                assert band[kind](a, None) in CODES


@pytest.mark.parametrize("seed", [1, 2])
def test_logits_plan_survives_mutated_headers(seed):
    rng = random.Random(seed)
    buf = ctypes.create_string_buffer(512)
    for _ in range(800):
        N, K = rng.choice([(10, 256), (1000, 5376), (300, 132)])
        h = LU.header(N, K, rng.choice(["bf16", "f16", "f32"]), rng.choice([1, 128]))
        hb = bytearray(h.tobytes()) + bytearray(4096)
        for _ in range(rng.randint(1, 6)):
            pos = rng.randrange(0, 32 + 72 * 2)
            if rng.random() < 0.5:
                hb[pos] = rng.randrange(256)
            else:
                w = rng.choice([4, 8])
                v = rng.choice([0, 1, 2, 0x7FFFFFFF, 0xFFFFFFFF, 1 << 31, 1 << 62, (1 << 63) - 1,
                                1 << 63, rng.randrange(1 << 32)])
                hb[pos:pos + w] = (v & ((1 << (8 * w)) - 1)).to_bytes(w, "little")
        ops, keep = TL._ops(M=rng.choice([1, 4]), N=N, K=K,
                            h=np.frombuffer(bytes(hb), np.uint8).copy())
        assert R.lib().r3d_gfx950_describe(b"logits_gemm_e4m3", ctypes.byref(ops.args),
                                           buf, 512) in CODES
