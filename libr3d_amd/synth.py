"""Seeded synthetic operands for gemm_nt_q (host numpy), shaped like the configs of BASELINE.json.

Weights and activations follow the configs' stated distributions:
  mxfp4a8  e2m1 codes uniform over the 16 codes (two per byte, low nibble = even k),
           E8M0 = 127 + U{-8..0};  activations x ~ bf16(N(0,1)) quantised per (row, 128)
           by quant_act_fp8's rule (scale = amax * (1/448), codes = e4m3(clamp(x/scale))).
  fp8a8    W ~ N(0, 0.02) quantised per output channel: s_n = bf16(amax_n / 448),
           codes e4m3(w / s_n); b_scale the per-row grid [N, K/128] filled with s_n;
           x ~ N(0,1) with one per-token scale replicated over [M, K/128].
The e4m3 encoding here uses torch's float8_e4m3fn conversion (round to nearest even)
after clamping to +-448, which is the saturating encoder for in-range values.
"""
import numpy as np


def _to_e4m3(x_f32):
    import torch
    t = torch.from_numpy(np.clip(np.ascontiguousarray(x_f32, np.float32), -448.0, 448.0))
    return t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def bf16_bits(x_f32):
    """float32 -> bf16 bits, round to nearest even (via torch)."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x_f32, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def bits_to_f32(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def quant_act_groups(x_bf16, group=128):
    """bf16 activations -> (e4m3 codes, f32 scale per (row, group))."""
    x = bits_to_f32(x_bf16)
    M, K = x.shape
    ng = (K + group - 1) // group
    pad = ng * group - K
    xp = np.pad(x, ((0, 0), (0, pad))) if pad else x
    g = xp.reshape(M, ng, group)
    amax = np.max(np.where(np.isnan(g), 0, np.abs(g)), axis=2).astype(np.float32)
    sc = np.where(amax > 0, amax * np.float32(1.0 / 448.0), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / sc).astype(np.float32)
    c = (g * inv[:, :, None]).astype(np.float32).reshape(M, ng * group)[:, :K]
    return _to_e4m3(c), sc


def activations(M, K, seed):
    rng = np.random.default_rng(seed)
    x = bf16_bits(rng.standard_normal((M, K), dtype=np.float32))
    q, sc = quant_act_groups(x, 128)
    return x, q, sc


def mxfp4_weights(N, K, seed, exp_lo=-8, exp_hi=0):
    rng = np.random.default_rng(seed)
    B = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    BS = (127 + rng.integers(exp_lo, exp_hi + 1, size=(N, K // 32))).astype(np.uint8)
    return B, BS


def fp8_weights(N, K, seed, std=0.02):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(std)).astype(np.float32)
    amax = np.max(np.abs(W), axis=1)
    s_bits = bf16_bits(np.where(amax > 0, amax / np.float32(448.0), 1.0).astype(np.float32))
    s = bits_to_f32(s_bits)
    B = _to_e4m3(W / s[:, None])
    BS = np.repeat(s_bits[:, None], K // 128, axis=1)
    return B, BS


def fp8_activations_per_token(M, K, seed):
    """x ~ N(0,1) with ONE scale per token (amax/448 over the row), replicated per group."""
    rng = np.random.default_rng(seed)
    x = bits_to_f32(bf16_bits(rng.standard_normal((M, K), dtype=np.float32)))
    amax = np.max(np.abs(x), axis=1).astype(np.float32)
    sc = np.where(amax > 0, amax * np.float32(1.0 / 448.0), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / sc).astype(np.float32)
    q = _to_e4m3(x * inv[:, None])
    AS = np.repeat(sc[:, None], K // 128, axis=1).astype(np.float32)
    return q, AS


def random_e4m3_codes(shape, rng, nan_free=True):
    c = rng.integers(0, 256, size=shape, dtype=np.uint8)
    if nan_free:
        c = np.where((c & 0x7F) == 0x7F, c & 0xFE, c).astype(np.uint8)
    return c
