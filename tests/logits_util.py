"""Shared pieces of the logits_gemm tests: synthetic heads, the joined-planes header as
bytes (rad_planes.h's layout, written independently of the library so the two can be held
against each other), and the exact float64 sum the kernel and the oracle are bounded
against."""
import numpy as np

from libr3d_amd import synth

MAGIC = 0x534E4C50
HDR = 32                                 # magic, n_planes, transform[4], bytes
ENTRY0 = HDR                             # the entries follow the header
ENTRY_BYTES = 72                         # role[16], dtype, kind, block[2], rows, cols, row_bytes, offset
HEADER_BYTES = HDR + 2 * ENTRY_BYTES     # a two-plane blob's header and entries
DT_CODE = {"F32": 0, "BF16": 1, "F16": 2, "F8E4M3": 3, "F8E5M2": 4, "U8": 7}
SDT = {"bf16": "BF16", "f16": "F16", "f32": "F32"}
TILED = 0


def up256(v):
    return (v + 255) // 256 * 256


def header(N, K, sdt="bf16", br=1):
    """The header and entries of an N x K head's blob, written the way the reference's tools
    write a joined blob (tools/bench_skinny.cpp:206-220): header at 0 with magic, n_planes,
    transform[0] and bytes; the entries right after it; the first plane at the header and
    entries rounded up to 256 bytes, the next at its end rounded up (uint8 [HEADER_BYTES])."""
    esz = 4 if sdt == "f32" else 2
    srows, scols = (N + br - 1) // br, (K + 127) // 128
    c_off = up256(HEADER_BYTES)
    s_off = up256(c_off + N * K)
    h = np.zeros(HEADER_BYTES, np.uint8)
    u32 = h[:24].view(np.uint32)
    u32[0], u32[1] = MAGIC, 2
    h[24:32].view(np.int64)[0] = s_off + srows * scols * esz
    for i, (role, dt, blk, rows, cols, rb, off) in enumerate([
            ("codes", DT_CODE["F8E4M3"], (1, 1), N, K, K, c_off),
            ("scale", DT_CODE[SDT[sdt]], (br, 128), srows, scols, scols * esz, s_off)]):
        e = h[ENTRY0 + i * ENTRY_BYTES: ENTRY0 + (i + 1) * ENTRY_BYTES]
        e[:len(role)] = np.frombuffer(role.encode(), np.uint8)
        e[16:24].view(np.uint32)[:] = [dt, TILED]
        e[24:72].view(np.int64)[:] = [blk[0], blk[1], rows, cols, rb, off]
    return h


def set_field(h, field, value, entry=None):
    """Overwrite one header field in place (entry 0 = codes, 1 = scale)."""
    top = {"magic": (0, np.uint32), "n_planes": (4, np.uint32), "transform0": (8, np.uint32),
           "bytes": (24, np.int64)}
    ent = {"dtype": (16, np.uint32), "kind": (20, np.uint32), "block0": (24, np.int64),
           "block1": (32, np.int64), "rows": (40, np.int64), "cols": (48, np.int64),
           "row_bytes": (56, np.int64), "offset": (64, np.int64)}
    if field == "role":
        b = ENTRY0 + entry * ENTRY_BYTES
        h[b:b + 16] = 0
        h[b:b + len(value)] = np.frombuffer(value.encode(), np.uint8)
        return
    off, dt = top[field] if entry is None else ent[field]
    if entry is not None:
        off += ENTRY0 + entry * ENTRY_BYTES
    h[off:off + np.dtype(dt).itemsize].view(dt)[0] = value


def head(N, K, seed, sdt="bf16", br=1, std=0.02):
    """Synthetic lm_head: e4m3 codes of N(0, std) weights quantised per (br rows, 128
    columns) block (amax -> 448), the block scales in `sdt` (bf16 / f16 bits, or f32)."""
    import torch
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * std).astype(np.float32)
    srows, scols = (N + br - 1) // br, (K + 127) // 128
    amax = np.zeros((srows, scols), np.float32)
    for j in range(scols):
        blk = np.abs(w[:, 128 * j:128 * (j + 1)]).max(axis=1)
        pad = np.zeros(srows * br, np.float32)
        pad[:N] = blk
        amax[:, j] = pad.reshape(srows, br).max(axis=1)
    s = np.where(amax > 0, amax / 448.0, 1.0).astype(np.float32)
    if sdt == "bf16":
        sbits = synth.bf16_bits(s)
        sv = (sbits.astype(np.uint32) << 16).view(np.float32)
    elif sdt == "f16":
        sbits = s.astype(np.float16).view(np.uint16)
        sv = sbits.view(np.float16).astype(np.float32)
    else:
        sbits = s
        sv = s
    full = np.repeat(np.repeat(sv, br, axis=0)[:N], 128, axis=1)[:, :K]
    q = torch.from_numpy(np.clip(w / full, -448, 448)).to(torch.float8_e4m3fn)
    codes = q.view(torch.uint8).numpy().copy()
    return codes, sbits


def scale_values(sbits, sdt):
    if sdt == "bf16":
        return (np.asarray(sbits, np.uint16).astype(np.uint32) << 16).view(np.float32)
    if sdt == "f16":
        return np.asarray(sbits, np.uint16).view(np.float16).astype(np.float32)
    return np.asarray(sbits, np.float32)


def e4m3_values(codes):
    import torch
    return torch.from_numpy(np.ascontiguousarray(codes, np.uint8)).view(
        torch.float8_e4m3fn).float().numpy()


def exact(x_bits, codes, sbits, sdt, br):
    """float64 y = sum_k x * (code * s) with code * s rounded to f32 first (the product the
    reference forms; exact for bf16 / f16 scales), and the magnitude sum, in float64."""
    x = (np.asarray(x_bits, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    N, K = codes.shape
    sv = scale_values(sbits, sdt)
    full = np.repeat(np.repeat(sv, br, axis=0)[:N], 128, axis=1)[:, :K]
    w = (e4m3_values(codes) * full).astype(np.float32).astype(np.float64)
    return x @ w.T, np.abs(x) @ np.abs(w).T
