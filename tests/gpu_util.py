"""Helpers for GPU parity tests: guarded device operands, row launches through the C ABI,
and comparison against the oracle."""
import numpy as np
import torch

import libr3d_amd as R
import oracle as O

GUARD = 4096          # red-zone bytes on each side of every operand
GUARD_BYTE = 0xA5
Y_SENTINEL = 0xEEEE


class Guarded:
    """A device tensor embedded in a larger allocation with red zones on both sides."""

    def __init__(self, host, dev, fill=None):
        host = np.ascontiguousarray(host)
        nbytes = host.nbytes
        self.buf = torch.full((GUARD + nbytes + GUARD,), GUARD_BYTE, dtype=torch.uint8, device=dev)
        self.nbytes = nbytes
        view = self.buf[GUARD:GUARD + nbytes]
        if fill is None:
            view.copy_(torch.from_numpy(host.view(np.uint8).reshape(-1)).to(dev))
        else:
            view.fill_(fill)
        tdt = {np.dtype(np.uint8): torch.uint8, np.dtype(np.float32): torch.float32,
               np.dtype(np.uint16): torch.int16}[host.dtype]
        self.t = view.view(tdt).view(host.shape)

    def guards_intact(self):
        lo = self.buf[:GUARD]
        hi = self.buf[GUARD + self.nbytes:]
        return bool((lo == GUARD_BYTE).all().item()) and bool((hi == GUARD_BYTE).all().item())


def y_buffer(M, N, dev):
    host = np.full((M, N), Y_SENTINEL, np.uint16)
    return Guarded(host, dev)


def run_row(row, dtype, A, AS, B, BS, M, N, K, dev, y_shape=None, extra=None, tunables=None,
            scratch=None):
    """Launch `row` on guarded copies of the operands; returns (rc, Y uint16 [M,N], guards_ok).
    scratch: None (no launch scratch), "hook" (the bytes the row's scratch hook asks for) or
    a byte count -- a guarded buffer, poisoned, handed over as RadArgs::scratch."""
    gA, gAS, gB, gBS = (Guarded(x, dev) for x in (A, AS, B, BS))
    gY = y_buffer(M, N, dev)
    ops = R.GemmOperands(gA.t, gAS.t, gB.t, gBS.t, gY.t, dtype=dtype, N=N, K=K,
                         extra_params=extra, y_shape=y_shape, tunables=tunables)
    held = [gA, gAS, gB, gBS, gY]
    if scratch is not None:
        nbytes = R.row_scratch_bytes(row, ops) if scratch == "hook" else int(scratch)
        if nbytes > 0:
            gS = Guarded(np.zeros(nbytes, np.uint8), dev, fill=0x5A)
            ops.set_scratch(gS.t, nbytes)
            held.append(gS)
    stream = torch.cuda.current_stream().cuda_stream
    rc = R.launch_row(row, ops, stream)
    torch.cuda.synchronize()
    Y = gY.t.cpu().numpy().view(np.uint16).reshape(M, N)
    ok = all(g.guards_intact() for g in held)
    return rc, Y, ok


def hook_bytes(row, dtype, M, N, K):
    """The launch scratch `row`'s hook asks for at M x N x K (the hook reads only N, K and
    y's element count, so the other operands are stand-ins)."""
    t = torch.zeros((1, 16), dtype=torch.uint8)
    y = torch.zeros((M, N), dtype=torch.int16)
    ops = R.GemmOperands(t, t, t, t, y, dtype=dtype, N=N, K=K)
    return R.row_scratch_bytes(row, ops)


def record(case, row, shape, c, Y=None, Yref_bits=None):
    """Append one parity record (JSON line) to the file named by R3D_PARITY_LOG, if set:
    the case, the row, the shape, the comparison figures and, given both outputs, the
    fraction of elements whose bf16 bits equal the oracle's."""
    import json
    import os
    path = os.environ.get("R3D_PARITY_LOG")
    if not path:
        return
    rec = {"case": case, "row": row, "shape": shape}
    rec.update({k: c[k] for k in ("rel_l2", "row_rel_l2_max", "max_abs", "max_viol") if k in c})
    for k in ("row_max_abs", "row_rel_l2"):            # per output row, up to 16 rows listed
        v = np.asarray(c.get(k, []), np.float64)
        rec[k] = [float(x) for x in v] if v.size <= 16 else {
            "rows": int(v.size), "max": float(v.max()), "median": float(np.median(v))}
    if Y is not None and Yref_bits is not None:
        y = np.asarray(Y, np.uint16)
        r = np.asarray(Yref_bits, np.uint16)
        both_nan = np.isnan(O.bf16_to_f32(y)) & np.isnan(O.bf16_to_f32(r))
        rec["bits_equal_frac"] = float(np.mean((y == r) | both_nan))
    with open(path, "a") as f:
        f.write(json.dumps(rec) + "\n")


def compare(Y, Yref_bits, Yf, S, K, S8=None):
    """-> dict with max violation ratio of the per-element bound (oracle.error_bound),
    NaN/inf class mismatches, per-output-row (Y[m, :]) rel_l2 max, whole-tensor rel_l2,
    max-abs, and unwritten elements."""
    y = O.bf16_to_f32(Y).astype(np.float64)
    yr = O.bf16_to_f32(Yref_bits).astype(np.float64)
    nan_y, nan_r = np.isnan(y), np.isnan(yr)
    nan_mismatch = int(np.sum(nan_y != nan_r))
    fin = ~(nan_y | nan_r)
    inf_mismatch = int(np.sum((np.isinf(y) != np.isinf(yr)) & fin))
    both_inf = np.isinf(y) & np.isinf(yr) & fin
    inf_sign_mismatch = int(np.sum(np.sign(y[both_inf]) != np.sign(yr[both_inf])))
    ok = fin & ~np.isinf(y) & ~np.isinf(yr)
    # one bf16 ulp at the larger of the two magnitudes (a rounding flip across a binade
    # edge) plus the two f32 summation orders' bound on the magnitude sum
    big = np.maximum(np.abs(np.where(ok, y, 0.0)), np.abs(np.asarray(Yf, np.float64)))
    bound = O.error_bound(big, S, K, S8)
    err = np.abs(y - yr)
    viol = np.where(ok, err / np.maximum(bound, 1e-300), 0.0)
    num = np.sqrt(np.sum(np.where(ok, err, 0.0) ** 2, axis=1))
    den = np.sqrt(np.sum(np.where(ok, yr, 0.0) ** 2, axis=1))
    rel_row = np.where(den > 0, num / np.maximum(den, 1e-300), 0.0)
    tot = float(np.sqrt(np.sum(np.where(ok, err, 0) ** 2)) / max(np.sqrt(np.sum(np.where(ok, yr, 0) ** 2)), 1e-300))
    return {
        "max_viol": float(np.max(viol)) if viol.size else 0.0,
        "nan_mismatch": nan_mismatch,
        "inf_mismatch": inf_mismatch + inf_sign_mismatch,
        "row_rel_l2_max": float(np.max(rel_row)) if rel_row.size else 0.0,
        "rel_l2": tot,
        "max_abs": float(np.max(np.where(ok, err, 0.0))) if err.size else 0.0,
        # per output row (Y[m, :]): max-abs error and rel_l2 of each row
        "row_max_abs": np.max(np.where(ok, err, 0.0), axis=1) if err.size else np.zeros(0),
        "row_rel_l2": rel_row,
        "sentinel_left": int(np.sum((Y == Y_SENTINEL) & (Yref_bits != Y_SENTINEL))),
    }
