"""GPU parity over a seeded sweep of shapes: every gemm_nt_q row (mxfp4a8 / fp8a8, decode
and tile) at M, N, K drawn log-uniformly -- ragged N and M, K any multiple of 128 --
with and without hook-sized launch scratch and at both fp8a8 scale grids, so the launch
planner's arms (quad, line, 16-row and split-K GEMVs, the skinny band, the prefill tiles
and their splits) meet shapes no hand-picked case names.  Each case is held to the same
bar as tests/test_gpu_gemm.py: status, red zones, every element written, NaN classes, the
per-element bound and the reference's kbench rel_l2 (docs/COVERAGE.md:868,1296).  A
128 x 128 scale grid over fewer than 128 weight rows is refused, as libref refuses it."""
import numpy as np
import pytest

import libr3d_amd as R

from tests.test_gpu_gemm import F8_DEC, F8_TILE, MX_DEC, MX_TILE, _check, _f8_case, _mx_case

pytestmark = pytest.mark.gpu


def _draw(n_cases=96, seed=20261202):
    rng = np.random.default_rng(seed)
    rows = [(MX_DEC, "mxfp4a8"), (F8_DEC, "fp8a8"), (MX_TILE, "mxfp4a8"), (F8_TILE, "fp8a8")]
    cases = []
    for i in range(n_cases):
        row, dtype = rows[i % 4]
        dec = row in (MX_DEC, F8_DEC)
        M = int(rng.integers(1, 17)) if dec else int(np.exp(rng.uniform(0, np.log(2100))))
        N = max(1, int(np.exp(rng.uniform(0, np.log(24000)))))
        K = 128 * int(rng.integers(1, 161))
        while M * N * K > 2_000_000_000:                  # keep the oracle to seconds
            if K > 128:
                K = max(128, K // 256 * 128)
            elif M > 1:
                M //= 2
            else:
                N //= 2
        scratch = "hook" if (i // 4) % 2 == 0 else None
        rblk = 128 if dtype == "fp8a8" and (i // 8) % 2 else 1
        cases.append((row, dtype, M, N, K, scratch, rblk))
    return cases


CASES = _draw()


@pytest.mark.parametrize("row,dtype,M,N,K,scratch,rblk", CASES,
                         ids=["%s-M%d-N%d-K%d-%s-r%d" % (r.replace("gemm_nt_q_", ""), m, n, k,
                                                         s or "noscratch", b)
                              for r, _, m, n, k, s, b in CASES])
def test_shape_sweep(gpu, row, dtype, M, N, K, scratch, rblk):
    seed = 7 * M + 13 * N + K + rblk
    if dtype == "mxfp4a8":
        A, AS, B, BS = _mx_case(M, N, K, seed)
    else:
        A, AS, B, BS = _f8_case(M, N, K, seed, rblk)
    if rblk == 128 and 1 < N < 128:
        # one scale row over 2..127 weight rows implies a block of N, not 128 (libref
        # grid_block, src/r3d_gemm_mxfp4.hip:71-84): refused, Y untouched.  At N = 1 the
        # one row is the per-row grid, which the same bytes also are.
        from tests import gpu_util as gu
        rc, Y, ok = gu.run_row(row, dtype, A, AS, B, BS, M, N, K, gpu, scratch=scratch)
        assert rc == R.RAD_E_UNSUPPORTED and ok and (Y == gu.Y_SENTINEL).all()
        return
    _check(row, dtype, A, AS, B, BS, M, N, K, gpu, rblk=rblk, scratch=scratch)


@pytest.mark.parametrize("row,dtype,M,N,K", [(MX_TILE, "mxfp4a8", 20, 256, 21504),
                                             (F8_TILE, "fp8a8", 40, 256, 16384),
                                             (MX_DEC, "mxfp4a8", 8, 3200, 21504)])
def test_split_many_chunks(gpu, row, dtype, M, N, K):
    """A narrow N over a long K: one weight tile, so the split cuts K into more than 16
    chunks and the reduce sums its planes over several load batches (in chunk order)."""
    from tests import gpu_util as gu
    seed = M + N + K
    if dtype == "mxfp4a8":
        A, AS, B, BS = _mx_case(M, N, K, seed)
    else:
        A, AS, B, BS = _f8_case(M, N, K, seed, 1)
    kc = gu.hook_bytes(row, dtype, M, N, K) // (M * N * 4)        # the hook sizes kc planes
    assert kc > 16, kc
    _check(row, dtype, A, AS, B, BS, M, N, K, gpu, scratch="hook")
