"""R3D_DUMP end to end on the GPU: a child process with R3D_DUMP set launches every kind of
row this library registers (decode, prefill, bf16-in decode, mxfp4a16 with its scratch, the
three producers, the gated GEMM, the e4m3 lm_head), each through its row's launch pointer; the library writes
one capture per launch; tests/replay_dump.py then rebuilds each launch from its capture and
(1) checks what the GPU wrote against the oracle, (2) re-launches it on the GPU and requires
byte-identical outputs.  Also: R3D_DUMP_MAX bounds the captures per row, and R3D_DUMP_OPS
selects rows."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

_CHILD = r"""
import sys
sys.path.insert(0, %r)
import numpy as np
import torch
import libr3d_amd as R
from libr3d_amd import synth
from tests.test_gpu_gemm import _mx_case, _f8_case
dev = torch.device("cuda:0")
st = torch.cuda.current_stream().cuda_stream
T = lambda x: torch.from_numpy(np.ascontiguousarray(x.view(np.int16) if x.dtype == np.uint16 else x)).to(dev)
live = []                      # every device tensor stays referenced: the launches hold raw pointers
def gemm(row, dtype, A, AS, B, BS, rows, N, K, **kw):
    t = [T(A), None if AS is None else T(AS), T(B), T(BS), torch.empty((rows, N), dtype=torch.int16, device=dev)]
    live.extend(t)
    ops = R.GemmOperands(*t, dtype=dtype, N=N, K=K, **kw)
    if dtype == "mxfp4a16":
        live.append(torch.empty(R.row_scratch_bytes(row, ops), dtype=torch.uint8, device=dev))
        ops.set_scratch(live[-1])
    assert R.launch_row(row, ops, st) == 0, row
    return ops
keep = []
A, AS, B, BS = _mx_case(3, 200, 640, 1)
keep.append(gemm("gemm_nt_q_mxfp4_decode", "mxfp4a8", A, AS, B, BS, 3, 200, 640))
keep.append(gemm("gemm_nt_q_mxfp4_decode", "mxfp4a8", A[:1], AS[:1], B, BS, 1, 200, 640))
keep.append(gemm("gemm_nt_q_mxfp4_decode", "mxfp4a8", A[:2], AS[:2], B, BS, 2, 200, 640))   # third: past R3D_DUMP_MAX
A, AS, B, BS = _mx_case(130, 300, 384, 2)
keep.append(gemm("gemm_nt_q_mxfp4", "mxfp4a8", A, AS, B, BS, 130, 300, 384))
A, AS, B, BS = _f8_case(70, 260, 512, 3, 128)
keep.append(gemm("gemm_nt_q_fp8a8", "fp8a8", A, AS, B, BS, 70, 260, 512))
X = synth.bf16_bits(np.random.default_rng(4).standard_normal((1, 1024)).astype(np.float32))
B, BS = _f8_case(1, 300, 1024, 5, 1)[2:]
keep.append(gemm("gemm_nt_q_fp8a8_decode", "fp8a8", X, None, B, BS, 1, 300, 1024))
X = synth.bf16_bits(np.random.default_rng(6).standard_normal((150, 256)).astype(np.float32))
B, BS = synth.mxfp4_weights(200, 256, 7)
keep.append(gemm("gemm_nt_q_mxfp4a16", "mxfp4a16", X, None, B, BS, 150, 200, 256, group=32, M=150))
x = T(synth.bf16_bits(np.random.default_rng(8).standard_normal((4, 512)).astype(np.float32)))
q = torch.empty((4, 512), dtype=torch.uint8, device=dev); s = torch.empty((4, 4), dtype=torch.float32, device=dev)
assert R.quant_act_fp8(x, q, s, n=512, group=128, stream=st) == 0
gu = T(synth.bf16_bits(np.random.default_rng(9).standard_normal((2, 512)).astype(np.float32)))
q2 = torch.empty((2, 256), dtype=torch.uint8, device=dev); s2 = torch.empty((2, 2), dtype=torch.float32, device=dev)
o2 = torch.empty((2, 256), dtype=torch.int16, device=dev)
go = R.GatedQuantOperands(gu, q2, s2, o2, n=256, group=128, act="silu", M=2)
assert R.launch_row("gated_quant_fp8_act", go, st) == 0
xr = T(synth.bf16_bits(np.random.default_rng(10).standard_normal((3, 512)).astype(np.float32)))
rr = T(synth.bf16_bits(np.random.default_rng(11).standard_normal((3, 512)).astype(np.float32)))
w = torch.from_numpy(np.random.default_rng(12).standard_normal(512).astype(np.float32)).to(dev)
q3 = torch.empty((3, 512), dtype=torch.uint8, device=dev); s3 = torch.empty((3, 4), dtype=torch.float32, device=dev)
o3 = torch.empty((3, 512), dtype=torch.int16, device=dev)
ro = R.RmsNormQuantOperands(xr, rr, w, q3, s3, o3, n=512, group=128, M=3)
assert R.launch_row("rmsnorm_quant_fp8", ro, st) == 0
A, AS, B, BS = _f8_case(3, 512, 256, 13, 1)
qg = torch.empty((3, 256), dtype=torch.uint8, device=dev); sg = torch.empty((3, 2), dtype=torch.float32, device=dev)
t = [T(A), T(AS), T(B), T(BS)]
live.extend(t)
gg = R.GatedGemmOperands(*t, qg, sg, None, N=512, K=256, act="sigmoid", M=3)
live.append(torch.empty(R.row_scratch_bytes("gemm_nt_q_gated_fp8a8", gg), dtype=torch.uint8, device=dev))
gg.set_scratch(live[-1])
assert R.launch_row("gemm_nt_q_gated_fp8a8", gg, st) == 0
from tests import logits_util as LU
codes, sb = LU.head(300, 640, 14, "bf16", 1)
hb = torch.from_numpy(R.join_head(codes, sb)).to(dev)
xl = T(synth.bf16_bits(np.random.default_rng(15).standard_normal((3, 640)).astype(np.float32)))
yl = torch.empty((3, 300), dtype=torch.float32, device=dev)
live.extend([hb, xl, yl])
assert R.launch_row("logits_gemm_e4m3", R.LogitsOperands(xl, hb, yl, n_vocab=300, n_embd=640), st) == 0
torch.cuda.synchronize()
print("LAUNCHED")
"""

ROWS = {"gemm_nt_q_mxfp4_decode": 2, "gemm_nt_q_mxfp4": 1, "gemm_nt_q_fp8a8": 1,
        "gemm_nt_q_fp8a8_decode": 1, "gemm_nt_q_mxfp4a16": 1, "quant_act_fp8_act": 1,
        "gated_quant_fp8_act": 1, "rmsnorm_quant_fp8": 1, "gemm_nt_q_gated_fp8a8": 1,
        "logits_gemm_e4m3": 1}


def _capture(tmp_path, **env_extra):
    env = dict(os.environ, R3D_DUMP=str(tmp_path), R3D_DUMP_MAX="2", **env_extra)
    p = subprocess.run([sys.executable, "-c", _CHILD % ROOT], env=env, capture_output=True,
                       text=True, timeout=300)
    assert p.returncode == 0 and "LAUNCHED" in p.stdout, p.stdout[-2000:] + p.stderr[-2000:]
    return sorted(os.listdir(tmp_path))


def test_capture_and_replay(gpu, tmp_path):
    caps = _capture(tmp_path)
    got = {}
    for d in caps:
        row = d.split("_", 1)[1]
        got[row] = got.get(row, 0) + 1
    assert got == ROWS, caps                         # R3D_DUMP_MAX = 2 bounds the decode row
    from tests import replay_dump as RD
    for d in caps:
        ok, msg = RD.replay_oracle(RD.Capture(str(tmp_path / d)))
        assert ok, (d, msg)
    p = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "replay_dump.py"),
                        str(tmp_path), "--device"], capture_output=True, text=True, timeout=300)
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-2000:]
    assert "%d capture(s), 0 divergent" % len(caps) in p.stdout, p.stdout[-3000:]


def test_capture_selects_rows(gpu, tmp_path):
    caps = _capture(tmp_path, R3D_DUMP_OPS="quant_act,gated_quant")
    assert sorted(d.split("_", 1)[1] for d in caps) == ["gated_quant_fp8_act", "quant_act_fp8_act"]
