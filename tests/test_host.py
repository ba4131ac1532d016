"""Host-side pieces that need no GPU: the bench's one-GPU contract, the build entry, and
the synthetic generators' distributions."""
import os
import subprocess
import sys

import numpy as np

from libr3d_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr or "single" in r.stderr


def test_synth_distributions():
    B, BS = synth.mxfp4_weights(64, 256, 1)
    assert B.shape == (64, 128) and BS.shape == (64, 8)
    assert BS.min() >= 119 and BS.max() <= 127
    nib = np.concatenate([B & 15, B >> 4]).ravel()
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.5 * counts.mean()
    Bf, BSf = synth.fp8_weights(32, 256, 2)
    assert BSf.shape == (32, 2) and (BSf[:, 0] == BSf[:, 1]).all()   # per-channel, replicated
    A, AS = synth.fp8_activations_per_token(3, 256, 3)
    assert (AS[:, 0] == AS[:, 1]).all()
    codes = A.ravel()
    assert ((codes & 0x7F) != 0x7F).all()
