"""Benchmark of the gfx950 gemm_nt_q rows on one MI355X (BASELINE.json's metric).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--quick] [--no-extra] [--no-cpu]

A "step" is one gemm_nt_q launch over one batch.  The headline workload is BASELINE.json's
config 1 -- the fp8a8 W8A8 decode GEMV at M=1, K=5376, N=21504 -- read cold from HBM:
the weight planes rotate over enough copies to exceed 1 GiB, well past the 256 MB
Infinity Cache; each copy is read once (a read-only stream) before the warm-up, as a
serving loop's weights have been.  `value` is algorithmic bytes per step (weights + scales + activations +
output, counted once) times steps over the wall time between two synchronised points.
`roofline.achieved` divides the same bytes by the kernel's average duration measured with
HIP events on the launch stream, from the end of the first timed launch to the end of the
last (the first reaches the idle GPU one host launch path after the timed region opens).
The headline times exactly --steps launches after
exactly --warmup; it runs after the `floors` leg (the stream probe's ceilings and the
launch floor on the same box), which also leaves the GPU at its working clocks.  The other
configs (C0, C2, C3, C4) are reported under `extra`, each timed over at least 30 ms of GPU
time.  The CPU baseline is the C restatement of libref (oracle/) on every host core this
process may use, timed on a bounded sample.  One GPU only: --gpus above 1 exits with a
message.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP8_PEAK_TFLOPS = 5000.0       # dense MFMA fp8 (the rate of an fp8 x fp4 scaled MFMA)
FP4_PEAK_TFLOPS = 10100.0      # dense MFMA fp4 x fp4
ROTATE_BYTES = 1.1 * 2 ** 30
# HBM bytes per launch of the headline kernel from two rocprofv3 --pmc passes over this
# script (--quick), FETCH_SIZE x 2.00 + WRITE_SIZE x 1.00 -- the factors a plain 256 MiB
# device copy reads on the same counters (bench.py --copy-calib).  Re-measured whenever
# the decode kernel changes; profiles/gemv_quad_fp8a8_c1_pmc_traffic.md has the numbers.
HEADLINE_TRAFFIC_BYTES = 117733292


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def mx_bytes(M, N, K):
    """mxfp4a8 algorithmic bytes: nibbles + E8M0 + e4m3 A + f32 a_scale + bf16 Y."""
    return N * K // 2 + N * K // 32 + M * K + M * ((K + 127) // 128) * 4 + M * N * 2


def f8_bytes(M, N, K, rblk=1):
    srows = N if rblk == 1 else (N + 127) // 128
    return N * K + srows * (K // 128) * 2 + M * K + M * ((K + 127) // 128) * 4 + M * N * 2


class Case:
    """Device operands for one gemm_nt_q call, with `copies` rotated weight planes."""

    def __init__(self, dtype, A, AS, B, BS, M, N, K, copies, dev):
        import torch
        import libr3d_amd as R
        self.M, self.N, self.K, self.dtype = M, N, K, dtype
        self.a = torch.from_numpy(A).to(dev)
        self.as_ = torch.from_numpy(AS).to(dev)
        b0 = torch.from_numpy(B).to(dev)
        bs0 = torch.from_numpy(BS.view(np.int16) if BS.dtype == np.uint16 else BS).to(dev)
        self.b = [b0] + [b0.clone() for _ in range(copies - 1)]
        self.bs = [bs0] + [bs0.clone() for _ in range(copies - 1)]
        self.y = torch.empty((M, N), dtype=torch.int16, device=dev)
        self.ops = [R.GemmOperands(self.a, self.as_, b, bs, self.y, dtype=dtype, N=N, K=K)
                    for b, bs in zip(self.b, self.bs)]
        self.scratch = None
        self.sink = torch.zeros(4, dtype=torch.int32, device=dev)
        self.touched = False

    def touch(self, stream):
        """Read every weight copy once (the library's read-only stream probe), so the timed
        launches find the inputs resident as a serving loop's weights are: the first read
        of a freshly written copy runs 25-80 % slower than every later one."""
        if self.touched:
            return
        import libr3d_amd as R
        L = R.lib()
        for t in self.b + self.bs:
            rc = L.r3d_gfx950_stream_probe(ctypes_ptr(t), t.numel() * t.element_size(), 8, 22,
                                           ctypes_ptr(self.sink), ctypes_ptr_stream(stream))
            assert rc == 0, rc
        self.touched = True

    def hook_scratch(self, row):
        """Hand every call the launch scratch `row`'s hook asks for (one buffer: the calls
        run in order on one stream), as an engine's arena would; returns its bytes."""
        import torch
        import libr3d_amd as R
        need = R.row_scratch_bytes(row, self.ops[0])
        if need > 0:
            self.scratch = torch.empty(need, dtype=torch.uint8, device=self.y.device)
            for o in self.ops:
                o.set_scratch(self.scratch, need)
        return need


def copies_for(nbytes):
    return max(1, int(np.ceil(ROTATE_BYTES / nbytes)))


EXTRA_MIN_S = 0.03     # GPU time every non-headline measurement runs for, at least


def time_case(case, row, steps, warmup, stream, min_s=EXTRA_MIN_S):
    """-> (wall seconds for the timed back-to-back launches between two synchronised points,
    average launch duration in seconds from HIP events recorded on the launch stream
    between the same launches -- what rocprofv3's per-kernel average measures plus the
    back-to-back dispatch gaps).
    At least `steps` launches are timed, and (min_s) enough for min_s seconds of GPU time,
    after `warmup` untimed ones; case.last_steps holds the count.  The headline passes
    min_s = None: exactly the --steps / --warmup it was given.
    The timed region starts on an idle GPU, so the first launch reaches the device one host
    launch path (~4-5 us) after an event recorded ahead of it: that wait is host time, not
    the kernel's.  The event pair therefore spans launches 2..n (it opens when the first
    launch ends); case.last_kern_window holds the span from before the first launch over
    all n, for comparison."""
    import torch
    import libr3d_amd as R
    launch = R.row_launcher(row)
    n = len(case.ops)
    if hasattr(case, "touch"):   # rotated weight copies: read each once first
        case.touch(stream)
    ew = torch.cuda.Event(enable_timing=True)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    ew.record()                  # the events' device objects exist before the timed region
    e0.record()
    e1.record()
    for i in range(warmup):
        rc = launch(case.ops[i % n], stream)
        assert rc == 0, "row %s refused: %d" % (row, rc)
    if min_s:
        e0.record()
        for i in range(5):
            launch(case.ops[(warmup + i) % n], stream)
        e1.record()
        torch.cuda.synchronize()
        est = e0.elapsed_time(e1) * 1e-3 / 5
        steps = max(steps, int(np.ceil(min_s / max(est, 1e-7))))
    case.last_steps = steps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ew.record()
    for i in range(steps):
        launch(case.ops[i % n], stream)
        if i == 0 and steps > 1:
            e0.record()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    case.last_kern_window = ew.elapsed_time(e1) * 1e-3 / steps
    kern = e0.elapsed_time(e1) * 1e-3 / (steps - 1) if steps > 1 else case.last_kern_window
    return wall, kern


def time_min(launch, min_s=0.03, warm=10):
    """Average seconds per call of launch(i) for i = 0, 1, ... back to back on the current
    stream (HIP events around the timed calls): `warm` untimed calls, a short probe, then
    enough calls for at least min_s of GPU time -- so clocks and queues are steady whatever
    the kernel's length."""
    import torch
    for i in range(warm):
        launch(i)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(5):
        launch(i)
    e1.record()
    torch.cuda.synchronize()
    n = max(20, int(np.ceil(min_s / max(e0.elapsed_time(e1) * 1e-3 / 5, 1e-7))))
    e0.record()
    for i in range(n):
        launch(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / n, n


FLOOR_SIZES = {          # algorithmic bytes of the decode workloads the floors stand beside
    "c2_qkv_M1": lambda: mx_bytes(1, 8192, 5376),
    "c2_gate_up_M1": lambda: mx_bytes(1, 21504, 5376),
    "c1": lambda: f8_bytes(1, 21504, 5376),
    "lm_head_M4": lambda: f8_bytes(4, 262144, 5376),
    "c1_weight_plane": lambda: 21504 * 5376,
}
# a workload timed at one probe shape only: config 1's weight plane in the GEMV's own grid --
# 768 workgroups of 7 waves, each wave streaming 4 rows x 5376 bytes = 21 KB
FLOOR_ONLY_SHAPE = {"c1_weight_plane": [(21, 7)]}


def bench_floors(dev, stream, min_s=0.03):
    """The ceilings the decode GEMVs are held against, from committed code: at each decode
    workload's byte count, rotated over > 1 GiB like the GEMVs' weights, (a) the library's
    read-only stream probe (r3d_gfx950_stream_probe: 1 KB loads 8 deep, best of the runs a
    wave and waves a workgroup listed), (b) a stock torch kernel that only reads the bytes
    (an int32 sum), and (c) the empty-kernel launch floor at 1 / 1344 / 5376 workgroups."""
    import torch
    import libr3d_amd as R
    L = R.lib()
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    out = {}
    for name, fn in FLOOR_SIZES.items():
        nb = (fn() + 1023) // 1024 * 1024
        bufs = [torch.empty(nb, dtype=torch.uint8, device=dev) for _ in range(copies_for(nb))]
        for b in bufs:
            b.view(torch.int32)[: nb // 4].fill_(0x01020304)
        rec = {"bytes": nb, "copies": len(bufs), "probe": {}}
        best = None
        shapes = FLOOR_ONLY_SHAPE.get(name) or [(kb, wpg) for kb in (16, 22, 32, 64, 128)
                                                for wpg in (4, 8)]
        for kb, wpg in shapes:
            def go(i, kb=kb, wpg=wpg):
                rc = L.r3d_gfx950_stream_probe(ctypes_ptr(bufs[i % len(bufs)]), nb, wpg, kb,
                                               ctypes_ptr(sink), ctypes_ptr_stream(stream))
                assert rc == 0, rc
            t, n = time_min(go, min_s)
            rec["probe"]["%dKBx%d" % (kb, wpg)] = round(t * 1e6, 3)
            if best is None or t < best[0]:
                best = (t, "%d KB a wave, %d waves a workgroup" % (kb, wpg))
        rec["probe_us"] = round(best[0] * 1e6, 3)
        rec["probe_best"] = best[1]
        rec["probe_GBps"] = round(nb / best[0] / 1e9, 1)
        rec["probe_frac_hbm"] = round(nb / best[0] / 1e9 / HBM_PEAK_GBS, 4)
        t, n = time_min(lambda i: torch.sum(bufs[i % len(bufs)].view(torch.int32)), min_s)
        rec["torch_sum_us"] = round(t * 1e6, 3)
        rec["torch_sum_GBps"] = round(nb / t / 1e9, 1)
        out[name] = rec
        log("[bench] floor %s (%d B): probe %.2f us (%.1f%% of HBM, %s), torch sum %.2f us" % (
            name, nb, best[0] * 1e6, 100 * rec["probe_frac_hbm"], best[1], t * 1e6))
        del bufs
        torch.cuda.empty_cache()
    empty = {}
    for wgs in (1, 1344, 5376):
        def go(i, wgs=wgs):
            L.r3d_gfx950_stream_probe(ctypes_ptr(sink), 0, 4, 4 * wgs, ctypes_ptr(sink),
                                      ctypes_ptr_stream(stream))
        t, n = time_min(go, min_s)
        empty["%d_workgroups" % wgs] = round(t * 1e6, 3)
    out["empty_kernel_us"] = empty
    log("[bench] launch floor (empty kernel, back to back): %s us" % empty)
    return out


def ctypes_ptr(t):
    import ctypes
    return ctypes.c_void_p(t.data_ptr())


def ctypes_ptr_stream(s):
    import ctypes
    return ctypes.c_void_p(s)


def cpu_baseline(seconds=10.0):
    """The oracle (libref restatement, OpenMP over output rows) on config 1, repeated for
    about `seconds` of wall time."""
    import oracle as O
    from libr3d_amd import synth
    M, K, N = 1, 5376, 21504
    A, AS = synth.fp8_activations_per_token(M, K, 0x5EED + 10)
    B, BS = synth.fp8_weights(N, K, 0x5EED + 11)
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    nth = min(avail, omp) if omp > 0 else avail
    O.quant_dot_fp8a8(A, AS, B, BS, 1, nthreads=nth)         # warm
    calls, t0 = 0, time.perf_counter()
    while True:
        O.quant_dot_fp8a8(A, AS, B, BS, 1, nthreads=nth)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    gbs = f8_bytes(M, N, K) * calls / el / 1e9
    cpu = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": nth, "kind": "port",
            "nproc": os.cpu_count(), "affinity_cores": avail,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "cpu_model": cpu,
            "sample": "config 1 (fp8a8 GEMV M=1 K=5376 N=21504), full problem x %d calls, "
                      "%.1f s wall, oracle/ C restatement of libref quant_dot, OpenMP %d "
                      "threads (every core this process may run on, capped by OMP_NUM_THREADS "
                      "when set) on %s" % (calls, el, nth, cpu or "host CPU")}


def bench_overlap(dev, stream, iters=4096):
    """How much VALU work one wave hides under its own MFMAs (r3d_gfx950_mfma_valu_probe):
    shader-clock ticks per 16x16x128 e4m3 MFMA with nv independent f32 fused multiply-adds
    issued between consecutive MFMAs, and with 4 / 8 that read the result of the MFMA issued
    three earlier (the e4m3 prefill tile's flush).  Each case launched twice, the second
    timed."""
    import torch
    import libr3d_amd as R
    L = R.lib()
    work = torch.zeros(256, dtype=torch.int32, device=dev)
    cyc = torch.zeros(1, dtype=torch.int64, device=dev)
    out = {}
    for nv, lag3 in ((0, 0), (4, 0), (8, 0), (16, 0), (4, 1), (8, 1)):
        for _ in range(2):
            rc = L.r3d_gfx950_mfma_valu_probe(nv, lag3, iters, ctypes_ptr(work), ctypes_ptr(cyc),
                                              ctypes_ptr_stream(stream))
            assert rc == 0, rc
        torch.cuda.synchronize()
        out["nv%d%s" % (nv, "_lag3" if lag3 else "")] = round(int(cyc.item()) / (4 * iters), 2)
    return {"ticks_per_mfma": out, "iters": iters}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline workload only")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--floors", action="store_true",
                    help="only measure the HBM stream ceilings and the launch floor, print JSON")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only run a plain 256 MiB device copy (counter calibration for PMC runs)")
    ap.add_argument("--overlap", action="store_true",
                    help="only run the MFMA / VALU overlap probe (one wave), print JSON")
    ap.add_argument("--c3-only", action="store_true",
                    help="only time config 3 (mxfp4a16 prefill) and print its JSON (for profiling)")
    ap.add_argument("--case", default=None,
                    help="only run one named workload and print its JSON line (for profiling): "
                         + ", ".join(CASES))
    args = ap.parse_args()
    if args.copy_calib:
        import torch
        src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel(), "launches": 5}), flush=True)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the gemm_nt_q path is built and measured on a single "
              "MI355X (multi-GPU sharding is design only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import libr3d_amd as R
    from libr3d_amd import synth
    R.lib()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    if args.c3_only:
        print(json.dumps(bench_c3(dev, stream, steps=args.steps, warmup=args.warmup, min_s=None)),
              flush=True)
        return
    if args.floors:
        print(json.dumps(bench_floors(dev, stream)), flush=True)
        return
    if args.overlap:
        print(json.dumps(bench_overlap(dev, stream)), flush=True)
        return
    if args.case:
        print(json.dumps(run_case(args.case, dev, stream, args.steps, args.warmup)), flush=True)
        return

    # ---- the ceilings first: the stream probe and the launch floor on this box (they also
    # leave the GPU at its working clocks, as a serving loop keeps it, before the headline's
    # own --warmup launches)
    floors = None
    if not args.quick and not args.no_extra:
        log("[bench] floors: HBM stream ceilings and the launch floor")
        floors = bench_floors(dev, stream)

    # ---- headline: config 1, fp8a8 decode GEMV, cold
    M, K, N = 1, 5376, 21504
    log("[bench] config 1: fp8a8 decode GEMV M=%d K=%d N=%d" % (M, K, N))
    A, AS = synth.fp8_activations_per_token(M, K, 0x5EED + 10)
    B, BS = synth.fp8_weights(N, K, 0x5EED + 11)
    nbytes = f8_bytes(M, N, K)
    c1 = Case("fp8a8", A, AS, B, BS, M, N, K, copies_for(B.nbytes), dev)
    torch.cuda.synchronize()
    wall, kern = time_case(c1, "gemm_nt_q_fp8a8_decode", args.steps, args.warmup, stream,
                           min_s=None)
    c1_window = c1.last_kern_window
    value = nbytes * args.steps / wall / 1e9
    achieved = nbytes / kern / 1e9
    log("[bench] config 1: wall %.2f GB/s, kernel %.2f us -> %.1f GB/s (%.1f%% of HBM peak)"
        % (value, kern * 1e6, achieved, 100 * achieved / HBM_PEAK_GBS))
    del c1

    out = {
        "metric": "fp8 decode GEMV HBM GB/s @M=1 (BASELINE config 1)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3 x fp8e4m3 -> f32 accumulate, bf16 out",
        "data": "synthetic (seeded; BASELINE config 1 distributions)",
        "config": {"workload": "config 1: gemm_nt_q fp8a8 decode GEMV, M=1 K=5376 N=21504, "
                               "per-row bf16 weight scales, per-token a_scale, cold HBM "
                               "(weights rotated over >1 GiB, each copy read once before "
                               "the warm-up)",
                   "row": "gemm_nt_q_fp8a8_decode", "bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": HEADLINE_TRAFFIC_BYTES,
                     "kernel": "r3d::gemv_quad_kernel<1, 1, 1, 4, 0, 7> (fp8a8, MT=1, one quad per wave, 4-step ring, 7 waves a workgroup)",
                     "kernel_us": round(kern * 1e6, 3),
                     "kernel_window": "HIP events from the end of the first timed launch to the "
                                      "end of the last (launches 2..steps); over all steps, "
                                      "from before the first launch: %.3f us a launch"
                                      % (c1_window * 1e6)},
    }

    extra = {}
    if floors is not None:
        extra["floors"] = floors
    if not args.quick and not args.no_extra:
        ksteps = max(20, args.steps // 4)
        # C0: cache-fit parity config
        M, K, N = 1, 4096, 4096
        _, A, AS = synth.activations(M, K, 0x5EED)
        B, BS = synth.mxfp4_weights(N, K, 0x5EED + 1)
        c = Case("mxfp4a8", A, AS, B, BS, M, N, K, 1, dev)
        wall, kern = time_case(c, "gemm_nt_q_mxfp4_decode", ksteps, 10, stream)
        nb = mx_bytes(M, N, K)
        extra["c0_mxfp4_gemv_cachefit"] = {"M": M, "K": K, "N": N, "kernel_us": round(kern * 1e6, 3),
                                           "GBps_kernel": round(nb / kern / 1e9, 1)}
        del c
        # C2: mxfp4 decode, three shapes x M in {1, 4, 16}, cold
        for name, (K, N) in (("gate_up", (5376, 21504)), ("down", (21504, 5376)),
                             ("qkv", (5376, 8192))):
            B, BS = synth.mxfp4_weights(N, K, 0x5EED + 21 + K)
            for M in (1, 4, 16):
                _, A, AS = synth.activations(M, K, 0x5EED + 20 + M)
                c = Case("mxfp4a8", A, AS, B, BS, M, N, K, copies_for(B.nbytes + BS.nbytes), dev)
                row = "gemm_nt_q_mxfp4_decode"
                rec = {"K": K, "N": N}
                # the row as an engine runs it: with the launch scratch its hook asks for
                # (the K split where it applies), and the GEMV alone without scratch
                if c.hook_scratch(row):
                    c.ops = [R.GemmOperands(c.a, c.as_, b, bs, c.y, dtype="mxfp4a8", N=N, K=K)
                             for b, bs in zip(c.b, c.bs)]
                    _, k0 = time_case(c, row, ksteps, 10, stream)
                    rec.update({"kernel_us_noscratch": round(k0 * 1e6, 3),
                                "arm_noscratch": R.describe(row, c.ops[0])[1].split()[1]})
                    c.hook_scratch(row)
                wall, kern = time_case(c, row, ksteps, 10, stream)
                nb = mx_bytes(M, N, K)
                gbs = nb / kern / 1e9
                rec.update({"kernel_us": round(kern * 1e6, 3), "GBps_kernel": round(gbs, 1),
                            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                            "GBps_wall": round(nb * c.last_steps / wall / 1e9, 1),
                            "launches": c.last_steps,
                            "arm": " ".join(R.describe(row, c.ops[0])[1].split()[:2])})
                extra["c2_mxfp4_%s_M%d" % (name, M)] = rec
                log("[bench] C2 %s M=%d: %.2f us, %.1f GB/s (%.1f%%) %s" % (
                    name, M, kern * 1e6, gbs, 100 * gbs / HBM_PEAK_GBS, rec["arm"]))
                del c
        # C3 as configured: bf16 activations quantised in-library to mxfp8, mxfp4a16 row;
        # its GEMM kernel alone carries the compute roofline
        # the prefill kernels run ~0.2-0.5 ms a launch: 100 launches after 20 warm-ups (over
        # 10, the GPU's clock ramp from idle showed as 10-15 % more time a launch)
        extra.update(bench_c3(dev, stream, steps=100, warmup=20))
        g = run_case("c3_a16_gemm", dev, stream, 100, 20)
        out["roofline_c3"] = {"bound": "mfma", "achieved": g["TFLOPs"], "peak": FP8_PEAK_TFLOPS,
                              "unit": "TFLOP/s", "frac": g["frac_fp8_peak"], "flops": g["flops"],
                              "kernel": g["kernel"], "kernel_us": g["kernel_us"],
                              "note": "config 3's GEMM alone (stage 2 of gemm_nt_q_mxfp4a16), "
                                      "dense fp8-rate peak: an fp4 x fp8 scaled MFMA issues "
                                      "at the fp8 rate"}
        # C3 on the reference's activation contract (e4m3 + f32 per 128): mxfp4a8 row
        M, K, N = 2048, 5376, 21504
        _, A, AS = synth.activations(M, K, 0x5EED + 30)
        B, BS = synth.mxfp4_weights(N, K, 0x5EED + 31)
        c = Case("mxfp4a8", A, AS, B, BS, M, N, K, 1, dev)
        wall, kern = time_case(c, "gemm_nt_q_mxfp4", 100, 20, stream)
        tf = 2.0 * M * N * K / kern / 1e12
        extra["c3_mxfp4a8_prefill"] = {"M": M, "K": K, "N": N, "kernel_us": round(kern * 1e6, 1),
                                       "TFLOPs": round(tf, 1),
                                       "frac_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4)}
        log("[bench] C3 mxfp4a8 prefill: %.1f us, %.1f TFLOP/s" % (kern * 1e6, tf))
        del c
        # the same shape on the fp8a8 row (config 1's weight law)
        A8, AS8 = synth.fp8_activations_per_token(M, K, 0x5EED + 35)
        B8, BS8 = synth.fp8_weights(N, K, 0x5EED + 36)
        c = Case("fp8a8", A8, AS8, B8, BS8, M, N, K, 1, dev)
        wall, kern = time_case(c, "gemm_nt_q_fp8a8", 100, 20, stream)
        tf = 2.0 * M * N * K / kern / 1e12
        extra["c3_shape_fp8a8_prefill"] = {"M": M, "K": K, "N": N, "kernel_us": round(kern * 1e6, 1),
                                           "TFLOPs": round(tf, 1),
                                           "frac_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4)}
        log("[bench] C3-shape fp8a8 prefill: %.1f us, %.1f TFLOP/s" % (kern * 1e6, tf))
        del c
        # and on the reference fp8a8 rows' checkpoint grid: one bf16 scale per 128 x 128
        # weight tile (the same scales, one row of them per 128 weight rows)
        c = Case("fp8a8", A8, AS8, B8, BS8[::128].copy(), M, N, K, 1, dev)
        wall, kern = time_case(c, "gemm_nt_q_fp8a8", 100, 20, stream)
        tf = 2.0 * M * N * K / kern / 1e12
        extra["c3_shape_fp8a8_prefill_block128"] = {
            "M": M, "K": K, "N": N, "kernel_us": round(kern * 1e6, 1), "TFLOPs": round(tf, 1),
            "frac_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4),
            "scales": "one bf16 per 128 x 128 weight tile"}
        log("[bench] C3-shape fp8a8 prefill, 128 x 128 scale blocks: %.1f us, %.1f TFLOP/s"
            % (kern * 1e6, tf))
        del c
        torch.cuda.empty_cache()
        extra.update(bench_quant(dev, stream))
        extra.update(bench_fused_decode(dev, stream))
        extra.update(bench_gated(dev, stream))
        extra.update(bench_skinny(dev, stream, ksteps))
        extra.update(bench_c4(dev, stream, steps=5))
        torch.cuda.empty_cache()
        for m in (1, 4):                 # the reference's lm_head row on the 27B head
            r = run_case("lm_head_e4m3_M%d" % m, dev, stream, 300, 30)   # ~70 ms: steady clocks
            extra["lm_head_e4m3_M%d" % m] = {k: r[k] for k in ("M", "K", "N", "bytes", "kernel",
                                                                "kernel_us", "GBps", "frac_hbm")}
            log("[bench] lm_head logits_gemm_e4m3 M=%d: %.1f us, %.1f GB/s (%.1f%%)" % (
                m, r["kernel_us"], r["GBps"], 100 * r["frac_hbm"]))
            torch.cuda.empty_cache()
    if extra:
        out["extra"] = extra

    if not args.no_cpu:
        log("[bench] CPU baseline (oracle, bounded sample) ...")
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


CASES = (["c0", "c1", "c3_a16", "c3_a16_quant", "c3_a16_gemm", "c3_a8", "c3_f8", "c3_f8_b128",
          "lm_head_M4"] +
         ["c2_%s_M%d" % (s, m) for s in ("gate_up", "down", "qkv") for m in (1, 4, 16)] +
         ["c4_%s_M4" % s for s in ("q", "kv", "o")] +
         ["skinny_%s_M%d" % (s, m) for s in ("gate_up", "down", "qkv") for m in (17, 32, 64)] +
         ["lm_head_e4m3_M%d" % m for m in (1, 4, 8, 16)])
C2_SHAPES = {"gate_up": (5376, 21504), "down": (21504, 5376), "qkv": (5376, 8192)}
C4_SHAPES = {"q": (5376, 4096), "kv": (5376, 2048), "o": (4096, 5376)}


def run_case(name, dev, stream, steps, warmup):
    """One named workload, cold where its weights exceed the cache (rotated copies), timed
    with HIP events on the launch stream: kernel (or op) microseconds and the rate against
    its roofline.  The names are the profiling targets of profiles/."""
    import torch
    import libr3d_amd as R
    from libr3d_amd import synth
    if name not in CASES:
        raise SystemExit("unknown case %r; one of: %s" % (name, ", ".join(CASES)))
    res = {"case": name, "steps": steps}
    if name.startswith("c3_a16"):
        M, K, N = 2048, 5376, 21504
        rng = np.random.default_rng(0x5EED + 32)
        X = synth.bf16_bits(rng.standard_normal((M, K), dtype=np.float32))
        B, BS = synth.mxfp4_weights(N, K, 0x5EED + 31)
        x = torch.from_numpy(X.view(np.int16)).to(dev)
        b, bs = torch.from_numpy(B).to(dev), torch.from_numpy(BS).to(dev)
        y = torch.empty((M, N), dtype=torch.int16, device=dev)
        ops = R.GemmOperands(x, None, b, bs, y, dtype="mxfp4a16", N=N, K=K, group=32, M=M)
        scratch = torch.empty(R.row_scratch_bytes("gemm_nt_q_mxfp4a16", ops), dtype=torch.uint8,
                              device=dev)
        ops.set_scratch(scratch)
        stage = {"c3_a16": 0, "c3_a16_quant": 1, "c3_a16_gemm": 2}[name]
        assert R.mxfp4a16_stage(ops, 1, stream) == 0           # the planes the GEMM reads
        for _ in range(warmup):
            assert R.mxfp4a16_stage(ops, stage, stream) == 0
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            R.mxfp4a16_stage(ops, stage, stream)
        e1.record()
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / steps
        fl = 2.0 * M * N * K
        res.update({"M": M, "K": K, "N": N, "kernel_us": round(t * 1e6, 2), "flops": fl})
        if stage == 1:
            nb = M * K * 2 + M * K + M * K // 32
            res.update({"kernel": "r3d::quant_mx8_kernel", "GBps": round(nb / t / 1e9, 1),
                        "frac_hbm": round(nb / t / 1e9 / HBM_PEAK_GBS, 4)})
        else:
            d = R.describe("gemm_nt_q_mxfp4a16", ops)[1]
            bn = int(d.split("bn=")[1].split()[0])
            res.update({"kernel": "r3d::prefill_kernel<1, %d, 4>" % (bn // 32)
                        + (" (+ r3d::quant_mx8_kernel)" if stage == 0 else ""),
                        "TFLOPs": round(fl / t / 1e12, 1),
                        "frac_fp8_peak": round(fl / t / 1e12 / FP8_PEAK_TFLOPS, 4)})
        return res
    if name in ("c3_a8", "c3_f8", "c3_f8_b128"):
        M, K, N = 2048, 5376, 21504
        if name == "c3_a8":
            _, A, AS = synth.activations(M, K, 0x5EED + 30)
            B, BS = synth.mxfp4_weights(N, K, 0x5EED + 31)
            c, row = Case("mxfp4a8", A, AS, B, BS, M, N, K, 1, dev), "gemm_nt_q_mxfp4"
        else:
            A, AS = synth.fp8_activations_per_token(M, K, 0x5EED + 35)
            B, BS = synth.fp8_weights(N, K, 0x5EED + 36)
            if name == "c3_f8_b128":
                BS = BS[::128].copy()             # one scale per 128 x 128 weight tile
            c, row = Case("fp8a8", A, AS, B, BS, M, N, K, 1, dev), "gemm_nt_q_fp8a8"
        wall, kern = time_case(c, row, steps, warmup, stream)
        fl = 2.0 * M * N * K
        res.update({"M": M, "K": K, "N": N, "row": row, "kernel_us": round(kern * 1e6, 2),
                    "flops": fl, "TFLOPs": round(fl / kern / 1e12, 1),
                    "frac_fp8_peak": round(fl / kern / 1e12 / FP8_PEAK_TFLOPS, 4),
                    "plan": R.describe(row, c.ops[0])[1]})
        return res
    if name.startswith("lm_head_e4m3_"):
        return bench_lm_head_e4m3(int(name.rsplit("_M", 1)[1]), dev, stream, steps, warmup, res)
    # bandwidth-bound workloads
    if name == "c1" or name == "lm_head_M4":
        M, K, N = (1, 5376, 21504) if name == "c1" else (4, 5376, 262144)
        A, AS = synth.fp8_activations_per_token(M, K, 0x5EED + 10 if name == "c1" else 0x5EED + 40)
        B, BS = synth.fp8_weights(N, K, 0x5EED + 11 if name == "c1" else 0x5EED + 41)
        dtype, row, nb = "fp8a8", "gemm_nt_q_fp8a8_decode", f8_bytes(M, N, K)
    else:
        if name == "c0":
            M, K, N, seed = 1, 4096, 4096, 0x5EED
        elif name.startswith("c2_") or name.startswith("skinny_"):
            shape, m = name.split("_", 1)[1].rsplit("_M", 1)
            M = int(m)
            K, N = C2_SHAPES[shape]
            seed = 0x5EED + 20 + M if name.startswith("c2_") else 0x5EED + 50 + M
        else:
            shape = name[3:].rsplit("_M", 1)[0]
            M = 4
            K, N = C4_SHAPES[shape]
            seed = 0x5EED + 50 + K
        _, A, AS = synth.activations(M, K, seed)
        B, BS = synth.mxfp4_weights(N, K, 0x5EED + 21 + K)
        dtype, nb = "mxfp4a8", mx_bytes(M, N, K)
        row = "gemm_nt_q_mxfp4" if name.startswith("skinny_") else "gemm_nt_q_mxfp4_decode"
    copies = 1 if name == "c0" else copies_for(B.nbytes + BS.nbytes)
    c = Case(dtype, A, AS, B, BS, M, N, K, copies, dev)
    res["scratch_bytes"] = c.hook_scratch(row)              # split K where it applies
    wall, kern = time_case(c, row, steps, warmup, stream)
    res.update({"M": M, "K": K, "N": N, "row": row, "bytes": nb, "copies": copies,
                "kernel_us": round(kern * 1e6, 3), "GBps": round(nb / kern / 1e9, 1),
                "frac_hbm": round(nb / kern / 1e9 / HBM_PEAK_GBS, 4),
                "GBps_wall": round(nb * c.last_steps / wall / 1e9, 1), "steps": c.last_steps,
                "plan": R.describe(row, c.ops[0])[1]})
    return res


def bench_lm_head_e4m3(M, dev, stream, steps, warmup, res):
    """The 27B head as logits_gemm_e4m3 reads it: n_vocab 262144 x n_embd 5376 e4m3 codes
    (uniform over the 254 finite codes) with one bf16 scale per (row, 128 columns), joined
    in device memory; bf16 N(0,1) x [M, 5376]; f32 logits.  Bytes per launch: codes +
    scales + x + logits."""
    import torch
    import libr3d_amd as R
    from libr3d_amd import synth
    N, K = 262144, 5376
    hdr, c_off, s_off, nb_blob = R.head_header(N, K, "bf16", 1)
    blob = torch.empty(nb_blob, dtype=torch.uint8, device=dev)
    blob[:hdr.size].copy_(torch.from_numpy(hdr))
    g = torch.Generator(device=dev)
    g.manual_seed(0x5EED + 60)
    codes = torch.randint(0, 256, (N * K,), dtype=torch.int32, device=dev, generator=g)
    codes = torch.where((codes & 0x7F) == 0x7F, codes - 1, codes)       # no NaN codes
    blob[c_off:c_off + N * K].copy_(codes.to(torch.uint8))
    del codes
    scols = (K + 127) // 128
    sv = (torch.rand((N * scols,), device=dev, generator=g) + 0.5) * (0.02 / 448)
    blob[s_off:s_off + N * scols * 2].copy_(sv.to(torch.bfloat16).view(torch.uint8))
    del sv
    X = synth.bf16_bits(np.random.default_rng(0x5EED + 61).standard_normal((M, K)).astype(np.float32))
    x = torch.from_numpy(X.view(np.int16)).to(dev)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)

    class _Case:
        ops = [R.LogitsOperands(x, blob, y, n_vocab=N, n_embd=K)]
    row = "logits_gemm_e4m3"
    wall, kern = time_case(_Case, row, steps, warmup, stream)
    R.forget_head(blob)
    nb = N * K + N * scols * 2 + M * K * 2 + M * N * 4
    res.update({"M": M, "K": K, "N": N, "row": row, "bytes": nb,
                "kernel": "r3d::logits_e4m3_kernel<%d, %d, 0>" % (2 if M <= 4 else 1, 1 if M <= 4 else 2),
                "kernel_us": round(kern * 1e6, 3),
                "GBps": round(nb / kern / 1e9, 1), "frac_hbm": round(nb / kern / 1e9 / HBM_PEAK_GBS, 4),
                "GBps_wall": round(nb * _Case.last_steps / wall / 1e9, 1),
                "steps": _Case.last_steps})
    return res


def bench_c3(dev, stream, steps=10, warmup=3, min_s=EXTRA_MIN_S):
    """Config 3 as written: M=2048, K=5376, N=21504, mxfp4 weights (E8M0 exponents in
    [-8, 0]), bf16 N(0,1) activations quantised by the row itself to mxfp8 (e4m3 + E8M0
    per 32) -- gemm_nt_q_mxfp4a16, quantiser and GEMM both inside the timed launches."""
    import torch
    import libr3d_amd as R
    from libr3d_amd import synth
    M, K, N = 2048, 5376, 21504
    rng = np.random.default_rng(0x5EED + 32)
    X = synth.bf16_bits(rng.standard_normal((M, K), dtype=np.float32))
    B, BS = synth.mxfp4_weights(N, K, 0x5EED + 31)
    x = torch.from_numpy(X.view(np.int16)).to(dev)
    b = torch.from_numpy(B).to(dev)
    bs = torch.from_numpy(BS).to(dev)
    y = torch.empty((M, N), dtype=torch.int16, device=dev)
    ops = R.GemmOperands(x, None, b, bs, y, dtype="mxfp4a16", N=N, K=K, group=32, M=M)
    need = R.row_scratch_bytes("gemm_nt_q_mxfp4a16", ops)
    scratch = torch.empty(need, dtype=torch.uint8, device=dev)
    ops.set_scratch(scratch)
    launch = R.row_launcher("gemm_nt_q_mxfp4a16")
    assert launch(ops, stream) == 0
    if min_s:
        t, n = time_min(lambda i: launch(ops, stream), min_s, warm=warmup)
    else:                        # exactly `steps` launches after `warmup` (profiling runs)
        for _ in range(warmup):
            launch(ops, stream)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            launch(ops, stream)
        e1.record()
        torch.cuda.synchronize()
        t, n = e0.elapsed_time(e1) * 1e-3 / steps, steps
    tf = 2.0 * M * N * K / t / 1e12
    log("[bench] C3 mxfp4a16 prefill (quantiser + GEMM): %.1f us, %.1f TFLOP/s (%.1f%% of fp8 dense)"
        % (t * 1e6, tf, 100 * tf / FP8_PEAK_TFLOPS))
    return {"c3_mxfp4a16_prefill": {"M": M, "K": K, "N": N, "op_us": round(t * 1e6, 1), "launches": n,
                                    "TFLOPs": round(tf, 1),
                                    "frac_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4),
                                    "includes": "bf16->mxfp8 quantiser + block-scaled MFMA GEMM"}}


def bench_quant(dev, stream):
    """The quant_act_fp8 producer (bf16 in, e4m3 codes + f32 scale per 128 out) on the
    configs' activation shapes: config 3's 2048 x 5376 and a decode step's 4 x 5376."""
    import torch
    import libr3d_amd as R
    res = {}
    for M in (2048, 4):
        n, g = 5376, 128
        x = torch.randn((M, n), device=dev, dtype=torch.float32).to(torch.bfloat16).view(torch.int16)
        q = torch.empty((M, n), dtype=torch.uint8, device=dev)
        s = torch.empty((M, n // g), dtype=torch.float32, device=dev)
        ops = R.QuantActOperands(x, q, s, n=n, group=g, M=M, x_dtype="BF16")
        f = R.row_launcher("quant_act_fp8_act")
        assert f(ops, stream) == 0
        t, _ = time_min(lambda i: f(ops, stream), EXTRA_MIN_S)
        nb = M * n * 2 + M * n + M * (n // g) * 4
        res["quant_act_fp8_M%d" % M] = {"n": n, "group": g, "kernel_us": round(t * 1e6, 2),
                                         "GBps": round(nb / t / 1e9, 1),
                                         "frac_hbm": round(nb / t / 1e9 / HBM_PEAK_GBS, 4)}
        log("[bench] quant_act_fp8 M=%d n=%d: %.2f us, %.1f GB/s" % (M, n, t * 1e6, nb / t / 1e9))
        # rmsnorm_quant_fp8 on the same rows, with a residual and the bf16 normed output
        r = torch.randn((M, n), device=dev, dtype=torch.float32).to(torch.bfloat16).view(torch.int16)
        w = torch.ones(n, dtype=torch.float32, device=dev)
        o = torch.empty((M, n), dtype=torch.int16, device=dev)
        rops = R.RmsNormQuantOperands(x, r, w, q, s, o, n=n, group=g, M=M)
        fr = R.row_launcher("rmsnorm_quant_fp8")
        assert fr(rops, stream) == 0
        t, _ = time_min(lambda i: fr(rops, stream), EXTRA_MIN_S)
        nb = M * n * 2 * 4 + n * 4 + M * n + M * (n // g) * 4    # x, residual in/out, out, w, q, s
        res["rmsnorm_quant_fp8_M%d" % M] = {"n": n, "group": g, "kernel_us": round(t * 1e6, 2),
                                             "GBps": round(nb / t / 1e9, 1)}
        log("[bench] rmsnorm_quant_fp8 (+residual, +out) M=%d n=%d: %.2f us, %.1f GB/s"
            % (M, n, t * 1e6, nb / t / 1e9))
    return res


def bench_fused_decode(dev, stream):
    """A decode call fed bf16 activations, two ways, cold weights: the quant_act_fp8 row then
    the decode row (two launches), and the decode row taking the bf16 rows itself (the
    producer fused into its LDS staging, one launch: the default at M = 1, the rows' "fuse"
    tunable at M = 4).  Config 1's shape (fp8a8), config 2's gate_up (mxfp4a8) and C4's o
    (mxfp4a8, K = 4096 N = 5376)."""
    import torch
    import libr3d_amd as R
    from libr3d_amd import synth
    res = {}
    for name, dtype, M, K, N in (("c1_fp8a8_M1", "fp8a8", 1, 5376, 21504),
                                 ("c2_mxfp4_gate_up_M1", "mxfp4a8", 1, 5376, 21504),
                                 ("c1_fp8a8_M4", "fp8a8", 4, 5376, 21504),
                                 ("c2_mxfp4_gate_up_M4", "mxfp4a8", 4, 5376, 21504),
                                 ("c4_mxfp4_o_M4", "mxfp4a8", 4, 4096, 5376)):
        if dtype == "fp8a8":
            B, BS = synth.fp8_weights(N, K, 0x5EED + 11)
            BS = BS.view(np.int16)
            row, nb = "gemm_nt_q_fp8a8_decode", f8_bytes(M, N, K)
        else:
            B, BS = synth.mxfp4_weights(N, K, 0x5EED + 21 + K)
            row, nb = "gemm_nt_q_mxfp4_decode", mx_bytes(M, N, K)
        copies = copies_for(B.nbytes + BS.nbytes)
        bs = [torch.from_numpy(B).to(dev)]
        bss = [torch.from_numpy(BS).to(dev)]
        for _ in range(copies - 1):
            bs.append(bs[0].clone())
            bss.append(bss[0].clone())
        x = torch.randn((M, K), device=dev, dtype=torch.float32).to(torch.bfloat16).view(torch.int16)
        q = torch.empty((M, K), dtype=torch.uint8, device=dev)
        sc = torch.empty((M, K // 128), dtype=torch.float32, device=dev)
        y = torch.empty((M, N), dtype=torch.int16, device=dev)
        qa = R.QuantActOperands(x, q, sc, n=K, group=128, M=M, x_dtype="BF16")
        two = [R.GemmOperands(q, sc, b, s_, y, dtype=dtype, N=N, K=K) for b, s_ in zip(bs, bss)]
        tv = [("fuse", 1)] if M > 1 else None
        one = [R.GemmOperands(x, None, b, s_, y, dtype=dtype, N=N, K=K, tunables=tv)
               for b, s_ in zip(bs, bss)]
        fq, fg = R.row_launcher("quant_act_fp8_act"), R.row_launcher(row)

        def timed(body):
            return time_min(body, EXTRA_MIN_S)[0]

        def unfused(i):
            assert fq(qa, stream) == 0 and fg(two[i % copies], stream) == 0

        def fused(i):
            assert fg(one[i % copies], stream) == 0

        t2, t1 = timed(unfused), timed(fused)
        res["fused_decode_" + name] = {
            "M": M, "K": K, "N": N, "two_launch_us": round(t2 * 1e6, 2),
            "fused_us": round(t1 * 1e6, 2), "GBps_fused": round(nb / t1 / 1e9, 1)}
        log("[bench] bf16-fed decode %s: quant + GEMV %.2f us, fused %.2f us" % (
            name, t2 * 1e6, t1 * 1e6))
        del bs, bss, one, two
        torch.cuda.empty_cache()
    return res


def bench_gated(dev, stream):
    """gemm_nt_q_gated at fp8a8 on config 1's plane read as a gate_up pair (N = 2n = 21504,
    K = 5376, per-row weight scales, cold), silu: the gated row against its two rows
    (gemm_nt_q, then gated_quant_fp8) at M = 1 and 4 -- the same kernels, so the gap is the
    host work of the second row's launch."""
    import torch
    import libr3d_amd as R
    from libr3d_amd import synth
    res = {}
    K, N = 5376, 21504
    n = N // 2
    B, BS = synth.fp8_weights(N, K, 0x5EED + 11)
    copies = copies_for(B.nbytes)
    bs = [torch.from_numpy(B).to(dev)]
    bss = [torch.from_numpy(BS.view(np.int16)).to(dev)]
    for _ in range(copies - 1):
        bs.append(bs[0].clone())
        bss.append(bss[0].clone())
    for M in (1, 4):
        A, AS = synth.fp8_activations_per_token(M, K, 0x5EED + 40 + M)
        a, as_ = torch.from_numpy(A).to(dev), torch.from_numpy(AS).to(dev)
        q = torch.empty((M, n), dtype=torch.uint8, device=dev)
        sc = torch.empty((M, n // 128), dtype=torch.float32, device=dev)
        y = torch.empty((M, N), dtype=torch.int16, device=dev)
        scratch = torch.empty(64 * N * 2, dtype=torch.uint8, device=dev)
        fused = []
        for b, s_ in zip(bs, bss):
            o = R.GatedGemmOperands(a, as_, b, s_, q, sc, None, N=N, K=K, act="silu", M=M)
            o.set_scratch(scratch)
            fused.append(o)
        gemm = [R.GemmOperands(a, as_, b, s_, y, dtype="fp8a8", N=N, K=K) for b, s_ in zip(bs, bss)]
        gq = R.GatedQuantOperands(y, q, sc, None, n=n, group=128, act="silu", M=M)
        fg, fd, fq = (R.row_launcher(r) for r in
                      ("gemm_nt_q_gated_fp8a8", "gemm_nt_q_fp8a8_decode", "gated_quant_fp8_act"))

        def timed(body):
            return time_min(body, EXTRA_MIN_S)[0]

        def one(i):
            assert fg(fused[i % copies], stream) == 0

        def two(i):
            assert fd(gemm[i % copies], stream) == 0 and fq(gq, stream) == 0

        def prod(i):
            assert fq(gq, stream) == 0

        t1, t2, tp = timed(one), timed(two), timed(prod)
        nb = f8_bytes(M, N, K)
        res["gated_fp8a8_c1_plane_M%d" % M] = {
            "M": M, "K": K, "N": N, "gated_row_us": round(t1 * 1e6, 2),
            "two_rows_us": round(t2 * 1e6, 2), "gated_quant_fp8_us": round(tp * 1e6, 2),
            "GBps_gated_row": round(nb / t1 / 1e9, 1)}
        log("[bench] gated fp8a8 M=%d: row %.2f us, gemm_nt_q + gated_quant_fp8 %.2f us "
            "(producer alone %.2f us)" % (M, t1 * 1e6, t2 * 1e6, tp * 1e6))
    del bs, bss
    torch.cuda.empty_cache()
    return res


def bench_skinny(dev, stream, steps=50):
    """The skinny band (M = 17..64) on the tile rows at config 2's shapes, cold: the row's
    own dispatch with the launch scratch its hook asks for (split K where it applies), and
    without scratch (16-row decode passes on a narrow N, else the prefill pipeline)."""
    import torch
    import libr3d_amd as R
    from libr3d_amd import synth
    res = {}
    for dtype, row in (("mxfp4a8", "gemm_nt_q_mxfp4"), ("fp8a8", "gemm_nt_q_fp8a8")):
        for name, (K, N) in (("gate_up", (5376, 21504)), ("down", (21504, 5376)),
                             ("qkv", (5376, 8192))):
            if dtype == "mxfp4a8":
                B, BS = synth.mxfp4_weights(N, K, 0x5EED + 21 + K)
            else:
                B, BS = synth.fp8_weights(N, K, 0x5EED + 21 + K)
            for M in (17, 32, 64):
                _, A, AS = synth.activations(M, K, 0x5EED + 50 + M)
                c = Case(dtype, A, AS, B, BS, M, N, K, copies_for(B.nbytes + BS.nbytes), dev)
                nb = mx_bytes(M, N, K) if dtype == "mxfp4a8" else f8_bytes(M, N, K)
                out = {"K": K, "N": N}
                for tag in ("noscratch", "hook"):
                    if tag == "hook" and not c.hook_scratch(row):
                        break
                    wall, kern = time_case(c, row, steps, 10, stream)
                    arm = R.describe(row, c.ops[0])[1].split()[0]
                    out.update({"us_" + tag: round(kern * 1e6, 2), "arm_" + tag: arm})
                    log("[bench] skinny %s %s M=%d %s: %.2f us, %.1f GB/s (%s)" % (
                        dtype, name, M, tag, kern * 1e6, nb / kern / 1e9, arm))
                us = out.get("us_hook", out["us_noscratch"])
                out.update({"us": us, "GBps": round(nb / (us * 1e-6) / 1e9, 1),
                            "frac_hbm": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                            "arm": out.get("arm_hook", out["arm_noscratch"])})
                res["skinny_%s_%s_M%d" % ("mxfp4" if dtype == "mxfp4a8" else "fp8",
                                          name, M)] = out
                del c
        torch.cuda.empty_cache()
    return res


def bench_c4(dev, stream, steps=5):
    """Config 4: one decode step of a 27B-class model at M=4 -- 62 layers of q/k/v/o and
    gate/up/down in mxfp4a8 plus an fp8a8 lm_head (K=5376, N=262144).  Weights are random
    codes generated on the device (bandwidth does not depend on values; NaN-free); the
    435 launches run eagerly and as one captured HIP graph; then eagerly again with the
    reference's own lm_head row, logits_gemm_e4m3 over the joined e4m3 head.  Last, the
    same bytes in the engine's joined layouts -- q/k/v as one N = 8192 plane (config 2's
    qkv shape) and gate/up as one N = 43008 plane (the [M, 2n] gate_up plane the gated row
    consumes) -- 249 launches, eagerly and as a graph."""
    import torch
    import libr3d_amd as R
    M, H, I, L, V = 4, 5376, 21504, 62, 262144
    g = torch.Generator(device=dev)
    g.manual_seed(0x5EED + 4)

    def codes(n, fp8):
        t = torch.randint(0, 256, (n,), dtype=torch.uint8, device=dev, generator=g)
        if fp8:
            t = torch.where((t & 0x7F) == 0x7F, t & 0xFE, t)
        return t

    acts = {}
    for K in (H, 4096, I):
        a = codes(M * K, True).view(M, K)
        s = torch.full((M, K // 128), 0.01, dtype=torch.float32, device=dev)
        acts[K] = (a, s)
    mx_dec = R.row_launcher("gemm_nt_q_mxfp4_decode")
    f8_dec = R.row_launcher("gemm_nt_q_fp8a8_decode")

    def build(shapes):
        """-> (launches, kept tensors, bytes, split launches) for 62 layers of `shapes` and
        the fp8a8 lm_head; every launch gets the scratch its row's hook asks for from one
        arena (the launches run in order on one stream, as an engine's would)."""
        y_bufs, launches, keep, total = {}, [], [], 0
        for layer in range(L):
            for name, K, N in shapes:
                b = codes(N * K // 2, False).view(N, K // 2)
                bs = (127 - torch.randint(0, 9, (N, K // 32), dtype=torch.int32, device=dev,
                                          generator=g)).to(torch.uint8)
                y = y_bufs.setdefault(N, torch.empty((M, N), dtype=torch.int16, device=dev))
                a, s = acts[K]
                ops = R.GemmOperands(a, s, b, bs, y, dtype="mxfp4a8", N=N, K=K)
                keep.append((b, bs, ops))
                launches.append((mx_dec, ops))
                total += mx_bytes(M, N, K)
        b = codes(V * H, True).view(V, H)
        bs = torch.full((V, H // 128), 0x3C00, dtype=torch.int16, device=dev)   # bf16 2^-7
        y = torch.empty((M, V), dtype=torch.int16, device=dev)
        a, s = acts[H]
        ops = R.GemmOperands(a, s, b, bs, y, dtype="fp8a8", N=V, K=H)
        keep.append((b, bs, ops))
        launches.append((f8_dec, ops))
        total += f8_bytes(M, V, H)
        needs = [R.row_scratch_bytes("gemm_nt_q_mxfp4_decode" if fn is mx_dec
                                     else "gemm_nt_q_fp8a8_decode", o) for fn, o in launches]
        arena = torch.empty(max(max(needs), 256), dtype=torch.uint8, device=dev)
        keep.append(arena)
        for (fn, o), need in zip(launches, needs):
            if need > 0:
                o.set_scratch(arena, need)
        torch.cuda.synchronize()
        return launches, keep, total, sum(1 for n in needs if n > 0)

    def step(launches, st):
        for fn, o in launches:
            fn(o, st)

    def eager(launches):
        step(launches, stream)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step(launches, stream)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    def graphed(launches):
        s2 = torch.cuda.Stream()
        with torch.cuda.stream(s2):
            step(launches, s2.cuda_stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s2):
            step(launches, s2.cuda_stream)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            graph.replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    def rec(total, t, **kw):
        r = {"bytes": total, "ms": round(t * 1e3, 3), "GBps": round(total / t / 1e9, 1),
             "frac_hbm": round(total / t / 1e9 / HBM_PEAK_GBS, 4)}
        r.update(kw)
        return r

    separate = [("q", H, 4096), ("k", H, 2048), ("v", H, 2048), ("o", 4096, H),
                ("gate", H, I), ("up", H, I), ("down", I, H)]
    launches, keep, total, nsplit = build(separate)
    te = eager(launches)
    res = {"c4_decode_step_eager": rec(total, te, launches=len(launches), split_launches=nsplit)}
    try:
        tg = graphed(launches)
        res["c4_decode_step_graph"] = rec(total, tg)
        log("[bench] C4 decode step: eager %.3f ms (%.1f GB/s), graph %.3f ms (%.1f GB/s)" % (
            te * 1e3, total / te / 1e9, tg * 1e3, total / tg / 1e9))
    except Exception as e:          # graph capture unavailable: report eager only
        res["c4_decode_step_graph"] = {"error": repr(e)[:200]}
        log("[bench] C4 graph capture failed: %r" % (e,))
    # the same step with the reference's own lm_head row: bf16 x through logits_gemm_e4m3
    # over the joined e4m3 head (codes + one bf16 scale per row and 128 columns), f32 logits
    hdr, c_off, s_off, nb_blob = R.head_header(V, H, "bf16", 1)
    blob = torch.empty(nb_blob, dtype=torch.uint8, device=dev)
    blob[:hdr.size].copy_(torch.from_numpy(hdr))
    blob[c_off:c_off + V * H].copy_(codes(V * H, True))
    scols = (H + 127) // 128
    blob[s_off:s_off + V * scols * 2].view(torch.int16).fill_(0x3C00)     # bf16 0.0078125
    xh = torch.randn((M, H), device=dev, generator=g).to(torch.bfloat16).view(torch.int16)
    yl = torch.empty((M, V), dtype=torch.float32, device=dev)
    lops = R.LogitsOperands(xh, blob, yl, n_vocab=V, n_embd=H)
    launches[-1] = (R.row_launcher("logits_gemm_e4m3"), lops)
    total_e4 = total - f8_bytes(M, V, H) + V * H + V * scols * 2 + M * H * 2 + M * V * 4
    t4 = eager(launches)
    R.forget_head(blob)
    res["c4_decode_step_eager_e4m3_head"] = rec(
        total_e4, t4, lm_head="logits_gemm_e4m3 (bf16 x, joined e4m3 + bf16 scale head, f32 logits)")
    log("[bench] C4 decode step with the e4m3 logits head: eager %.3f ms (%.1f GB/s)" % (
        t4 * 1e3, total_e4 / t4 / 1e9))
    del keep, launches, blob
    torch.cuda.empty_cache()
    # the joined layouts: the same weight bytes in 4 launches a layer
    joined = [("qkv", H, 8192), ("o", 4096, H), ("gate_up", H, 2 * I), ("down", I, H)]
    launches, keep, total_j, nsplit = build(joined)     # the activation rows read once less
    tj = eager(launches)
    res["c4_decode_step_eager_joined"] = rec(
        total_j, tj, launches=len(launches), split_launches=nsplit,
        layout="q/k/v joined (N = 8192) and gate/up joined (N = 43008): the same weight bytes")
    try:
        tjg = graphed(launches)
        res["c4_decode_step_graph_joined"] = rec(total_j, tjg)
    except Exception as e:
        res["c4_decode_step_graph_joined"] = {"error": repr(e)[:200]}
        tjg = float("nan")
    log("[bench] C4 decode step, joined q/k/v and gate/up planes: eager %.3f ms (%.1f GB/s), "
        "graph %.3f ms" % (tj * 1e3, total_j / tj / 1e9, tjg * 1e3))
    del keep, launches
    torch.cuda.empty_cache()
    return res


if __name__ == "__main__":
    main()
