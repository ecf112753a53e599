"""Benchmark of the hot path on one MI355X.

Headline (BASELINE.json metric, config 2): fp32 GEMM C = A @ B at
M = N = K = 4096, NN layout, A/B ~ N(0,1), inputs resident in HBM. A "step" is
one GEMM. Prints ONE JSON line:

  value        whole-job TFLOP/s over the timed K steps (2*M*N*K per step)
  roofline     the GEMM kernel's algorithmic TFLOP/s from HIP-event launch times
               on the backend's stream, against the fp32 MFMA peak (157.3 TFLOP/s)
  cpu_baseline the CPU oracle (the C restatement of vkML's CPU matmul) on a row
               sample of the same problem, on this host's cores
  secondary    the other hot-path kernels at their BASELINE shapes (GB/s against
               8 TB/s for bandwidth kernels; bandwidth cases rotate buffers larger
               than the 256 MB Infinity Cache)

Warm-up: W untimed launches of the headline GEMM, and at least --warmup-seconds
(default 0.3 s) of them: the part raises its clocks over the first tens of
milliseconds of sustained matrix load (back-to-back launches of one 4096^3 GEMM
fall from about 1.3 ms to 1.03 ms over the first ~25 in a kernel trace), and the
timed steps are meant to see the sustained clock. The secondary cases are each
queued behind ~25 ms of GEMM for the same reason.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--warmup-seconds S]
       [--no-secondary] [--no-cpu-baseline] [--case NAME[,NAME] [--no-gate]]
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

MFMA_FP32_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0
# fp32 VALU rate for rounded multiplies and adds issued separately (no FMA, no
# packed fp32): 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz, one FLOP per lane-op.
# The exact arm rounds every product and sum on its own, so this is its roof.
VALU_FP32_SEPARATE_TFLOPS = 39.3
METRIC = "fp32 GEMM TFLOP/s @4096³ (% fp32 MFMA peak); im2col/softmax GB/s; steps/s"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--warmup-seconds", type=float, default=0.3,
                   help="minimum untimed warm-up of the headline GEMM (clock ramp)")
    p.add_argument("--m", type=int, default=4096)
    p.add_argument("--n", type=int, default=4096)
    p.add_argument("--k", type=int, default=4096)
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="target CPU work for the baseline sample")
    p.add_argument("--case", default="",
                   help="run only these secondary cases (comma-separated names) and print them; "
                        "the headline, training and CPU lines are skipped (profiling runs)")
    p.add_argument("--no-gate", action="store_true",
                   help="do not queue the ~25 ms of GEMM before each timed batch (profiling runs: "
                        "counters then see the case's kernels only)")
    p.add_argument("--train-modes", default="",
                   help="training modes the train_mlp / train_cnn cases run (comma-separated; default "
                        "all: dropin,eager,replay,graph,graph_queued,exact), for profiling one mode")
    p.add_argument("--calibrate", action="store_true",
                   help="also run the plain 16-byte copy kernel 5x over 256 MiB (the byte-counter "
                        "calibration for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    return p.parse_args()


class Timer:
    """HIP events recorded on the backend's own stream, through the C ABI."""

    def event(self):
        from vkml_amd.device import Event

        return Event().record()


_GATE = None
_GATE_ON = True


def gate(launches: int = 24):
    """Enqueues ~25 ms of GEMM so the host can queue the timed launches ahead of
    the GPU (event pairs then bracket GPU time only, not Python launch gaps) and
    the clocks are back up after the host-side set-up of the case."""
    global _GATE
    from vkml_amd import ops
    from vkml_amd.device import DeviceArray

    if not _GATE_ON:
        return
    if _GATE is None:
        a = DeviceArray.from_numpy(np.ones((4096, 4096), np.float32))
        _GATE = (a, DeviceArray((4096, 4096), np.float32))
    a, c = _GATE
    for _ in range(launches):
        ops.matmul(a, a, out=c)


def time_launches(fn, timer: Timer, reps: int, warmup: int = 3):
    """Per-launch durations (ms) from event pairs around each call (for
    launches long enough that event overhead is negligible)."""
    for _ in range(warmup):
        fn(0)
    gate()
    pairs = []
    for i in range(reps):
        s = timer.event()
        fn(i)
        e = timer.event()
        pairs.append((s, e))
    return [s.elapsed_ms(e) for s, e in pairs]


def time_batch(fn, timer: Timer, reps: int, warmup: int = 3) -> float:
    """Mean time (ms) of `reps` back-to-back launches between ONE event pair,
    queued behind the gate so the GPU never waits for the host."""
    for _ in range(warmup):
        fn(0)
    gate()
    s = timer.event()
    for i in range(reps):
        fn(i)
    e = timer.event()
    return s.elapsed_ms(e) / reps


def gemm_headline(args, hip, ops, timer):
    from vkml_amd.device import DeviceArray

    m, n, k = args.m, args.n, args.k
    rng = np.random.default_rng(20260726)
    a = DeviceArray.from_numpy(rng.standard_normal((m, k), dtype=np.float32))
    b = DeviceArray.from_numpy(rng.standard_normal((k, n), dtype=np.float32))
    c = DeviceArray((m, n), np.float32)
    t_end = time.perf_counter() + args.warmup_seconds
    done = 0
    while done < args.warmup or time.perf_counter() < t_end:
        for _ in range(8):
            ops.matmul(a, b, out=c)
        done += 8
        hip.synchronize()
    events = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        s = timer.event()
        ops.matmul(a, b, out=c)
        e = timer.event()
        events.append((s, e))
    hip.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = [s.elapsed_ms(e) for s, e in events]
    flop = 2.0 * m * n * k
    value = flop * args.steps / wall / 1e12
    avg_ms = float(np.mean(launch_ms))
    achieved = flop / (avg_ms * 1e-3) / 1e12
    return value, wall * 1e3 / args.steps, avg_ms, achieved, float(np.min(launch_ms)), done


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _host_threads() -> int:
    """The host cores this process may use: its affinity set, capped by
    OMP_NUM_THREADS when that is set (the GPU box gives each GPU a share of
    the host and says so there)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def _timed(fn, seconds: float, reps_min: int = 1):
    """Best-of time of fn() over at least reps_min calls and about `seconds`."""
    best, spent, reps = float("inf"), 0.0, 0
    while reps < reps_min or spent < seconds:
        t0 = time.perf_counter()
        fn()
        dt = time.perf_counter() - t0
        best = min(best, dt)
        spent += dt
        reps += 1
        if reps >= 5 and spent >= seconds:
            break
    return best


def cpu_baseline(args):
    """The CPU oracle (the C restatement of vkML's CPU backend, the
    reference's own algorithms) timed on this host: single-threaded, as the
    reference CPU backend runs (include/vkml/backend/cpu/cpu_backend.h:16), and
    over every host core this process may use (OpenMP over outputs only: the
    same bits). Each case runs on a bounded sample of the workload, scaled to
    the metric's unit; the rate is the sample's, labelled "sampled" (the whole
    problem would take minutes to hours single-threaded)."""
    import oracle as O
    from vkml_amd import nn, optim
    from vkml_amd import tensor as T

    threads_all = _host_threads()
    rng = np.random.default_rng(1)
    m, n, k = args.m, args.n, args.k
    per_case = max(0.5, args.cpu_seconds / 10.0)
    lines = []

    def line(case, value, unit, threads, sample):
        lines.append({"case": case, "value": round(value, 6), "unit": unit, "cores": threads,
                      "sample": sample})

    b = rng.standard_normal((k, n), dtype=np.float32)
    img = rng.uniform(-1, 1, (8, 64, 32, 32)).astype(np.float32)
    logits = (rng.standard_normal((4096, 1000)) * 2).astype(np.float32)
    red = rng.standard_normal((1024, 4096)).astype(np.float32)
    mlp_x = rng.uniform(0, 1, (64, 1, 28, 28)).astype(np.float32)
    mlp_y = rng.integers(0, 10, 64).astype(np.int64)
    sk_b = rng.standard_normal((65536, 256), dtype=np.float32)
    gv_a = rng.standard_normal((4096, 4096), dtype=np.float32)
    gv_x = rng.standard_normal((4096, 1), dtype=np.float32)
    cols = O.im2col(img, 3, 1, 1)
    wide = (rng.standard_normal((16, 32768)) * 2).astype(np.float32)
    S = _streams()
    cnn_x, cnn_y = next(S.batches(S.CONFIG5, 1, 8))
    for threads in sorted({1, threads_all}):
        # GEMM 4096^3 on a row sample sized to ~1/3 of the budget
        probe_rows = max(threads, 4)
        a = rng.standard_normal((probe_rows, k), dtype=np.float32)
        t0 = time.perf_counter()
        O.matmul(a, b, threads=threads)
        probe = time.perf_counter() - t0
        rows = int(min(m, max(probe_rows, probe_rows * (3 * per_case) / max(probe, 1e-3))))
        rows = max(threads, rows - rows % threads)
        a = rng.standard_normal((rows, k), dtype=np.float32)
        dt = _timed(lambda: O.matmul(a, b, threads=threads), 0.0)
        line("gemm_nn_4096x4096x4096", 2.0 * rows * n * k / dt / 1e9, "GFLOP/s", threads,
             f"{rows} of {m} rows, {dt:.2f} s")
        # im2col conv2 geometry on 8 of 128 images (read image + write cols)
        dt = _timed(lambda: O.im2col(img, 3, 1, 1, threads=threads), per_case, 2)
        byt = img.nbytes + img.shape[0] * 576 * 1024 * 4
        line("im2col_conv2", byt / dt / 1e9, "GB/s", threads, f"8 of 128 images, best {dt * 1e3:.1f} ms")
        # softmax [4096, 1000] (read + write once)
        dt = _timed(lambda: O.softmax(logits, -1, threads=threads), per_case, 2)
        line("softmax_4096x1000", 2 * logits.nbytes / dt / 1e9, "GB/s", threads,
             f"whole problem, best {dt * 1e3:.1f} ms")
        # sum over the last axis of [8192, 4096] on 1024 rows
        dt = _timed(lambda: O.sum(red, [1], threads=threads), per_case, 2)
        line("sum_8192x4096", (red.nbytes + 1024 * 4) / dt / 1e9, "GB/s", threads,
             f"1024 of 8192 rows, best {dt * 1e3:.1f} ms")
        # one config-1 MLP training step (forward, backward, SGD) on the oracle backend
        be = O.OracleBackend(threads=threads)
        nn.manual_seed(20260726)
        model = nn.Sequential(nn.Flatten(), nn.Linear(784, 128, backend=be), nn.ReLU(),
                              nn.Linear(128, 10, backend=be))
        opt = optim.SGD(model.parameters(), lr=0.1, momentum=0.9)

        def mlp_step():
            opt.zero_grad()
            loss = nn.cross_entropy(model(T.tensor(mlp_x, backend=be)), T.tensor(mlp_y, backend=be))
            loss.backward()
            opt.step()
            loss.item()

        dt = _timed(mlp_step, per_case, 3)
        line("mlp_784_128_10_b64_step", 1.0 / dt, "steps/s", threads,
             f"whole step, best {dt * 1e3:.2f} ms")
        # split-K shape 256x256x65536 on a row sample (the oracle has no split:
        # one pairwise sum per output)
        sk_rows = max(threads, 8)
        sk_a = rng.standard_normal((sk_rows, 65536), dtype=np.float32)
        dt = _timed(lambda: O.matmul(sk_a, sk_b, threads=threads), per_case, 1)
        line("splitk_256x256x65536", 2.0 * sk_rows * 256 * 65536 / dt / 1e9, "GFLOP/s", threads,
             f"{sk_rows} of 256 rows, best {dt:.2f} s")
        # GEMV 4096x4096 . 4096 (read the matrix once)
        dt = _timed(lambda: O.matmul(gv_a, gv_x, threads=threads), per_case, 2)
        line("gemv_4096", (gv_a.nbytes + 2 * 4096 * 4) / dt / 1e9, "GB/s", threads,
             f"whole problem, best {dt * 1e3:.1f} ms")
        # col2im conv2 geometry on 8 of 128 images (read cols + write image)
        dt = _timed(lambda: O.col2im(cols, (32, 32), 3, 1, 1, threads=threads), per_case, 2)
        line("col2im_conv2", (cols.nbytes + img.nbytes) / dt / 1e9, "GB/s", threads,
             f"8 of 128 images, best {dt * 1e3:.1f} ms")
        # softmax [256, 32768] on 16 of the 256 rows
        dt = _timed(lambda: O.softmax(wide, -1, threads=threads), per_case, 2)
        line("softmax_256x32768", 2 * wide.nbytes / dt / 1e9, "GB/s", threads,
             f"16 of 256 rows, best {dt * 1e3:.1f} ms")
        # one config-5 CNN training step at batch 8 (the whole network, a
        # sixteenth of the batch): steps/s at batch 8 and, labelled, the
        # batch-128 rate it implies (the step's work is linear in the batch)
        nn.manual_seed(S.CONFIG5.model_seed)
        cnn = S.model(S.CONFIG5, be)
        copt = optim.SGD(cnn.parameters(), lr=S.CONFIG5.lr, momentum=S.CONFIG5.momentum)

        def cnn_step():
            copt.zero_grad()
            loss = nn.cross_entropy(cnn(T.tensor(cnn_x, backend=be)), T.tensor(cnn_y, backend=be))
            loss.backward()
            copt.step()
            loss.item()

        dt = _timed(cnn_step, per_case, 2)
        line("cifar_cnn_b128_step", 8.0 / 128.0 / dt, "steps/s", threads,
             f"batch 8 of 128 (extrapolated linearly to 128), best {dt * 1e3:.1f} ms per batch-8 step")

    head = next(l for l in lines if l["case"].startswith("gemm") and l["cores"] == threads_all)
    return {"value": round(head["value"] / 1e3, 6), "unit": "TFLOP/s", "cores": threads_all,
            "kind": "port", "sample": f"CPU oracle matmul (C restatement of reference "
                                      f"kernels_matmul.cpp:34-87, pairwise K-sum, -O2 "
                                      f"-ffp-contract=off), {head['sample']} of the {m}x{n}x{k} "
                                      f"problem, {threads_all} threads over outputs",
            "nproc": os.cpu_count(), "cpu_model": _cpu_model(),
            "threads_note": "single-threaded (the reference CPU backend's design) and every core "
                            "this process may use (affinity, capped by OMP_NUM_THREADS)",
            "lines": lines}


# ---- secondary cases ------------------------------------------------------------
# Each case measures one hot-path kernel family at its BASELINE shape and adds
# its entries to `out`. `python bench.py --case NAME[,NAME]` runs only the
# named cases (the profiling runs behind profiles/ use this with rocprofv3).

def _rotate(rng, shape, count, scale=1.0):
    from vkml_amd.device import DeviceArray

    return [DeviceArray.from_numpy(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))
            for _ in range(count)]


def _bw(out, name, ms, byt):
    out[name] = {"ms": round(ms, 5), "gbs": round(byt / ms / 1e6, 1),
                 "frac_of_hbm": round(byt / ms / 1e6 / HBM_PEAK_GBS, 4)}


GEMM_CASES = {"gemm_512": ((512, 512, 512), "nn"), "gemm_1024": ((1024, 1024, 1024), "nn"),
              "gemm_2048": ((2048, 2048, 2048), "nn"), "gemm_nn_4096": ((4096, 4096, 4096), "nn"),
              "gemm_nt_4096": ((4096, 4096, 4096), "nt"), "gemm_tn_4096": ((4096, 4096, 4096), "tn"),
              "gemm_8192x1024x4096": ((8192, 1024, 4096), "nn"), "gemm_8192": ((8192, 8192, 8192), "nn"),
              "splitk_256x256x65536": ((256, 256, 65536), "nn"),
              "wgrad_128x784x16384": ((128, 784, 16384), "nn")}


def case_gemm(name, hip, ops, timer, rng, out):
    """GEMM variants (compute-bound: no rotation)."""
    from vkml_amd.device import DeviceArray

    (m, n, k), lay = GEMM_CASES[name]
    a = DeviceArray.from_numpy(rng.standard_normal((m, k) if lay[0] == "n" else (k, m), dtype=np.float32))
    b = DeviceArray.from_numpy(rng.standard_normal((k, n) if lay[1] == "n" else (n, k), dtype=np.float32))
    av = a if lay[0] == "n" else a.T
    bv = b if lay[1] == "n" else b.T
    c = DeviceArray((m, n), np.float32)
    ms = time_batch(lambda i: ops.matmul(av, bv, out=c), timer, 10 if m * n * k > 2**36 else 20)
    splits, _ = ops.gemm_plan(1, m, n, k)
    tf = 2.0 * m * n * k / ms / 1e9
    out[name] = {"ms": round(ms, 5), "tflops": round(tf, 2),
                 "frac_of_peak": round(tf / MFMA_FP32_PEAK_TFLOPS, 4), "splits": splits}


def case_gemm_exact(name, hip, ops, timer, rng, out):
    """The exact arm (VKHIP_GEMM_EXACT: the oracle's bits) at 4096^3 NN, against
    the VALU rate of separately rounded multiplies and adds."""
    from vkml_amd import _lib
    from vkml_amd.device import DeviceArray

    m = n = k = 4096
    a = DeviceArray.from_numpy(rng.standard_normal((m, k), dtype=np.float32))
    b = DeviceArray.from_numpy(rng.standard_normal((k, n), dtype=np.float32))
    c = DeviceArray((m, n), np.float32)
    ms = time_batch(lambda i: ops.matmul(a, b, kernel=_lib.GEMM_EXACT, out=c), timer, 3, warmup=1)
    tf = 2.0 * m * n * k / ms / 1e9
    out[name] = {"ms": round(ms, 4), "tflops": round(tf, 2),
                 "frac_of_valu_separate": round(tf / VALU_FP32_SEPARATE_TFLOPS, 4),
                 "frac_of_mfma_peak": round(tf / MFMA_FP32_PEAK_TFLOPS, 4)}


def case_copy(name, hip, ops, timer, rng, out):
    """Practical HBM ceiling: the library's plain 16-byte copy, 4 x 256 MiB."""
    from vkml_amd.device import DeviceArray

    bufs = [DeviceArray((64 << 20,), np.float32) for _ in range(4)]
    ms = time_batch(lambda i: hip.copy_device_to_device([(bufs[(i + 1) % 4], bufs[i % 4])]), timer, 20)
    _bw(out, name, ms, 2 * (64 << 20) * 4)


def case_gemv(name, hip, ops, timer, rng, out):
    """GEMV 4096x4096 . 4096 (bandwidth): 8 rotated matrices (512 MB)."""
    from vkml_amd.device import DeviceArray

    mats = _rotate(rng, (4096, 4096), 8)
    x = DeviceArray.from_numpy(rng.standard_normal(4096, dtype=np.float32))
    y = DeviceArray((4096,), np.float32)
    ms = time_batch(lambda i: ops.gemv(mats[i % 8], x, out=y), timer, 40)
    _bw(out, name, ms, 4096 * 4096 * 4 + 4096 * 4 * 2)
    # the floor of one launch that reads these bytes: the library's row sum of
    # the same rotated matrices (the same reads, no vector, no products)
    ms_sum = time_batch(lambda i: ops.sum(mats[i % 8], [1], out=y), timer, 40)
    out[name]["row_sum_same_matrix_ms"] = round(ms_sum, 5)
    out[name]["frac_of_row_sum"] = round(ms_sum / ms, 4)


def case_im2col_col2im(name, hip, ops, timer, rng, out):
    """im2col / col2im conv2 [128,64,32,32] <-> [128,576,1024] (335.5 MB each way)."""
    from vkml_amd.device import DeviceArray

    imgs = _rotate(rng, (128, 64, 32, 32), 2)
    cols = [ops.im2col(im, 3, 1, 1) for im in imgs]
    img_out = DeviceArray((128, 64, 32, 32), np.float32)
    hip.synchronize()
    byt = 128 * 64 * 32 * 32 * 4 + 128 * 576 * 1024 * 4
    if name in ("im2col_conv2", "im2col_col2im"):
        ms = time_batch(lambda i: ops.im2col(imgs[i % 2], 3, 1, 1, out=cols[(i + 1) % 2]), timer, 20)
        _bw(out, "im2col_conv2", ms, byt)
    if name in ("col2im_conv2", "im2col_col2im"):
        ms = time_batch(lambda i: ops.col2im(cols[i % 2], (32, 32), 3, 1, 1, out=img_out), timer, 20)
        _bw(out, "col2im_conv2", ms, byt)


CONV_CASES = {"conv_128x64x32x32_c128": ((128, 64, 32, 32), 128),
              "conv_cnn1_128x3x32x32_c64": ((128, 3, 32, 32), 64),
              "conv_cnn2_128x64x16x16_c128": ((128, 64, 16, 16), 128)}


def case_conv(name, hip, ops, timer, rng, out):
    """Convolution forward and weight gradient: one implicit-im2col GEMM each,
    against the reference lowering (im2col into a column matrix, then the
    batch-broadcast GEMM)."""
    from vkml_amd.device import DeviceArray

    xs_shape, cout = CONV_CASES[name]
    n_, cin, h, w_ = xs_shape

    def roof(entry, flops, byt, ms):
        """frac_of_roofline: the larger of the two floors (MFMA FLOP, HBM
        bytes read + written once) over the measured time; `bound` names it."""
        t_flop = flops / (MFMA_FP32_PEAK_TFLOPS * 1e9)
        t_byte = byt / (HBM_PEAK_GBS * 1e6)
        entry["algorithmic_bytes"] = int(byt)
        entry["bound"] = "hbm" if t_byte > t_flop else "mfma"
        entry["frac_of_roofline"] = round(max(t_flop, t_byte) / ms, 4)
        entry["floor_us"] = round(max(t_flop, t_byte) * 1e3, 3)

    x_bytes, y_bytes = 4 * n_ * cin * h * w_, 4 * n_ * cout * h * w_
    w_bytes = 4 * cout * cin * 9
    x = DeviceArray.from_numpy(rng.standard_normal(xs_shape, dtype=np.float32))
    wt = DeviceArray.from_numpy(rng.standard_normal((cout, cin, 3, 3), dtype=np.float32))
    y = DeviceArray((n_, cout, h, w_), np.float32)
    ck, L = cin * 9, h * w_
    cols = DeviceArray((n_, ck, L), np.float32)
    wf = wt.reshape(1, 1, cout, ck).broadcast_to((1, n_, cout, ck))
    flops = 2.0 * n_ * cout * L * ck
    ms_i = time_batch(lambda i: ops.conv2d(x, wt, 1, 1, out=y), timer, 20)

    def explicit(i):
        ops.im2col(x, 3, 1, 1, out=cols)
        ops.matmul(wf, cols.reshape(1, n_, ck, L), out=y.reshape(1, n_, cout, L))

    ms_e = time_batch(explicit, timer, 20)
    out[name] = {"ms": round(ms_i, 5), "tflops": round(flops / ms_i / 1e9, 2),
                 "frac_of_peak": round(flops / ms_i / 1e9 / MFMA_FP32_PEAK_TFLOPS, 4),
                 "explicit_ms": round(ms_e, 5), "speedup_vs_explicit": round(ms_e / ms_i, 3)}
    roof(out[name], flops, x_bytes + w_bytes + y_bytes, ms_i)
    g = DeviceArray.from_numpy(rng.standard_normal((n_, cout, h, w_), dtype=np.float32))
    wg = DeviceArray((n_, cout, ck), np.float32)
    g4 = g.reshape(1, n_, cout, L)
    colsT = cols.reshape(1, n_, ck, L).transpose(-2, -1)
    ms_i = time_batch(lambda i: ops.conv2d_weight_grad(x, g, 3, 1, 1, out=wg), timer, 20)

    def explicit_wg(i):
        ops.im2col(x, 3, 1, 1, out=cols)
        ops.matmul(g4, colsT, out=wg.reshape(1, n_, cout, ck))

    ms_e = time_batch(explicit_wg, timer, 20)
    out[name.replace("conv_", "conv_wgrad_")] = {
        "ms": round(ms_i, 5), "tflops": round(flops / ms_i / 1e9, 2),
        "frac_of_peak": round(flops / ms_i / 1e9 / MFMA_FP32_PEAK_TFLOPS, 4),
        "explicit_ms": round(ms_e, 5), "speedup_vs_explicit": round(ms_e / ms_i, 3)}
    roof(out[name.replace("conv_", "conv_wgrad_")], flops,
         x_bytes + y_bytes + 4 * n_ * cout * cin * 9, ms_i)
    # dW itself (summed over the batch): the per-image products followed by
    # the batch SUM (the reference graph's two nodes) against one product
    # with the batch folded into K
    dw = DeviceArray((cout, ck), np.float32)

    def per_image_then_sum(i):
        ops.conv2d_weight_grad(x, g, 3, 1, 1, out=wg)
        ops.sum(wg, [0], out=dw)

    ms_s = time_batch(per_image_then_sum, timer, 20)
    ms_f = time_batch(lambda i: ops.conv2d_weight_grad_sum(x, g, 3, 1, 1, out=dw), timer, 20)
    out[name.replace("conv_", "conv_dw_")] = {
        "ms": round(ms_f, 5), "tflops": round(flops / ms_f / 1e9, 2),
        "frac_of_peak": round(flops / ms_f / 1e9 / MFMA_FP32_PEAK_TFLOPS, 4),
        "per_image_then_sum_ms": round(ms_s, 5), "speedup_vs_per_image": round(ms_s / ms_f, 3)}
    roof(out[name.replace("conv_", "conv_dw_")], flops, x_bytes + y_bytes + w_bytes, ms_f)
    # dX: the reference graph's TN product into the column matrix and col2im,
    # against one convolution of the gradient with the flipped weight
    dx = DeviceArray(xs_shape, np.float32)

    def tn_then_col2im(i):
        ops.matmul(wf.transpose(-2, -1), g4, out=cols.reshape(1, n_, ck, L))
        ops.col2im(cols, (h, w_), 3, 1, 1, out=dx)

    ms_t = time_batch(tn_then_col2im, timer, 20)
    ms_f = time_batch(lambda i: ops.conv2d_input_grad(g, wt, (h, w_), 1, 1, out=dx), timer, 20)
    out[name.replace("conv_", "conv_dx_")] = {
        "ms": round(ms_f, 5), "tflops": round(flops / ms_f / 1e9, 2),
        "frac_of_peak": round(flops / ms_f / 1e9 / MFMA_FP32_PEAK_TFLOPS, 4),
        "tn_then_col2im_ms": round(ms_t, 5), "speedup_vs_tn_col2im": round(ms_t / ms_f, 3)}
    roof(out[name.replace("conv_", "conv_dx_")], flops, y_bytes + w_bytes + x_bytes, ms_f)


SOFTMAX_CASES = {"softmax_4096x1000": ((4096, 1000), 20), "softmax_256x32768": ((256, 32768), 10)}


def case_softmax(name, hip, ops, timer, rng, out):
    """Softmax (read + write once), rotated past the MALL, against the
    library's plain copy of the same bytes (the floor of a one-pass kernel at
    that size, launch ramp and drain included)."""
    from vkml_amd.device import DeviceArray

    shape, count = SOFTMAX_CASES[name]
    xs = _rotate(rng, shape, count, 2.0)
    ys = [DeviceArray(shape, np.float32) for _ in range(2)]
    ms = time_batch(lambda i: ops.softmax(xs[i % count], -1, out=ys[i % 2]), timer, 40)
    _bw(out, name, ms, 2 * shape[0] * shape[1] * 4)
    flat = [xv.reshape(shape[0] * shape[1]) for xv in xs]
    yflat = [yv.reshape(shape[0] * shape[1]) for yv in ys]
    ms_copy = time_batch(lambda i: hip.copy_device_to_device([(yflat[i % 2], flat[i % count])]),
                         timer, 40)
    out[name]["copy_same_bytes_ms"] = round(ms_copy, 5)
    out[name]["frac_of_copy"] = round(ms_copy / ms, 4)


def case_reduce(name, hip, ops, timer, rng, out):
    """sum / max over the last axis of [8192, 4096] (134 MB read), 4 buffers."""
    from vkml_amd.device import DeviceArray

    xs = _rotate(rng, (8192, 4096), 4)
    r = DeviceArray((8192,), np.float32)
    fns = {"sum_8192x4096": ops.sum, "max_8192x4096": ops.amax}
    for key, fn in fns.items():
        if name in (key, "reduce_8192x4096"):
            ms = time_batch(lambda i: fn(xs[i % 4], [1], out=r), timer, 20)
            _bw(out, key, ms, 8192 * 4096 * 4 + 8192 * 4)


CASES = {**{k: case_gemm for k in GEMM_CASES}, "gemm_exact_4096": case_gemm_exact,
         "copy_256MiB": case_copy, "gemv_4096": case_gemv,
         "im2col_conv2": case_im2col_col2im, "col2im_conv2": case_im2col_col2im,
         **{k: case_conv for k in CONV_CASES}, **{k: case_softmax for k in SOFTMAX_CASES},
         "sum_8192x4096": case_reduce, "max_8192x4096": case_reduce}
DEFAULT_RUN = [k for k in GEMM_CASES if k != "gemm_nn_4096"] + [
    "gemm_exact_4096", "copy_256MiB", "gemv_4096", "im2col_col2im", *CONV_CASES, *SOFTMAX_CASES, "reduce_8192x4096"]
CASES["im2col_col2im"] = case_im2col_col2im
CASES["reduce_8192x4096"] = case_reduce


def secondary(hip, ops, timer, names=None):
    """The other hot-path kernels at BASELINE shapes: mean per-launch time of
    back-to-back launches into preallocated outputs."""
    rng = np.random.default_rng(7)
    out = {}
    for name in names or DEFAULT_RUN:
        if name not in CASES:
            raise SystemExit(f"unknown case {name!r}; known: {sorted(CASES)}")
        CASES[name](name, hip, ops, timer, rng, out)
    return out


def case_training(name, hip, ops, timer, rng, out):
    """One training config (config 1 "train_mlp" or config 5 "train_cnn") in
    every mode training_steps runs."""
    only = {"train_mlp": 1, "train_cnn": 5}[name]
    modes = tuple(m for m in _TRAIN_MODES_ARG.split(",") if m) or TRAIN_MODES
    unknown = set(modes) - set(TRAIN_MODES)
    if unknown:
        raise SystemExit(f"unknown training modes {sorted(unknown)}; known: {TRAIN_MODES}")
    out.update(training_steps(only=only, modes=modes))


_TRAIN_MODES_ARG = ""


TRAIN_MODES = ("dropin", "eager", "replay", "graph", "graph_queued", "resident", "resident_queued", "exact")


def _streams():
    """tests/golden/streams.py: the configs' seeded data streams, models and
    the committed CPU-oracle trajectories the parity tests compare against."""
    golden = ROOT / "tests" / "golden"
    if str(golden) not in sys.path:
        sys.path.insert(0, str(golden))
    import streams

    return streams


def _pinned_stream(hip, data):
    """The stream's batches in pinned host memory, as a data loader's reusable
    pinned buffers hold them, each DMA'd once to the device (untimed): the
    first DMA out of newly pinned pages costs several times a later one, and a
    loader's buffers are reused epoch after epoch."""
    import ctypes

    from vkml_amd import _lib
    from vkml_amd.device import DeviceArray, Event, pinned_copy

    pinned = [(pinned_copy(x), pinned_copy(y)) for x, y in data]
    done = Event()
    scratch = {}
    for pair in pinned:
        for a in pair:
            key = (a.shape, a.dtype.str)
            if key not in scratch:
                scratch[key] = DeviceArray(a.shape, a.dtype)
            _lib.check(hip.lib.vkhip_copy_from_host_async(
                ctypes.c_void_p(scratch[key].ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes, None,
                ctypes.c_void_p(done.handle)), "copy_from_host_async")
    done.synchronize()
    return pinned


def training_steps(only: int | None = None, modes=TRAIN_MODES):
    """BASELINE configs 1 and 5 as training loops on the device, on the very
    streams the parity tests check (tests/golden/streams.py: 100 steps, a
    fresh seeded batch per step, all generated before the timed loop), each
    mode from freshly initialised weights:

      dropin        the reference's node graph only (tensor.reference_graph(),
                    SGD(fused=False)), built and flushed every step: what
                    vkML's executor would hand a drop-in HipBackend::compute
      eager         the host core's rewritten graph, built every step
      replay        the step recorded once, its calls replayed from C; each
                    call uploads the next batch on the copy stream while its
                    step runs (CapturedStep prefetch; the stream's batches in
                    pinned host memory, which the DMA reads in place), and
                    reads its loss back
      graph         the replay captured once into a HIP graph
      graph_queued  "graph" with no per-step loss read-back: the host queues
                    step after step, the last loss is read inside the timed
                    region
      resident      "replay" with the stream's batches resident in HBM
                    (uploaded before the timed loop, 157 MB for config 5):
                    each step copies its batch on the device instead of
                    uploading it from the host, and reads its loss back
      resident_queued  "resident" with no per-step read-back: each step's
                    loss is copied on the device into a 100-entry log that is
                    read once, inside the timed region
      exact         "replay" in the exact numerics mode (vkhip_set_numerics):
                    every node the oracle's bits

    Step 0 (the recording, for the replayed modes) is untimed; steps 1-99 are
    timed by wall clock, each step uploading its batch and (but for
    graph_queued) reading its loss back. Every mode reports its largest loss
    drift over the 100 steps from the committed oracle trajectory
    (tests/golden/config*_losses.json) and the step where it occurs;
    graph_queued reads only its last loss, which must be the graph mode's
    bits, and reports the graph mode's drift. `oracle_libm_drift` is the
    distance between the oracle trajectory with its named exp/log and with
    the platform libm's (the reference's std::exp / std::log): how far two
    valid builds of the reference's own CPU arithmetic separate."""
    from vkml_amd import nn, optim
    from vkml_amd import tensor as T
    from vkml_amd.device import DeviceArray

    S = _streams()
    hip = T.default_backend().hip
    res = {}
    for num, cfg in S.CONFIGS.items():
        if only is not None and num != only:
            continue
        data = list(S.batches(cfg))
        want = S.oracle_losses(cfg)
        envelope, env_step = S.max_drift(want, S.oracle_losses(cfg, libm=True))
        pinned = None
        entry = {"steps": cfg.steps, "timed_steps": cfg.steps - 1, "stream": "tests/golden/streams.py",
                 "oracle_fixture": S.fixture_path(cfg).name,
                 "oracle_libm_drift": envelope, "oracle_libm_drift_step": env_step}
        for mode in modes:
            nn.manual_seed(cfg.model_seed)
            ref_ctx = T.reference_graph() if mode == "dropin" else None
            if mode == "exact":
                hip.set_numerics("exact")
            try:
                if ref_ctx:
                    ref_ctx.__enter__()
                model = S.model(cfg)
                opt = optim.SGD(model.parameters(), lr=cfg.lr, momentum=cfg.momentum,
                                fused=mode != "dropin")

                def fn(x, y):
                    opt.zero_grad()
                    loss = nn.cross_entropy(model(x), y)
                    loss.backward()
                    opt.step()
                    return loss

                losses = []
                captured = None
                if mode in ("dropin", "eager"):
                    def step(i):
                        x, y = data[i]
                        return fn(T.tensor(x), T.tensor(y)).item()
                    losses.append(step(0))
                else:
                    captured = T.CapturedStep(fn, *data[0], graph=mode.startswith("graph"))
                    losses.append(float(captured.first[0]))
                    queued = mode == "graph_queued"
                    # host-fed modes read their batches from pinned host memory, as a
                    # data loader with pinned buffers fills them (the DMA reads them in
                    # place), allocated and mapped once per configuration (_pinned_stream)
                    if pinned is None:
                        pinned = _pinned_stream(hip, data)
                    feed = pinned
                    if mode.startswith("resident"):
                        feed = [(DeviceArray.from_numpy(x), DeviceArray.from_numpy(y)) for x, y in data]
                    if mode == "resident_queued":
                        loss_t = captured.outputs[0]
                        log = DeviceArray((cfg.steps,) + tuple(loss_t.shape), np.float32)

                        def step(i):
                            captured(*feed[i], read=False)
                            captured.outputs_to(DeviceArray(loss_t.shape, np.float32, None, log.buffer,
                                                            offset=i * max(loss_t.numel(), 1)))
                    else:
                        ahead = not mode.startswith("resident")  # host batches: upload i + 1 during step i

                        def step(i):
                            nxt = feed[i + 1] if ahead and i + 1 < cfg.steps else None
                            out = captured(*feed[i], read=not queued, prefetch=nxt)
                            return None if out is None else float(out[0])
                # the collector runs before the timed loop, not inside it (the
                # eager modes leave many graph objects behind; a full
                # collection inside a ~40 ms loop costs ~0.1 ms/step), as timeit does
                gc.collect()
                gc.disable()
                hip.synchronize()
                t0 = time.perf_counter()
                if captured is not None and not mode.startswith("resident"):
                    captured.prefetch(*feed[1])
                for i in range(1, cfg.steps):
                    losses.append(step(i))
                if mode == "graph_queued":
                    losses[-1] = float(captured.outputs_now()[0])
                if mode == "resident_queued":
                    losses[1:] = [float(v) for v in log.numpy().reshape(cfg.steps, -1)[1:, 0]]
                dt = time.perf_counter() - t0
            finally:
                gc.enable()
                if ref_ctx:
                    ref_ctx.__exit__(None, None, None)
                if mode == "exact":
                    hip.set_numerics("fast")
            timed = cfg.steps - 1
            out = {"ms_per_step": round(dt * 1e3 / timed, 4), "steps_per_s": round(timed / dt, 2),
                   "last_loss": losses[-1]}
            if mode == "graph_queued" and "graph" not in entry:
                out["max_loss_drift_vs_oracle"] = None
                out["drift_from"] = "graph mode not run"
            elif mode == "graph_queued":
                same = np.float32(losses[-1]).tobytes() == np.float32(entry["graph"]["last_loss"]).tobytes()
                out["last_loss_same_bits_as_graph"] = bool(same)
                out["max_loss_drift_vs_oracle"] = entry["graph"]["max_loss_drift_vs_oracle"] if same else None
                out["drift_from"] = "graph (same steps; last loss checked bit for bit)"
            else:
                got = np.array(losses, np.float32)
                d, at = S.max_drift(got, want)
                out["max_loss_drift_vs_oracle"] = d
                out["max_drift_step"] = at
                out["steps_within_1e-4"] = int(np.argmax(np.abs(got.astype(np.float64) - want) > 1e-4)) \
                    if d > 1e-4 else cfg.steps
                out["bit_identical_steps"] = int(np.sum(got.view(np.uint32) == want.view(np.uint32)))
            if captured is not None:
                out.update(captured.info())
                captured.close()
            entry[mode] = out
        res[cfg.key] = entry
    return res


CASES["train_mlp"] = case_training
CASES["train_cnn"] = case_training


def read_traffic(args):
    """HBM bytes per launch of the headline GEMM, from the committed rocprofv3
    PMC summary (FETCH_SIZE + WRITE_SIZE, each scaled by the copy-kernel
    calibration in the same summary); None when no summary matches."""
    path = ROOT / "profiles" / f"gemm_nn_{args.m}x{args.n}x{args.k}_pmc.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not implemented)"}))
        sys.exit(2)
    from vkml_amd import ops
    from vkml_amd.device import backend

    hip = backend()
    timer = Timer()
    if args.case:
        global _GATE_ON, _TRAIN_MODES_ARG
        _GATE_ON = not args.no_gate
        _TRAIN_MODES_ARG = args.train_modes
        names = [c for c in args.case.split(",") if c]
        print(json.dumps({"cases": secondary(hip, ops, timer, names), "gate": _GATE_ON}), flush=True)
        return
    value, ms_step, avg_ms, achieved, min_ms, warm = gemm_headline(args, hip, ops, timer)
    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_launches": warm,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"gemm_nn_{args.m}x{args.n}x{args.k}_fp32", "m": args.m,
                   "n": args.n, "k": args.k, "layout": "NN", "parallelism": "none"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3),
                     "peak": MFMA_FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_FP32_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "gemm_nn_direct_kernel",
                     "avg_launch_ms": round(avg_ms, 4), "min_launch_ms": round(min_ms, 4)},
    }
    if args.calibrate:
        from vkml_amd.device import DeviceArray

        src, dst = DeviceArray((64 << 20,), np.float32), DeviceArray((64 << 20,), np.float32)
        for _ in range(5):
            hip.copy_device_to_device([(dst, src)])
        hip.synchronize()
    traffic = read_traffic(args)
    if traffic is not None:
        result["roofline"]["traffic"] = traffic
    if not args.no_secondary:
        result["secondary"] = secondary(hip, ops, timer)
        result["training"] = training_steps()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
