#!/usr/bin/env python
"""bench.py — MI355X measurement of vkflame's quantized-linear hot path.

One step = one pass of the hot path over one batch: the Q4_K decode GEMV of
the 14B-class FFN (W 13824x5120 Q4_K, x fp16 [1, 5120], y fp32), reading its
weights cold from HBM.  The timed graph holds exactly --steps launches, each
on the next of a set of weight copies totalling more than 1 GiB, so the
256 MB Infinity Cache never holds a launch's weights; it is replayed
--replays times (at least 50), each replay bracketed by HIP events on the
stream the graph runs on, and the headline is the median replay's time per
launch.  torch.cuda.synchronize() brackets the timed region.

Prints ONE JSON line (the benchmark contract) with:
  value      effective weight GB/s of the primary step (BASELINE metric),
  roofline   the GEMV kernel's algorithmic bytes (weights + x + y) per launch
             / its median launch duration, against 8 TB/s HBM,
  cpu_baseline  the numpy port (oracle/oracle.py) on the box's host cores:
             the primary step and one line per BASELINE configuration, with
             the dequantisation and the BLAS product timed separately,
  suite      every BASELINE configuration (GEMV GB/s and GEMM TOPS with the
             fraction of the MI355X roofline), measured the same way.
Diagnostics go to stderr.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--replays R]
                       [--no-suite] [--no-cpu] [--no-primary] [--suite-only S]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)


def _cpu_threads() -> int:
    """Host threads for the CPU baseline: the affinity mask, capped by the
    thread count the box grants this job (OMP_NUM_THREADS)."""
    n = len(os.sched_getaffinity(0))
    try:
        n = min(n, int(os.environ.get("OMP_NUM_THREADS", n)))
    except ValueError:
        pass
    return max(1, n)


# numpy's BLAS reads its thread count when numpy is first imported
CPU_THREADS = _cpu_threads()
for _v in ("OPENBLAS_NUM_THREADS", "OMP_NUM_THREADS", "MKL_NUM_THREADS"):
    os.environ.setdefault(_v, str(CPU_THREADS))

METRIC = "Q4_K/Q8_0 GEMV weight GB/s + int8/fp16 GEMM TOPS, % of MI355X roofline"
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0
ROTATE_BYTES = 1 << 30
SUITE_GEMV_LAUNCHES = 200


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _seed(cfg, sub=0):
    return 1000 + 10 * cfg + sub


def median(v):
    s = sorted(v)
    n = len(s)
    return s[n // 2] if n % 2 else 0.5 * (s[n // 2 - 1] + s[n // 2])


def time_graph(torch, launches, replays: int, warmup_launches: int = 0) -> list[float]:
    """Captures `launches` (zero-argument callables) in one HIP graph, replays
    it `replays` times back to back and returns each replay's time per launch
    in ms, from HIP events recorded on the stream the graph runs on."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in launches[:2]:      # eager warm-up (module load, first touch)
            f()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    # captured on the warm-up stream: launches that keep per-stream state
    # (the stream-K GEMM's workspace, made on a stream's first eager call)
    # find it there
    with torch.cuda.graph(g, stream=s):
        for f in launches:
            f()
    for _ in range(max(1, math.ceil(warmup_launches / len(launches)))):
        g.replay()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
    torch.cuda.synchronize()
    for e0, e1 in ev:
        e0.record(stream)
        g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    out = [e0.elapsed_time(e1) / len(launches) for e0, e1 in ev]
    del g
    return out


def _rotating_copies(torch, base, nbytes_each, at_least=2):
    n = max(at_least, int(ROTATE_BYTES // max(nbytes_each, 1)) + 1)
    return [base] + [base.clone() for _ in range(n - 1)]


def gemv_case(torch, ops, O, qt, N, K, M, xkind, seed, replays, quant_on_gpu=False):
    """Returns (median ms per launch, weight bytes, algorithmic bytes per
    launch, median Q8_1 quantise ms or None)."""
    import numpy as np
    dev = torch.device("cuda:0")
    w = torch.from_numpy(O.gen_weight(qt, N, K, seed)).to(dev)
    wbytes = w.numel()
    copies = _rotating_copies(torch, w, wbytes)
    rng = np.random.default_rng(seed + 1)
    x32 = rng.normal(0, 1, (M, K)).astype(np.float32)
    if xkind == "f16":
        x = torch.from_numpy(x32.astype(np.float16)).to(dev)
        xbytes = M * K * 2
    elif xkind == "f32":
        x = torch.from_numpy(x32).to(dev)
        xbytes = M * K * 4
    else:
        xf = torch.from_numpy(x32).to(dev)
        x = ops.quantize_q8_1(xf)
        xbytes = M * (K // 32) * 36
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    # as many launches per graph as the primary step's default, cycling over
    # the copies, so that the graph's own start is spread as thinly
    launches = [(lambda c=copies[i % len(copies)]: ops.gemm_q(c, qt, x, N, K, out=y))
                for i in range(max(SUITE_GEMV_LAUNCHES, len(copies)))]
    ms = median(time_graph(torch, launches, replays))
    t_q = None
    if quant_on_gpu:
        t_q = median(time_graph(torch, [lambda: ops.quantize_q8_1(xf)] * 8, replays))
    del copies, w
    torch.cuda.empty_cache()
    return ms, wbytes, wbytes + xbytes + M * N * 4, t_q


def run_suite(torch, ops, O, replays, only=None):
    import numpy as np
    dev = torch.device("cuda:0")
    out = []

    def want(name):
        return only is None or any(o in name for o in only.split("|"))

    def gemv_line(name, qt, N, K, M, xkind, cfg, sub, quant=False):
        if not want(name):
            return
        ms, wb, ab, tq = gemv_case(torch, ops, O, qt, N, K, M, xkind, _seed(cfg, sub), replays, quant)
        gbs = wb / (ms * 1e-3) / 1e9
        line = {"config": name, "kernel_us": round(ms * 1e3, 2), "weight_GBps": round(gbs, 1),
                "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                "algorithmic_GBps": round(ab / (ms * 1e-3) / 1e9, 1)}
        if tq is not None:
            line["q8_1_quantize_us"] = round(tq * 1e3, 2)
            line["with_quantize_weight_GBps"] = round(wb / ((ms + tq) * 1e-3) / 1e9, 1)
        log(json.dumps(line))
        out.append(line)

    gemv_line("C1 Q8_0 GEMV 4096x4096 M=1 x fp32", O.Q8_0, 4096, 4096, 1, "f32", 1, 0)
    for qt, nm in ((O.Q4_0, "Q4_0"), (O.Q4_1, "Q4_1")):
        for M in (1, 4, 16):
            gemv_line(f"C2 {nm} GEMV 11008x4096 M={M} x fp16", qt, 11008, 4096, M, "f16", 2, qt * 3 + M)
    for (N, K) in ((13824, 5120), (5120, 13824)):
        for M in (1, 8):
            gemv_line(f"C3 Q4_K GEMV {N}x{K} M={M} x fp16", O.Q4_K, N, K, M, "f16", 3, M + (0 if N == 13824 else 5))
    gemv_line("C5 Q6_K x Q8_1 GEMV 152064x5120 M=1", O.Q6_K, 152064, 5120, 1, "q8_1", 5, 0, quant=True)

    def gemm_line(name, flops, peak, unit_peak, fn_list):
        ms = median(time_graph(torch, fn_list, max(5, replays // 4)))
        t = flops / (ms * 1e-3) / 1e12
        line = {"config": name, "kernel_us": round(ms * 1e3, 2), "TOPS": round(t, 1),
                "mfma_frac": round(t / peak, 4), "peak_TOPS": peak, "peak": unit_peak,
                "weight_copies": len(fn_list)}
        log(json.dumps(line))
        out.append(line)

    # C3 prefill, both shapes: Q4_K weights (rotated), x fp16 [512, K]
    for (N, K, sub) in ((13824, 5120, 0), (5120, 13824, 5)):
        name = f"C3 Q4_K prefill 512x{N}x{K} (weights decoded to fp16 between fp16 MFMA steps)"
        if not want(name):
            continue
        M = 512
        w = torch.from_numpy(O.gen_weight(O.Q4_K, N, K, _seed(3, sub))).to(dev)
        copies = _rotating_copies(torch, w, w.numel())
        x = torch.from_numpy(np.random.default_rng(_seed(3, 512 + sub)).normal(0, 1, (M, K)).astype(np.float16)).to(dev)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        gemm_line(name, 2.0 * M * N * K, FP16_PEAK_TFLOPS, "fp16 dense MFMA",
                  [(lambda c=c: ops.gemm_q(c, O.Q4_K, x, N, K, out=y)) for c in copies])
        del w, copies, x, y
        torch.cuda.empty_cache()
    # C4 int8 linear: weights and activations rotated
    name = "C4 int8 linear 512x5120x5120 (+scales, bias, fp16 out)"
    if want(name):
        M, N, K = 512, 5120, 5120
        inp = O.gen_int8_linear(M, N, K, _seed(4))
        A, W = torch.from_numpy(inp.A).to(dev), torch.from_numpy(inp.W).to(dev)
        Ws = _rotating_copies(torch, W, W.numel() + A.numel())
        As = [A] + [A.clone() for _ in range(len(Ws) - 1)]
        a_s, w_s = torch.from_numpy(inp.a_scale).to(dev), torch.from_numpy(inp.w_scale).to(dev)
        bias = torch.from_numpy(inp.bias).to(dev)
        D = torch.empty((M, N), dtype=torch.float16, device=dev)
        gemm_line(name, 2.0 * M * N * K, INT8_PEAK_TOPS, "int8 dense MFMA",
                  [(lambda a=a, wc=wc: ops.linear_int8(a, a_s, wc, w_s, bias, out=D)) for a, wc in zip(As, Ws)])
        del A, W, Ws, As, D
        torch.cuda.empty_cache()
    # C5 prefill: Q6_K x Q8_1, M = 512, full vocab projection (two weight copies, 1.28 GB)
    name = "C5 Q6_K x Q8_1 prefill 512x152064x5120 (activations decoded once to fp16, weight tiles between MFMA steps)"
    if want(name):
        N, K, M = 152064, 5120, 512
        w = torch.from_numpy(O.gen_weight(O.Q6_K, N, K, _seed(5))).to(dev)
        copies = _rotating_copies(torch, w, w.numel())
        xf = torch.from_numpy(np.random.default_rng(_seed(5, 1)).normal(0, 1, (M, K)).astype(np.float32)).to(dev)
        xq = ops.quantize_q8_1(xf)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        gemm_line(name, 2.0 * M * N * K, INT8_PEAK_TOPS, "int8 dense MFMA (the config's 'integer dot' peak)",
                  [(lambda c=c: ops.gemm_q(c, O.Q6_K, xq, N, K, out=y)) for c in copies])
        del w, copies, xf, xq, y
        torch.cuda.empty_cache()
    # dense fp16 linear (vkflame_dispatch_linear / hipblasGemmEx): the M = 512
    # FFN shape, and the six torch.mm shapes of the reference's only published
    # run (added-files/Test-Run-RCOM-Vulkan.md:22-27; torch.mm(a, b) with a
    # contiguous b is B [K, N], the NN layout), B rotated through cold copies;
    # torch.mm on the same inputs (ROCm's library) timed beside for context
    from vkflame_amd._lib import DTYPE_FP16
    dense = [("fp16 linear 512x5120x5120 NT (B [N, K])", 512, 5120, 5120, 1)]
    dense += [(f"fp16 torch.mm ({m},{k},{n}) NN (B [K, N])", m, n, k, 0)
              for (m, k, n) in ((256, 256, 256), (1024, 1024, 1024), (4096, 4096, 4096), (1, 4096, 4096),
                                (32, 4096, 4096), (128, 8192, 8192))]
    for (name, M, N, K, tb) in dense:
        if not want(name):
            continue
        rng = np.random.default_rng(_seed(6, M + N + K + tb))
        a = torch.from_numpy(rng.normal(0, 1, (M, K)).astype(np.float16)).to(dev)
        b = torch.from_numpy(rng.normal(0, 1, (N, K) if tb else (K, N)).astype(np.float16)).to(dev)
        # at most 64 copies: a B of a few MB stays in the 256 MB MALL whatever
        # the rotation, so small shapes gain nothing from thousands of copies
        copies = _rotating_copies(torch, b, max(b.numel() * 2, ROTATE_BYTES // 64))
        d = torch.empty((M, N), dtype=torch.float16, device=dev)
        nl = max(32, len(copies))
        fl = 2.0 * M * N * K
        ms = median(time_graph(torch, [(lambda c=copies[i % len(copies)]: ops.linear(a, c, M, N, K, DTYPE_FP16,
                                                                                      transB=tb, out=d))
                                       for i in range(nl)], max(5, replays // 4)))
        bt = [c.t() if tb else c for c in copies]  # torch.mm(a, B) with B [K, N]
        ms_t = median(time_graph(torch, [(lambda c=bt[i % len(bt)]: torch.mm(a, c, out=d)) for i in range(nl)],
                                 max(5, replays // 4)))
        t = fl / (ms * 1e-3) / 1e12
        line = {"config": name, "kernel_us": round(ms * 1e3, 2), "TOPS": round(t, 2),
                "mfma_frac": round(t / FP16_PEAK_TFLOPS, 4), "peak_TOPS": FP16_PEAK_TFLOPS, "peak": "fp16 dense MFMA",
                "B_GBps": round(b.numel() * 2 / (ms * 1e-3) / 1e9, 1),
                "hbm_frac_B": round(b.numel() * 2 / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "torch_mm_us": round(ms_t * 1e3, 2), "weight_copies": len(copies)}
        log(json.dumps(line))
        out.append(line)
        del a, b, copies, bt, d
        torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------
# CPU baseline: the oracle's numpy port on the host cores
# ---------------------------------------------------------------------------

def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _blas_name() -> str:
    try:
        import numpy as _np
        return _np.__config__.CONFIG["Build Dependencies"]["blas"]["name"]
    except Exception:
        return "unknown"


def _par_dequant(O, pool, qt, w, chunks):
    """np_dequant over row chunks on the thread pool (numpy releases the GIL
    in the vectorised work)."""
    import numpy as np
    parts = list(pool.map(lambda r: O.np_dequant(qt, w[r[0]:r[1]]), chunks))
    return np.concatenate(parts)


def cpu_baseline(O, budget_s: float = 25.0):
    """The numpy port of every configuration on the host: dequantise with
    O.np_dequant on all CPU_THREADS threads (row chunks), then the product
    through numpy's BLAS.  Each line is the median of 3 runs after one
    warm-up, on a row sample of the weights where the full matrix would
    exceed the time budget (rates scale with rows)."""
    import concurrent.futures as cf
    import numpy as np
    t_start = time.perf_counter()
    pool = cf.ThreadPoolExecutor(CPU_THREADS)
    lines = []

    def run(name, qt, N, K, M, rows, unit, x_f16=True, int8=None):
        rng = np.random.default_rng(7)
        if int8 is not None:
            A, W = int8
            Af, Wf = A.astype(np.float64), W.astype(np.float64)   # exact: |acc| < 2^53
            deq = lambda: None                                      # noqa: E731
            prod = lambda _: Af @ Wf.T                              # noqa: E731
            work = 2.0 * A.shape[0] * W.shape[0] * A.shape[1]
        else:
            w = O.gen_weight(qt, rows, K, 100 + qt)
            x = rng.normal(0, 1, (M, K)).astype(np.float16 if x_f16 else np.float32).astype(np.float32)
            # small row chunks (measured faster than one per thread: each
            # chunk's temporaries stay in cache)
            step = max(64, rows // (8 * CPU_THREADS))
            chunks = [(i, min(rows, i + step)) for i in range(0, rows, step)]
            deq = lambda: _par_dequant(O, pool, qt, w, chunks).reshape(rows, K)  # noqa: E731
            prod = lambda wd: x @ wd.T                                          # noqa: E731
            work = w.nbytes if unit == "GB/s" else 2.0 * M * rows * K
        td, tp = [], []
        for i in range(4):
            t0 = time.perf_counter()
            wd = deq()
            t1 = time.perf_counter()
            prod(wd)
            t2 = time.perf_counter()
            if i:
                td.append(t1 - t0)
                tp.append(t2 - t1)
        d_s, p_s = median(td), median(tp)
        tot = d_s + p_s
        val = work / tot / 1e9 if unit == "GB/s" else work / tot / 1e12
        line = {"config": name, "value": round(val, 4), "unit": unit, "dequant_ms": round(d_s * 1e3, 2),
                "blas_ms": round(p_s * 1e3, 2), "rows_sampled": rows, "rows_full": N}
        log("cpu " + json.dumps(line))
        lines.append(line)
        return line

    primary = run("C3 Q4_K GEMV 13824x5120 M=1 (primary)", O.Q4_K, 13824, 5120, 1, 13824, "GB/s")
    plan = [
        ("C1 Q8_0 GEMV 4096x4096 M=1 x fp32", O.Q8_0, 4096, 4096, 1, 4096, "GB/s", False),
        ("C2 Q4_0 GEMV 11008x4096 M=1", O.Q4_0, 11008, 4096, 1, 11008, "GB/s", True),
        ("C2 Q4_1 GEMV 11008x4096 M=16", O.Q4_1, 11008, 4096, 16, 11008, "GB/s", True),
        ("C3 Q4_K GEMV 5120x13824 M=8", O.Q4_K, 5120, 13824, 8, 5120, "GB/s", True),
        ("C5 Q6_K x Q8_1 GEMV 152064x5120 M=1", O.Q6_K, 152064, 5120, 1, 19008, "GB/s", False),
        ("C3 Q4_K prefill 512x13824x5120", O.Q4_K, 13824, 5120, 512, 3456, "TOPS", True),
        ("C5 Q6_K x Q8_1 prefill 512x152064x5120", O.Q6_K, 152064, 5120, 512, 4752, "TOPS", False),
    ]
    for (name, qt, N, K, M, rows, unit, xf16) in plan:
        if time.perf_counter() - t_start > budget_s:
            log(f"cpu baseline: time budget reached, skipped {name}")
            continue
        run(name, qt, N, K, M, rows, unit, xf16)
    if time.perf_counter() - t_start <= budget_s:
        inp = O.gen_int8_linear(512, 5120, 5120, _seed(4))
        run("C4 int8 linear 512x5120x5120", None, 5120, 5120, 512, 5120, "TOPS", int8=(inp.A, inp.W))
    pool.shutdown()
    return {"value": primary["value"], "unit": "GB/s", "cores": CPU_THREADS, "kind": "port",
            "cpu_model": _cpu_model(), "blas": _blas_name(),
            "dequant_ms": primary["dequant_ms"], "gemv_ms": primary["blas_ms"],
            "sample": (f"numpy port (oracle/oracle.py): full 13824x5120 Q4_K weight, M=1, dequant on "
                       f"{CPU_THREADS} threads (row chunks) then x @ W^T through {_blas_name()}; median of 3 "
                       f"after 1 warm-up; configs below on the stated row samples"),
            "configs": lines}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="launches in the timed graph")
    ap.add_argument("--warmup", type=int, default=20, help="untimed launches before the timed replays")
    ap.add_argument("--replays", type=int, default=50, help="timed replays of the graph (at least 50)")
    ap.add_argument("--no-suite", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-primary", action="store_true",
                    help="suite lines only, to stderr (profiling runs); no contract line")
    ap.add_argument("--suite-only", default=None,
                    help="run only suite lines whose name contains one of these '|'-separated strings")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="only run 10 plain device copies of this many MiB (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build's path runs on a single MI355X "
              f"(got --gpus {args.gpus}); multi-GPU sharding is a design note, not a measured mode.",
              file=sys.stderr)
        sys.exit(2)
    steps = max(1, args.steps)
    replays = max(50, args.replays)

    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    from vkflame_amd import ops

    dev = torch.device("cuda:0")
    if args.calib_copy_mib:
        # A copy of known size: its FETCH_SIZE / WRITE_SIZE per dispatch give
        # the factor between those counters and bytes moved.
        n = args.calib_copy_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: 10 x {n} bytes")
        return
    props = torch.cuda.get_device_properties(0)
    log(f"device: {props.name} {props.gcnArchName} CUs={props.multi_processor_count}")
    if args.no_primary:
        run_suite(torch, ops, O, replays=20, only=args.suite_only)
        return

    # ---- primary step: C3 Q4_K decode GEMV 13824x5120, M=1 ----
    N, K, M = 13824, 5120, 1
    seed = _seed(3)
    w = torch.from_numpy(O.gen_weight(O.Q4_K, N, K, seed)).to(dev)
    wbytes = w.numel()
    copies = _rotating_copies(torch, w, wbytes)
    x = torch.from_numpy(np.random.default_rng(seed + 1).normal(0, 1, (M, K)).astype(np.float16)).to(dev)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    launches = [(lambda c=copies[i % len(copies)]: ops.gemm_q(c, O.Q4_K, x, N, K, out=y)) for i in range(steps)]
    torch.cuda.synchronize()
    per_replay = time_graph(torch, launches, replays, warmup_launches=args.warmup)
    torch.cuda.synchronize()
    ms = median(per_replay)
    # correctness of the measured configuration (one extra launch, checked on rows)
    ops.gemm_q(copies[0], O.Q4_K, x, N, K, out=y)
    torch.cuda.synchronize()
    rows = np.arange(0, N, 97)
    ref = O.ref_gemv(x.cpu().numpy().astype(np.float64),
                     O.np_dequant(O.Q4_K, w.cpu().numpy()[rows]).reshape(len(rows), K))
    err = O.max_rel_err(y.cpu().numpy()[:, rows], ref)
    log(f"primary: median {ms * 1e3:.2f} us/launch (min {min(per_replay) * 1e3:.2f}, max "
        f"{max(per_replay) * 1e3:.2f}) over {replays} replays of {steps} launches, {len(copies)} rotating copies, "
        f"max rel err {err:.2e}")
    # measured read-bandwidth reference: a plain coalesced read of the same
    # weight copies, timed the same way (library kernel vkf_stream_read)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    s_launches = [(lambda c=copies[i % len(copies)]: ops.stream_read(c, sink)) for i in range(steps)]
    ms_stream = median(time_graph(torch, s_launches, replays, warmup_launches=args.warmup))
    stream_gbs = wbytes / (ms_stream * 1e-3) / 1e9
    log(f"stream read of the same {wbytes} B: {ms_stream * 1e3:.2f} us/launch, {stream_gbs:.0f} GB/s")
    del copies
    torch.cuda.empty_cache()

    value = wbytes / (ms * 1e-3) / 1e9
    alg_bytes = wbytes + M * K * 2 + M * N * 4
    achieved = alg_bytes / (ms * 1e-3) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_q4_k_gemv_13824x5120.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "vkf_gemv_dotl_q4_k_f16", "algorithmic_bytes_per_launch": alg_bytes,
                "launch_us_median": round(ms * 1e3, 3),
                "stream_read_GBps": round(stream_gbs, 1), "frac_of_stream_read": round(value / stream_gbs, 4)}

    suite = None if args.no_suite else run_suite(torch, ops, O, replays=20, only=args.suite_only)
    cpu = None if args.no_cpu else cpu_baseline(O)

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "replays": replays, "ms_per_step": round(ms, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k x i8 (v_dot4, i32 acc) -> f32",
        "data": "synthetic (seeded ggml blocks per BASELINE configs)",
        "config": {"workload": "C3 Q4_K decode GEMV: W 13824x5120 Q4_K (39.8 MB, cold), x fp16 [1,5120], "
                               "y fp32 [1,13824]", "global_batch": 1, "seq_len": 1, "parallelism": "single GPU",
                   "max_rel_err": err,
                   "timing": f"median over {replays} graph replays of {steps} launches, HIP events"},
        "roofline": roofline, "cpu_baseline": cpu, "suite": suite,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
