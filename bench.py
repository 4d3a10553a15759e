#!/usr/bin/env python3
"""MhcPre benchmark on one MI355X: tokens/s and achieved HBM bandwidth.

Workload (default): the headline prefill shape n=4, D=7168, T=8192, bf16 x,
gamma on -- one "step" is one MhcPre launch over all T rows with every input
already resident in HBM.  Prints ONE JSON line.

  value      tokens/s = T / (mean launch time): the timed steps are launched
             back to back between one pair of HIP events recorded on the
             launch stream
  roofline   algorithmic bytes per launch / mean launch time, against 8 TB/s;
             bytes = x + phi + gamma + bias + alpha + hIn + hPost + hRes, each
             counted once (hPre is not part of the operator contract);
             traffic = HBM bytes per launch from the committed rocprofv3 PMC
             record for the workload (profiles/*.traffic.json), when present
  cpu_baseline  the scalar C oracle (reference floating-point order), OpenMP
             over rows on the host's cores, timed on a bounded sample of the
             same inputs (about --cpu-seconds of work), and beside it the same
             oracle on one thread (bitwise identical results) and the CPU model

Before the --warmup launches, launches run back to back for --settle-ms of
wall time (the device's clocks take about 20 ms of load to settle; reported
as settle_ms / settle_launches).  Also reported, outside the timed region:
  host_latency_us  the reference harness's method (cloud_runner/runner.cpp:
             458-490): 1 warm-up, then 20 x (launch + stream synchronize)
             timed on the host clock; min / median / avg
  cold_us    per-launch event-timed duration after a 512 MiB scratch write
             (evicts the 256 MB MALL); the roofline figure for workloads whose
             working set fits the MALL (configs 1, 2 and 4)
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E peak, GB/s
COPY_BYTES = 256 << 20  # size of the calibration copy (--copy-probe)
CEILING_BYTES = 512 << 20  # size of the copy whose rate is reported as the measured ceiling

WORKLOADS = {
    # name: (n, D, T, bf16, gamma, outlier rows x50)
    1: (4, 256, 128, False, False, False),
    2: (4, 4096, 1024, True, True, False),
    3: (4, 7168, 8192, True, True, False),
    4: (8, 7168, 64, False, False, False),
    5: (8, 8192, 5472, True, True, True),
}
METRIC = "MhcPre tokens/s + achieved HBM GB/s (% of peak), n=4 D=7168 T=8192 bf16"


def algorithmic_bytes(n: int, D: int, T: int, bf16_or_f16: bool, gamma: bool) -> int:
    sx = 2
    M = n * n + 2 * n
    K = n * D
    b = T * K * sx + K * M * 4 + (K * 4 if gamma else 0) + M * 4 + 12
    b += T * D * sx + T * n * 4 + T * n * n * 4
    return b


def make_inputs(cfg: int, device):
    import torch

    n, D, T, bf16, gamma, outliers = WORKLOADS[cfg]
    K, M = n * D, n * n + 2 * n
    gen = torch.Generator(device=device)
    gen.manual_seed(20261201 + cfg)
    x = torch.randn((T, n, D), generator=gen, device=device, dtype=torch.float32)
    if outliers:
        idx = torch.arange(0, T, 100, device=device)
        x[idx] *= 50.0
        x[T - 1] *= 50.0
    x = x.to(torch.bfloat16 if bf16 else torch.float16)
    phi = torch.randn((M, K), generator=gen, device=device) * (1.0 / K ** 0.5)
    bias = torch.rand((M,), generator=gen, device=device) * 0.2 - 0.1
    alpha = torch.full((3,), 0.01, device=device)
    g = (1.0 + 0.1 * torch.randn((K,), generator=gen, device=device)) if gamma else None
    return x, phi.contiguous(), alpha, bias, g


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def _time_oracle(orc, x_h, bf16, phi_h, alpha_h, bias_h, g_h, threads, block, target_s):
    """Rows per second of the C oracle over blocks of the same inputs, repeated
    for about target_s seconds."""
    T = x_h.shape[0]
    rows = 0
    t0 = time.perf_counter()
    elapsed = 0.0
    start = 0
    while elapsed < target_s:
        xs = x_h[start:start + block]
        orc.mhc_pre(xs, bf16, phi_h, alpha_h, bias_h, g_h, nthreads=threads)
        rows += xs.shape[0]
        start = (start + block) % T
        elapsed = time.perf_counter() - t0
    return rows, elapsed


def cpu_baseline(x, phi, alpha, bias, gamma, bf16: bool, target_s: float) -> dict:
    """Time the C oracle (reference fp order) on this host: OpenMP over rows on
    all host cores (the reported value), and on one thread.

    The sample is the full workload's rows, processed in blocks of up to 512
    rows (64 on one thread) and repeated until about target_s (target_s / 2
    on one thread) seconds have passed: a bounded sample; the rate is rows /
    second.  Both variants give bitwise identical outputs (rows are
    independent)."""
    import numpy as np
    import torch

    from oracle import oracle as orc

    T = x.shape[0]
    threads = orc.max_threads()
    phi_h = phi.cpu().numpy()
    alpha_h, bias_h = alpha.cpu().numpy(), bias.cpu().numpy()
    g_h = gamma.cpu().numpy() if gamma is not None else None
    x_h = x.view(torch.int16).cpu().numpy().view(np.uint16)
    block = min(T, 512)
    rows, elapsed = _time_oracle(orc, x_h, bf16, phi_h, alpha_h, bias_h, g_h, threads, block,
                                 target_s)
    block1 = min(T, 64)
    rows1, elapsed1 = _time_oracle(orc, x_h, bf16, phi_h, alpha_h, bias_h, g_h, 1, block1,
                                   target_s / 2)
    return {"value": rows / elapsed, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{rows} rows ({rows / T:.2f} passes over the {T} rows of the same inputs, "
                      f"in blocks of {block}) in {elapsed:.1f} s, OpenMP over rows "
                      f"({threads} threads)",
            "single_thread": {"value": rows1 / elapsed1, "unit": "tokens/s", "cores": 1,
                              "sample": f"{rows1} rows in blocks of {block1} in "
                                        f"{elapsed1:.1f} s"},
            "cpu_model": cpu_model()}


def host_call_cost(pkg, op, x, phi, alpha, bias, gamma, prepared: bool) -> dict:
    """Host cost of one call, outside the timed region: (a) mhcPre on a
    prebuilt executor (MhcPreOp.launch), (b) the torch operator
    torch.ops.mhcpre.mhc_pre, which runs phase 1 (a plan-cache hit after the
    first call), allocates its outputs and workspace and launches.  For each,
    the host time per call of 100 calls enqueued back to back (one
    synchronize after them) and the reference harness's latency (one call +
    stream synchronize, median of 20).  The operator is not timed with
    prepared weights (it takes phi and gamma)."""
    import torch

    def enqueue(fn, n=100):
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        return (t1 - t0) / n * 1e6

    def latency(fn):
        fn()
        torch.cuda.synchronize()
        ls = []
        for _ in range(20):
            h0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ls.append((time.perf_counter() - h0) * 1e6)
        ls.sort()
        return (ls[9] + ls[10]) / 2

    out = {"launch": {"enqueue_us": enqueue(op.launch), "latency_us": latency(op.launch)}}
    if not prepared:
        pkg.torch_ops()
        call = lambda: torch.ops.mhcpre.mhc_pre(x, phi, alpha, bias, gamma)
        out["torch_op"] = {"enqueue_us": enqueue(call), "latency_us": latency(call)}
    return out


def measured_traffic(workload: str, path: str, prepared: bool = False):
    """HBM bytes per launch for this workload from the committed rocprofv3 PMC
    record (FETCH_SIZE + WRITE_SIZE, scaled by a copy of known size) of the
    kernel path this launch takes (and the same weights mode), or None."""
    for f in sorted((ROOT / "profiles").glob("*.traffic.json")):
        rec = json.loads(f.read_text())
        if (rec.get("workload") == workload and rec.get("path") == path
                and bool(rec.get("prepared_weights", False)) == prepared):
            return rec
    return None


def measure_stream_ceiling(pkg, x, write_bytes: int, cold: bool, device, stream) -> dict:
    """A measured ceiling for this workload's own byte mix: the library's
    stream probe (mhcPreStreamProbe) reads x's bytes and writes hIn's bytes
    with no arithmetic, in the access pattern the device serves best.  The
    best of two grid sizes (one workgroup per CU, and 7/8 of that); each the
    mean of 20 back-to-back launches between one event pair, or for workloads
    that fit the MALL the median of 10 launches each after a 512 MiB scratch
    write, like the operator's cold figure."""
    import torch

    read_bytes = (x.numel() * x.element_size()) // 4096 * 4096
    write_bytes = write_bytes // 1024 * 1024
    dst = torch.empty(max(write_bytes, 1024) // 4, dtype=torch.float32, device=device)
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    flush = torch.empty(CEILING_BYTES // 4, dtype=torch.float32, device=device) if cold else None
    best = None
    for wg in (cus, cus * 7 // 8):
        for _ in range(5):
            pkg.stream_probe(x, read_bytes, dst, write_bytes, wg, stream)
        torch.cuda.synchronize()
        if cold:
            ts = []
            for _ in range(10):
                flush.fill_(1.0)
                c0 = torch.cuda.Event(enable_timing=True)
                c1 = torch.cuda.Event(enable_timing=True)
                c0.record(stream)
                pkg.stream_probe(x, read_bytes, dst, write_bytes, wg, stream)
                c1.record(stream)
                torch.cuda.synchronize()
                ts.append(c0.elapsed_time(c1) * 1e3)
            us = sorted(ts)[len(ts) // 2]
        else:
            c0 = torch.cuda.Event(enable_timing=True)
            c1 = torch.cuda.Event(enable_timing=True)
            c0.record(stream)
            for _ in range(20):
                pkg.stream_probe(x, read_bytes, dst, write_bytes, wg, stream)
            c1.record(stream)
            torch.cuda.synchronize()
            us = c0.elapsed_time(c1) * 1e3 / 20
        gbs = (read_bytes + write_bytes) / (us * 1e-6) / 1e9
        if best is None or gbs > best["gbs"]:
            best = {"gbs": gbs, "us": us, "workgroups": wg, "read_bytes": read_bytes,
                    "write_bytes": write_bytes, "timing": "cold" if cold else "warm back-to-back"}
    del dst, flush
    return best


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # Defaults: the device's clocks settle within about 20 ms of sustained load
    # (launches 20-50 of a cold start run up to 30% slower than the steady
    # state), so 300 warm-up launches (~35 ms) precede 1000 timed ones (~0.12 s).
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--settle-ms", type=float, default=100.0,
                    help="wall time of back-to-back launches before the warm-up (clock settling)")
    ap.add_argument("--config", type=int, default=3, choices=sorted(WORKLOADS))
    ap.add_argument("--shape", type=str, default=None,
                    help="n,D,T,bf16,gamma (e.g. 8,8192,2048,1,1): another workload in place of "
                         "--config, with the same input distributions (seed of config 0)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target duration of the CPU-baseline sample (0 disables it)")
    ap.add_argument("--prepared", action="store_true",
                    help="launch an executor built from prepared weights (mhcPrePrepareWeights)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a device copy of a known size (calibrates profiler byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); MhcPre shards "
              "over rows with no exchange, so N GPUs run N independent copies.", file=sys.stderr)
        return 2

    import torch

    from __graft_entry__ import load_package

    pkg = load_package()
    pkg.load_library()
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")
    cfg = args.config
    if args.shape is not None:
        parts = [int(v) for v in args.shape.split(",")]
        if len(parts) != 5:
            print("--shape takes n,D,T,bf16,gamma", file=sys.stderr)
            return 2
        cfg = 0
        WORKLOADS[cfg] = (parts[0], parts[1], parts[2], bool(parts[3]), bool(parts[4]), False)
    n, D, T, bf16, gamma_on, _ = WORKLOADS[cfg]
    x, phi, alpha, bias, gamma = make_inputs(cfg, device)
    weights = None
    if args.prepared:
        # B = gamma * phi prepared once, outside the timed region (the
        # weights of a layer do not change between steps).
        weights = pkg.MhcPreWeights(phi, gamma, n)
        op = pkg.MhcPreOp(x, None, alpha, bias, None, weights=weights)
    else:
        op = pkg.MhcPreOp(x, phi, alpha, bias, gamma)
    stream = torch.cuda.current_stream()

    # Clock settling: launches back to back for settle_ms of wall time (the
    # host enqueues ahead of the device, so the check runs every 16 launches
    # and the device is kept busy throughout), then the --warmup launches.
    settle_launches = 0
    t_settle = time.perf_counter()
    while True:
        for _ in range(16):
            op.launch(stream)
        settle_launches += 16
        torch.cuda.synchronize()
        settle_ms = (time.perf_counter() - t_settle) * 1e3
        if settle_ms >= args.settle_ms:
            break
    for _ in range(args.warmup):
        op.launch(stream)
    torch.cuda.synchronize()

    # Timed region: K launches back to back on the launch stream, between one
    # pair of HIP events recorded on that stream.  (An event pair around each
    # launch puts a marker between consecutive dispatches, which costs about
    # 10 us of idle GPU per launch; those per-launch figures come from a
    # separate pass below and only describe the spread.)
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for _ in range(args.steps):
        op.launch(stream)
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    mean_ms = total_ms / args.steps

    n_ev = min(args.steps, 20)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    for i in range(n_ev):
        starts[i].record(stream)
        op.launch(stream)
        ends[i].record(stream)
    torch.cuda.synchronize()
    durs = sorted(s.elapsed_time(e) for s, e in zip(starts, ends))  # ms per launch
    status = op.device_status(stream)
    if status != 0:
        print(f"device status {status}", file=sys.stderr)
        return 1

    # Host wall-clock latency, the reference harness's method
    # (cloud_runner/runner.cpp:458-490): 1 warm-up, then 20 iterations of one
    # launch followed by a stream synchronize, on the host clock.
    op.launch(stream)
    stream.synchronize()
    lat = []
    for _ in range(20):
        h0 = time.perf_counter()
        op.launch(stream)
        stream.synchronize()
        lat.append((time.perf_counter() - h0) * 1e6)
    lat.sort()
    host_latency = {"min": lat[0], "median": (lat[9] + lat[10]) / 2, "avg": sum(lat) / len(lat),
                    "iterations": 20, "warmup": 1}
    op_cost = host_call_cost(pkg, op, x, phi, alpha, bias, gamma, args.prepared)

    # Cold cache: a 512 MiB scratch write before each event-timed launch
    # evicts the MALL (256 MB) and the L2s; median of 20.
    flush = torch.empty(CEILING_BYTES // 4, dtype=torch.float32, device=device)
    cold = []
    for _ in range(21):
        flush.fill_(1.0)
        c0 = torch.cuda.Event(enable_timing=True)
        c1 = torch.cuda.Event(enable_timing=True)
        c0.record(stream)
        op.launch(stream)
        c1.record(stream)
        torch.cuda.synchronize()
        cold.append(c0.elapsed_time(c1) * 1e3)
    cold = sorted(cold[1:])
    cold_us = (cold[9] + cold[10]) / 2
    del flush
    if op.device_status(stream) != 0:
        print("device status after the latency passes", file=sys.stderr)
        return 1

    if args.copy_probe:
        # A plain device-to-device copy of exactly COPY_BYTES: under rocprofv3
        # --pmc its FETCH_SIZE / WRITE_SIZE give the counters' scale factor.
        src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=device).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # Measured ceiling: a plain device-to-device copy of 512 MiB (read + write
    # bytes over its event-timed duration, median of 5, after 2 untimed
    # copies), beside the spec peak.  It runs after the timed region.
    csrc = torch.empty(CEILING_BYTES // 4, dtype=torch.float32, device=device).fill_(1.0)
    cdst = torch.empty_like(csrc)
    for _ in range(2):
        cdst.copy_(csrc)
    cts = []
    for _ in range(5):
        c0 = torch.cuda.Event(enable_timing=True)
        c1 = torch.cuda.Event(enable_timing=True)
        c0.record(stream)
        cdst.copy_(csrc)
        c1.record(stream)
        torch.cuda.synchronize()
        cts.append(c0.elapsed_time(c1))
    copy_gbs = 2 * CEILING_BYTES / (sorted(cts)[len(cts) // 2] * 1e-3) / 1e9
    del csrc, cdst

    b_alg = algorithmic_bytes(n, D, T, bf16, gamma_on)
    # Working sets that fit the 256 MB MALL are judged on the cold-cache
    # figure (a warm back-to-back launch re-reads them from the cache).
    fits_mall = b_alg < (256 << 20)
    stream_ceiling = measure_stream_ceiling(pkg, x, T * D * 2, fits_mall, device, stream)
    roof_us = cold_us if fits_mall else mean_ms * 1e3
    achieved = b_alg / (roof_us * 1e-6) / 1e9
    workload = (f"mhc_pre n={n} D={D} T={T} {'bf16' if bf16 else 'fp16'} "
                f"gamma={'on' if gamma_on else 'off'}")
    traffic = measured_traffic(workload, op.path, args.prepared)
    result = {
        "metric": METRIC,
        "value": T / (mean_ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": total_ms / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if bf16 else "fp16",
        "data": "synthetic",
        "settle_ms": settle_ms,
        "settle_launches": settle_launches,
        "config": {"workload": workload,
                   "n": n, "D": D, "T": T, "gamma": gamma_on, "path": op.path,
                   "prepared_weights": args.prepared,
                   "launch_us": mean_ms * 1e3,
                   "event_pair_median_us": durs[len(durs) // 2] * 1e3,
                   "event_pair_min_us": durs[0] * 1e3,
                   "cold_us": cold_us,
                   "host_latency_us": host_latency,
                   "host_call_us": op_cost,
                   "algorithmic_bytes": b_alg,
                   "traffic_source": traffic["summary"] if traffic else None},
        "roofline": {"bound": "hbm", "timing": "cold" if fits_mall else "warm back-to-back",
                     "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic["traffic_bytes"] if traffic else None,
                     "copy_ceiling": copy_gbs, "frac_of_copy": achieved / copy_gbs,
                     "stream_ceiling": stream_ceiling["gbs"],
                     "frac_of_stream_ceiling": achieved / stream_ceiling["gbs"],
                     "stream_ceiling_detail": stream_ceiling},
    }
    if args.cpu_seconds > 0:
        result["cpu_baseline"] = cpu_baseline(x, phi, alpha, bias, gamma, bf16,
                                              args.cpu_seconds)
    op.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
