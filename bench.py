#!/usr/bin/env python3
"""FP8 GEMM throughput on one MI355X (BASELINE.json metric).

    python bench.py [--steps K] [--warmup W] [--shape M,N,K] [--variant auto]

A step is one GEMM launch (C = sa*sb * A . B_T^T, e4m3 in, fp32 accumulate,
bf16 out) through the C ABI on inputs already resident in HBM.  Default
workload: M = N = K = 8192, normal(0, 1) e4m3
inputs, per-tensor scales uniform in [0.5, 2], rotating A/B sets totalling at
least 512 MiB so consecutive launches do not hit in the 256 MB MALL (the
reference's bench.cpp:24 does the same).

Prints ONE JSON line on stdout (rank 0, N = 1):
  value      whole-job TFLOP/s = 2*M*N*K*steps / wall time of the timed loop
  prewarm    the declared steady-state pre-warm that ran before the
             --warmup launches (--prewarm-seconds of back-to-back launches)
  roofline   the GEMM kernel's average launch duration from one pair of HIP
             events on its stream around the timed loop -> achieved TFLOP/s
             against the 5.0 PFLOP/s dense-FP8 MFMA peak; `traffic` (HBM bytes
             per launch, rocprofv3 FETCH_SIZE / WRITE_SIZE) and
             `mfma_busy_pct` come from the committed counter summary of this
             workload (profiles/counters.json -> `counters_source`) when one
             exists
  cpu_baseline  the reference's CPU GEMM (test.cpp:19-30, built from its
             sources into oracle/_ref) -- or the oracle port of it when that
             build is absent -- timed on a row slab of the same workload
Diagnostics go to stderr.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP8_TFLOPS = 5000.0      # MI355X dense FP8 MFMA peak (published)
PEAK_CLOCK_MHZ = 2400.0       # the GFX clock that peak is quoted at
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E (published)
ROTATE_BYTES = 512 << 20      # bench.cpp:24


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--prewarm-seconds", type=float, default=3.0,
                    help="steady-state pre-warm before the --warmup launches: "
                         "back-to-back launches for at least this much wall "
                         "time, so that the timed loop runs at the clock the "
                         "GPU settles at under this load (0 = none)")
    ap.add_argument("--shape", default="8192,8192,8192",
                    help="M,N,K of the timed GEMM")
    ap.add_argument("--variant", default="auto")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU time of the cpu_baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ceiling", action="store_true",
                    help="skip the MFMA ceiling probe")
    ap.add_argument("--ceiling-seconds", type=float, default=2.0,
                    help="pre-warm of the MFMA ceiling probe")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="before the GEMMs, run one elementwise copy kernel "
                         "over this many MiB (reads N, writes N bytes) as the "
                         "known-size reference for rocprof FETCH_SIZE / "
                         "WRITE_SIZE")
    return ap.parse_args()


def counters_for(workload: str, variant: str) -> dict:
    """The committed rocprofv3 counter summary of this workload and schedule
    (profiles/counters.json), or {}: HBM bytes per launch (FETCH_SIZE /
    WRITE_SIZE scaled by a copy kernel), MFMA-busy %, and the file they come
    from."""
    path = os.path.join(ROOT, "profiles", "counters.json")
    try:
        with open(path) as f:
            return json.load(f).get(workload, {}).get(variant, {}) or {}
    except (OSError, ValueError):
        return {}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(A_host, B_host, M, N, K, target_s):
    """Time the reference CPU GEMM on rows [0, R) of the workload."""
    import numpy as np
    from oracle import pyoracle as po
    kind = "reference"
    try:
        ref = po.RefLib()
        fn = ref.gemm_cpu

        def run(rows):
            return fn(np.ascontiguousarray(A_host[:rows]), B_host)
        try:
            omp = ctypes.CDLL("/opt/rocm/llvm/lib/libomp.so")
            cores = int(omp.omp_get_max_threads())
        except OSError:
            cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count()))
        what = "reference gemm_cpu (test.cpp:19-30) built from its sources"
    except (FileNotFoundError, OSError):
        kind = "port"
        o = po.get()

        def run(rows):
            return o.gemm(np.ascontiguousarray(A_host[:rows]), B_host,
                          faithful=True)
        cores = o.num_threads()
        what = "oracle port of gemm_cpu (oracle/oracle.c hg_gemm_ref)"
    rows = 8
    t0 = time.perf_counter()
    run(rows)
    t = time.perf_counter() - t0
    rows = int(max(8, min(M, rows * target_s / max(t, 1e-3))))
    t0 = time.perf_counter()
    run(rows)
    t = time.perf_counter() - t0
    tflops = 2.0 * rows * N * K / t / 1e12
    return {
        "value": round(tflops, 6), "unit": "TFLOP/s", "cores": cores,
        "cpu_model": cpu_model(), "kind": kind,
        "sample": (f"rows 0..{rows - 1} of the {M}x{N}x{K} workload "
                   f"({rows}x{N}x{K}, {t:.1f} s, {what}); TFLOP/s of the "
                   f"slab, which equals the full-size rate (cost is linear "
                   f"in M)"),
    }


def mfma_ceiling(dev, stream, prewarm_s, steps=100, iters=256):
    """Sustained v_mfma_f32_16x16x128_f8f6f4 rate with register-resident
    normal(0,1) e4m3 operands and no memory traffic
    (hipgemm_amd/probe/mfma_ceiling.hip): the rate this GPU holds under its
    power limit when the matrix unit alone draws power.  One workgroup of 4
    waves per CU, each wave issuing the 64 MFMA of one K-step of the 4-wave
    schedule `iters` times per launch (iters 256: the flop of one 8192^3
    GEMM).  Timed like the GEMM: pre-warm, then `steps` launches between one
    event pair."""
    import torch
    path = os.path.join(ROOT, "hipgemm_amd", "libhipgemm_probe.so")
    if not os.path.exists(path):
        raise SystemExit(f"{path} is missing: build first "
                         "(python -c 'import __graft_entry__ as g; g.build()')")
    L = ctypes.CDLL(path)
    L.hipgemm_probe_ops_bytes.restype = ctypes.c_size_t
    L.hipgemm_probe_mfma_ceiling.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_int, ctypes.c_int,
                                            ctypes.c_void_p]
    L.hipgemm_probe_mfma_ceiling.restype = ctypes.c_int
    nbytes = int(L.hipgemm_probe_ops_bytes())
    gen = torch.Generator(device=dev)
    gen.manual_seed(4242)
    ops = (torch.randn(nbytes, generator=gen, device=dev)
           .clamp_(-448, 448).to(torch.float8_e4m3fn))
    grid = torch.cuda.get_device_properties(dev).multi_processor_count
    out = torch.empty(grid * 256, dtype=torch.float32, device=dev)
    sptr = stream.cuda_stream

    def launch(_i):
        code = L.hipgemm_probe_mfma_ceiling(ops.data_ptr(), out.data_ptr(),
                                            grid, iters, sptr)
        if code != 0:
            raise RuntimeError(f"hipgemm_probe_mfma_ceiling returned {code}")

    monitor = GpuMonitor(0).start()
    res = time_kernel(launch, 20, steps, stream, prewarm_s, monitor)
    monitor.stop()
    live = None
    if "timed_end" in monitor.marks:
        live = monitor.window(monitor.marks["timed_end"] - 1.0,
                              monitor.marks["timed_end"])
    flop = grid * 4 * iters * 64 * 2.0 * 16 * 16 * 128
    tflops = flop / (res["event_ms"] * 1e-3) / 1e12
    return {"achieved": round(tflops, 1), "unit": "TFLOP/s",
            "kernel_ms_avg": round(res["event_ms"], 5),
            "gpu_monitor": live,
            "kernel": "mfma_ceiling_16x16x128 (hipgemm_amd/probe/"
                      "mfma_ceiling.hip)",
            "what": (f"{grid} workgroups x 4 waves, {iters} x 64 "
                     "register-resident 16x16x128 e4m3 MFMA per wave, "
                     "normal(0,1) operands, no memory traffic; "
                     f"{res['prewarm_launches']} pre-warm launches")}


class GpuMonitor:
    """The GPU's GFX clock and socket power while a kernel runs, sampled by a
    background thread through amdsmi (the ROCm SMI library): the mean of
    the per-XCD current_gfxclks and current_socket_power of the GPU's
    metrics table, every 5 ms, each sample with its host time.  window()
    summarises the samples between two marks.  Every field is None where
    amdsmi or a metric is unavailable; the monitor never fails the bench."""

    def __init__(self, dev_index=0):
        import threading
        self.ok, self.h, self.samples, self.marks = False, None, [], {}
        self.cap_w = None
        self._stop = threading.Event()
        self._thread = None
        try:
            import amdsmi
            self.smi = amdsmi
            amdsmi.amdsmi_init()
            hs = amdsmi.amdsmi_get_processor_handles()
            if len(hs) == 1:
                self.h = hs[0]
            else:
                import torch
                p = torch.cuda.get_device_properties(dev_index)
                want = (getattr(p, "pci_domain_id", 0), p.pci_bus_id,
                        p.pci_device_id)
                for h in hs:
                    bdf = amdsmi.amdsmi_get_gpu_device_bdf(h)
                    dom, bus, rest = bdf.split(":")
                    if (int(dom, 16), int(bus, 16),
                            int(rest.split(".")[0], 16)) == want:
                        self.h = h
            if self.h is not None:
                self._sample()
                self.ok = bool(self.samples)
                self.samples.clear()
                try:
                    cap = amdsmi.amdsmi_get_power_cap_info(self.h)["power_cap"]
                    # microwatts in the ROCm 7 API, watts in older ones
                    self.cap_w = round(cap / 1e6 if cap > 1e5 else cap, 1)
                except Exception:
                    self.cap_w = None
        except Exception:
            self.ok = False

    def _sample(self):
        m = self.smi.amdsmi_get_gpu_metrics_info(self.h)
        clks = [c for c in (m.get("current_gfxclks") or [])
                if isinstance(c, (int, float)) and c > 0]
        if not clks and isinstance(m.get("current_gfxclk"), (int, float)):
            clks = [m["current_gfxclk"]]
        pw = m.get("current_socket_power")
        if clks:
            self.samples.append((time.perf_counter(), sum(clks) / len(clks),
                                 pw if isinstance(pw, (int, float)) else None))

    def _run(self):
        while not self._stop.is_set():
            try:
                self._sample()
            except Exception:
                return
            self._stop.wait(0.005)

    def start(self):
        import threading
        if self.ok:
            self._thread = threading.Thread(target=self._run, daemon=True)
            self._thread.start()
        return self

    def mark(self, name):
        self.marks[name] = time.perf_counter()

    def stop(self):
        if self._thread:
            self._stop.set()
            self._thread.join()

    def window(self, t0, t1):
        s = [x for x in self.samples if t0 <= x[0] <= t1]
        if not s:
            return None
        clk = [x[1] for x in s]
        pw = [x[2] for x in s if x[2] is not None]
        return {"gfxclk_mhz": round(sum(clk) / len(clk), 1),
                "gfxclk_mhz_range": [round(min(clk), 1), round(max(clk), 1)],
                "socket_power_w": round(sum(pw) / len(pw), 1) if pw else None,
                "power_cap_w": self.cap_w, "samples": len(s)}


def prewarm(launch, seconds):
    """Back-to-back launches until at least `seconds` of wall time have
    passed (checked between chunks of about 0.1 s).  The GPU ramps its clock
    and settles its power state over the first few thousand launches of a
    heavy kernel; this runs the timed loop at the steady state.  Returns
    (launches, seconds)."""
    import torch
    if seconds <= 0:
        return 0, 0.0
    t0 = time.perf_counter()
    n, chunk = 0, 4
    while True:
        c0 = time.perf_counter()
        for _ in range(chunk):
            launch(n)
            n += 1
        torch.cuda.synchronize()
        now = time.perf_counter()
        if now - t0 >= seconds:
            return n, now - t0
        per = (now - c0) / chunk
        chunk = max(1, min(100000, int(0.1 / max(per, 1e-7))))


def time_kernel(launch, warmup, steps, stream, prewarm_s=0.0, monitor=None):
    """The contract's timed loop, then a per-launch pass for diagnostics.

    Pre-warm (prewarm_s seconds of launches, then `warmup` more), then the
    timed loop: `steps` launches back to back with nothing between them,
    bracketed by a device synchronize on both sides; wall time from the host
    clock and, over the same region, one pair of HIP events on the launch
    stream (-> average time per launch).  Per-launch pass: the same number of
    launches, each between its own event pair (median, best, drift)."""
    import numpy as np
    import torch
    pre_n, pre_s = prewarm(launch, prewarm_s)
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    if monitor:
        monitor.mark("timed_start")
    e0.record(stream)
    for i in range(steps):
        launch(warmup + i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if monitor:
        monitor.mark("timed_end")
    event_ms = e0.elapsed_time(e1) / steps
    ev = [(torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record(stream)
        launch(warmup + steps + i)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    per = np.array([a.elapsed_time(b) for a, b in ev])
    return {"wall_ms": wall * 1e3 / steps, "event_ms": event_ms,
            "prewarm_launches": pre_n, "prewarm_s": pre_s,
            "median_ms": float(np.median(per)), "best_ms": float(per.min()),
            "tenths": [float(p.mean()) for p in
                       np.array_split(per, min(10, len(per)))]}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} "
              "is not supported (on several GPUs the GEMM shards by M or N "
              "with no exchange; each GPU runs this same kernel).",
              file=sys.stderr)
        return 2
    import numpy as np
    import torch

    import hipgemm_amd as hg

    M, N, K = (int(x) for x in args.shape.split(","))
    variant = hg.VARIANTS.get(args.variant)
    if variant is None:
        raise SystemExit(f"unknown variant {args.variant}")
    vname = hg.variant_name(hg.select_variant(M, N, K) if variant == 0
                            else variant)
    n1 = hg.split_columns(M, N, K) if variant == 0 else 0
    if n1:  # AUTO's column split: two schedules, two launches per step
        vname = f"{vname}[0:{n1}]+{hg.variant_name(5)}[{n1}:{N}]"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    hg.lib()

    per_set = M * K + N * K
    nsets = max(1, math.ceil(ROTATE_BYTES / per_set))
    gen = torch.Generator(device=dev)
    gen.manual_seed(2024)
    As, Bs = [], []
    for _ in range(nsets):
        As.append(torch.randn((M, K), generator=gen, device=dev)
                  .clamp_(-448, 448).to(torch.float8_e4m3fn))
        Bs.append(torch.randn((N, K), generator=gen, device=dev)
                  .clamp_(-448, 448).to(torch.float8_e4m3fn))
    sa = (torch.rand(1, generator=gen, device=dev) * 1.5 + 0.5)
    sb = (torch.rand(1, generator=gen, device=dev) * 1.5 + 0.5)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream(dev)
    torch.cuda.synchronize()
    log(f"bench: {M}x{N}x{K} variant={vname} rotating_sets={nsets} "
        f"steps={args.steps} warmup={args.warmup}")

    # Launch through the C ABI on raw pointers: the per-launch host cost stays
    # far below the kernel time, so the stream never runs dry.
    ptrs = [(As[i].data_ptr(), Bs[i].data_ptr()) for i in range(nsets)]
    cptr, sap, sbp, sptr = (out.data_ptr(), sa.data_ptr(), sb.data_ptr(),
                            stream.cuda_stream)
    # A caller-owned workspace (zero-filled once) for schedules that split K.
    ws_bytes = hg.workspace_size(M, N, K, variant)
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    wsp = ws.data_ptr() if ws_bytes else 0

    def launch(i):
        a, b = ptrs[i % nsets]
        code = hg.gemm_raw_ws(a, b, cptr, M, N, K, K, K, N, sap, sbp, variant,
                              wsp, ws_bytes, sptr)
        if code != 0:
            raise hg.HipGemmError(f"hipgemm_fp8_gemm_bf16_ws returned {code}",
                                  code)

    if args.calibrate_copy_mib > 0:
        n = (args.calibrate_copy_mib << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.neg(src, out=dst)  # one kernel: n*4 bytes in, n*4 bytes out
        torch.cuda.synchronize()
        del src, dst

    flop = 2.0 * M * N * K
    monitor = GpuMonitor(0).start()
    res = time_kernel(launch, args.warmup, args.steps, stream,
                      args.prewarm_seconds, monitor)
    monitor.stop()
    # The clock of the timed loop: the samples of its last second of
    # back-to-back launches (the pre-warm's end, the warm-up and the loop;
    # the metrics table refreshes far more slowly than a short loop lasts).
    live = None
    if "timed_end" in monitor.marks:
        live = monitor.window(monitor.marks["timed_end"] - 1.0,
                              monitor.marks["timed_end"])
    log(f"bench: GPU monitor over the timed loop's last second: {live}")
    ms_per_step = res["wall_ms"]
    value = flop / (ms_per_step * 1e-3) / 1e12
    avg_ms = res["event_ms"]
    achieved = flop / (avg_ms * 1e-3) / 1e12
    log(f"bench: timed loop {ms_per_step:.4f} ms/step wall, {avg_ms:.4f} "
        f"ms/launch by events -> {value:.1f} TFLOP/s wall, {achieved:.1f} "
        f"by events; per-launch pass median={res['median_ms']:.4f} "
        f"best={res['best_ms']:.4f}")
    log(f"bench: pre-warm {res['prewarm_launches']} launches in "
        f"{res['prewarm_s']:.2f} s before the {args.warmup} warm-up launches")
    log("bench: per-launch ms by tenth of the per-launch pass: "
        + " ".join(f"{x:.4f}" for x in res["tenths"]))

    workload = f"fp8_gemm_{M}x{N}x{K}"
    # Algorithmic work of one launch: 2MNK flop; A and B_T read once, C
    # written once.  Below the ridge point (peak flop / peak bytes) the
    # kernel is bounded by HBM, above it by the MFMA.
    alg_bytes = M * K + N * K + 2 * M * N
    ctr = counters_for(workload, vname)
    measured = {"traffic": ctr.get("hbm_bytes_per_launch"),
                "mfma_busy_pct": ctr.get("mfma_busy_pct"),
                "counters_source": ctr.get("source")}
    if flop / max(alg_bytes, 1) < PEAK_FP8_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9):
        gbs = alg_bytes / (avg_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(gbs, 1),
                    "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(gbs / PEAK_HBM_GBS, 4),
                    **measured, "algorithmic_bytes": alg_bytes}
    else:
        roofline = {"bound": "mfma", "achieved": round(achieved, 3),
                    "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(achieved / PEAK_FP8_TFLOPS, 4),
                    **measured}
        # The same peak at the clock the GPU ran the loop at (measured in
        # this run): the rate the matrix unit allows at that clock, and the
        # share of it the kernel reaches.
        if live and live.get("gfxclk_mhz"):
            pk = PEAK_FP8_TFLOPS * live["gfxclk_mhz"] / PEAK_CLOCK_MHZ
            roofline["peak_at_measured_clock"] = round(pk, 1)
            roofline["frac_at_measured_clock"] = round(achieved / pk, 4)
    roofline["gpu_monitor"] = live
    result = {
        "metric": ("FP8 GEMM TFLOP/s at M=N=K=8192 (% of dense FP8 peak) "
                   "+ MFMA busy %"),
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm": {"seconds": round(res["prewarm_s"], 3),
                    "launches": res["prewarm_launches"]},
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3",
        "data": "synthetic",
        "config": {
            "workload": workload,
            "M": M, "N": N, "K": K,
            "inputs": "normal(0,1) clipped +-448 -> e4m3, per-tensor fp32 "
                      "scales U[0.5,2)",
            "accumulate": "fp32", "output": "bf16",
            "variant": vname, "rotating_sets": nsets,
            "pct_of_peak": round(100.0 * value / PEAK_FP8_TFLOPS, 2),
        },
        "roofline": dict(roofline, kernel_ms_avg=round(avg_ms, 5),
                         kernel_ms_median=round(res["median_ms"], 5),
                         kernel_ms_best=round(res["best_ms"], 5)),
        "cpu_baseline": None,
    }
    if not args.no_ceiling and roofline["bound"] == "mfma":
        # After the GEMM, so that its timed loop ran first on a GPU in the
        # state bench.py always leaves it in.
        ceil = mfma_ceiling(dev, stream, args.ceiling_seconds)
        ceil["frac"] = round(achieved / ceil["achieved"], 4)
        result["roofline"]["mfma_ceiling"] = ceil
        log(f"bench: MFMA ceiling {ceil}")
    if not args.no_cpu_baseline:
        A_host = As[0].view(torch.uint8).cpu().numpy()
        B_host = Bs[0].view(torch.uint8).cpu().numpy()
        result["cpu_baseline"] = cpu_baseline(A_host, B_host, M, N, K,
                                              args.cpu_seconds)
        log(f"bench: cpu_baseline {result['cpu_baseline']}")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
