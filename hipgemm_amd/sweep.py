"""Schedule sweep: time every applicable schedule on given shapes and report
AUTO's pick against the fastest.

    python -m hipgemm_amd.sweep 64x4096x4096,128x8192x8192 [--variants 3,5,6]
    python -m hipgemm_amd.sweep --grid 16,32:4096,8192:2048,8192 \
        [--grid ...] [--show-above 1.02]

For each M x N x K: e4m3 operands drawn from normal(0, 1) (rotating sets
of at least 512 MiB, so that the L2 and the MALL do not hold them between
launches), per-tensor scales, bf16 C, one caller workspace
(hipgemm_fp8_gemm_bf16_ws).  The schedules are timed in alternating blocks
of launches (four rounds, the order reversed every other round) with HIP
events on one stream; a schedule that rejects the shape is left out.  One
line per shape: microseconds per launch for each schedule, AUTO's pick
(hipgemm_select_variant; for AUTO's column split the 4-wave schedule is
reported), the fastest, and AUTO's time over the fastest (with
--show-above R, only the shapes whose ratio exceeds R).  The summary gives
the mean and worst ratio and how many shapes fall in each ratio bucket.
--grid M,..:N,..:K,.. adds every combination of the listed sizes.

Measurement only: it checks no results (the tests do).
"""
from __future__ import annotations

import argparse
import sys

from . import VARIANTS, lib, variant_name, workspace_size


def parse_shapes(text: str):
    shapes = []
    for item in text.split(","):
        m, n, k = (int(x) for x in item.lower().split("x"))
        if min(m, n, k) <= 0:
            raise ValueError(f"bad shape {item!r}")
        shapes.append((m, n, k))
    return shapes


def parse_grid(text: str):
    """'M1,M2:N1,N2:K1,K2' -> every (M, N, K) combination, M outermost."""
    parts = text.split(":")
    if len(parts) != 3:
        raise ValueError(f"bad grid {text!r}")
    ms, ns, ks = ([int(x) for x in p.split(",")] for p in parts)
    if min(ms + ns + ks) <= 0:
        raise ValueError(f"bad grid {text!r}")
    return [(m, n, k) for m in ms for n in ns for k in ks]


BUCKETS = (1.0, 1.02, 1.05, 1.10)


def sweep(shapes, variants, rounds: int = 4, launches: int = 100, out=sys.stdout,
          show_above: float = 0.0):
    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    L = lib()
    ratios = []
    for (M, N, K) in shapes:
        nsets = max(1, -(-(512 << 20) // (M * K + N * K)))
        g = torch.Generator(device=dev)
        g.manual_seed(7)
        As = [torch.randn((M, K), generator=g, device=dev).clamp_(-448, 448)
              .to(torch.float8_e4m3fn) for _ in range(nsets)]
        Bs = [torch.randn((N, K), generator=g, device=dev).clamp_(-448, 448)
              .to(torch.float8_e4m3fn) for _ in range(nsets)]
        sa = torch.rand(1, generator=g, device=dev) + 0.5
        sb = torch.rand(1, generator=g, device=dev) + 0.5
        C = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        need = max(workspace_size(M, N, K, v) for v in variants)
        ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=dev)

        def launch(v, i):
            return L.hipgemm_fp8_gemm_bf16_ws(
                As[i % nsets].data_ptr(), Bs[i % nsets].data_ptr(), C.data_ptr(),
                M, N, K, K, K, N, sa.data_ptr(), sb.data_ptr(), v,
                ws.data_ptr(), ws.numel(), stream.cuda_stream)

        ok = [v for v in variants if launch(v, 0) == 0]
        torch.cuda.synchronize()
        if not ok:
            print(f"{M}x{N}x{K}: no schedule takes this shape", file=out, flush=True)
            continue
        for v in ok:
            for i in range(launches // 2):
                code = launch(v, i)
                if code != 0:
                    raise RuntimeError(f"{variant_name(v)} on {M}x{N}x{K}: error {code}")
        torch.cuda.synchronize()
        us = {v: 0.0 for v in ok}
        for r in range(rounds):
            for v in (ok if r % 2 == 0 else ok[::-1]):
                for i in range(launches // 10):
                    launch(v, i)
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for i in range(launches):
                    launch(v, i)
                e1.record(stream)
                torch.cuda.synchronize()
                us[v] += e0.elapsed_time(e1) * 1000.0 / launches / rounds
        auto = int(L.hipgemm_select_variant(M, N, K))
        best = min(us, key=us.get)
        line = "  ".join(f"{variant_name(v)} {us[v]:.2f}" for v in ok)
        ratio = None
        if auto in us:
            ratio = us[auto] / us[best]
            ratios.append(ratio)
            tail = f"auto={variant_name(auto)} best={variant_name(best)} ratio {ratio:.3f}"
        else:
            tail = f"auto={variant_name(auto)} (not timed) best={variant_name(best)}"
        if ratio is None or ratio > show_above:
            print(f"{M}x{N}x{K}: {line}  | {tail}", file=out, flush=True)
        del As, Bs, C, ws
    if ratios:
        print(f"summary: {len(ratios)} shapes, AUTO / fastest mean "
              f"{sum(ratios) / len(ratios):.4f}, worst {max(ratios):.3f}, "
              f"{sum(r > 1.02 for r in ratios)} above 1.02", file=out, flush=True)
        edges = BUCKETS + (float("inf"),)
        counts = [sum(lo < r <= hi for r in ratios) if i else
                  sum(r <= hi for r in ratios)
                  for i, (lo, hi) in enumerate(zip((0.0,) + BUCKETS, edges))]
        names = ["= 1.00"] + [f"({lo:.2f}, {hi:.2f}]" for lo, hi in
                              zip(BUCKETS[:-1], BUCKETS[1:])] + [f"> {BUCKETS[-1]:.2f}"]
        print("ratio buckets: " + ", ".join(f"{n} {c}" for n, c in zip(names, counts)),
              file=out, flush=True)
    return ratios


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("shapes", nargs="?", default="",
                    help="comma-separated MxNxK list")
    ap.add_argument("--grid", action="append", default=[],
                    help="M,..:N,..:K,.. -- every combination (repeatable)")
    ap.add_argument("--show-above", type=float, default=0.0,
                    help="print only shapes whose AUTO / fastest ratio exceeds this")
    ap.add_argument("--variants", default="",
                    help="comma-separated schedule codes or names "
                         "(default: every schedule but AUTO)")
    ap.add_argument("--rounds", type=int, default=4)
    ap.add_argument("--launches", type=int, default=100)
    a = ap.parse_args(argv)
    if a.variants:
        vs = [VARIANTS[x] if x in VARIANTS else int(x) for x in a.variants.split(",")]
    else:
        vs = [v for k, v in VARIANTS.items() if k != "auto"]
    shapes = parse_shapes(a.shapes) if a.shapes else []
    for g in a.grid:
        shapes += parse_grid(g)
    seen = set()
    shapes = [s for s in shapes if not (s in seen or seen.add(s))]
    if not shapes:
        ap.error("no shapes: give a list or --grid")
    sweep(shapes, vs, a.rounds, a.launches, show_above=a.show_above)
    return 0


if __name__ == "__main__":
    sys.exit(main())
