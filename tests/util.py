"""Shared helpers for the parity tests (comparison metric, device I/O)."""
from __future__ import annotations

import sys

import numpy as np

# north_star tolerance: max relative error 1e-2 on bf16 outputs against the
# CPU fp32-accumulate GEMM, with a floor for cancellation-prone entries:
#   rel = |c - r| / max(|r|, DELTA_FRAC * rms(r)),   max(rel) <= REL_TOL
REL_TOL = 1e-2
DELTA_FRAC = 1e-2


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits).astype(np.uint32) << 16).view(np.float32)


def compare(c_bits: np.ndarray, r_bits: np.ndarray):
    """Return (max_rel, exact_fraction, n_nan) and assert NaN positions agree."""
    c = bf16_to_f32(c_bits).astype(np.float64)
    r = bf16_to_f32(r_bits).astype(np.float64)
    nc, nr = np.isnan(c), np.isnan(r)
    assert np.array_equal(nc, nr), (
        f"NaN positions differ: gpu {int(nc.sum())} vs oracle {int(nr.sum())}")
    ok = ~nr
    if not ok.any():
        return 0.0, 1.0, int(nr.sum())
    cf, rf = c[ok], r[ok]
    inf_c, inf_r = np.isinf(cf), np.isinf(rf)
    assert np.array_equal(inf_c, inf_r) and np.array_equal(
        cf[inf_c], rf[inf_r]), "infinities differ"
    fin = ~inf_r
    cf, rf = cf[fin], rf[fin]
    rms = float(np.sqrt(np.mean(rf * rf))) if rf.size else 0.0
    delta = max(DELTA_FRAC * rms, np.finfo(np.float32).tiny)
    rel = np.abs(cf - rf) / np.maximum(np.abs(rf), delta)
    exact = float(np.mean(c_bits[~nr][fin] == r_bits[~nr][fin])) if rf.size else 1.0
    return (float(rel.max()) if rel.size else 0.0), exact, int(nr.sum())


def to_dev(torch, a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def from_dev_bf16(t) -> np.ndarray:
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def scale_tensor(torch, v: float):
    return torch.tensor([v], dtype=torch.float32, device="cuda")
