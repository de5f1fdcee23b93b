"""Child process of tests/test_capture_gpu.py (not collected by pytest).

Runs in a fresh process, so that hipgemm_gemm_noalloc's first use on the GPU
-- the lookup of its static scratch array and the load of the code object
that holds it -- happens while a stream is being captured.  Mode "capture":
the first noalloc calls are captured into a CUDA graph for shapes whose
schedules use scratch (the strip schedule's K-slices with arrival counters,
the 128 x 128 schedule's K-slices with the reduce kernel); the graph is
replayed several times, with eager work and synchronisations between the
replays, and every replay must equal the oracle bit for bit (ternary inputs:
every sum exact).  Mode "footprint": device memory in use before and after
the first noalloc call that needs scratch, after other GEMMs have run; the
array must appear only then.  Prints one line per step and "OK" at the end;
exits non-zero on any mismatch.
"""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import torch  # noqa: E402

import hipgemm_amd as hg  # noqa: E402
from oracle import pyoracle as po  # noqa: E402

TERNARY = np.array([0xB8, 0x00, 0x38], np.uint8)  # -1, 0, +1
SHAPES = [(16, 4096, 8192), (256, 4096, 14336)]
# HIPGEMM_NOALLOC_SCRATCH_BYTES (include/hipgemm.h)
SCRATCH_BYTES = 16384 + (32 << 20)


def say(msg):
    print(msg, flush=True)


def case(M, N, K, seed):
    rng = np.random.default_rng(seed)
    A = TERNARY[rng.integers(0, 3, (M, K))]
    B = TERNARY[rng.integers(0, 3, (N, K))]
    a = torch.from_numpy(A).cuda()
    b = torch.from_numpy(B).cuda()
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    sa = torch.tensor([0.5], device="cuda")
    sb = torch.tensor([0.25], device="cuda")
    d = hg.GemmDesc(A=a.data_ptr(), B_T=b.data_ptr(), C=out.data_ptr(), M=M,
                    N=N, K=K, lda=K, ldb=K, ldc=N, scale_a=sa.data_ptr(),
                    scale_b=sb.data_ptr())
    return A, B, (a, b, sa, sb), out, d


def bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def capture():
    o = po.get()
    cases = [case(M, N, K, 50 + i) for i, (M, N, K) in enumerate(SHAPES)]
    wants = [o.gemm(A, B, 0.5, 0.25) for A, B, _, _, _ in cases]
    for (M, N, K), c in zip(SHAPES, cases):
        need = int(hg.lib().hipgemm_gemm_workspace_size(ctypes.byref(c[4])))
        say(f"shape {M}x{N}x{K}: scratch need {need} bytes")
        assert need > 0
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    say("capture: first hipgemm_gemm_noalloc calls of this process")
    with torch.cuda.graph(graph, stream=s):
        for _, _, _, out, d in cases:
            code = hg.gemm_desc_noalloc_raw(d, s.cuda_stream)
            assert code == 0, f"noalloc under capture: hipError {code}"
    torch.cuda.synchronize()
    for r in range(4):
        for _, _, _, out, _ in cases:
            out.fill_(float("nan"))  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for (M, N, K), (_, _, _, out, _), want in zip(SHAPES, cases, wants):
            got = bits(out)
            bad = int((got != want).sum())
            say(f"replay {r} {M}x{N}x{K}: {bad} of {M * N} outputs differ")
            assert bad == 0
    # and eagerly after the replays (the scratch's counters left at zero)
    for (M, N, K), (_, _, _, out, d), want in zip(SHAPES, cases, wants):
        out.fill_(float("nan"))
        assert hg.gemm_desc_noalloc_raw(d, 0) == 0
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), want), f"eager {M}x{N}x{K}"
        say(f"eager after replays {M}x{N}x{K}: equal")


def footprint():
    M, N, K = SHAPES[0]
    _, _, _, out, d = case(M, N, K, 60)
    a = torch.zeros((512, 512), dtype=torch.uint8, device="cuda")
    c = torch.empty((512, 512), dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    # Other schedules first (their code objects load), no scratch.
    for v in (0, 2, 5):
        assert hg.gemm_raw(a.data_ptr(), a.data_ptr(), c.data_ptr(), 512, 512,
                           512, 512, 512, 512, 0, 0, v, 0) == 0
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    assert hg.gemm_desc_noalloc_raw(d, 0) == 0
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    grew = free0 - free1
    say(f"device memory in use grew by {grew} bytes at the first noalloc call "
        f"(scratch array {SCRATCH_BYTES} bytes)")
    assert grew >= SCRATCH_BYTES


if __name__ == "__main__":
    {"capture": capture, "footprint": footprint}[sys.argv[1]]()
    say("OK")
