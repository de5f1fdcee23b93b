"""GPU check of hipgemm_gemm_noalloc (include/hipgemm.h), the entry point
that allocates nothing: schedules that need scratch use the library's static
per-GPU array instead of a workspace.  Its output must equal hipgemm_gemm's
(the same kernels; both deterministic) bit for bit, on consecutive calls
whose second input is smaller than the first, and the static array's
counter region must be left at zero between calls (a skinny split-K call
after a K-split 128 x 128 call).  Calls go through the C ABI (ctypes).
"""
import ctypes

import numpy as np
import pytest

import hipgemm_amd as hg
from oracle import pyoracle as po
from util import compare, from_dev_bf16, say, to_dev

pytestmark = pytest.mark.gpu

TERNARY = np.array([0xB8, 0x00, 0x38], np.uint8)  # -1, 0, +1


def both(torch, oracle, M, N, K, seed, general=True):
    """hipgemm_gemm (with a zeroed workspace of its own) and
    hipgemm_gemm_noalloc on the same inputs; returns both outputs."""
    if general:
        A = oracle.fill((M, K), seed, po.NORMAL, 0.0, 1.0)
        B = oracle.fill((N, K), seed + 1, po.NORMAL, 0.0, 1.0)
    else:
        rng = np.random.default_rng(seed)
        A = TERNARY[rng.integers(0, 3, (M, K))]
        B = TERNARY[rng.integers(0, 3, (N, K))]
    a, b = to_dev(torch, A), to_dev(torch, B)
    sa = torch.tensor([0.75], device="cuda")
    sb = torch.tensor([1.5], device="cuda")
    outs = []
    stream = torch.cuda.current_stream().cuda_stream
    for noalloc in (False, True):
        out = torch.full((M, N), float("nan"), dtype=torch.bfloat16,
                         device="cuda")
        d = hg.GemmDesc(A=a.data_ptr(), B_T=b.data_ptr(), C=out.data_ptr(),
                        M=M, N=N, K=K, lda=K, ldb=K, ldc=N,
                        scale_a=sa.data_ptr(), scale_b=sb.data_ptr())
        need = int(hg.lib().hipgemm_gemm_workspace_size(ctypes.byref(d)))
        if noalloc:
            code = hg.gemm_desc_noalloc_raw(d, stream)
        else:
            ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda")
            d.workspace = ws.data_ptr() if need else None
            d.workspace_bytes = need
            code = hg.gemm_desc_raw(d, stream)
        assert code == 0, f"noalloc={noalloc}: hipError {code}"
        torch.cuda.synchronize()
        outs.append(from_dev_bf16(out))
    return A, B, outs[0], outs[1], need


# Shapes whose AUTO schedules use scratch: split-K with the separate reduce
# kernel (128 rows), the strip schedule with K-slices and in-kernel arrival
# counters (16 and 64 rows at narrow N), the 128 x 128 schedule's K-slices
# (256 x 4096 x 14336); and shapes that need none (512^3, 16 x 8192 x 8192
# on one strip per CU).  Each pair: the second call smaller.
PAIRS = [((128, 8192, 8192), (100, 2048, 4096)),
         ((16, 4096, 8192), (16, 1024, 2048)),
         ((64, 4096, 8192), (33, 2048, 4096)),
         ((256, 4096, 14336), (32, 4096, 4096)),
         ((512, 512, 512), (16, 8192, 8192))]


@pytest.mark.parametrize("first,second", PAIRS,
                         ids=["splitk128", "strip16", "strip64", "ksplit",
                              "none"])
def test_noalloc_equals_gemm(gpu, oracle, first, second):
    torch = gpu
    for i, (M, N, K) in enumerate((first, second)):
        say(f"case noalloc call {i} M={M} N={N} K={K} "
            f"(variant {hg.variant_name(hg.select_variant(M, N, K))})")
        A, B, ref, got, need = both(torch, oracle, M, N, K, 4100 + 10 * i)
        say(f"    scratch need {need} bytes")
        assert np.array_equal(ref, got)
        # and against the oracle, on a few rows
        rows = np.unique(np.array([0, M // 2, M - 1], np.int32))
        max_rel, _, _ = compare(got[rows], oracle.gemm_rows(A, B, rows, 0.75, 1.5))
        assert max_rel <= 1e-2


def test_noalloc_ternary_bit_exact_after_ksplit(gpu, oracle):
    """Counters stay zero across schedules in the one static array: a K-split
    128 x 128 call (partials after the counter region), then strip calls
    with in-kernel arrival counters and a split-K call, bit-exact against
    the oracle."""
    torch = gpu
    for (M, N, K) in [(256, 4096, 14336), (16, 4096, 8192), (32, 4096, 8192),
                      (16, 2048, 8192), (100, 8192, 4096), (16, 4096, 8192)]:
        say(f"case noalloc ternary M={M} N={N} K={K}")
        A, B, ref, got, _ = both(torch, oracle, M, N, K, 4200, general=False)
        assert np.array_equal(ref, got)
        if M <= 32:
            assert np.array_equal(got, oracle.gemm(A, B, 0.75, 1.5))


def test_noalloc_rejects_workspace_argument(gpu):
    torch = gpu
    say("case noalloc rejects a workspace argument")
    a = torch.zeros((16, 256), dtype=torch.uint8, device="cuda")
    out = torch.empty((16, 256), dtype=torch.bfloat16, device="cuda")
    d = hg.GemmDesc(A=a.data_ptr(), B_T=a.data_ptr(), C=out.data_ptr(), M=16,
                    N=16, K=256, lda=256, ldb=256, ldc=256,
                    workspace=a.data_ptr(), workspace_bytes=4096)
    assert hg.gemm_desc_noalloc_raw(d, 0) == hg.hipErrorInvalidValue
