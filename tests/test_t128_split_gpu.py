"""GPU parity of the 128 x 128 schedule's K-slices.  With the per-tensor
bf16 epilogue and at most 4 slices, the slice that finishes a 64 x 64
quadrant last sums the quadrant's partials in slice order and writes C
inside the split kernel; with more slices the reduce kernel sums them.

Cases: the BASELINE skinny shape 128 x 8192 x 8192 (4 slices), two and
three slices, ragged M and N with K ending inside a step, C rows that rule
out 16-byte stores (ldc not a multiple of 8: the 2-byte epilogue), and two
8-slice shapes (the reduce kernel, on the same workspace protocol).
Ternary inputs (every sum exact) must equal the oracle bit for bit, with a
canary-guarded C; each case runs twice on one workspace, which must give
the same bits and leave the workspace's arrival counters at zero.  Normal
inputs at the skinny BASELINE shape stay within the tolerance, and with
normal inputs the in-kernel sum and the reduce kernel give the same bits.
"""
import numpy as np
import pytest

import hipgemm_amd as hg
from oracle import pyoracle as po
from util import REL_TOL, compare, say, scale_tensor, to_dev

pytestmark = pytest.mark.gpu

TILE128 = hg.VARIANTS["tile128"]
CANARY = 0x7FA5
TERNARY = np.array([0xB8, 0x00, 0x38], np.uint8)  # -1, 0, +1
COUNTER_BYTES = 16384  # HIPGEMM_WS_COUNTER_BYTES


def run(torch, A, B, M, N, K, ldc, sa, sb, ws):
    a, b = to_dev(torch, A), to_dev(torch, B)
    buf = torch.full((M + 4, ldc), CANARY, dtype=torch.int16, device="cuda")
    ta, tb = scale_tensor(torch, sa), scale_tensor(torch, sb)
    code = hg.gemm_raw_ws(a.data_ptr(), b.data_ptr(),
                          buf.data_ptr() + 2 * ldc * 2, M, N, K, K, K, ldc,
                          ta.data_ptr(), tb.data_ptr(), TILE128, ws.data_ptr(),
                          ws.numel(), torch.cuda.current_stream().cuda_stream)
    assert code == 0, code
    torch.cuda.synchronize()
    got = buf.cpu().numpy().view(np.uint16)
    guard = (np.all(got[:2] == CANARY) and np.all(got[M + 2:] == CANARY)
             and np.all(got[2:M + 2, N:] == CANARY))
    return np.ascontiguousarray(got[2:M + 2, :N]), guard


@pytest.mark.parametrize("M,N,K,ldc", [
    (128, 8192, 8192, 8192),    # 64 tiles x 4 slices
    (128, 8192, 8192, 8196),    # the same with 2-byte C stores
    (256, 8192, 8192, 8192),    # 128 tiles x 2 slices
    (128, 10240, 8192, 10240),  # 80 tiles x 3 slices
    (128, 2048, 8192, 2048),    # 16 tiles x 8 slices: reduce kernel
    (200, 1000, 4112, 1000),    # ragged M, N; K ends inside a step
    (200, 1000, 4112, 1004),    # the same with 2-byte C stores
    (96, 4096, 28672, 4096),    # 32 tiles x 8 slices: reduce kernel
])
def test_t128_split_bit_exact(gpu, oracle, M, N, K, ldc):
    torch = gpu
    need = hg.workspace_size(M, N, K, TILE128)
    say(f"case t128-split M={M} N={N} K={K} ldc={ldc} ws={need} seed=31")
    assert need > COUNTER_BYTES, "expected a K-split plan"
    rng = np.random.default_rng(31)
    A = TERNARY[rng.integers(0, 3, (M, K))]
    B = TERNARY[rng.integers(0, 3, (N, K))]
    want = oracle.gemm(A, B, 0.5, 4.0)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    first = None
    for call in range(2):
        C, guard = run(torch, A, B, M, N, K, ldc, 0.5, 4.0, ws)
        assert guard, f"call {call}: write outside M x N"
        assert np.array_equal(C, want), (
            f"call {call}: {int((C != want).sum())} of {M * N} outputs differ")
        assert not ws[:COUNTER_BYTES].cpu().numpy().any(), (
            f"call {call}: arrival counters not reset")
        if first is None:
            first = C
        assert np.array_equal(C, first)


def test_t128_split_fused_normal_within_tolerance(gpu, oracle):
    torch = gpu
    M, N, K = 128, 8192, 8192
    sa, sb = oracle.draw_scale(81), oracle.draw_scale(82)
    say(f"case t128-split-fused normal M={M} N={N} K={K} sa={sa} sb={sb}")
    A = oracle.fill((M, K), 8101, po.NORMAL, 0.0, 1.0)
    B = oracle.fill((N, K), 8102, po.NORMAL, 0.0, 1.0)
    ws = torch.zeros(hg.workspace_size(M, N, K, TILE128), dtype=torch.uint8,
                     device="cuda")
    C, guard = run(torch, A, B, M, N, K, N, sa, sb, ws)
    assert guard
    max_rel, exact, _ = compare(C, oracle.gemm(A, B, sa, sb))
    say(f"    max_rel={max_rel:.3e} exact={exact:.6f}")
    assert max_rel <= REL_TOL


@pytest.mark.parametrize("M,N,K", [(128, 8192, 8192), (256, 8192, 8192),
                                   (128, 10240, 8192)])
def test_t128_split_sum_in_kernel_equals_reduce_kernel(gpu, oracle, M, N, K):
    """Normal inputs (sums not exact): the in-kernel sum (caller workspace)
    and the reduce kernel (no workspace: the library allocates one for the
    call and sums in a second kernel) add the same slices in the same order,
    so C is the same bit for bit."""
    torch = gpu
    say(f"case t128-split fused-vs-reduce M={M} N={N} K={K} seed=91")
    A = oracle.fill((M, K), 9101, po.NORMAL, 0.0, 1.0)
    B = oracle.fill((N, K), 9102, po.NORMAL, 0.0, 1.0)
    ws = torch.zeros(hg.workspace_size(M, N, K, TILE128), dtype=torch.uint8,
                     device="cuda")
    fused, guard = run(torch, A, B, M, N, K, N, 0.75, 1.5, ws)
    assert guard
    a, b = to_dev(torch, A), to_dev(torch, B)
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    ta, tb = scale_tensor(torch, 0.75), scale_tensor(torch, 1.5)
    code = hg.gemm_raw(a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, K,
                       K, N, ta.data_ptr(), tb.data_ptr(), TILE128,
                       torch.cuda.current_stream().cuda_stream)
    assert code == 0
    torch.cuda.synchronize()
    reduced = out.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(fused, reduced), (
        f"{int((fused != reduced).sum())} of {M * N} outputs differ")
    max_rel, _, _ = compare(fused, oracle.gemm(A, B, 0.75, 1.5))
    assert max_rel <= REL_TOL
