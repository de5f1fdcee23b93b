"""GPU parity of the skinny schedules (M <= 128) against the CPU oracle, through
the C ABI: the split-K schedule (HIPGEMM_VARIANT_SKINNY) and the column-strip
schedule (HIPGEMM_VARIANT_STRIP).

The schedule sums K-slices in a fixed order, so results are deterministic but
not the sequential fp32 sum: general inputs are checked with the north_star
tolerance (util.compare), ternary inputs (exact sums in any order) bit-exactly,
with canaries around C.  Every case prints its name before it runs.
"""
import numpy as np
import pytest

import hipgemm_amd as hg
from oracle import pyoracle as po
from util import REL_TOL, compare, from_dev_bf16, say, scale_tensor, to_dev

pytestmark = pytest.mark.gpu

SKINNY = hg.VARIANTS["skinny"]
STRIP = hg.VARIANTS["strip"]
BOTH = [pytest.param(SKINNY, id="splitk"), pytest.param(STRIP, id="strip")]
CANARY = 0x7FA5
TERNARY = np.array([0xB8, 0x00, 0x38], np.uint8)  # -1, 0, +1


def ternary(shape, seed):
    return TERNARY[np.random.default_rng(seed).integers(0, 3, shape)]


def run_ws(torch, A, B, M, N, K, ldc=None, sa=None, sb=None, variant=SKINNY,
           ws=None):
    """Call hipgemm_fp8_gemm_bf16_ws into a canary-guarded C; returns
    (C, guard_ok, workspace)."""
    ldc = ldc or N
    a, b = to_dev(torch, A), to_dev(torch, B)
    buf = torch.full((M + 4, ldc), CANARY, dtype=torch.int16, device="cuda")
    need = hg.workspace_size(M, N, K, variant)
    if ws is None and need:
        ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    ta = scale_tensor(torch, sa) if sa is not None else None
    tb = scale_tensor(torch, sb) if sb is not None else None
    code = hg.gemm_raw_ws(a.data_ptr(), b.data_ptr(),
                          buf.data_ptr() + 2 * ldc * 2, M, N, K, K, K, ldc,
                          ta.data_ptr() if ta is not None else 0,
                          tb.data_ptr() if tb is not None else 0, variant,
                          ws.data_ptr() if ws is not None else 0, need,
                          torch.cuda.current_stream().cuda_stream)
    assert code == 0, code
    torch.cuda.synchronize()
    got = buf.cpu().numpy().view(np.uint16)
    guard = (np.all(got[:2] == CANARY) and np.all(got[M + 2:] == CANARY)
             and np.all(got[2:M + 2, N:] == CANARY))
    return np.ascontiguousarray(got[2:M + 2, :N]), guard, ws


@pytest.mark.parametrize("variant", BOTH)
@pytest.mark.parametrize("M,N,K", [
    (1, 300, 16), (16, 8192, 8192), (17, 1000, 272), (33, 4100, 1040),
    (64, 512, 4096), (100, 2050, 528), (128, 8192, 8192), (5, 260, 8192),
    (32, 8192, 8192), (128, 2048, 8192), (20, 16384, 1024), (48, 70, 4112),
    # 17-32 rows on 32-column strips (A staged through LDS): K tails,
    # ragged N, many K-slices
    (24, 3000, 4112), (31, 96, 20000), (29, 5000, 1008),
    # long K: the split-K plan takes two workgroups per CU (8 and 16 slices)
    (128, 8192, 12288), (96, 4096, 28672)])
def test_skinny_ternary_bit_exact(gpu, oracle, M, N, K, variant):
    torch = gpu
    say(f"case skinny-ternary [v{variant}] M={M} N={N} K={K} seed=21 "
        f"ws={hg.workspace_size(M, N, K, variant)}")
    A, B = ternary((M, K), 21), ternary((N, K), 22)
    ldc = N + 12 if N % 4 else N + 8  # N % 4 != 0 takes the 2-byte stores
    C, guard, _ = run_ws(torch, A, B, M, N, K, ldc=ldc, sa=0.5, sb=4.0,
                         variant=variant)
    assert guard, "write outside M x N"
    want = oracle.gemm(A, B, 0.5, 4.0)
    assert np.array_equal(C, want)


@pytest.mark.parametrize("variant", BOTH)
@pytest.mark.parametrize("M,N,K", [(16, 8192, 8192), (128, 8192, 8192),
                                   (40, 3000, 2064), (64, 28672, 4096),
                                   (128, 8192, 16384)])
def test_skinny_uniform_within_tolerance(gpu, oracle, M, N, K, variant):
    torch = gpu
    sa, sb = oracle.draw_scale(51), oracle.draw_scale(52)
    say(f"case skinny-uniform [v{variant}] M={M} N={N} K={K} seed=5 sa={sa} sb={sb}")
    A = oracle.fill((M, K), 5001, po.UNIFORM, -1.0, 1.0)
    B = oracle.fill((N, K), 5002, po.UNIFORM, -1.0, 1.0)
    C, guard, _ = run_ws(torch, A, B, M, N, K, sa=sa, sb=sb, variant=variant)
    assert guard
    max_rel, exact, _ = compare(C, oracle.gemm(A, B, sa, sb))
    say(f"    max_rel={max_rel:.3e} exact={exact:.6f}")
    assert max_rel <= REL_TOL


def test_skinny_deterministic_and_workspace_left_zero(gpu, oracle):
    """Same bits on every call (the slice sum order is fixed, whichever
    workgroup arrives last), and the workspace counters are zero again after
    each call, so one workspace serves consecutive calls."""
    torch = gpu
    M, N, K = 64, 4096, 8192
    say(f"case skinny-determinism M={M} N={N} K={K}")
    A = oracle.fill((M, K), 61, po.NORMAL, 0.0, 1.0)
    B = oracle.fill((N, K), 62, po.NORMAL, 0.0, 1.0)
    C0, _, ws = run_ws(torch, A, B, M, N, K)
    tiles_n = (N + 255) // 256
    for _ in range(3):
        counters = ws[:4 * tiles_n].cpu().numpy()
        assert not counters.any(), "arrival counters not reset"
        C1, _, ws = run_ws(torch, A, B, M, N, K, ws=ws)
        assert np.array_equal(C0, C1)
    max_rel, _, _ = compare(C0, oracle.gemm(A, B))
    assert max_rel <= REL_TOL


@pytest.mark.parametrize("M,N,K,splits", [
    (16, 1024, 32768, True),   # 1.5 MiB of A and B_T per strip: K-slices
    (16, 2048, 4096, False),   # 192 KiB per strip: one K-slice
])
def test_strip_plain_entry_without_workspace(gpu, oracle, M, N, K, splits):
    """hipgemm_fp8_gemm_bf16 (no workspace argument) on the strip schedule:
    where each strip would stream more than 1 MiB of A and B_T it takes a
    stream-ordered allocation for its K-slices and equals the workspace
    entry point bit for bit; below that it runs one K-slice, allocating
    nothing, and stays within the tolerance of the oracle (its sums run in
    another order than the workspace entry point's)."""
    torch = gpu
    say(f"case strip-plain M={M} N={N} K={K} splits={splits}")
    assert hg.select_variant(M, N, K) == STRIP
    assert hg.workspace_size(M, N, K, 0) > 0
    A = oracle.fill((M, K), 71, po.UNIFORM, -1.0, 1.0)
    B = oracle.fill((N, K), 72, po.UNIFORM, -1.0, 1.0)
    a, b = to_dev(torch, A), to_dev(torch, B)
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    code = hg.gemm_raw(a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K,
                       K, K, N, 0, 0, 0,
                       torch.cuda.current_stream().cuda_stream)
    assert code == 0
    torch.cuda.synchronize()
    C_plain = from_dev_bf16(out)
    C_ws, _, _ = run_ws(torch, A, B, M, N, K, variant=STRIP)
    if splits:
        assert np.array_equal(C_plain, C_ws)
    max_rel, _, _ = compare(C_plain, oracle.gemm(A, B))
    say(f"    max_rel={max_rel:.3e}")
    assert max_rel <= REL_TOL


def test_skinny_torch_helper(gpu, oracle):
    torch = gpu
    M, N, K = 128, 1024, 2048
    say(f"case skinny-torch-helper M={M} N={N} K={K}")
    A, B = ternary((M, K), 81), ternary((N, K), 82)
    out = hg.fp8_gemm_bf16(to_dev(torch, A), to_dev(torch, B))
    torch.cuda.synchronize()
    assert np.array_equal(from_dev_bf16(out), oracle.gemm(A, B))
