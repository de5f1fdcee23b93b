"""GPU parity of AUTO's picks in the regions its rules name one by one
(hipgemm_select_variant): up to 64 rows (column strips of 32 or 64 columns,
one or more K-slices; 128 x 128 tiles for N > 64 x CUs from 17 rows and,
above 48 rows, for K > 8192), 65-128 rows (strips for a B_T of
at most 8 MiB, the split-K schedule on half-filled K-splits of 3 slices or
more, else 128 x 128 tiles), and M > 128 where 128 x 128 tiles take under
two rounds while 256 x 256 ones fill at most half the CUs. Each case checks
the pick, then runs AUTO through the plain entry point (a workspace
allocated for the call) and through the workspace entry point on ternary
inputs (every sum exact): both must equal the oracle bit for bit.
"""
import numpy as np
import pytest

import hipgemm_amd as hg
from util import from_dev_bf16, say, scale_tensor, to_dev

pytestmark = pytest.mark.gpu

V = hg.VARIANTS
TERNARY = np.array([0xB8, 0x00, 0x38], np.uint8)  # -1, 0, +1


@pytest.mark.parametrize("M,N,K,pick", [
    (64, 4096, 4096, "strip"),      # 32-column strips, 2 K-slices
    (40, 2048, 8192, "strip"),      # 4 K-slices
    (33, 6144, 2048, "strip"),      # 192 strips, one K-slice
    (48, 3072, 8192, "strip"),      # 64-column strips fill the CUs better
    (40, 14336, 8192, "strip"),     # 64-column strips: 448 of 32 > CUs
    (64, 8192, 8192, "strip"),
    (16, 28672, 8192, "strip"),     # up to 16 rows: strips throughout
    (32, 28672, 8192, "tile128"),   # N > 64 x CUs from 17 rows
    (28, 20480, 1536, "tile128"),
    (40, 24576, 8192, "tile128"),
    (56, 8192, 14336, "tile128"),   # above 48 rows, K > 8192
    (48, 8192, 14336, "strip"),     # three 16-row blocks
    (40, 3072, 1024, "strip"),      # K <= 1024, 96 strips
    (40, 2048, 1024, "tile128"),    # ... 64 strips
    (96, 2048, 4096, "strip"),      # 65-128 rows, B_T of at most 8 MiB
    (128, 6144, 2048, "tile128"),   # half-filled, but 2 slices
    (120, 2560, 4096, "skinny"),    # half-filled, 4 slices
    (100, 4096, 4096, "skinny"),
    (1536, 4096, 4096, "tile128"),  # 96 tiles of 256, 384 of 128
    (1152, 4096, 4096, "tile128"),
    (640, 8192, 4096, "4wave_mfma16"),   # the same region, a side of 8192
    (2048, 4096, 4096, "4wave_mfma16"),  # 512 tiles of 128: two full rounds
])
def test_auto_pick_bit_exact(gpu, oracle, M, N, K, pick):
    torch = gpu
    say(f"case auto-pick M={M} N={N} K={K} want={pick} seed=17")
    assert hg.select_variant(M, N, K) == V[pick]
    rng = np.random.default_rng(17)
    A = TERNARY[rng.integers(0, 3, (M, K))]
    B = TERNARY[rng.integers(0, 3, (N, K))]
    want = oracle.gemm(A, B, 0.5, 2.0)
    a, b = to_dev(torch, A), to_dev(torch, B)
    sa, sb = scale_tensor(torch, 0.5), scale_tensor(torch, 2.0)
    stream = torch.cuda.current_stream().cuda_stream
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert hg.gemm_raw(a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, K,
                       K, N, sa.data_ptr(), sb.data_ptr(), 0, stream) == 0
    torch.cuda.synchronize()
    got = from_dev_bf16(out)
    assert np.array_equal(got, want), (
        f"plain entry: {int((got != want).sum())} of {M * N} outputs differ")
    need = hg.workspace_size(M, N, K, 0)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device="cuda")
    out.fill_(float("nan"))
    assert hg.gemm_raw_ws(a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K,
                          K, K, N, sa.data_ptr(), sb.data_ptr(), 0,
                          ws.data_ptr(), need, stream) == 0
    torch.cuda.synchronize()
    got = from_dev_bf16(out)
    assert np.array_equal(got, want), (
        f"workspace entry: {int((got != want).sum())} of {M * N} outputs differ")
    if need:
        assert not ws[:16384].cpu().numpy().any(), "counters not left zero"


def test_sweep_module_reports_auto(gpu):
    """hipgemm_amd.sweep times the schedules that take a shape and reports
    AUTO's pick against the fastest (measurement only)."""
    import io

    from hipgemm_amd import sweep

    say("case sweep 64x1024x1024 strip/tile128, 128x256x256 all")
    buf = io.StringIO()
    r = sweep.sweep([(64, 1024, 1024), (128, 256, 256)], [V["strip"], V["tile128"], V["skinny"]],
                    rounds=2, launches=10, out=buf)
    text = buf.getvalue()
    assert len(r) == 2 and all(x >= 1.0 for x in r), text
    assert "64x1024x1024:" in text and "summary: 2 shapes" in text
