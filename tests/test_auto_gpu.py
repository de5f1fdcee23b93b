"""GPU parity of AUTO's picks in the regions its rules name one by one
(hipgemm_select_variant): 33-128 rows (the split-K schedule on half-filled
K-splits, the 128 x 128 one for short K, wide N or, above 48 rows, long K,
the strip elsewhere up to 64 rows), and M > 128 where 128 x 128 tiles take
under two rounds while 256 x 256 ones fill at most half the CUs.  Each case
checks the pick, then runs AUTO through the plain entry point (a workspace
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
    (64, 4096, 4096, "skinny"),     # half-filled K-split, 16 MiB of B_T
    (40, 2048, 8192, "skinny"),
    (128, 6144, 2048, "tile128"),   # half-filled, but 2 slices
    (64, 2048, 2048, "skinny"),     # half-filled, small B_T
    (48, 1024, 1024, "tile128"),    # 33-64 rows, K <= 1024
    (120, 2560, 4096, "skinny"),
    (40, 28672, 4096, "tile128"),   # N >= 12288
    (36, 14336, 4096, "tile128"),
    (64, 8192, 14336, "tile128"),   # above 48 rows, K >= 12288
    (48, 8192, 14336, "strip"),
    (64, 8192, 8192, "strip"),
    (32, 28672, 8192, "strip"),     # up to 32 rows
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
