"""GPU parity of the 4-wave schedule's overlapped epilogue.

Where the rows of C start on 128-byte lines (ldc a multiple of 64, C 128-byte
aligned) the 16x16x128 4-wave kernel converts and stores each 64 x 64
accumulator quadrant inside the MFMA stream of the tile boundary
(gemm_4wave.hpp, kLine); elsewhere it keeps the epilogue after the K loop.
These cases put C inside a larger buffer with guard rows and columns, so
that one call with a line-aligned C and one with the same C moved by 16
bytes exercise both epilogues on the same inputs: ragged M and N, one or
several tiles per persistent workgroup (the drain after the last tile and
the quadrant stores woven into the next tile's first steps), K from one
step up, K ending inside a step.  Ternary inputs (every sum exact): both
must equal the oracle bit for bit, and every guard element must keep its
canary.
"""
import numpy as np
import pytest

import hipgemm_amd as hg
from util import say, scale_tensor, to_dev

pytestmark = pytest.mark.gpu

CANARY = 0x7FA5  # a NaN bit pattern no epilogue produces
TERNARY = np.array([0xB8, 0x00, 0x38], np.uint8)  # -1, 0, +1
MFMA16 = 2  # HIPGEMM_VARIANT_4WAVE_MFMA16


@pytest.mark.parametrize("M,N,K,ldc", [
    (4352, 4352, 256, 4352),   # 289 tiles: workgroups with one and two tiles
    (4000, 5000, 1216, 5056),  # ragged M, N; K ends inside a step
    (300, 5000, 208, 5056),    # one tile row, ragged N
    (513, 257, 128, 320),      # one K-step, ragged both ways
    (1, 64, 16, 64),           # one row, one 16-byte K chunk
    (8448, 512, 400, 576),     # 33 x 2 tiles, K tail
    (2048, 2048, 4096, 2048),  # 64 tiles, long K
])
def test_overlapped_epilogue_bit_exact(gpu, oracle, M, N, K, ldc):
    torch = gpu
    say(f"case overlap M={M} N={N} K={K} ldc={ldc} seed=23")
    rng = np.random.default_rng(23)
    A = TERNARY[rng.integers(0, 3, (M, K))]
    B = TERNARY[rng.integers(0, 3, (N, K))]
    want = oracle.gemm(A, B, 0.5, 0.25)
    a, b = to_dev(torch, A), to_dev(torch, B)
    sa, sb = scale_tensor(torch, 0.5), scale_tensor(torch, 0.25)
    stream = torch.cuda.current_stream().cuda_stream
    # C at a 128-byte boundary of a flat buffer (torch's allocations are
    # 512-byte aligned), or 16 bytes past it; at least two rows of ldc
    # elements of guard before C and after its last row.
    front = 2 * ldc + 64
    total = front + M * ldc + 2 * ldc + 64
    for shift, what in ((0, "line-aligned"), (8, "shifted by 16 bytes")):
        dev = torch.from_numpy(
            np.full(total, CANARY, np.uint16).view(np.int16)).to("cuda")
        assert dev.data_ptr() % 512 == 0
        c0 = front + shift
        base = dev.data_ptr() + 2 * c0
        assert base % 128 == (0 if shift == 0 else 16)
        say(f"    {what}: C at element {c0}")
        code = hg.gemm_raw(a.data_ptr(), b.data_ptr(), base, M, N, K, K, K, ldc,
                           sa.data_ptr(), sb.data_ptr(), MFMA16, stream)
        assert code == 0
        torch.cuda.synchronize()
        got = dev.cpu().numpy().view(np.uint16)
        idx = c0 + np.arange(M)[:, None] * ldc + np.arange(N)[None, :]
        C = got[idx]
        assert np.array_equal(C, want), (
            f"{what}: {int((C != want).sum())} of {M * N} outputs differ")
        mask = np.ones(got.size, bool)
        mask[idx.reshape(-1)] = False
        assert np.all(got[mask] == CANARY), f"{what}: write outside C"
