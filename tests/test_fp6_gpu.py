"""GPU parity of fp6 (OCP E2M3 / E3M2) operands on the 128 x 128 and 4-wave
16x16x128 schedules against the oracle's hg_gemm_ex.

Operands are packed LSB first, element k of a row at bits [6k, 6k + 6) of
its little-endian bit string (include/hipgemm.h).  The inputs keep every
fp32 partial sum exact in any order, so the GPU must match the oracle bit
for bit: E2M3 products are multiples of 2^-6 below 56.25 and K <= 4096
keeps sums below 2^18; E3M2 codes are drawn with magnitudes <= 3.5
(products multiples of 2^-8 below 12.25, sums below 2^16).  Covered: the
four format pairs, K tails (half a 96-byte step), ragged M / N, the K-split
path, every output type with row / column scales, bias and relu on both
schedules, canaries.
Every case prints its name before it touches the GPU.
"""
import ctypes

import numpy as np
import pytest

import hipgemm_amd as hg
from oracle import pyoracle as po
from util import say, to_dev

pytestmark = pytest.mark.gpu

ES = {po.OUT_BF16: 2, po.OUT_F16: 2, po.OUT_F32: 4, po.OUT_FP8: 1}
NP = {2: np.uint16, 4: np.uint32, 1: np.uint8}
TV = {2: np.int16, 4: np.int32, 1: np.uint8}
CANARY = {2: 0x7FA5, 4: 0x7FA5A5A5, 1: 0xA5}
E2M3, E3M2 = po.FMT_FP6_E2M3, po.FMT_FP6_E3M2


def pack6(codes: np.ndarray) -> np.ndarray:
    """rows x K 6-bit codes -> rows x 3K/4 bytes, LSB first."""
    c = codes.astype(np.uint32).reshape(codes.shape[0], -1, 4)
    w = c[..., 0] | (c[..., 1] << 6) | (c[..., 2] << 12) | (c[..., 3] << 18)
    b = np.stack([w & 255, (w >> 8) & 255, (w >> 16) & 255], axis=2)
    return b.reshape(codes.shape[0], -1).astype(np.uint8)


def rand_codes(fmt, shape, seed):
    rng = np.random.default_rng(seed)
    if fmt == E2M3:
        return rng.integers(0, 64, shape).astype(np.uint8)
    # E3M2 magnitudes <= 3.5: exponent field <= 4 (codes 0..19), either sign
    return (rng.integers(0, 20, shape) | (rng.integers(0, 2, shape) << 5)).astype(np.uint8)


def run(torch, A, B, K, fa, fb, out=0, act=0, sa=None, sr=None, sc=None,
        bias=None, variant=0, guard_cols=24):
    M, N = A.shape[0], B.shape[0]
    es = ES[out]
    ldc = N + guard_cols
    a, b = to_dev(torch, A), to_dev(torch, B)

    def dev(x):
        return None if x is None else torch.from_numpy(
            np.ascontiguousarray(x, np.float32).reshape(-1)).to("cuda")
    t = {k: dev(v) for k, v in dict(sa=sa, sr=sr, sc=sc, bias=bias).items()}
    host = np.full((M + 4) * ldc, CANARY[es], NP[es])
    buf = torch.from_numpy(host.view(TV[es])).to("cuda")
    ptr = (lambda x: x.data_ptr() if x is not None else 0)
    d = hg.GemmDesc(A=a.data_ptr(), B_T=b.data_ptr(),
                    C=buf.data_ptr() + 2 * ldc * es, M=M, N=N, K=K,
                    lda=A.shape[1], ldb=B.shape[1], ldc=ldc, a_format=fa,
                    b_format=fb, out_dtype=out, activation=act,
                    scale_a=ptr(t["sa"]), scale_rows=ptr(t["sr"]),
                    scale_cols=ptr(t["sc"]), bias=ptr(t["bias"]),
                    variant=variant)
    need = int(hg.lib().hipgemm_gemm_workspace_size(ctypes.byref(d)))
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda")
    d.workspace = ws.data_ptr() if need else None
    d.workspace_bytes = need
    code = hg.gemm_desc_raw(d, torch.cuda.current_stream().cuda_stream)
    assert code == 0, code
    torch.cuda.synchronize()
    got = buf.cpu().numpy().view(NP[es]).reshape(M + 4, ldc)
    guard = (np.all(got[:2] == CANARY[es]) and np.all(got[M + 2:] == CANARY[es])
             and np.all(got[2:M + 2, N:] == CANARY[es]))
    return np.ascontiguousarray(got[2:M + 2, :N]), guard


PAIRS = [(E2M3, E2M3), (E3M2, E3M2), (E2M3, E3M2), (E3M2, E2M3)]


@pytest.mark.parametrize("fa,fb", PAIRS, ids=["e2m3", "e3m2", "mixed", "mixed2"])
@pytest.mark.parametrize("variant", [0, 2, 5], ids=["auto", "4wave16", "tile128"])
@pytest.mark.parametrize("M,N,K", [(300, 260, 192), (512, 512, 1024),
                                   (129, 1000, 64), (1100, 700, 4096),
                                   (200, 300, 4032), (256, 2048, 3072),
                                   (2304, 3840, 256)])
def test_fp6_bit_exact(gpu, oracle, M, N, K, fa, fb, variant):
    # 2304 x 3840: 135 tiles of 256 x 256, so AUTO takes the 4-wave schedule
    say(f"case [v{variant}] fp6 a={fa} b={fb} M={M} N={N} K={K} seed=121 "
        f"auto={hg.select_variant(M, N, K // 4 * 3)} "
        f"ws={hg.lib().hipgemm_workspace_size(M, N, K // 4 * 3, 5)}")
    A = pack6(rand_codes(fa, (M, K), 121))
    B = pack6(rand_codes(fb, (N, K), 122))
    C, guard = run(gpu, A, B, K, fa, fb, sa=[0.5], variant=variant)
    assert guard, "write outside the M x N window"
    want = oracle.gemm_ex(A, B, a_fmt=fa, b_fmt=fb, scale_a=0.5)
    assert np.array_equal(C, want), f"{int((C != want).sum())} of {C.size} differ"


@pytest.mark.parametrize("out", [0, 1, 2, 3], ids=["bf16", "f16", "f32", "e4m3"])
@pytest.mark.parametrize("shape,variant", [((384, 520, 512), 5), ((256, 2048, 3072), 5),
                                           ((384, 520, 512), 2), ((300, 1040, 1088), 2)],
                         ids=["plain", "ksplit", "4wave16", "4wave16-ragged"])
def test_fp6_epilogue(gpu, oracle, out, shape, variant):
    M, N, K = shape
    say(f"case [v{variant}] fp6-epilogue out={out} M={M} N={N} K={K} seed=123")
    rng = np.random.default_rng(123)
    A = pack6(rand_codes(E2M3, (M, K), 123))
    B = pack6(rand_codes(E3M2, (N, K), 124))
    sr = np.exp2(rng.integers(-3, 4, M)).astype(np.float32)
    sc = np.exp2(rng.integers(-6, -1, N)).astype(np.float32)
    bias = rng.uniform(-4, 4, N).astype(np.float32)
    C, guard = run(gpu, A, B, K, E2M3, E3M2, out=out, act=1, sa=[0.25], sr=sr,
                   sc=sc, bias=bias, variant=variant)
    assert guard
    want = oracle.gemm_ex(A, B, a_fmt=E2M3, b_fmt=E3M2, out=out, act=1,
                          scale_a=0.25, scale_rows=sr, scale_cols=sc, bias=bias)
    assert np.array_equal(C, want), f"{int((C != want).sum())} differ"


def test_fp6_torch_helper(gpu, oracle):
    torch = gpu
    M, N, K = 256, 384, 1024
    say(f"case fp6-helper M={M} N={N} K={K}")
    A = pack6(rand_codes(E3M2, (M, K), 125))
    B = pack6(rand_codes(E2M3, (N, K), 126))
    y = hg.gemm(torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda(),
                a_format=hg.FMT_FP6_E3M2, b_format=hg.FMT_FP6_E2M3,
                out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (M, N)
    assert np.array_equal(y.cpu().numpy().view(np.uint32),
                          oracle.gemm_ex(A, B, a_fmt=E3M2, b_fmt=E2M3,
                                         out=po.OUT_F32))
