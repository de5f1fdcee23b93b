"""GPU parity of fp4 (OCP E2M1) operands on the 128 x 128 schedule and the
4-wave 16x16x128 one (per-tensor epilogue) against the oracle's hg_gemm_ex.

Every product of two fp4 values is a multiple of 1/4 below 36 and every
partial sum over K <= 8192 stays below 2^19, so fp32 sums are exact in any
order: random bytes (all 16 codes in both nibbles, -0 included) are
bit-exact against the oracle, for bf16, fp16, fp32 and e4m3 outputs, with
the extended epilogue, K tails, ragged M / N, the K-split path and
canaries.  Every case prints its name before it touches the GPU.
"""
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


def run(torch, A, B, K, out=0, act=0, sa=None, sr=None, sc=None, bias=None,
        variant=0, guard_cols=24):
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
                    lda=A.shape[1], ldb=B.shape[1], ldc=ldc, a_format=4,
                    b_format=4, out_dtype=out, activation=act,
                    scale_a=ptr(t["sa"]), scale_rows=ptr(t["sr"]),
                    scale_cols=ptr(t["sc"]), bias=ptr(t["bias"]),
                    variant=variant)
    code = hg.gemm_desc_raw(d, torch.cuda.current_stream().cuda_stream)
    assert code == 0, code
    torch.cuda.synchronize()
    got = buf.cpu().numpy().view(NP[es]).reshape(M + 4, ldc)
    guard = (np.all(got[:2] == CANARY[es]) and np.all(got[M + 2:] == CANARY[es])
             and np.all(got[2:M + 2, N:] == CANARY[es]))
    return np.ascontiguousarray(got[2:M + 2, :N]), guard


def rand_fp4(shape, seed):
    return np.random.default_rng(seed).integers(0, 256, shape).astype(np.uint8)


@pytest.mark.parametrize("variant", [0, 2, 5], ids=["auto", "4wave", "tile128"])
@pytest.mark.parametrize("M,N,K", [(300, 260, 224), (512, 512, 1024),
                                   (129, 1000, 96), (1100, 700, 4128),
                                   (200, 300, 8192),
                                   # 81 tiles of 256, K 2176 bytes: AUTO's
                                   # 4-wave schedule
                                   (2304, 2304, 4352)])
def test_fp4_bit_exact(gpu, oracle, M, N, K, variant):
    say(f"case [v{variant}] fp4 M={M} N={N} K={K} seed=111")
    A, B = rand_fp4((M, K // 2), 111), rand_fp4((N, K // 2), 112)
    C, guard = run(gpu, A, B, K, sa=[0.5], variant=variant)
    assert guard, "write outside the M x N window"
    want = oracle.gemm_ex(A, B, a_fmt=4, b_fmt=4, scale_a=0.5)
    assert np.array_equal(C, want), f"{int((C != want).sum())} of {C.size} differ"


@pytest.mark.parametrize("variant", [2, 5], ids=["4wave", "tile128"])
@pytest.mark.parametrize("out", [0, 1, 2, 3], ids=["bf16", "f16", "f32", "e4m3"])
@pytest.mark.parametrize("shape", [(384, 520, 512), (200, 300, 8192)],
                         ids=["plain", "ksplit"])
def test_fp4_epilogue(gpu, oracle, out, shape, variant):
    M, N, K = shape
    say(f"case [v{variant}] fp4-epilogue out={out} M={M} N={N} K={K} seed=113")
    rng = np.random.default_rng(113)
    A, B = rand_fp4((M, K // 2), 113), rand_fp4((N, K // 2), 114)
    sr = np.exp2(rng.integers(-3, 4, M)).astype(np.float32)
    sc = np.exp2(rng.integers(-6, -1, N)).astype(np.float32)
    bias = rng.uniform(-4, 4, N).astype(np.float32)
    C, guard = run(gpu, A, B, K, out=out, act=1, sa=[0.25], sr=sr, sc=sc,
                   bias=bias, variant=variant)
    assert guard
    want = oracle.gemm_ex(A, B, a_fmt=4, b_fmt=4, out=out, act=1, scale_a=0.25,
                          scale_rows=sr, scale_cols=sc, bias=bias)
    assert np.array_equal(C, want), f"{int((C != want).sum())} differ"


def test_fp4_torch_dtype(gpu, oracle):
    torch = gpu
    M, N, K = 256, 384, 1024
    say(f"case fp4-helper M={M} N={N} K={K}")
    A, B = rand_fp4((M, K // 2), 115), rand_fp4((N, K // 2), 116)
    a = torch.from_numpy(A).cuda().view(torch.float4_e2m1fn_x2)
    b = torch.from_numpy(B).cuda().view(torch.float4_e2m1fn_x2)
    y = hg.gemm(a, b, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (M, N)
    assert np.array_equal(y.cpu().numpy().view(np.uint32),
                          oracle.gemm_ex(A, B, a_fmt=4, b_fmt=4, out=po.OUT_F32))
