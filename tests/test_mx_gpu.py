"""GPU parity of MX block scales (hipgemm_gemm with mx_scale_a / mx_scale_b)
against the oracle's hg_gemm_mx, and of the scale packing.

Ternary operands with E8M0 scales in 2^-2 .. 2^2 keep every partial sum
exact in fp32 (at most 2^16 in magnitude, in units of 2^-4, for K up to
4128), so any summation order gives the oracle's result: bit-exact, for every
operand-format pair, with canaries.  General inputs are
held to the north_star tolerance.  Every case prints its name before it
touches the GPU.
"""
import numpy as np
import pytest

import hipgemm_amd as hg
from oracle import pyoracle as po
from util import REL_TOL, compare, from_dev_bf16, say, to_dev

pytestmark = pytest.mark.gpu

CANARY = 0x7FA5
TERN = {0: np.array([0xB8, 0x00, 0x38], np.uint8),
        1: np.array([0xBC, 0x00, 0x3C], np.uint8)}


def np_pack(S, rows, K):
    """The packed layout, restated from its definition (MxArgs)."""
    kb = (K + 31) // 32
    P = ((K + 127) // 128 + 1) // 2
    W = (rows + 127) // 128
    i = np.arange(W * P * 1024)
    f, st, l, wp = i & 7, (i >> 3) & 1, (i >> 4) & 63, i >> 10
    p, w = wp % P, wp // P
    row = 128 * w + 16 * f + (l & 15)
    blk = 4 * (2 * p + st) + (l >> 4)
    out = np.full(i.shape, 127, np.uint8)
    ok = (row < rows) & (blk < kb)
    out[ok] = S[row[ok], blk[ok]]
    return out


def run(torch, A, B, sa, sb, fa=0, fb=0, s_a=None, variant=0, ldc_pad=24,
        K=None):
    """K: elements per row (default the bytes of A's rows; fp4: twice)."""
    M, Kb = A.shape
    K = K or Kb
    N = B.shape[0]
    ldc = N + ldc_pad
    a, b = to_dev(torch, A), to_dev(torch, B)
    pa = hg.mx_pack_scales(torch.from_numpy(np.ascontiguousarray(sa)).cuda(), K)
    pb = hg.mx_pack_scales(torch.from_numpy(np.ascontiguousarray(sb)).cuda(), K)
    tsa = torch.tensor([s_a], device="cuda") if s_a is not None else None
    buf = torch.full((M + 4, ldc), CANARY, dtype=torch.int16, device="cuda")
    d = hg.GemmDesc(A=a.data_ptr(), B_T=b.data_ptr(),
                    C=buf.data_ptr() + 2 * ldc * 2, M=M, N=N, K=K, lda=Kb,
                    ldb=Kb, ldc=ldc, a_format=fa, b_format=fb,
                    scale_a=tsa.data_ptr() if tsa is not None else 0,
                    variant=variant, mx_scale_a=pa.data_ptr(),
                    mx_scale_b=pb.data_ptr())
    code = hg.gemm_desc_raw(d, torch.cuda.current_stream().cuda_stream)
    assert code == 0, code
    torch.cuda.synchronize()
    got = buf.cpu().numpy().view(np.uint16)
    guard = (np.all(got[:2] == CANARY) and np.all(got[M + 2:] == CANARY)
             and np.all(got[2:M + 2, N:] == CANARY))
    return np.ascontiguousarray(got[2:M + 2, :N]), guard


def scales(rng, rows, K, lo=125, hi=130):
    return rng.integers(lo, hi, (rows, (K + 31) // 32)).astype(np.uint8)


@pytest.mark.parametrize("rows,K", [(1, 32), (100, 160), (128, 256),
                                    (300, 4128), (1000, 96)])
def test_pack_layout(gpu, rows, K):
    say(f"case mx-pack rows={rows} K={K}")
    rng = np.random.default_rng(rows + K)
    S = rng.integers(0, 256, (rows, (K + 31) // 32)).astype(np.uint8)
    got = hg.mx_pack_scales(gpu.from_numpy(S).cuda(), K)
    gpu.cuda.synchronize()
    want = np_pack(S, rows, K)
    assert got.numel() == want.size == hg.mx_scales_bytes(rows, K)
    assert np.array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("variant", [2, 5], ids=["mfma16", "tile128"])
@pytest.mark.parametrize("fa,fb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(300, 260, 224), (512, 512, 1024),
                                   (257, 1000, 96), (1100, 1300, 4128),
                                   (200, 300, 4096)])
def test_mx_ternary_bit_exact(gpu, oracle, M, N, K, fa, fb, variant):
    say(f"case [v{variant}] mx-ternary a={fa} b={fb} M={M} N={N} K={K} seed=91")
    rng = np.random.default_rng(91)
    A = TERN[fa][rng.integers(0, 3, (M, K))]
    B = TERN[fb][rng.integers(0, 3, (N, K))]
    sa, sb = scales(rng, M, K), scales(rng, N, K)
    C, guard = run(gpu, A, B, sa, sb, fa, fb, s_a=0.75, variant=variant)
    assert guard, "write outside the M x N window"
    want = oracle.gemm_mx(A, B, sa, sb, fa, fb, scale_a=0.75)
    assert np.array_equal(C, want), f"{int((C != want).sum())} of {C.size} differ"


@pytest.mark.parametrize("spread", [4, 15])
def test_mx_general_inputs(gpu, oracle, spread):
    """Normal(0, 1) e4m3 operands with block scales 2^-spread .. 2^spread,
    against the exact product (float64 of the decoded, scaled operands):
    |C - R| <= 2^-8 |R| + K 2^-24 S, S = sum_k |a_k b_k| -- one bf16 ulp
    plus the standard bound for a K-term float32 sum.  (The MFMA's internal
    accumulation is not correctly rounded: on plain fp8 operands about 1 % of
    outputs already land beyond half an ulp; with block scales the products
    span a wider range and the same absolute error weighs more against the
    north_star metric's floor, so this bound is the parity criterion here.)"""
    M, N, K = 2048, 1536, 2048
    say(f"case mx-normal spread={spread} M={M} N={N} K={K}")
    rng = np.random.default_rng(92 + spread)
    A = oracle.fill((M, K), 92001, po.NORMAL, 0.0, 1.0)
    B = oracle.fill((N, K), 92002, po.NORMAL, 0.0, 1.0)
    sa = scales(rng, M, K, 127 - spread, 128 + spread)
    sb = scales(rng, N, K, 127 - spread, 128 + spread)
    C, guard = run(gpu, A, B, sa, sb)
    assert guard
    Af = oracle.decode(A, 0).astype(np.float64) * np.exp2(
        np.repeat(sa.astype(np.float64) - 127, 32, axis=1))
    Bf = oracle.decode(B, 0).astype(np.float64) * np.exp2(
        np.repeat(sb.astype(np.float64) - 127, 32, axis=1))
    R = Af @ Bf.T
    S = np.abs(Af) @ np.abs(Bf).T
    Cf = (C.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    excess = np.abs(Cf - R) - (2.0 ** -8 * np.abs(R) + K * 2.0 ** -24 * S)
    max_rel, exact, _ = compare(C, oracle.gemm_mx(A, B, sa, sb))
    say(f"    vs oracle: max_rel={max_rel:.3e} exact={exact:.6f}; "
        f"bound violations={int((excess > 0).sum())}")
    assert np.all(excess <= 0)
    assert exact > 0.98


def test_mx_unit_scales_equal_plain(gpu, oracle):
    """All scales 1.0 (127): the plain entry's result on general inputs."""
    torch = gpu
    M, N, K = 768, 640, 1024
    say(f"case mx-unit M={M} N={N} K={K}")
    A = oracle.fill((M, K), 93001, po.NORMAL, 0.0, 1.0)
    B = oracle.fill((N, K), 93002, po.NORMAL, 0.0, 1.0)
    C, _ = run(torch, A, B, np.full((M, K // 32), 127, np.uint8),
               np.full((N, K // 32), 127, np.uint8), variant=2, ldc_pad=0)
    ref = hg.fp8_gemm_bf16(to_dev(torch, A), to_dev(torch, B), variant=2)
    torch.cuda.synchronize()
    max_rel, exact, _ = compare(C, from_dev_bf16(ref))
    say(f"    vs plain: max_rel={max_rel:.3e} exact={exact:.6f}")
    assert max_rel <= REL_TOL
    assert compare(C, oracle.gemm(A, B))[0] <= REL_TOL


@pytest.mark.parametrize("variant", [0, 2, 5], ids=["auto", "4wave", "tile128"])
@pytest.mark.parametrize("M,N,K", [(300, 260, 256), (129, 1000, 96),
                                   (1100, 700, 4128), (200, 300, 4096),
                                   # 81 tiles of 256, K 2176 bytes: AUTO's
                                   # 4-wave schedule
                                   (2304, 2304, 4352)])
def test_mxfp4_bit_exact(gpu, oracle, M, N, K, variant):
    """MXFP4: fp4 operands (random bytes) with block scales 2^-1 .. 2^1 on
    the 128 x 128 schedule (whole K and K-slices) and the 4-wave one:
    products are multiples of 2^-4 below 144, sums below 2^20 for
    K <= 7000, exact in fp32 in any order -- bit-exact against
    hg_gemm_mx."""
    say(f"case [v{variant}] mxfp4 M={M} N={N} K={K} seed=121")
    rng = np.random.default_rng(121)
    A = rng.integers(0, 256, (M, K // 2)).astype(np.uint8)
    B = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    sa, sb = scales(rng, M, K, 126, 129), scales(rng, N, K, 126, 129)
    C, guard = run(gpu, A, B, sa, sb, 4, 4, s_a=0.5, variant=variant, K=K)
    assert guard, "write outside the M x N window"
    want = oracle.gemm_mx(A, B, sa, sb, 4, 4, scale_a=0.5)
    assert np.array_equal(C, want), f"{int((C != want).sum())} of {C.size} differ"


def test_mx_nan_scale(gpu, oracle):
    """A scale of 255 is NaN for every output of its row (A) or column (B)."""
    M, N, K = 300, 400, 256
    say(f"case mx-nan M={M} N={N} K={K}")
    rng = np.random.default_rng(94)
    A = TERN[0][rng.integers(0, 3, (M, K))]
    B = TERN[0][rng.integers(0, 3, (N, K))]
    sa, sb = scales(rng, M, K), scales(rng, N, K)
    sa[17, 3] = 255
    sb[250, 7] = 255
    C, guard = run(gpu, A, B, sa, sb)
    assert guard
    want = oracle.gemm_mx(A, B, sa, sb)
    nan_c, nan_w = (C & 0x7FFF) > 0x7F80, (want & 0x7FFF) > 0x7F80
    assert nan_w[17].all() and nan_w[:, 250].all()
    assert np.array_equal(nan_c, nan_w)
    assert np.array_equal(C[~nan_w], want[~nan_w])


def test_mx_torch_helper(gpu, oracle):
    torch = gpu
    M, N, K = 256, 384, 512
    say(f"case mx-helper M={M} N={N} K={K}")
    rng = np.random.default_rng(95)
    A = TERN[1][rng.integers(0, 3, (M, K))]
    B = TERN[0][rng.integers(0, 3, (N, K))]
    sa, sb = scales(rng, M, K), scales(rng, N, K)
    a = torch.from_numpy(A).cuda().view(torch.float8_e5m2)
    b = torch.from_numpy(B).cuda().view(torch.float8_e4m3fn)
    y = hg.gemm(a, b, mx_scale_a=hg.mx_pack_scales(torch.from_numpy(sa).cuda(), K),
                mx_scale_b=hg.mx_pack_scales(torch.from_numpy(sb).cuda(), K))
    torch.cuda.synchronize()
    assert np.array_equal(from_dev_bf16(y), oracle.gemm_mx(A, B, sa, sb, 1, 0))
