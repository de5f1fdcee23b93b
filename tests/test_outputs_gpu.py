"""GPU parity of the fp32 and e4m3 outputs of hipgemm_gemm against the
oracle's hg_gemm_ex, on every schedule that takes them (AUTO, 4-wave
16x16x128, skinny, 128 x 128 with and without K-slices, AUTO's column
split), with canaries sized to the element.

fp32 output is the epilogue's fp32 value itself, e4m3 output its
saturating conversion (hg_f32_to_e4m3, pinned against the HIP header): both
bit-exact wherever the epilogue is exact arithmetic (ternary sums,
power-of-two scales, bias through one fma, relu).  The e4m3 conversion is
also pinned directly: rows of zeros in A make C the conversion of the bias
vector, which holds ties, the saturation boundary, Inf, NaN and subnormals.
silu / gelu are held to the north_star tolerance.
"""
import numpy as np
import pytest

import hipgemm_amd as hg
from oracle import pyoracle as po
from util import DELTA_FRAC, REL_TOL, say, to_dev

pytestmark = pytest.mark.gpu

TERN = {0: np.array([0xB8, 0x00, 0x38], np.uint8),
        1: np.array([0xBC, 0x00, 0x3C], np.uint8)}
ES = {po.OUT_F32: 4, po.OUT_FP8: 1}
NP = {4: np.uint32, 1: np.uint8}
CANARY = {4: 0x7FA5A5A5, 1: 0xA5}
# (variant, shape): AUTO on a tiled shape, the 4-wave schedule, skinny,
# 128 x 128 without and with K-slices.
CASES = [pytest.param(0, (520, 600, 336), id="auto"),
         pytest.param(2, (520, 600, 336), id="mfma16"),
         pytest.param(3, (96, 1000, 528), id="skinny"),
         pytest.param(6, (96, 1000, 528), id="strip"),
         pytest.param(6, (20, 9000, 1040), id="strip-wide"),
         pytest.param(5, (300, 520, 336), id="tile128"),
         pytest.param(5, (300, 1000, 4112), id="tile128-ksplit")]


def ternary(fmt, shape, seed):
    return TERN[fmt][np.random.default_rng(seed).integers(0, 3, shape)]


def run(torch, A, B, out, *, fa=0, fb=0, act=0, sa=None, sr=None, sc=None,
        bias=None, so=None, variant=0, guard_cols=24, c_offset=0):
    """hipgemm_gemm into a canary-guarded C of the output's element type;
    c_offset shifts C by that many elements (alignment cases)."""
    M, K = A.shape
    N = B.shape[0]
    es = ES[out]
    ldc = N + guard_cols
    a, b = to_dev(torch, A), to_dev(torch, B)

    def dev(x):
        return None if x is None else torch.from_numpy(
            np.ascontiguousarray(x, np.float32).reshape(-1)).to("cuda")
    t = {k: dev(v) for k, v in dict(sa=sa, sr=sr, sc=sc, bias=bias, so=so).items()}
    total = (M + 4) * ldc + c_offset
    host = np.full(total, CANARY[es], NP[es])
    buf = torch.from_numpy(host.view(np.int32 if es == 4 else np.uint8)).to("cuda")
    need = hg.workspace_size(M, N, K, variant)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda")
    ptr = (lambda x: x.data_ptr() if x is not None else 0)
    d = hg.GemmDesc(A=a.data_ptr(), B_T=b.data_ptr(),
                    C=buf.data_ptr() + (c_offset + 2 * ldc) * es, M=M, N=N,
                    K=K, lda=K, ldb=K, ldc=ldc, a_format=fa, b_format=fb,
                    out_dtype=out, activation=act, scale_a=ptr(t["sa"]),
                    scale_rows=ptr(t["sr"]), scale_cols=ptr(t["sc"]),
                    bias=ptr(t["bias"]), scale_out=ptr(t["so"]),
                    variant=variant, workspace=ws.data_ptr() if need else 0,
                    workspace_bytes=need)
    code = hg.gemm_desc_raw(d, torch.cuda.current_stream().cuda_stream)
    assert code == 0, code
    torch.cuda.synchronize()
    got = buf.cpu().numpy().view(NP[es])
    body = got[c_offset:].reshape(M + 4, ldc)
    guard = (np.all(got[:c_offset] == CANARY[es]) and
             np.all(body[:2] == CANARY[es]) and np.all(body[M + 2:] == CANARY[es])
             and np.all(body[2:M + 2, N:] == CANARY[es]))
    return np.ascontiguousarray(body[2:M + 2, :N]), guard


def e4m3_value(bits, oracle):
    return oracle.e4m3_to_f32(bits).astype(np.float64)


@pytest.mark.parametrize("variant,shape", CASES)
@pytest.mark.parametrize("out", [po.OUT_F32, po.OUT_FP8], ids=["f32", "e4m3"])
@pytest.mark.parametrize("act", [0, 1], ids=["none", "relu"])
def test_outputs_exact(gpu, oracle, variant, shape, out, act):
    M, N, K = shape
    say(f"case [v{variant}] out={out} act={act} M={M} N={N} K={K} seed=91")
    rng = np.random.default_rng(91)
    A, B = ternary(0, (M, K), 91), ternary(1, (N, K), 92)
    sr = np.exp2(rng.integers(-3, 4, M)).astype(np.float32)
    sc = np.exp2(rng.integers(-3, 4, N)).astype(np.float32)
    bias = rng.uniform(-4, 4, N).astype(np.float32)
    so = [0.25] if out == po.OUT_FP8 else None
    C, guard = run(gpu, A, B, out, fb=1, act=act, sa=[0.5], sr=sr, sc=sc,
                   bias=bias, so=so, variant=variant)
    assert guard, "write outside the M x N window"
    want = oracle.gemm_ex(A, B, b_fmt=1, out=out, act=act, scale_a=0.5,
                          scale_rows=sr, scale_cols=sc, bias=bias,
                          scale_out=so[0] if so else 1.0)
    assert np.array_equal(C, want), f"{int((C != want).sum())} of {C.size} differ"


@pytest.mark.parametrize("variant", [2, 3, 5])
def test_e4m3_conversion_pinned(gpu, oracle, variant):
    """Rows of zeros in A: C[m, n] = e4m3(bias[n] * scale_out), as
    fma(+0, s, b) = b + 0 (so -0 becomes +0), over ties, the saturation
    boundary, Inf, NaN of both signs, subnormals and a sweep of
    magnitudes."""
    special = [0.0, -0.0, 448.0, -448.0, 449.0, 464.0, 464.1, 480.0, 500.0,
               1e30, -1e30, np.inf, -np.inf, np.nan, -np.nan, 2.0 ** -9,
               2.0 ** -10, 3 * 2.0 ** -10, 2.0 ** -10 + 2.0 ** -20, 2.0 ** -7,
               1.0625, 1.1875, 1.125 + 2 ** -20, 240.0, 248.0, 256.0, 272.0,
               -0.001953125, 0.0029296875]
    rng = np.random.default_rng(93)
    sweep = (rng.standard_normal(4000) * np.exp2(rng.uniform(-12, 10, 4000)))
    bias = np.concatenate([special, sweep]).astype(np.float32)
    N = bias.size + (-bias.size) % 8
    bias = np.pad(bias, (0, N - bias.size))
    M, K = (64 if variant in (3, 6) else 256), 128
    say(f"case [v{variant}] e4m3-pin M={M} N={N} K={K}")
    A = np.zeros((M, K), np.uint8)
    B = ternary(0, (N, K), 94)
    C, guard = run(gpu, A, B, po.OUT_FP8, bias=bias, so=[1.0], variant=variant)
    assert guard
    want = oracle.f32_to_e4m3(bias + np.float32(0.0))
    assert np.array_equal(oracle.gemm_ex(A[:1], B, out=po.OUT_FP8, bias=bias)[0],
                          want)
    bad = np.nonzero(C[0] != want)[0][:20]
    assert np.array_equal(C[0], want), [(float(bias[i]), int(C[0, i]), int(want[i]))
                                        for i in bad]
    assert np.all(C == C[0])


@pytest.mark.parametrize("out", [po.OUT_F32, po.OUT_FP8], ids=["f32", "e4m3"])
def test_outputs_unaligned(gpu, oracle, out):
    """N and ldc not multiples of 4, C off the vector alignment: the
    one-store-per-element paths, on the tiled, 128 x 128 and skinny
    schedules."""
    for variant, (M, N, K) in [(2, (300, 257, 208)), (5, (200, 257, 208)),
                               (3, (40, 257, 208))]:
        say(f"case [v{variant}] unaligned out={out} M={M} N={N} K={K}")
        A, B = ternary(0, (M, K), 95), ternary(0, (N, K), 96)
        bias = np.random.default_rng(97).uniform(-2, 2, N).astype(np.float32)
        C, guard = run(gpu, A, B, out, bias=bias, sa=[0.75], variant=variant,
                       guard_cols=3, c_offset=1)
        assert guard
        want = oracle.gemm_ex(A, B, out=out, scale_a=0.75, bias=bias)
        assert np.array_equal(C, want), f"{int((C != want).sum())} differ"


def test_outputs_auto_column_split(gpu, oracle):
    """AUTO's column split with fp32 output: the 128 x 128 half's C columns
    are offset in bytes of the element."""
    M, N, K = 4000, 5000, 64
    n1 = hg.split_columns(M, N, K)
    say(f"case [auto] split f32 M={M} N={N} K={K} n1={n1}")
    A, B = ternary(0, (M, K), 98), ternary(1, (N, K), 99)
    bias = np.random.default_rng(100).uniform(-4, 4, N).astype(np.float32)
    for out in (po.OUT_F32, po.OUT_FP8):
        C, guard = run(gpu, A, B, out, fb=1, act=1, bias=bias, variant=0)
        assert guard
        want = oracle.gemm_ex(A, B, b_fmt=1, out=out, act=1, bias=bias)
        assert np.array_equal(C, want), f"{int((C != want).sum())} differ"


@pytest.mark.parametrize("variant,shape", [CASES[1], CASES[2], CASES[4]])
@pytest.mark.parametrize("act", [2, 3], ids=["gelu_tanh", "silu"])
def test_outputs_transcendental(gpu, oracle, variant, shape, act):
    M, N, K = shape
    say(f"case [v{variant}] f32/e4m3 act={act} M={M} N={N} K={K}")
    A = oracle.fill((M, K), 101, po.NORMAL, 0.0, 1.0)
    B = oracle.fill((N, K), 102, po.NORMAL, 0.0, 1.0)
    bias = np.random.default_rng(103).uniform(-2, 2, N).astype(np.float32)
    C, guard = run(gpu, A, B, po.OUT_F32, act=act, sa=[1.0 / 16], bias=bias,
                   variant=variant)
    assert guard
    want = oracle.gemm_ex(A, B, out=po.OUT_F32, act=act, scale_a=1.0 / 16, bias=bias)
    c, r = C.view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
    delta = DELTA_FRAC * float(np.sqrt(np.mean(r * r)))
    rel = float((np.abs(c - r) / np.maximum(np.abs(r), delta)).max())
    say(f"    f32 max_rel={rel:.3e}")
    assert rel <= REL_TOL
    C8, guard = run(gpu, A, B, po.OUT_FP8, act=act, sa=[1.0 / 16], bias=bias,
                    so=[8.0], variant=variant)
    assert guard
    want8 = oracle.gemm_ex(A, B, out=po.OUT_FP8, act=act, scale_a=1.0 / 16,
                           bias=bias, scale_out=8.0)
    c8, r8 = e4m3_value(C8, oracle), e4m3_value(want8, oracle)
    # one e4m3 step (2^-3 relative) where the fp32 values round apart
    step = np.maximum(np.abs(r8), 2.0 ** -6) * 2.0 ** -3
    assert np.all(np.abs(c8 - r8) <= step + 1e-30)
    say(f"    e4m3 exact={np.mean(C8 == want8):.4f}")


def test_torch_helper_outputs(gpu, oracle):
    torch = gpu
    M, N, K = 256, 384, 256
    say(f"case gemm-helper f32/e4m3 M={M} N={N} K={K}")
    A, B = ternary(1, (M, K), 104), ternary(0, (N, K), 105)
    a = torch.from_numpy(A).cuda().view(torch.float8_e5m2)
    b = torch.from_numpy(B).cuda().view(torch.float8_e4m3fn)
    bias = torch.linspace(-3, 3, N, device="cuda")
    y = hg.gemm(a, b, out_dtype=torch.float32, bias=bias, activation="relu")
    y8 = hg.gemm(a, b, out_dtype=torch.float8_e4m3fn, bias=bias,
                 activation="relu", scale_out=torch.tensor([0.5], device="cuda"))
    torch.cuda.synchronize()
    assert y.dtype == torch.float32 and y8.dtype == torch.float8_e4m3fn
    bb = bias.cpu().numpy()
    assert np.array_equal(y.cpu().numpy().view(np.uint32),
                          oracle.gemm_ex(A, B, a_fmt=1, out=po.OUT_F32, act=1, bias=bb))
    assert np.array_equal(y8.view(torch.uint8).cpu().numpy(),
                          oracle.gemm_ex(A, B, a_fmt=1, out=po.OUT_FP8, act=1,
                                         bias=bb, scale_out=0.5))
