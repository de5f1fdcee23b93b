"""GPU parity of the general entry point hipgemm_gemm against the oracle's
hg_gemm_ex: operand formats (e4m3 / e5m2, mixed), fp16 output, per-tensor
and per-row / per-column scales, bias and activations, on every schedule
that takes them.

Bit-exact where the sums are exact in any order (ternary values, which
e4m3 and e5m2 both hold) and the epilogue is exact arithmetic (scales,
bias through one fma, relu, rounding to bf16 / fp16).  The hardware
exponential of silu / gelu and general inputs are held to the north_star
tolerance.  Canaries around C catch writes outside M x N.  Every case
prints its name before it touches the GPU.
"""
import numpy as np
import pytest

import hipgemm_amd as hg
from oracle import pyoracle as po
from util import DELTA_FRAC, REL_TOL, say, to_dev

pytestmark = pytest.mark.gpu

CANARY = 0x7FA5
TERN = {po.FMT_E4M3: np.array([0xB8, 0x00, 0x38], np.uint8),   # -1, 0, +1
        po.FMT_E5M2: np.array([0xBC, 0x00, 0x3C], np.uint8)}
FMTS = [(0, 0), (1, 0), (0, 1), (1, 1)]
TILED = [pytest.param(0, id="auto"), pytest.param(2, id="mfma16"),
         pytest.param(4, id="8wave"), pytest.param(5, id="tile128")]
ALL = TILED + [pytest.param(3, id="skinny"), pytest.param(6, id="strip")]


def ternary(fmt, shape, seed):
    idx = np.random.default_rng(seed).integers(0, 3, shape)
    return TERN[fmt][idx]


def general(oracle, fmt, shape, seed):
    """Normal(0, 1) values on the format's grid."""
    x = oracle.e4m3_to_f32(oracle.fill(shape, seed, po.NORMAL, 0.0, 1.0))
    return oracle.f32_to_e5m2(x) if fmt == po.FMT_E5M2 else oracle.f32_to_e4m3(x)


def shape_for(variant, M, N, K):
    skinny = variant in (hg.VARIANTS["skinny"], hg.VARIANTS["strip"])
    return (min(M, 96), N, K) if skinny else (M, N, K)


def run(torch, A, B, *, fa=0, fb=0, out=0, act=0, sa=None, sb=None, sr=None,
        sc=None, bias=None, variant=0, guard_cols=24):
    """hipgemm_gemm into a canary-guarded C; returns (C bits, guard_ok)."""
    M, K = A.shape
    N = B.shape[0]
    ldc = N + guard_cols
    a, b = to_dev(torch, A), to_dev(torch, B)

    def dev(x):
        return None if x is None else torch.from_numpy(
            np.ascontiguousarray(x, np.float32).reshape(-1)).to("cuda")
    t = {k: dev(v) for k, v in dict(sa=sa, sb=sb, sr=sr, sc=sc, bias=bias).items()}
    buf = torch.full((M + 4, ldc), CANARY, dtype=torch.int16, device="cuda")
    need = hg.workspace_size(M, N, K, variant)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda")
    ptr = (lambda x: x.data_ptr() if x is not None else 0)
    d = hg.GemmDesc(A=a.data_ptr(), B_T=b.data_ptr(),
                    C=buf.data_ptr() + 2 * ldc * 2, M=M, N=N, K=K, lda=K,
                    ldb=K, ldc=ldc, a_format=fa, b_format=fb, out_dtype=out,
                    activation=act, scale_a=ptr(t["sa"]), scale_b=ptr(t["sb"]),
                    scale_rows=ptr(t["sr"]), scale_cols=ptr(t["sc"]),
                    bias=ptr(t["bias"]), variant=variant,
                    workspace=ws.data_ptr() if need else 0,
                    workspace_bytes=need)
    code = hg.gemm_desc_raw(d, torch.cuda.current_stream().cuda_stream)
    assert code == 0, code
    torch.cuda.synchronize()
    got = buf.cpu().numpy().view(np.uint16)
    guard = (np.all(got[:2] == CANARY) and np.all(got[M + 2:] == CANARY)
             and np.all(got[2:M + 2, N:] == CANARY))
    return np.ascontiguousarray(got[2:M + 2, :N]), guard


def to_f32(bits, out):
    if out == po.OUT_F16:
        return bits.view(np.float16).astype(np.float32)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def max_rel(got, want, out):
    """north_star metric (util.compare) for bf16 or fp16 bits."""
    c = to_f32(got, out).astype(np.float64)
    r = to_f32(want, out).astype(np.float64)
    assert np.array_equal(np.isnan(c), np.isnan(r))
    ok = np.isfinite(r)
    assert np.array_equal(c[~ok & ~np.isnan(r)], r[~ok & ~np.isnan(r)])
    c, r = c[ok], r[ok]
    delta = max(DELTA_FRAC * float(np.sqrt(np.mean(r * r))), 1e-30)
    return float((np.abs(c - r) / np.maximum(np.abs(r), delta)).max())


@pytest.mark.parametrize("variant", ALL)
@pytest.mark.parametrize("fa,fb", FMTS)
@pytest.mark.parametrize("M,N,K", [(300, 260, 208), (512, 512, 1024),
                                   (257, 1000, 80)])
def test_formats_ternary_bit_exact(gpu, oracle, M, N, K, fa, fb, variant):
    M, N, K = shape_for(variant, M, N, K)
    say(f"case [v{variant}] formats a={fa} b={fb} M={M} N={N} K={K} seed=71")
    A, B = ternary(fa, (M, K), 71), ternary(fb, (N, K), 72)
    C, guard = run(gpu, A, B, fa=fa, fb=fb, sa=[1.25], sb=[0.5], variant=variant)
    assert guard
    want = oracle.gemm_ex(A, B, a_fmt=fa, b_fmt=fb, scale_a=1.25, scale_b=0.5)
    assert np.array_equal(C, want), f"{int((C != want).sum())} differ"


@pytest.mark.parametrize("variant", ALL)
@pytest.mark.parametrize("fa,fb", [(1, 1), (0, 1)])
def test_formats_general_inputs(gpu, oracle, fa, fb, variant):
    M, N, K = shape_for(variant, 640, 768, 2048)
    say(f"case [v{variant}] formats-normal a={fa} b={fb} M={M} N={N} K={K}")
    A, B = general(oracle, fa, (M, K), 73), general(oracle, fb, (N, K), 74)
    C, guard = run(gpu, A, B, fa=fa, fb=fb, variant=variant)
    assert guard
    want = oracle.gemm_ex(A, B, a_fmt=fa, b_fmt=fb)
    rel = max_rel(C, want, 0)
    say(f"    max_rel={rel:.3e}")
    assert rel <= REL_TOL


@pytest.mark.parametrize("variant", ALL)
@pytest.mark.parametrize("out", [0, 1], ids=["bf16", "f16"])
@pytest.mark.parametrize("act", [0, 1], ids=["none", "relu"])
def test_epilogue_exact_options(gpu, oracle, variant, out, act):
    """Scalars, row / column vectors, bias (one fma), relu and the output
    type together, bit-exact on ternary sums (power-of-two scales keep every
    product exact; the bias rounds once)."""
    M, N, K = shape_for(variant, 384, 520, 336)
    say(f"case [v{variant}] epilogue out={out} act={act} M={M} N={N} K={K}")
    rng = np.random.default_rng(75)
    A, B = ternary(0, (M, K), 75), ternary(1, (N, K), 76)
    sr = np.exp2(rng.integers(-3, 4, M)).astype(np.float32)
    sc = np.exp2(rng.integers(-3, 4, N)).astype(np.float32)
    bias = rng.uniform(-4, 4, N).astype(np.float32)
    C, guard = run(gpu, A, B, fb=1, out=out, act=act, sa=[0.5], sb=[3.0],
                   sr=sr, sc=sc, bias=bias, variant=variant)
    assert guard
    want = oracle.gemm_ex(A, B, b_fmt=1, out=out, act=act, scale_a=0.5,
                          scale_b=3.0, scale_rows=sr, scale_cols=sc, bias=bias)
    assert np.array_equal(C, want), f"{int((C != want).sum())} differ"


@pytest.mark.parametrize("variant", ALL)
@pytest.mark.parametrize("act", [2, 3], ids=["gelu_tanh", "silu"])
def test_epilogue_transcendental(gpu, oracle, variant, act):
    M, N, K = shape_for(variant, 384, 1024, 512)
    say(f"case [v{variant}] epilogue act={act} M={M} N={N} K={K}")
    A = general(oracle, 0, (M, K), 77)
    B = general(oracle, 0, (N, K), 78)
    bias = np.random.default_rng(79).uniform(-2, 2, N).astype(np.float32)
    for out in (0, 1):
        C, guard = run(gpu, A, B, out=out, act=act, sa=[1.0 / 16], bias=bias,
                       variant=variant)
        assert guard
        want = oracle.gemm_ex(A, B, out=out, act=act, scale_a=1.0 / 16, bias=bias)
        rel = max_rel(C, want, out)
        say(f"    out={out} max_rel={rel:.3e} exact={np.mean(C == want):.4f}")
        assert rel <= REL_TOL


@pytest.mark.parametrize("out,act", [(0, 0), (1, 1)])
def test_tile128_k_split(gpu, oracle, out, act):
    """The 128 x 128 schedule with K-slices (3 x 8 tiles, 4 slices of 10
    steps, a K tail) and the reduce kernel's epilogue: formats, scales, bias,
    relu, fp16; bit-exact on ternary sums, canaries around C."""
    M, N, K = 300, 1000, 4112
    say(f"case [v5] k-split out={out} act={act} M={M} N={N} K={K}")
    assert hg.workspace_size(M, N, K, 5) > 0
    rng = np.random.default_rng(87)
    A, B = ternary(1, (M, K), 87), ternary(0, (N, K), 88)
    sr = np.exp2(rng.integers(-3, 4, M)).astype(np.float32)
    sc = np.exp2(rng.integers(-3, 4, N)).astype(np.float32)
    bias = rng.uniform(-4, 4, N).astype(np.float32)
    ext = dict(sr=sr, sc=sc, bias=bias) if out or act else {}
    C, guard = run(gpu, A, B, fa=1, out=out, act=act, sa=[0.5], sb=[2.0],
                   variant=5, **ext)
    assert guard
    want = oracle.gemm_ex(A, B, a_fmt=1, out=out, act=act, scale_a=0.5,
                          scale_b=2.0, scale_rows=ext.get("sr"),
                          scale_cols=ext.get("sc"), bias=ext.get("bias"))
    assert np.array_equal(C, want), f"{int((C != want).sum())} differ"


@pytest.mark.parametrize("M,N,K", [(100, 500, 12272), (128, 256, 20480)])
def test_tile128_k_split_many_slices(gpu, oracle, M, N, K):
    """The reduce kernel loads 8 slices per batch: 12 slices (one full batch
    and a part, ragged M and N, a K tail) and 20 (two full batches and a
    part), bit-exact on ternary sums, canaries around C."""
    say(f"case [v5] k-split many slices M={M} N={N} K={K}")
    ws = hg.workspace_size(M, N, K, 5)
    tiles = -(-M // 128) * -(-N // 128)
    slices = (ws - 16384) // (tiles * 65536)  # HIPGEMM_WS_COUNTER_BYTES first
    say(f"    tiles={tiles} slices={slices}")
    assert slices > 8 and slices % 8, slices
    A, B = ternary(0, (M, K), 91), ternary(0, (N, K), 92)
    C, guard = run(gpu, A, B, sa=[0.25], sb=[4.0], variant=5)
    assert guard
    want = oracle.gemm_ex(A, B, scale_a=0.25, scale_b=4.0)
    assert np.array_equal(C, want), f"{int((C != want).sum())} differ"


def test_tile128_k_split_half_filled(gpu, oracle):
    """Tiles that fill between a quarter and half of the CUs split K in two
    when K has 64+ steps: 3 x 40 tiles (ragged M and N), 65 steps (a K
    tail), 2 slices; AUTO takes it; bit-exact on ternary sums, canaries."""
    M, N, K = 300, 5000, 8272
    say(f"case [auto] k-split half-filled M={M} N={N} K={K}")
    assert hg.select_variant(M, N, K) == 5
    ws = hg.workspace_size(M, N, K, 0)
    assert ws == 16384 + 3 * 40 * 2 * 65536, ws
    A, B = ternary(0, (M, K), 95), ternary(1, (N, K), 96)
    C, guard = run(gpu, A, B, fb=1, sa=[2.0], sb=[0.125], variant=0)
    assert guard
    want = oracle.gemm_ex(A, B, b_fmt=1, scale_a=2.0, scale_b=0.125)
    assert np.array_equal(C, want), f"{int((C != want).sum())} differ"


def test_auto_split_epilogue(gpu, oracle):
    """AUTO's column split with every column-indexed option: the column
    scales and the bias of the 128 x 128 half are offset by the split
    column.  Ternary e4m3 x e5m2, power-of-two scales, relu, fp16: bit-exact
    against the oracle, canaries around C."""
    M, N, K = 4000, 5000, 3584
    n1 = hg.split_columns(M, N, K)
    say(f"case [auto] split-epilogue M={M} N={N} K={K} n1={n1}")
    rng = np.random.default_rng(85)
    A, B = ternary(0, (M, K), 85), ternary(1, (N, K), 86)
    sr = np.exp2(rng.integers(-3, 4, M)).astype(np.float32)
    sc = np.exp2(rng.integers(-3, 4, N)).astype(np.float32)
    bias = rng.uniform(-4, 4, N).astype(np.float32)
    C, guard = run(gpu, A, B, fb=1, out=1, act=1, sa=[0.5], sr=sr, sc=sc,
                   bias=bias, variant=0)
    assert guard
    want = oracle.gemm_ex(A, B, b_fmt=1, out=1, act=1, scale_a=0.5,
                          scale_rows=sr, scale_cols=sc, bias=bias)
    assert np.array_equal(C, want), f"{int((C != want).sum())} differ"


def test_defaults_equal_plain_entry(gpu, oracle):
    """A default descriptor is hipgemm_fp8_gemm_bf16, bit for bit, on every
    schedule (general inputs: the same kernel and accumulation order)."""
    torch = gpu
    for variant, (M, N, K) in [(0, (700, 900, 1040)), (1, (512, 768, 512)),
                               (3, (64, 2048, 2048)), (4, (512, 512, 512)),
                               (5, (600, 520, 784))]:
        say(f"case [v{variant}] desc-defaults M={M} N={N} K={K}")
        A = general(oracle, 0, (M, K), 80)
        B = general(oracle, 0, (N, K), 81)
        C, _ = run(torch, A, B, sa=[0.75], sb=[2.0], variant=variant,
                   guard_cols=0)
        a, b = to_dev(torch, A), to_dev(torch, B)
        ref = hg.fp8_gemm_bf16(a, b, torch.tensor([0.75], device="cuda"),
                               torch.tensor([2.0], device="cuda"),
                               variant=variant)
        torch.cuda.synchronize()
        assert np.array_equal(C, ref.view(torch.int16).cpu().numpy().view(np.uint16))


def test_torch_helper_dtypes(gpu, oracle):
    """hipgemm_amd.gemm with float8_e5m2 / float8_e4m3fn tensors, an fp16
    output and fused bias + relu."""
    torch = gpu
    M, N, K = 320, 448, 256
    say(f"case gemm-helper M={M} N={N} K={K}")
    A, B = ternary(1, (M, K), 82), ternary(0, (N, K), 83)
    a = torch.from_numpy(A).cuda().view(torch.float8_e5m2)
    b = torch.from_numpy(B).cuda().view(torch.float8_e4m3fn)
    bias = torch.linspace(-3, 3, N, device="cuda")
    y = hg.gemm(a, b, out_dtype=torch.float16, bias=bias, activation="relu")
    torch.cuda.synchronize()
    want = oracle.gemm_ex(A, B, a_fmt=1, b_fmt=0, out=1, act=1,
                          bias=bias.cpu().numpy())
    assert y.dtype == torch.float16
    assert np.array_equal(y.view(torch.int16).cpu().numpy().view(np.uint16), want)
