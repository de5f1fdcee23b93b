"""GPU parity of the per-row / per-column scaled GEMM
(hipgemm_fp8_gemm_bf16_rowcol) against the CPU oracle, through the C ABI.

C[m, n] = bf16_rne(acc[m, n] * (scale_rows[m] * scale_cols[n])).  With ternary
inputs (e4m3 -1, 0, +1) every partial sum is a small integer, exact in any
order, and the scale product is one fp32 multiply on both sides: the GPU must
equal the oracle bit for bit for ANY fp32 scale vectors.  General inputs are
checked with the north_star tolerance on the unscaled product (scaled_rel).
Canaries around C check that nothing outside the M x N window is written.
Every case prints its name before it touches the GPU.
"""
import numpy as np
import pytest

import hipgemm_amd as hg
from oracle import pyoracle as po
from util import DELTA_FRAC, REL_TOL, bf16_to_f32, from_dev_bf16, say, to_dev

pytestmark = pytest.mark.gpu

CANARY = 0x7FA5
TERNARY = np.array([0xB8, 0x00, 0x38], np.uint8)  # -1, 0, +1

# Every schedule the row/column entry point accepts (AUTO resolves per shape).
VARIANTS = [pytest.param(0, id="auto"), pytest.param(2, id="mfma16"),
            pytest.param(4, id="8wave"), pytest.param(3, id="skinny"),
            pytest.param(5, id="tile128"), pytest.param(6, id="strip")]


def ternary(shape, seed):
    return TERNARY[np.random.default_rng(seed).integers(0, 3, shape)]


def scales(n, seed, lo=0.25, hi=4.0):
    return np.random.default_rng(seed).uniform(lo, hi, n).astype(np.float32)


def scaled_rel(C, want, sr, sc):
    """The north_star metric (util.compare) on the unscaled product: both
    outputs divided by scale_rows[m] * scale_cols[n] first, so that the
    cancellation floor (1e-2 of the rms) is that of the accumulator, not one
    dominated by the largest scales.  bf16 rounding is relative, so the
    division keeps each element's relative error."""
    s = np.outer(sr.astype(np.float64), sc.astype(np.float64))
    c = bf16_to_f32(C).astype(np.float64) / s
    r = bf16_to_f32(want).astype(np.float64) / s
    assert np.isfinite(c).all() and np.isfinite(r).all()
    delta = DELTA_FRAC * float(np.sqrt(np.mean(r * r)))
    return float((np.abs(c - r) / np.maximum(np.abs(r), delta)).max())


def usable(variant, M):
    return variant not in (hg.VARIANTS["skinny"], hg.VARIANTS["strip"]) or M <= 128


def run_rowcol(torch, A, B, sr, sc, variant, ldc=None):
    """Call the row/column entry point into a canary-guarded C (2 guard rows
    above and below, ldc - N guard columns); returns (C, guard_ok)."""
    M, K = A.shape
    N = B.shape[0]
    ldc = ldc or N
    a, b = to_dev(torch, A), to_dev(torch, B)
    tr = torch.from_numpy(sr).to("cuda") if sr is not None else None
    tc = torch.from_numpy(sc).to("cuda") if sc is not None else None
    buf = torch.full((M + 4, ldc), CANARY, dtype=torch.int16, device="cuda")
    need = hg.workspace_size(M, N, K, variant)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda")
    code = hg.gemm_raw_rowcol(a.data_ptr(), b.data_ptr(),
                              buf.data_ptr() + 2 * ldc * 2, M, N, K, K, K, ldc,
                              tr.data_ptr() if tr is not None else 0,
                              tc.data_ptr() if tc is not None else 0, variant,
                              ws.data_ptr() if need else 0, need,
                              torch.cuda.current_stream().cuda_stream)
    assert code == 0, code
    torch.cuda.synchronize()
    got = buf.cpu().numpy().view(np.uint16)
    guard = (np.all(got[:2] == CANARY) and np.all(got[M + 2:] == CANARY)
             and np.all(got[2:M + 2, N:] == CANARY))
    return np.ascontiguousarray(got[2:M + 2, :N]), guard


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("M,N,K", [
    (512, 512, 512), (300, 260, 208), (257, 255, 80), (1, 1, 16),
    (17, 513, 48), (128, 4100, 1040), (513, 17, 1040), (4000, 5000, 64),
    (1024, 2048, 4112)])
def test_rowcol_ternary_bit_exact(gpu, oracle, M, N, K, variant):
    if not usable(variant, M):
        pytest.skip("skinny schedule: M <= 128 only")
    say(f"case [v{variant}] rowcol-ternary M={M} N={N} K={K} seed=41")
    A, B = ternary((M, K), 41), ternary((N, K), 42)
    sr, sc = scales(M, 43), scales(N, 44)
    C, guard = run_rowcol(gpu, A, B, sr, sc, variant, ldc=N + 24)
    assert guard, "write outside the M x N window"
    want = oracle.gemm_rowcol(A, B, sr, sc)
    assert np.array_equal(C, want), (
        f"{int((C != want).sum())} of {C.size} differ")


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("which", ["rows", "cols", "none"])
def test_rowcol_one_side_null(gpu, oracle, variant, which):
    """A NULL vector means all ones: equal to the oracle with that vector
    omitted, and with both NULL equal to the unscaled per-tensor oracle."""
    M, N, K = (96, 700, 528) if variant in (3, 6) else (320, 700, 528)
    say(f"case [v{variant}] rowcol-null-{which} M={M} N={N} K={K} seed=45")
    A, B = ternary((M, K), 45), ternary((N, K), 46)
    sr = scales(M, 47) if which == "rows" else None
    sc = scales(N, 48) if which == "cols" else None
    C, guard = run_rowcol(gpu, A, B, sr, sc, variant)
    assert guard
    assert np.array_equal(C, oracle.gemm_rowcol(A, B, sr, sc))
    if which == "none":
        assert np.array_equal(C, oracle.gemm(A, B))


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("M,N,K,dist", [
    (512, 512, 512, "uniform"), (2048, 2048, 2048, "normal"),
    (96, 8192, 8192, "normal"), (1000, 3000, 1104, "uniform")])
def test_rowcol_general_inputs(gpu, oracle, M, N, K, dist, variant):
    if not usable(variant, M):
        pytest.skip("skinny schedule: M <= 128 only")
    say(f"case [v{variant}] rowcol-{dist} M={M} N={N} K={K} seed=49")
    if dist == "uniform":
        A = oracle.fill((M, K), 49001, po.UNIFORM, -1.0, 1.0)
        B = oracle.fill((N, K), 49002, po.UNIFORM, -1.0, 1.0)
    else:
        A = oracle.fill((M, K), 49001, po.NORMAL, 0.0, 1.0)
        B = oracle.fill((N, K), 49002, po.NORMAL, 0.0, 1.0)
    # scales spanning 2^-10 .. 2^10, as per-channel quantisation produces
    sr = np.exp2(np.random.default_rng(50).uniform(-10, 10, M)).astype(np.float32)
    sc = np.exp2(np.random.default_rng(51).uniform(-10, 10, N)).astype(np.float32)
    C, guard = run_rowcol(gpu, A, B, sr, sc, variant)
    assert guard
    want = oracle.gemm_rowcol(A, B, sr, sc)
    max_rel = scaled_rel(C, want, sr, sc)
    say(f"    max_rel={max_rel:.3e} exact={np.mean(C == want):.6f}")
    assert max_rel <= REL_TOL


@pytest.mark.parametrize("variant", VARIANTS)
def test_rowcol_special_scales(gpu, oracle, variant):
    """Zero, huge and tiny scales: products that overflow to inf, 0 * inf =
    NaN where the sum is zero, subnormal products -- bit-exact with ternary
    inputs, NaN positions included."""
    M, N, K = (64, 300, 272) if variant in (3, 6) else (300, 300, 272)
    say(f"case [v{variant}] rowcol-special M={M} N={N} K={K} seed=52")
    A, B = ternary((M, K), 52), ternary((N, K), 53)
    # 2^-126 * 0.25 and 2^-130 (itself subnormal) give subnormal products
    special = np.array([0.0, 1e30, 1e-30, 2.0 ** -126, 2.0 ** -130, 0.25,
                        65504.0, 1.0, -3.5], np.float32)
    rng = np.random.default_rng(54)
    sr = special[rng.integers(0, len(special), M)]
    sc = special[rng.integers(0, len(special), N)]
    C, guard = run_rowcol(gpu, A, B, sr, sc, variant)
    assert guard
    want = oracle.gemm_rowcol(A, B, sr, sc)
    nan_c = (C & 0x7FFF) > 0x7F80
    nan_w = (want & 0x7FFF) > 0x7F80
    assert np.array_equal(nan_c, nan_w)
    assert np.array_equal(C[~nan_w], want[~nan_w])


def test_rowcol_matches_per_tensor_entry(gpu, oracle):
    """Constant vectors give the per-tensor entry point's result, bit for bit,
    on general inputs and every schedule (the same accumulator, one scale
    product per element either way)."""
    torch = gpu
    M, N, K = 700, 900, 1040
    A = oracle.fill((M, K), 55001, po.NORMAL, 0.0, 1.0)
    B = oracle.fill((N, K), 55002, po.NORMAL, 0.0, 1.0)
    sa, sb = np.float32(0.37), np.float32(2.9)
    for variant in (0, 2, 4):
        say(f"case [v{variant}] rowcol-vs-per-tensor M={M} N={N} K={K}")
        C, _ = run_rowcol(torch, A, B, np.full(M, sa, np.float32),
                          np.full(N, sb, np.float32), variant)
        a, b = to_dev(torch, A), to_dev(torch, B)
        ref = hg.fp8_gemm_bf16(a, b, torch.tensor([sa], device="cuda"),
                               torch.tensor([sb], device="cuda"),
                               variant=variant)
        torch.cuda.synchronize()
        assert np.array_equal(C, from_dev_bf16(ref))


def test_rowcol_torch_helper(gpu, oracle):
    """The torch convenience wrapper: vectors as device tensors, strided
    operands, a preallocated output on a side stream."""
    torch = gpu
    M, N, K = 384, 520, 288
    say(f"case rowcol-torch M={M} N={N} K={K} seed=56")
    A, B = ternary((M, K + 32), 56), ternary((N, K + 64), 57)
    sr, sc = scales(M, 58), scales(N, 59)
    a = to_dev(torch, A)[:, :K]
    b = to_dev(torch, B)[:, :K]
    out = torch.empty((M, N + 8), dtype=torch.bfloat16, device="cuda")[:, :N]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        hg.fp8_gemm_bf16_rowcol(a, b, torch.from_numpy(sr).to("cuda"),
                                torch.from_numpy(sc).to("cuda"), out=out,
                                stream=s)
    s.synchronize()
    want = oracle.gemm_rowcol(np.ascontiguousarray(A[:, :K]),
                              np.ascontiguousarray(B[:, :K]), sr, sc)
    assert np.array_equal(from_dev_bf16(out), want)
    with pytest.raises(hg.HipGemmError):
        hg.fp8_gemm_bf16_rowcol(a, b, torch.ones(M + 1, device="cuda"), None)
    with pytest.raises(hg.HipGemmError):
        hg.fp8_gemm_bf16_rowcol(a, b, None, torch.ones(N, device="cuda"),
                                variant=hg.VARIANTS["4wave"])
