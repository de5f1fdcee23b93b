"""Pins for the CPU oracle (oracle/): the checker every parity test relies on.

Each oracle function is checked against something independent of it:
  * codecs: exhaustive 2^32 sweeps against the HIP header conversions the
    reference calls (utils.hpp:32, test.cpp:25/27), plus OCP closed forms;
  * reference-test generator: bit-exact against init_random (utils.hpp:27-34)
    compiled from the reference sources (oracle/_ref);
  * GEMM: bit-exact against gemm_cpu (test.cpp:19-30) compiled from the
    reference sources, exact fp64 brute force where fp32 sums are exact,
    permutation / all-ones / zero closed forms, and committed golden vectors;
  * own generators: committed golden hashes and distribution moments.
"""
import hashlib
import json
import os

import numpy as np
import pytest

from oracle import pyoracle as po

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def bits_f32(u):
    return np.array([u], dtype=np.uint32).view(np.float32)[0]


# ---------------------------------------------------------------- codecs ---

def test_e4m3_encode_exhaustive_vs_hip_header():
    pin = po.HipConvPin()
    n, bad, tiny = pin.sweep(0)
    assert n == 0, [hex(b) for b in bad]
    assert tiny > 0  # the |x| < 2^-69 range was compared to signed zero


def test_bf16_encode_exhaustive_vs_hip_header():
    pin = po.HipConvPin()
    n, bad, _ = pin.sweep(1)
    assert n == 0, [hex(b) for b in bad]


def test_e4m3_decode_all_codes_vs_hip_header(oracle):
    pin = po.HipConvPin()
    for b in range(256):
        x = oracle.lib.hg_e4m3_to_f32(b)
        y = pin.lib.hg_pin_hip_e4m3_to_f32(b)
        assert (np.isnan(x) and np.isnan(y)) or (x == y and
                                                 np.signbit(x) == np.signbit(y)), b


def test_e4m3_closed_forms(oracle):
    dec, enc = oracle.lib.hg_e4m3_to_f32, oracle.lib.hg_f32_to_e4m3
    assert dec(0x38) == 1.0 and dec(0xB8) == -1.0
    assert dec(0x7E) == 448.0 and dec(0xFE) == -448.0
    assert dec(0x01) == 2.0 ** -9 and dec(0x08) == 2.0 ** -6
    assert dec(0x07) == 7 * 2.0 ** -9
    assert np.isnan(dec(0x7F)) and np.isnan(dec(0xFF))
    assert dec(0x80) == 0.0 and np.signbit(dec(0x80))
    # every finite code round-trips
    for b in range(256):
        if b & 0x7F != 0x7F:
            assert enc(dec(b)) == b, hex(b)
    assert enc(449.0) == 0x7E and enc(1e30) == 0x7E and enc(-1e30) == 0xFE
    assert enc(float("inf")) == 0x7F and enc(float("-inf")) == 0xFF
    assert enc(float("nan")) & 0x7F == 0x7F
    assert enc(2.0 ** -10) == 0x00            # tie -> even (zero)
    assert enc(1.5 * 2.0 ** -10) == 0x01      # above the tie
    assert enc(1.0625) == 0x38                # tie 1.0 / 1.125 -> even
    assert enc(1.1875) == 0x3A                # tie 1.125 / 1.25 -> even
    assert enc(-0.0) == 0x80


def test_bf16_closed_forms(oracle):
    f = oracle.lib.hg_f32_to_bf16
    assert f(1.0) == 0x3F80 and f(-2.0) == 0xC000
    assert f(1.0 + 2.0 ** -8) == 0x3F80          # tie -> even
    assert f(1.0 + 3 * 2.0 ** -8) == 0x3F82      # tie -> even (up)
    assert f(1.0 + 2.0 ** -8 + 2.0 ** -20) == 0x3F81
    assert f(3.4e38) == 0x7F80                   # rounds up to +inf
    assert f(float("inf")) == 0x7F80
    nanb = f(float("nan"))
    assert (nanb & 0x7F80) == 0x7F80 and (nanb & 0x7F) != 0


# ------------------------------------------------------------ generators ---

def test_reftest_generator_matches_reference_init_random(oracle):
    if not po.RefLib.available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    ref = po.RefLib()
    for seed in (0, 1, 2, 123):
        n = 50_000 + seed
        assert np.array_equal(ref.init_random(n, seed),
                              oracle.fill_reftest((n,), seed)), seed


def test_generator_golden_hashes(oracle):
    with open(os.path.join(GOLDEN, "generators.json")) as f:
        gold = json.load(f)
    for case in gold["cases"]:
        if case["dist"] == "reftest":
            a = oracle.fill_reftest((case["n"],), case["seed"])
        else:
            d = po.UNIFORM if case["dist"] == "uniform" else po.NORMAL
            a = oracle.fill((case["n"],), case["seed"], d, case["p0"], case["p1"])
        assert hashlib.sha256(a.tobytes()).hexdigest() == case["sha256"], case
    for case in gold["scales"]:
        assert oracle.draw_scale(case["seed"]) == case["value"]


def test_generator_moments(oracle):
    n = 1 << 20
    u = oracle.e4m3_to_f32(oracle.fill((n,), 11, po.UNIFORM, -1.0, 1.0))
    assert abs(u.mean()) < 5e-3 and abs(u.var() - 1 / 3) < 5e-3
    assert u.min() >= -1.0 and u.max() <= 1.0
    z = oracle.e4m3_to_f32(oracle.fill((n,), 12, po.NORMAL, 0.0, 1.0))
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1.0) < 1e-2
    h = oracle.e4m3_to_f32(oracle.fill((n,), 13, po.NORMAL, 0.0, 0.5))
    assert abs(h.std() - 0.5) < 5e-3
    # different seeds, different streams; same seed, same stream
    assert not np.array_equal(oracle.fill((4096,), 1), oracle.fill((4096,), 2))
    assert np.array_equal(oracle.fill((4096,), 3), oracle.fill((4096,), 3))
    s = [oracle.draw_scale(k) for k in range(64)]
    assert min(s) >= 0.5 and max(s) < 2.0 and len(set(s)) > 60


# ------------------------------------------------------------------ GEMM ---

def _inputs(oracle, M, N, K, seed=1, dist=po.NORMAL, p0=0.0, p1=1.0):
    return (oracle.fill((M, K), 2 * seed, dist, p0, p1),
            oracle.fill((N, K), 2 * seed + 1, dist, p0, p1))


@pytest.mark.parametrize("shape", [(64, 48, 96), (33, 17, 160), (1, 1, 16),
                                   (128, 96, 512), (7, 130, 48)])
def test_gemm_matches_reference_gemm_cpu(oracle, shape):
    if not po.RefLib.available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    ref = po.RefLib()
    M, N, K = shape
    for dist, p0, p1 in ((po.NORMAL, 0.0, 1.0), (po.UNIFORM, -1.0, 1.0)):
        A, B = _inputs(oracle, M, N, K, 3, dist, p0, p1)
        want = ref.gemm_cpu(A, B)
        assert np.array_equal(oracle.gemm(A, B, faithful=True), want)
        assert np.array_equal(oracle.gemm(A, B), want)


def test_gemm_reftest_inputs_match_reference(oracle):
    """The reference's own test inputs (utils.hpp:27-34), A != B."""
    if not po.RefLib.available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    ref = po.RefLib()
    M = N = K = 256
    A = ref.init_random(M * K, 0).reshape(M, K)
    B = ref.init_random(N * K, 1).reshape(N, K)
    assert np.array_equal(oracle.gemm(A, B), ref.gemm_cpu(A, B))


def test_gemm_exact_bruteforce_fp64(oracle):
    """U[-1,1] e4m3 values are multiples of 2^-9, so products are multiples of
    2^-18; with |partial sums| < 2^6 every fp32 sum is exact and the oracle
    must equal bf16(exact fp64 sum) bit for bit."""
    M, N, K = 40, 56, 256
    A, B = _inputs(oracle, M, N, K, 5, po.UNIFORM, -1.0, 1.0)
    a = oracle.e4m3_to_f32(A).astype(np.float64)
    b = oracle.e4m3_to_f32(B).astype(np.float64)
    exact = a @ b.T
    partial = np.abs(np.cumsum(a[:, None, :] * b[None, :, :], axis=2)).max()
    assert partial < 64.0
    want = oracle.f32_to_bf16(exact.astype(np.float32))
    assert np.array_equal(oracle.gemm(A, B), want)
    # and the transposed product is a different matrix (orientation is pinned)
    assert not np.array_equal(oracle.gemm(B, A), want[:N, :M])


def test_gemm_closed_forms(oracle):
    rng = np.random.default_rng(0)
    K = 64
    B = oracle.fill((48, K), 9, po.NORMAL, 0.0, 1.0)
    # permutation A: C row i = B row-sums picked by one-hot positions
    perm = rng.permutation(K)[:32]
    A = np.zeros((32, K), np.uint8)
    A[np.arange(32), perm] = 0x38  # 1.0
    bf = oracle.e4m3_to_f32(B)
    want = oracle.f32_to_bf16(bf[:, perm].T + np.float32(0))  # -0 sums to +0
    assert np.array_equal(oracle.gemm(A, B), want)
    # all-ones A: every row equals the row sums of B (exact: small integers*2^-9)
    Bu = oracle.fill((48, K), 10, po.UNIFORM, -1.0, 1.0)
    ones = np.full((5, K), 0x38, np.uint8)
    sums = oracle.e4m3_to_f32(Bu).astype(np.float64).sum(axis=1)
    want = np.tile(oracle.f32_to_bf16(sums.astype(np.float32)), (5, 1))
    assert np.array_equal(oracle.gemm(ones, Bu), want)
    # zero A
    assert np.all(oracle.gemm(np.zeros((3, K), np.uint8), B) == 0)


def test_gemm_scale_extension(oracle):
    """C = bf16(acc * (sa*sb)) with the fp32 accumulator of the same order."""
    M, N, K = 24, 40, 320
    A, B = _inputs(oracle, M, N, K, 7)
    sa, sb = np.float32(1.7), np.float32(0.6)
    rows = np.arange(M)
    acc = oracle.gemm_rows_acc(A, B, rows)
    want = oracle.f32_to_bf16((acc * np.float32(sa * sb)).astype(np.float32))
    assert np.array_equal(oracle.gemm(A, B, float(sa), float(sb)), want)
    assert np.array_equal(oracle.gemm(A, B, float(sa), float(sb), faithful=True),
                          want)
    assert np.array_equal(oracle.gemm(A, B, 1.0, 1.0), oracle.f32_to_bf16(acc))


def test_gemm_rowcol_reduces_to_per_tensor(oracle):
    """Per-row / per-column scales, pinned by reduction to the per-tensor path
    (itself pinned against the reference's gemm_cpu):
    * constant vectors equal the two scalars;
    * element (m, n) equals the per-tensor product with scale_a = sr[m],
      scale_b = sc[n] (the scale product is formed first, in fp32);
    * column scales are row scales of the transposed product (same products,
      same K order, so the same fp32 sums)."""
    M, N, K = 37, 45, 208
    A, B = _inputs(oracle, M, N, K, 31)
    rng = np.random.default_rng(31)
    sr = rng.uniform(0.25, 4.0, M).astype(np.float32)
    sc = rng.uniform(0.25, 4.0, N).astype(np.float32)
    assert np.array_equal(
        oracle.gemm_rowcol(A, B, np.full(M, 1.7, np.float32),
                           np.full(N, 0.6, np.float32)),
        oracle.gemm(A, B, float(np.float32(1.7)), float(np.float32(0.6))))
    assert np.array_equal(oracle.gemm_rowcol(A, B), oracle.gemm(A, B))
    C = oracle.gemm_rowcol(A, B, sr, sc)
    for m in (0, 5, 36):
        for n in (0, 11, 44):
            one = oracle.gemm_rows(A, B, [m], float(sr[m]), float(sc[n]))
            assert C[m, n] == one[0, n], (m, n)
    Cr = oracle.gemm_rowcol(A, B, sr, None)
    for m in (0, 20, 36):
        assert np.array_equal(Cr[m], oracle.gemm_rows(A, B, [m], float(sr[m]))[0])
    Cc = oracle.gemm_rowcol(A, B, None, sc)
    assert np.array_equal(Cc, oracle.gemm_rowcol(B, A, sc, None).T)
    # a wrong column index (here the vector reversed) is caught
    assert not np.array_equal(C, oracle.gemm_rowcol(A, B, sr, sc[::-1].copy()))


def test_gemm_rows_subset(oracle):
    M, N, K = 50, 70, 192
    A, B = _inputs(oracle, M, N, K, 8)
    full = oracle.gemm(A, B, 1.3, 0.9)
    rows = [0, 7, 49, 7, 13]
    assert np.array_equal(oracle.gemm_rows(A, B, rows, 1.3, 0.9), full[rows])
    ex = oracle.gemm_rows_f64(A, B, rows)
    acc = oracle.gemm_rows_acc(A, B, rows)
    assert np.allclose(ex, acc, rtol=1e-5, atol=1e-4)


def test_gemm_nan_and_saturation(oracle):
    K = 64
    A = np.full((4, K), 0x7E, np.uint8)   # 448
    B = np.full((3, K), 0x7E, np.uint8)
    want = oracle.lib.hg_f32_to_bf16(448.0 * 448.0 * K)
    assert np.all(oracle.gemm(A, B) == want)
    A[2, 5] = 0x7F  # NaN
    C = oracle.gemm(A, B)
    assert np.all(np.isnan(oracle.bf16_to_f32(C[2])))
    assert not np.any(np.isnan(oracle.bf16_to_f32(C[[0, 1, 3]])))


def test_golden_vectors(oracle):
    """Committed vectors made by tests/golden/make_golden.py (oracle output,
    cross-checked at generation time against the reference's gemm_cpu)."""
    path = os.path.join(GOLDEN, "gemm_small.npz")
    z = np.load(path)
    names = sorted({k.rsplit("_", 1)[0] for k in z.files})
    assert names
    for nm in names:
        A, B, C = z[nm + "_A"], z[nm + "_B"], z[nm + "_C"]
        sa, sb = (float(x) for x in z[nm + "_S"])
        assert np.array_equal(oracle.gemm(A, B, sa, sb), C), nm
        assert np.array_equal(oracle.gemm(A, B, sa, sb, faithful=True), C), nm


# ---- extensions: e5m2 operands, f16 output, bias, activations -------------

def _f16_bits(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def test_e5m2_decode_is_upper_byte_of_binary16(oracle):
    """Closed form: an e5m2 byte b is the binary16 with bits b << 8."""
    codes = np.arange(256, dtype=np.uint8)
    got = oracle.e5m2_to_f32(codes)
    want = (codes.astype(np.uint16) << 8).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])
    assert got[0x7b] == 57344.0 and got[0x01] == 2.0 ** -16 and np.isinf(got[0x7c])


def _probe_floats(seed, n=1 << 21):
    """Every binary16 value (so every e5m2 / f16 grid point), its float32
    neighbours and midpoints, plus random floats over the whole range."""
    h = np.arange(1 << 16, dtype=np.uint16).view(np.float16).astype(np.float32)
    h = h[np.isfinite(h)]
    mids = ((h[:-1].astype(np.float64) + h[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(seed)
    rnd = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    near = np.concatenate([np.nextafter(h, np.float32(np.inf)),
                           np.nextafter(h, np.float32(-np.inf))])
    extra = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 61440.0, 61439.996,
                      65504.0, 65519.996, 65520.0, 2.0 ** -17, 2.0 ** -25,
                      3 * 2.0 ** -25], np.float32)
    return np.concatenate([h, mids, near, rnd, extra])


def test_e5m2_encode_vs_torch(oracle):
    torch = pytest.importorskip("torch")
    x = _probe_floats(7)
    got = oracle.f32_to_e5m2(x)
    want = torch.from_numpy(x).to(torch.float8_e5m2).view(torch.uint8).numpy()
    nan_g = ((got & 0x7c) == 0x7c) & ((got & 3) != 0)
    nan_w = ((want & 0x7c) == 0x7c) & ((want & 3) != 0)
    assert np.array_equal(nan_g, nan_w)
    bad = np.flatnonzero((got != want) & ~nan_w)
    assert bad.size == 0, [(float(x[i]), int(got[i]), int(want[i])) for i in bad[:8]]


def test_f16_encode_vs_numpy(oracle):
    x = _probe_floats(8)
    got = oracle.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = _f16_bits(x)
    nan = np.isnan(x)
    assert np.all((got[nan] & 0x7c00) == 0x7c00) and np.all(got[nan] & 0x3ff)
    bad = np.flatnonzero((got != want) & ~nan)
    assert bad.size == 0, [(float(x[i]), int(got[i]), int(want[i])) for i in bad[:8]]


def test_gemm_ex_defaults_equal_per_tensor_and_rowcol(oracle):
    M, N, K = 37, 45, 208
    A, B = _inputs(oracle, M, N, K, 41)
    assert np.array_equal(oracle.gemm_ex(A, B, scale_a=1.5, scale_b=0.75),
                          oracle.gemm(A, B, 1.5, 0.75))
    rng = np.random.default_rng(41)
    sr = rng.uniform(0.25, 4, M).astype(np.float32)
    sc = rng.uniform(0.25, 4, N).astype(np.float32)
    assert np.array_equal(oracle.gemm_ex(A, B, scale_rows=sr, scale_cols=sc),
                          oracle.gemm_rowcol(A, B, sr, sc))


# values exact in both e4m3 and e5m2: {0, +-0.5, +-1, +-1.5, +-2, +-3}
_BOTH = np.array([0.0, 0.5, -0.5, 1.0, -1.0, 1.5, -1.5, 2.0, -2.0, 3.0, -3.0],
                 np.float32)


def test_gemm_ex_formats_pinned_by_reencoding(oracle):
    """The same values encoded as e4m3 or e5m2 give the same product, for
    every format pair, and that product is the fp64 one (all partial sums
    of these values are exact in fp32).  A swapped format, a wrong exponent
    bias or the wrong table for one operand fails this."""
    M, N, K = 23, 31, 272
    rng = np.random.default_rng(42)
    va = _BOTH[rng.integers(0, len(_BOTH), (M, K))]
    vb = _BOTH[rng.integers(0, len(_BOTH), (N, K))]
    enc = {po.FMT_E4M3: oracle.f32_to_e4m3, po.FMT_E5M2: oracle.f32_to_e5m2}
    want = oracle.f32_to_bf16((va.astype(np.float64) @ vb.T.astype(np.float64))
                              .astype(np.float32))
    for fa in (po.FMT_E4M3, po.FMT_E5M2):
        for fb in (po.FMT_E4M3, po.FMT_E5M2):
            A, B = enc[fa](va), enc[fb](vb)
            assert np.array_equal(oracle.decode(A, fa), va)
            got = oracle.gemm_ex(A, B, a_fmt=fa, b_fmt=fb)
            assert np.array_equal(got, want), (fa, fb)
    # e5m2-only magnitudes (beyond e4m3's 448 and below its 2^-9)
    A = oracle.f32_to_e5m2(np.array([[2.0 ** 14], [2.0 ** -16]], np.float32))
    B = oracle.f32_to_e5m2(np.array([[2.0], [2.0 ** 10]], np.float32))
    got = oracle.bf16_to_f32(oracle.gemm_ex(A, B, a_fmt=po.FMT_E5M2,
                                            b_fmt=po.FMT_E5M2))
    assert got[0, 0] == 2.0 ** 15 and got[1, 1] == 2.0 ** -6


def test_gemm_ex_bias_is_one_fma(oracle):
    """v = fma(acc, scale, bias): with exact sums, scale a power of two and
    the bias on a nearby exponent, the fp64 sum is exact and its rounding is
    the fma's; a separately rounded product would differ on ties."""
    M, N, K = 16, 64, 256
    rng = np.random.default_rng(43)
    A = np.array([0xB8, 0x00, 0x38], np.uint8)[rng.integers(0, 3, (M, K))]
    B = np.array([0xB8, 0x00, 0x38], np.uint8)[rng.integers(0, 3, (N, K))]
    bias = rng.uniform(-8, 8, N).astype(np.float32)
    got = oracle.gemm_ex(A, B, scale_a=0.25, bias=bias)
    acc = oracle.e4m3_to_f32(A).astype(np.float64) @ oracle.e4m3_to_f32(B).T.astype(np.float64)
    want = oracle.f32_to_bf16((acc * 0.25 + bias.astype(np.float64)).astype(np.float32))
    assert np.array_equal(got, want)
    # no bias: exactly acc * scale, -0 kept
    neg0 = oracle.gemm_ex(np.zeros((1, 16), np.uint8), np.zeros((1, 16), np.uint8),
                          scale_a=-1.0)
    assert neg0[0, 0] == 0x8000 == oracle.gemm(np.zeros((1, 16), np.uint8),
                                               np.zeros((1, 16), np.uint8), -1.0)[0, 0]


def test_gemm_ex_activations_vs_library_routines(oracle):
    """relu exactly; silu against scipy's expit, gelu (tanh form) against
    torch's, both in float64, within one bf16 ulp of the oracle's output."""
    torch = pytest.importorskip("torch")
    from scipy.special import expit
    M, N, K = 24, 96, 128
    A, B = _inputs(oracle, M, N, K, 44)
    bias = np.random.default_rng(44).uniform(-2, 2, N).astype(np.float32)
    base = oracle.gemm_ex(A, B, scale_a=0.125, bias=bias, out=po.OUT_BF16)
    rows = np.arange(M, dtype=np.int32)
    acc = oracle.gemm_rows_acc(A, B, rows)
    # fma(acc, 1/8, bias): the fp64 value acc/8 + bias is exact (acc has 24
    # bits, bias is within 2^4 of it), so rounding it once is the fma
    v = (acc.astype(np.float64) * 0.125 + bias).astype(np.float32)
    assert np.array_equal(oracle.f32_to_bf16(v), base)
    relu = oracle.gemm_ex(A, B, scale_a=0.125, bias=bias, act=po.ACT_RELU)
    assert np.array_equal(relu, oracle.f32_to_bf16(np.where(v < 0, 0, v).astype(np.float32)))
    x = v.astype(np.float64)
    refs = {po.ACT_SILU: x * expit(x),
            po.ACT_GELU_TANH: torch.nn.functional.gelu(torch.from_numpy(x),
                                                       approximate="tanh").numpy()}
    for act, ref in refs.items():
        got = oracle.bf16_to_f32(oracle.gemm_ex(A, B, scale_a=0.125, bias=bias, act=act))
        want = oracle.bf16_to_f32(oracle.f32_to_bf16(ref.astype(np.float32)))
        ulp = np.abs(want) * 2.0 ** -7 + 1e-30
        assert np.all(np.abs(got - want) <= ulp), act
        assert np.mean(got == want) > 0.99, act


def test_gemm_ex_f16_output(oracle):
    M, N, K = 20, 40, 160
    A, B = _inputs(oracle, M, N, K, 45)
    acc = oracle.gemm_rows_acc(A, B, np.arange(M, dtype=np.int32))
    got = oracle.gemm_ex(A, B, scale_a=3.0, out=po.OUT_F16)
    with np.errstate(over="ignore"):
        assert np.array_equal(got, _f16_bits(acc * np.float32(3.0)))


# ---- MX block scales -------------------------------------------------------

def test_gemm_mx_pinned(oracle):
    """Unit scales: hg_gemm_ex.  Scales constant along each row: the row /
    column vectors of hg_gemm_ex with 2^(e-127), bit for bit (powers of two
    commute with fp32 rounding).  Per-block scales on ternary sums: fp64.
    A scale of 255 is NaN for every output it touches."""
    M, N, K = 21, 35, 320
    kb = K // 32
    A, B = _inputs(oracle, M, N, K, 51)
    one_a = np.full((M, kb), 127, np.uint8)
    one_b = np.full((N, kb), 127, np.uint8)
    assert np.array_equal(oracle.gemm_mx(A, B, one_a, one_b, scale_a=2.0),
                          oracle.gemm_ex(A, B, scale_a=2.0))
    rng = np.random.default_rng(51)
    er = rng.integers(117, 138, M).astype(np.uint8)
    ec = rng.integers(117, 138, N).astype(np.uint8)
    got = oracle.gemm_mx(A, B, np.repeat(er[:, None], kb, 1),
                         np.repeat(ec[:, None], kb, 1))
    want = oracle.gemm_ex(A, B, scale_rows=np.exp2(er.astype(np.float64) - 127).astype(np.float32),
                          scale_cols=np.exp2(ec.astype(np.float64) - 127).astype(np.float32))
    assert np.array_equal(got, want)
    # per-block, exact sums
    T = np.array([0xB8, 0x00, 0x38], np.uint8)
    A = T[rng.integers(0, 3, (M, K))]
    B = T[rng.integers(0, 3, (N, K))]
    sa = rng.integers(120, 135, (M, kb)).astype(np.uint8)
    sb = rng.integers(120, 135, (N, kb)).astype(np.uint8)
    af = oracle.e4m3_to_f32(A).astype(np.float64) * np.repeat(np.exp2(sa - 127.0), 32, 1)
    bf = oracle.e4m3_to_f32(B).astype(np.float64) * np.repeat(np.exp2(sb - 127.0), 32, 1)
    want = oracle.f32_to_bf16((af @ bf.T).astype(np.float32))
    assert np.array_equal(oracle.gemm_mx(A, B, sa, sb), want)
    # a swapped block index (scales of block b applied to block b+1) fails
    assert not np.array_equal(oracle.gemm_mx(A, B, np.roll(sa, 1, 1), sb), want)
    sa2 = sa.copy()
    sa2[3, 2] = 255
    nan = (oracle.gemm_mx(A, B, sa2, sb) & 0x7FFF) > 0x7F80
    assert nan[3].all() and not nan[np.arange(M) != 3].any()


def test_fp4_decode_and_gemm_pinned(oracle):
    """OCP E2M1: the value table of the OCP Microscaling v1.0 spec (written
    out, not derived); the fp4 GEMM against fp64 sums of the decoded
    values; nibble order: swapping the nibbles of every byte of both
    operands is a common permutation of K (same result), of one operand
    only it is not."""
    table = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    got = oracle.fp4_to_f32(np.arange(16))
    assert list(got[:8]) == table and list(-got[8:]) == table
    assert np.signbit(got[8])  # 0x8 is -0
    rng = np.random.default_rng(61)
    M, N, K = 37, 29, 160
    A = rng.integers(0, 256, (M, K // 2)).astype(np.uint8)
    B = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)

    def unpack(X):
        return np.stack([X & 15, X >> 4], axis=2).reshape(X.shape[0], -1)
    t = got.astype(np.float64)
    want = (t[unpack(A)] @ t[unpack(B)].T).astype(np.float32)
    C = oracle.gemm_ex(A, B, a_fmt=po.FMT_FP4, b_fmt=po.FMT_FP4, out=po.OUT_F32)
    assert np.array_equal(C.view(np.float32), want)
    swap = lambda X: ((X & 15) << 4 | (X >> 4)).astype(np.uint8)
    assert np.array_equal(oracle.gemm_ex(swap(A), swap(B), a_fmt=4, b_fmt=4,
                                         out=po.OUT_F32), C)
    assert not np.array_equal(oracle.gemm_ex(swap(A), B, a_fmt=4, b_fmt=4,
                                             out=po.OUT_F32), C)
    # bf16 output of the same sums: the bf16 rounding of the fp32 values
    assert np.array_equal(oracle.gemm_ex(A, B, a_fmt=4, b_fmt=4),
                          oracle.f32_to_bf16(want))


# OCP Microscaling v1.0, FP6 value tables (magnitudes of codes 0..31, the
# sign bit is 0x20), written out from the spec's definitions, not computed:
# E2M3: exponent bias 1, 3 mantissa bits, subnormals m/8; E3M2: bias 3,
# 2 mantissa bits, subnormals m/16.
E2M3_TABLE = [0.0, 0.125, 0.25, 0.375, 0.5, 0.625, 0.75, 0.875,
              1.0, 1.125, 1.25, 1.375, 1.5, 1.625, 1.75, 1.875,
              2.0, 2.25, 2.5, 2.75, 3.0, 3.25, 3.5, 3.75,
              4.0, 4.5, 5.0, 5.5, 6.0, 6.5, 7.0, 7.5]
E3M2_TABLE = [0.0, 0.0625, 0.125, 0.1875, 0.25, 0.3125, 0.375, 0.4375,
              0.5, 0.625, 0.75, 0.875, 1.0, 1.25, 1.5, 1.75,
              2.0, 2.5, 3.0, 3.5, 4.0, 5.0, 6.0, 7.0,
              8.0, 10.0, 12.0, 14.0, 16.0, 20.0, 24.0, 28.0]


def fp6_unpack_bits(X: np.ndarray) -> np.ndarray:
    """The packing rule restated on the bit string: element k of a row is
    bits [6k, 6k + 6) of the row's bytes read as one little-endian bit
    string (bit 0 = the low bit of byte 0)."""
    bits = np.unpackbits(X, axis=1, bitorder="little")
    k = bits.shape[1] // 6
    b = bits[:, :6 * k].reshape(X.shape[0], k, 6).astype(np.uint8)
    return (b * (1 << np.arange(6, dtype=np.uint8))).sum(axis=2).astype(np.uint8)


@pytest.mark.parametrize("fmt,table", [(po.FMT_FP6_E2M3, E2M3_TABLE),
                                       (po.FMT_FP6_E3M2, E3M2_TABLE)],
                         ids=["e2m3", "e3m2"])
def test_fp6_decode_pinned(oracle, fmt, table):
    got = oracle.fp6_to_f32(np.arange(64), fmt)
    assert list(got[:32]) == table and list(-got[32:]) == table
    assert np.signbit(got[32])  # 0x20 is -0
    # only the low 6 bits count
    assert np.array_equal(oracle.fp6_to_f32(np.arange(64) + 64, fmt), got)


@pytest.mark.parametrize("fa,fb", [(2, 2), (3, 3), (2, 3), (3, 2)])
def test_fp6_gemm_pinned(oracle, fa, fb):
    """The fp6 GEMM against fp64 sums of the table values of the codes the
    bits-string restatement unpacks (exact: products are multiples of 2^-8
    below 2^10, and these sums stay below 2^15).  Plausible packing slips
    change the result: each 3-byte group read big-endian, or the four codes
    of a group taken MSB first in one operand only (in both it is a common
    permutation of K, which leaves the sums alone)."""
    rng = np.random.default_rng(67)
    M, N, K = 33, 21, 256
    A = rng.integers(0, 256, (M, 3 * K // 4)).astype(np.uint8)
    B = rng.integers(0, 256, (N, 3 * K // 4)).astype(np.uint8)
    ta = np.array(E2M3_TABLE if fa == 2 else E3M2_TABLE, np.float64)
    tb = np.array(E2M3_TABLE if fb == 2 else E3M2_TABLE, np.float64)
    val = lambda t, c: np.where(c & 32, -t[c & 31], t[c & 31])
    want = val(ta, fp6_unpack_bits(A)) @ val(tb, fp6_unpack_bits(B)).T
    assert np.all(np.abs(want) < 2 ** 15)
    C = oracle.gemm_ex(A, B, a_fmt=fa, b_fmt=fb, out=po.OUT_F32)
    assert np.array_equal(C.view(np.float32), want.astype(np.float32))
    def codes(X, big_endian=False, msb_first=False):
        w = X.reshape(X.shape[0], -1, 3).astype(np.uint32)
        if big_endian:
            w = w[..., ::-1]
        w = w[..., 0] | (w[..., 1] << 8) | (w[..., 2] << 16)
        sh = [18 - 6 * t if msb_first else 6 * t for t in range(4)]
        return np.stack([(w >> s) & 63 for s in sh], axis=2).reshape(
            X.shape[0], -1).astype(np.uint8)
    assert np.array_equal(codes(A), fp6_unpack_bits(A))
    for ka, kb in [(dict(big_endian=True), dict(big_endian=True)),
                   (dict(msb_first=True), {})]:
        wrong = val(ta, codes(A, **ka)) @ val(tb, codes(B, **kb)).T
        assert not np.array_equal(wrong.astype(np.float32), C.view(np.float32))
    # bf16 output of the same sums
    assert np.array_equal(oracle.gemm_ex(A, B, a_fmt=fa, b_fmt=fb),
                          oracle.f32_to_bf16(want.astype(np.float32)))
