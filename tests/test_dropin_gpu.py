"""GPU parity of the C++ drop-in header (include/fp8_4wave.hpp).

Both kernel templates of the reference header's launch surface,
fp8_gemm_4wave_256x256x128<M, N, K> (fp8_4wave.hpp:334-338) and
fp8_gemm_4wave_256x256x128_ref<M, N, K> (fp8_4wave.hpp:594-598), are launched
exactly as the reference's callers launch them (test.cpp:79: a grid of
(M * N) / 65536 workgroups of 256 threads, no dynamic LDS) through
tests/dropin/libdropin.so, and compared with the oracle: bit-exactly on
ternary inputs (every partial sum a small integer), within the 1e-2 metric
on general ones, with canaries around C (no write outside M x N).  At the
reference bench's shapes (8192^3, bench.cpp:4-14, and 8192 x 8192 x 28672)
the whole of C is compared for ternary inputs at 8192^3; for general inputs
and the long-K shape, about 200 rows (every tile row's edges and random
ones) plus the row- and column-sum identities of the whole output.
"""
import ctypes
import os

import numpy as np
import pytest

from oracle import pyoracle as po
from test_gemm_gpu import check_rows, check_sums, sample_rows
from util import REL_TOL, compare, say, to_dev

pytestmark = pytest.mark.gpu

CANARY = 0x7FA5
PAD = 64  # guard elements on each side of C (keeps C 16-byte aligned)
LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "dropin",
                   "libdropin.so")
TERNARY = np.array([0xB8, 0x00, 0x38], np.uint8)  # -1, 0, +1


@pytest.fixture(scope="module")
def dropin(gpu):
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (make -C tests/dropin)")
    L = ctypes.CDLL(LIB)
    vp, ci = ctypes.c_void_p, ctypes.c_int
    L.dropin_launch.argtypes = [ci, ci, vp, vp, vp, ci, vp]
    L.dropin_launch.restype = ci
    L.dropin_shape.argtypes = [ci, ctypes.POINTER(ci), ctypes.POINTER(ci),
                               ctypes.POINTER(ci)]
    L.dropin_shape.restype = ci
    return L


def shape_of(L, i):
    M, N, K = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    assert L.dropin_shape(i, M, N, K) == 0
    return M.value, N.value, K.value


def launch(torch, L, kernel, shape, A, B, grid=0):
    M, N, K = shape_of(L, shape)
    a, b = to_dev(torch, A), to_dev(torch, B)
    buf = torch.full((M * N + 2 * PAD,), CANARY, dtype=torch.int16,
                     device="cuda")
    code = L.dropin_launch(kernel, shape, a.data_ptr(), b.data_ptr(),
                           buf.data_ptr() + 2 * PAD, grid,
                           torch.cuda.current_stream().cuda_stream)
    assert code == 0, f"launch returned hipError {code}"
    torch.cuda.synchronize()
    got = buf.cpu().numpy().view(np.uint16)
    assert np.all(got[:PAD] == CANARY) and np.all(got[PAD + M * N:] == CANARY)
    return np.ascontiguousarray(got[PAD:PAD + M * N].reshape(M, N))


KERNELS = [pytest.param(0, id="main"), pytest.param(1, id="ref")]


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("shape", [0, 1, 2], ids=["512", "4096", "4000x5000x3584"])
def test_dropin_ternary_bit_exact(gpu, oracle, dropin, kernel, shape):
    M, N, K = shape_of(dropin, shape)
    say(f"case dropin kernel={kernel} {M}x{N}x{K} ternary seed=31")
    rng = np.random.default_rng(31)
    A = TERNARY[rng.integers(0, 3, (M, K))]
    B = TERNARY[rng.integers(0, 3, (N, K))]
    C = launch(gpu, dropin, kernel, shape, A, B)
    want = oracle.gemm(A, B, 1.0, 1.0)
    max_rel, exact, _ = compare(C, want)
    say(f"    max_rel={max_rel:.3e} exact={exact:.6f}")
    assert exact == 1.0


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("shape", [0, 1], ids=["512", "4096"])
def test_dropin_general_inputs(gpu, oracle, dropin, kernel, shape):
    M, N, K = shape_of(dropin, shape)
    say(f"case dropin kernel={kernel} {M}x{N}x{K} normal(0,1) seeds 32/33")
    A = oracle.fill((M, K), 32, po.NORMAL, 0.0, 1.0)
    B = oracle.fill((N, K), 33, po.NORMAL, 0.0, 1.0)
    C = launch(gpu, dropin, kernel, shape, A, B)
    max_rel, exact, _ = compare(C, oracle.gemm(A, B, 1.0, 1.0))
    say(f"    max_rel={max_rel:.3e} exact={exact:.6f}")
    assert max_rel <= REL_TOL


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("grid", [1, 3, 300])
def test_dropin_any_grid(gpu, oracle, dropin, kernel, grid):
    """Any grid >= 1 is correct (the reference's remap needs a multiple of 8
    and exactly one workgroup per tile)."""
    M, N, K = shape_of(dropin, 0)
    say(f"case dropin kernel={kernel} {M}x{N}x{K} grid={grid} ternary seed=34")
    rng = np.random.default_rng(34)
    A = TERNARY[rng.integers(0, 3, (M, K))]
    B = TERNARY[rng.integers(0, 3, (N, K))]
    C = launch(gpu, dropin, kernel, 0, A, B, grid=grid)
    _, exact, _ = compare(C, oracle.gemm(A, B, 1.0, 1.0))
    assert exact == 1.0


@pytest.mark.parametrize("kernel", KERNELS)
def test_dropin_bench_shape_ternary(gpu, oracle, dropin, kernel):
    """8192^3, the reference bench's default: the whole output, bit-exact."""
    M, N, K = shape_of(dropin, 3)
    say(f"case dropin kernel={kernel} {M}x{N}x{K} ternary seed=35")
    rng = np.random.default_rng(35)
    A = TERNARY[rng.integers(0, 3, (M, K))]
    B = TERNARY[rng.integers(0, 3, (N, K))]
    C = launch(gpu, dropin, kernel, 3, A, B)
    max_rel, exact, _ = compare(C, oracle.gemm(A, B, 1.0, 1.0))
    say(f"    max_rel={max_rel:.3e} exact={exact:.6f}")
    assert exact == 1.0


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("shape", [3, 4], ids=["8192", "8192x8192x28672"])
def test_dropin_bench_shapes_general(gpu, oracle, dropin, kernel, shape):
    M, N, K = shape_of(dropin, shape)
    say(f"case dropin kernel={kernel} {M}x{N}x{K} normal(0,1) seeds 36/37")
    A = oracle.fill((M, K), 36, po.NORMAL, 0.0, 1.0)
    B = oracle.fill((N, K), 37, po.NORMAL, 0.0, 1.0)
    C = launch(gpu, dropin, kernel, shape, A, B)
    check_rows(oracle, C, A, B, 1.0, 1.0, sample_rows(M, 38, 128))
    check_sums(oracle, C, A, B, 1.0)
