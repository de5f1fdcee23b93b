"""GPU checks of the workspace contract (include/hipgemm.h,
HIPGEMM_WS_COUNTER_BYTES) and of graph capture around it.

* One workspace serves every schedule in turn: the 128 x 128 schedule's
  K-split partial tiles sit after the counter region, so a skinny split-K
  call that follows on the same workspace still finds its arrival counters
  at zero (a prefill-then-decode sequence on one stream).
* The Python helpers never free a workspace a captured graph may hold, and
  create none while the stream is being captured.
* A call with no workspace on a capturing stream (the raw C ABI, or the
  Python helpers on a stream that has none) runs its schedule unsplit
  instead of recording an allocation and a memset into the caller's graph:
  the 128 x 128 schedule's K-slices at 256 x 8192 x 8192 and the strip
  schedule's at 16 x 4096 x 4096; every replay equals the oracle.
"""
import numpy as np
import pytest

import hipgemm_amd as hg
from util import compare, from_dev_bf16, say, to_dev

pytestmark = pytest.mark.gpu

TERNARY = np.array([0xB8, 0x00, 0x38], np.uint8)  # -1, 0, +1


def ternary(shape, seed):
    return TERNARY[np.random.default_rng(seed).integers(0, 3, shape)]


def test_one_workspace_prefill_then_decode(gpu, oracle):
    torch = gpu
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        # K-split on the 128 x 128 schedule: 16 MiB of fp32 partials.
        M, N, K = 256, 4096, 14336
        say(f"case ws-shared prefill {M}x{N}x{K} (AUTO: "
            f"{hg.variant_name(hg.select_variant(M, N, K))}, ws "
            f"{hg.workspace_size(M, N, K, 0)})")
        assert hg.workspace_size(M, N, K, 0) > 16384
        A, B = ternary((M, K), 91), ternary((N, K), 92)
        out = hg.fp8_gemm_bf16(to_dev(torch, A), to_dev(torch, B))
        torch.cuda.synchronize()
        rows = np.array([0, 1, 127, 128, 200, 255], np.int32)
        assert np.array_equal(from_dev_bf16(out)[rows],
                              oracle.gemm_rows(A, B, rows, 1.0, 1.0))
        # Then in-kernel reductions with arrival counters on the same
        # stream, hence the same workspace: the split-K schedule (16, 32
        # rows) and the strip schedule with K-slices (4096 columns).
        for M2, N2, K2, v in ((16, 8192, 8192, 3), (32, 8192, 8192, 3),
                              (16, 4096, 8192, 6), (16, 8192, 8192, 3),
                              (48, 2048, 8192, 6)):
            say(f"case ws-shared decode {M2}x{N2}x{K2} variant {v}")
            assert hg.workspace_size(M2, N2, K2, v) > 16384
            A2, B2 = ternary((M2, K2), 93), ternary((N2, K2), 94)
            out2 = hg.fp8_gemm_bf16(to_dev(torch, A2), to_dev(torch, B2),
                                    variant=v)
            torch.cuda.synchronize()
            assert np.array_equal(from_dev_bf16(out2), oracle.gemm(A2, B2))


def test_graph_replay_survives_workspace_growth(gpu, oracle):
    torch = gpu
    s = torch.cuda.Stream()
    M, N, K = 16, 2048, 4096
    say(f"case ws-graph capture {M}x{N}x{K}")
    A, B = ternary((M, K), 95), ternary((N, K), 96)
    a, b = to_dev(torch, A), to_dev(torch, B)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        hg.fp8_gemm_bf16(a, b)  # warm-up: creates this stream's workspace
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = hg.fp8_gemm_bf16(a, b)
    want = oracle.gemm(A, B)
    # A call that needs a larger workspace on the same stream replaces it;
    # the captured graph still holds (and may use) the old one.
    M3, N3, K3 = 128, 8192, 8192
    say(f"case ws-graph growth {M3}x{N3}x{K3} "
        f"({hg.workspace_size(M3, N3, K3, 0)} bytes)")
    A3, B3 = ternary((M3, K3), 97), ternary((N3, K3), 98)
    with torch.cuda.stream(s):
        big = hg.fp8_gemm_bf16(to_dev(torch, A3), to_dev(torch, B3))
    torch.cuda.synchronize()
    assert np.array_equal(from_dev_bf16(big), oracle.gemm(A3, B3))
    for r in range(3):
        say(f"case ws-graph replay {r}")
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(from_dev_bf16(out), want)
        with torch.cuda.stream(s):  # eager work between replays
            hg.fp8_gemm_bf16(a, b)
        torch.cuda.synchronize()


@pytest.mark.parametrize("M,N,K", [(256, 8192, 8192), (16, 4096, 4096)])
def test_capture_without_workspace_runs_unsplit(gpu, oracle, M, N, K):
    torch = gpu
    s = torch.cuda.Stream()
    need = hg.workspace_size(M, N, K, 0)
    say(f"case ws-capture-unsplit {M}x{N}x{K} (variant "
        f"{hg.variant_name(hg.select_variant(M, N, K))}, split workspace "
        f"{need} bytes)")
    assert need > 0  # AUTO splits K here when a workspace is available
    A, B = ternary((M, K), 70), ternary((N, K), 71)
    want = oracle.gemm(A, B, 1.0, 1.0)
    a, b = to_dev(torch, A), to_dev(torch, B)
    outs = [torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
            for _ in range(2)]
    # Stream handles come from a pool and may repeat: make sure this one has
    # no workspace yet (keeping any old one alive, as the helpers do).
    old = hg._workspaces.pop((0, s.cuda_stream), None)
    if old is not None:
        hg._retired.append(old)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):  # a fresh stream: no workspace
        hg.fp8_gemm_bf16(a, b, out=outs[0])
        code = hg.gemm_raw(a.data_ptr(), b.data_ptr(), outs[1].data_ptr(), M,
                           N, K, K, K, N, 0, 0, 0, s.cuda_stream)
    torch.cuda.synchronize()
    assert code == 0
    assert (0, s.cuda_stream) not in hg._workspaces  # none created
    for r in range(3):
        for o in outs:
            o.fill_(float("nan"))  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            got = from_dev_bf16(o)
            say(f"    replay {r} output {i}: "
                f"{int((got != want).sum())} of {M * N} differ")
            assert np.array_equal(got, want)
