"""torch.library operators (hipgemm_amd.torch_ops) and Fp8Linear.

CPU: registration, schemas, fake-tensor shape inference and tracing (no
kernel runs).  GPU (marked): results equal the C ABI's bit for bit, opcheck,
torch.compile without graph breaks, CUDA-graph replay, and Fp8Linear against
an fp32 computation on the same quantised operands.
"""
import numpy as np
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import hipgemm_amd as hg
import hipgemm_amd.torch_ops as ops
from oracle import pyoracle as po
from util import REL_TOL, compare, say

E4M3 = torch.float8_e4m3fn


def test_ops_registered_with_schemas():
    s1 = str(torch.ops.hipgemm.fp8_gemm.default._schema)
    s2 = str(torch.ops.hipgemm.fp8_gemm_rowcol.default._schema)
    assert "Tensor a, Tensor b_t, Tensor? scale_a=None" in s1
    assert s1.endswith("-> Tensor")
    assert "Tensor? scale_rows=None, Tensor? scale_cols=None" in s2


def test_fake_shapes_and_errors():
    with FakeTensorMode():
        a = torch.empty((300, 512), dtype=E4M3)
        b = torch.empty((700, 512), dtype=E4M3)
        y = torch.ops.hipgemm.fp8_gemm(a, b)
        assert tuple(y.shape) == (300, 700) and y.dtype == torch.bfloat16
        y = torch.ops.hipgemm.fp8_gemm_rowcol(a, b, torch.empty(300),
                                              torch.empty(700))
        assert tuple(y.shape) == (300, 700)
        with pytest.raises(hg.HipGemmError):
            torch.ops.hipgemm.fp8_gemm(a, torch.empty((700, 256), dtype=E4M3))
        with pytest.raises(hg.HipGemmError):
            torch.ops.hipgemm.fp8_gemm_rowcol(a, b, torch.empty(301), None)


def test_fp8_linear_traces_as_one_op():
    """make_fx over fake tensors: the layer's GEMM is one hipgemm op node
    (quantisation stays ordinary aten ops)."""
    from torch.fx.experimental.proxy_tensor import make_fx
    lin = torch.nn.Linear(256, 384)
    layer = ops.Fp8Linear.from_linear(lin)
    x = torch.randn(4, 8, 256)
    with FakeTensorMode(allow_non_fake_inputs=True) as mode:
        gm = make_fx(layer, tracing_mode="fake")(mode.from_tensor(x))
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert targets.count("hipgemm.gemm.default") == 1, targets


def test_general_op_fake_shapes():
    with FakeTensorMode():
        a = torch.empty((64, 256), dtype=torch.float8_e5m2)
        b = torch.empty((96, 256), dtype=E4M3)
        y = torch.ops.hipgemm.gemm(a, b, bias=torch.empty(96),
                                   activation="silu", out_f16=True)
        assert tuple(y.shape) == (64, 96) and y.dtype == torch.float16
        with pytest.raises(hg.HipGemmError):
            torch.ops.hipgemm.gemm(a, b, bias=torch.empty(95))
        with pytest.raises(hg.HipGemmError):
            torch.ops.hipgemm.gemm(a, b, activation="tanh")
        for dt in (torch.float32, torch.float8_e4m3fn, torch.bfloat16):
            y = torch.ops.hipgemm.gemm(a, b, out_dtype=dt)
            assert y.dtype == dt and tuple(y.shape) == (64, 96)
        with pytest.raises(hg.HipGemmError):
            torch.ops.hipgemm.gemm(a, b, out_dtype=torch.float64)


def test_cpu_tensors_fail_loudly():
    a = torch.zeros((64, 64), dtype=E4M3)
    with pytest.raises(hg.HipGemmError):
        torch.ops.hipgemm.fp8_gemm(a, a)


def test_quantize_rows_roundtrip():
    x = torch.randn(33, 64) * torch.logspace(-3, 3, 33)[:, None]
    x[5] = 0
    q, s = ops.quantize_rows(x)
    assert q.dtype == E4M3 and s.shape == (33,)
    assert float(s[5]) == 1.0 and not q[5].float().any()
    assert torch.all(q.float().abs().amax(1)[torch.arange(33) != 5] == 448)
    err = (q.float() * s[:, None] - x).abs() / x.abs().amax(1, keepdim=True).clamp(min=1e-30)
    assert float(err.max()) <= 2.0 ** -4  # half an e4m3 ulp at the row max


# ------------------------------------------------------------------ GPU ---

def _inputs(torch_, M, N, K, seed):
    g = torch_.Generator(device="cuda").manual_seed(seed)
    a = torch_.randn((M, K), generator=g, device="cuda").to(E4M3)
    b = torch_.randn((N, K), generator=g, device="cuda").to(E4M3)
    return a, b


@pytest.mark.gpu
def test_ops_equal_abi(gpu):
    torch_ = gpu
    for M, N, K in [(512, 512, 512), (96, 4096, 1024), (1000, 3000, 1104)]:
        say(f"case torch-op M={M} N={N} K={K}")
        a, b = _inputs(torch_, M, N, K, 61)
        sa = torch_.tensor([0.5], device="cuda")
        sb = torch_.tensor([3.0], device="cuda")
        y = torch_.ops.hipgemm.fp8_gemm(a, b, sa, sb)
        ref = hg.fp8_gemm_bf16(a, b, sa, sb)
        sr = torch_.rand(M, device="cuda") + 0.5
        sc = torch_.rand(N, device="cuda") + 0.5
        y2 = torch_.ops.hipgemm.fp8_gemm_rowcol(a, b, sr, sc)
        ref2 = hg.fp8_gemm_bf16_rowcol(a, b, sr, sc)
        torch_.cuda.synchronize()
        assert torch_.equal(y.view(torch_.int16), ref.view(torch_.int16))
        assert torch_.equal(y2.view(torch_.int16), ref2.view(torch_.int16))


@pytest.mark.gpu
def test_opcheck(gpu):
    torch_ = gpu
    say("case torch-op opcheck M=256 N=384 K=256")
    a, b = _inputs(torch_, 256, 384, 256, 62)
    # e4m3 bytes as uint8 (accepted by the ops): opcheck compares inputs
    # with arithmetic that float8 tensors do not implement
    a, b = a.view(torch_.uint8), b.view(torch_.uint8)
    tests = ("test_schema", "test_faketensor", "test_aot_dispatch_static")
    torch_.library.opcheck(torch_.ops.hipgemm.fp8_gemm.default,
                           (a, b, None, None, 0), test_utils=tests)
    torch_.library.opcheck(torch_.ops.hipgemm.fp8_gemm_rowcol.default,
                           (a, b, torch_.rand(256, device="cuda"), None, 0),
                           test_utils=tests)


@pytest.mark.gpu
def test_compile_fullgraph(gpu):
    """torch.compile with fullgraph (no graph break at the custom op); the
    aot_eager backend needs no code generator."""
    torch_ = gpu
    say("case torch-op compile M=384 N=512 K=256")
    a, b = _inputs(torch_, 384, 512, 256, 63)
    sr = torch_.rand(384, device="cuda") + 0.5

    def f(a, b, sr):
        return torch_.ops.hipgemm.fp8_gemm_rowcol(a, b, sr, None).float() * 2

    cf = torch_.compile(f, backend="aot_eager", fullgraph=True)
    got = cf(a, b, sr)
    want = f(a, b, sr)
    torch_.cuda.synchronize()
    assert torch_.equal(got, want)


@pytest.mark.gpu
def test_cuda_graph_replays(gpu):
    """Capture the op (and the skinny split-K schedule, whose workspace is
    allocated on first use, here during warm-up) in a CUDA graph; every
    replay, with eager work and synchronisation between replays, equals the
    eager result."""
    torch_ = gpu
    for M, N, K in [(512, 1024, 512), (64, 4096, 2048)]:
        say(f"case torch-op graph M={M} N={N} K={K}")
        a, b = _inputs(torch_, M, N, K, 64)
        s = torch_.cuda.Stream()
        s.wait_stream(torch_.cuda.current_stream())
        with torch_.cuda.stream(s):
            for _ in range(2):  # warm-up: workspace, caches
                torch_.ops.hipgemm.fp8_gemm(a, b)
        torch_.cuda.current_stream().wait_stream(s)
        torch_.cuda.synchronize()
        graph = torch_.cuda.CUDAGraph()
        with torch_.cuda.graph(graph, stream=s):  # the warmed-up stream
            out = torch_.ops.hipgemm.fp8_gemm(a, b)
        eager = torch_.ops.hipgemm.fp8_gemm(a, b)
        torch_.cuda.synchronize()
        for _ in range(3):
            out.zero_()
            graph.replay()
            torch_.cuda.synchronize()
            assert torch_.equal(out.view(torch_.int16), eager.view(torch_.int16))
            torch_.ops.hipgemm.fp8_gemm(b[:M], a)  # eager work between replays
            torch_.cuda.synchronize()


@pytest.mark.gpu
def test_general_op_equals_abi(gpu, oracle):
    torch_ = gpu
    M, N, K = 256, 384, 512
    say(f"case torch-op gemm M={M} N={N} K={K}")
    a, b = _inputs(torch_, M, N, K, 66)
    a5 = a.float().to(torch_.float8_e5m2)
    bias = torch_.randn(N, device="cuda")
    y = torch_.ops.hipgemm.gemm(a5, b, bias=bias, activation="gelu_tanh",
                                out_f16=True)
    ref = hg.gemm(a5, b, bias=bias, activation="gelu_tanh",
                  out_dtype=torch_.float16)
    torch_.cuda.synchronize()
    assert y.dtype == torch_.float16
    assert torch_.equal(y.view(torch_.int16), ref.view(torch_.int16))
    so = torch_.tensor([0.125], device="cuda")
    for dt in (torch_.float32, torch_.float8_e4m3fn):
        kw = dict(scale_out=so) if dt == torch_.float8_e4m3fn else {}
        y = torch_.ops.hipgemm.gemm(a5, b, bias=bias, activation="relu",
                                    out_dtype=dt, **kw)
        ref = hg.gemm(a5, b, bias=bias, activation="relu", out_dtype=dt, **kw)
        torch_.cuda.synchronize()
        assert y.dtype == dt
        assert torch_.equal(y.view(torch_.uint8), ref.view(torch_.uint8))


@pytest.mark.gpu
def test_fp8_linear_matches_fp32_on_quantised_operands(gpu, oracle):
    """Fp8Linear on an LLM-shaped projection, bias and activation fused,
    against the oracle's general GEMM of the same quantised operands
    (north_star tolerance)."""
    torch_ = gpu
    torch_.manual_seed(65)
    lin = torch_.nn.Linear(1024, 3072).cuda()
    layer = ops.Fp8Linear.from_linear(lin, activation="silu")
    x = torch_.randn(2, 160, 1024, device="cuda")
    say("case fp8-linear tokens=320 in=1024 out=3072 silu")
    y = layer(x)
    torch_.cuda.synchronize()
    assert tuple(y.shape) == (2, 160, 3072) and y.dtype == torch_.bfloat16
    q, s = ops.quantize_rows(x.reshape(-1, 1024))
    A = q.view(torch_.uint8).cpu().numpy()
    B = layer.weight.view(torch_.uint8).cpu().numpy()
    want = oracle.gemm_ex(A, B, act=po.ACT_SILU, scale_rows=s.cpu().numpy(),
                          scale_cols=layer.weight_scale.cpu().numpy(),
                          bias=layer.bias.cpu().numpy())
    got = y.reshape(-1, 3072).view(torch_.int16).cpu().numpy().view(np.uint16)
    max_rel, exact, _ = compare(got, want)
    say(f"    max_rel={max_rel:.3e} exact={exact:.4f}")
    assert max_rel <= REL_TOL
    # and the layer tracks the full-precision Linear to e4m3 accuracy
    with torch_.no_grad():
        ref = torch_.nn.functional.silu(lin(x))
    rel = float((y.float() - ref).norm() / ref.norm())
    say(f"    rel-vs-fp32-linear={rel:.3e}")
    assert rel < 0.05
