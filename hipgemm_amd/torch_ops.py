"""PyTorch custom operators over the hipgemm C ABI, and an FP8 linear layer.

Importing this module registers, in the ``hipgemm`` namespace:

  torch.ops.hipgemm.fp8_gemm(a, b_t, scale_a=None, scale_b=None, variant=0)
      bf16 (M x N) = scale_a * scale_b * a (M x K e4m3) . b_t (N x K e4m3)^T,
      per-tensor scales (1-element float32 device tensors) -- the C ABI's
      hipgemm_fp8_gemm_bf16_ws.
  torch.ops.hipgemm.fp8_gemm_rowcol(a, b_t, scale_rows=None, scale_cols=None,
                                    variant=0)
      the same with per-row (M) / per-column (N) float32 scale vectors --
      hipgemm_fp8_gemm_bf16_rowcol.
  torch.ops.hipgemm.gemm(a, b_t, scale_a=None, scale_b=None, scale_rows=None,
                         scale_cols=None, bias=None, activation="none",
                         out_f16=False, variant=0, out_dtype=None,
                         scale_out=None, mx_scale_a=None, mx_scale_b=None)
      the general entry point (hipgemm_gemm): a / b_t float8_e4m3fn or
      float8_e5m2 (uint8 bytes: e4m3), or both float4_e2m1fn_x2 (K / 2
      bytes per row); fused bias and activation ("none", "relu", "silu",
      "gelu_tanh"); output bf16, fp16 (out_f16 or out_dtype), fp32 or
      float8_e4m3fn (out_dtype; saturating, after multiplying by the
      1-element scale_out); MX block scales packed by
      hipgemm_amd.mx_pack_scales (mx_scale_a / mx_scale_b, uint8).

All have fake (meta) implementations, so they trace under torch.compile,
torch.export and FakeTensorMode without running, and they run inside CUDA
graph capture (the split-K workspace is allocated on first use per stream,
before capture if the caller warms up).  The device implementation is
libhipgemm.so; CPU tensors raise HipGemmError -- there is no CPU path.

Fp8Linear is a drop-in for torch.nn.Linear in LLM projections (the reference
has no layer; its LLM shapes are benchmark configurations): e4m3 weights with
one fp32 scale per output channel, activations quantised per token (row) on
the fly, the product through hipgemm::gemm with the bias and activation
fused into its epilogue.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ACTIVATIONS, HipGemmError, fp8_gemm_bf16, fp8_gemm_bf16_rowcol
from . import gemm as _gemm

__all__ = ["fp8_gemm", "fp8_gemm_rowcol", "gemm", "Fp8Linear",
           "quantize_rows"]

E4M3_MAX = 448.0


@torch.library.custom_op("hipgemm::fp8_gemm", mutates_args=())
def fp8_gemm(a: torch.Tensor, b_t: torch.Tensor,
             scale_a: Optional[torch.Tensor] = None,
             scale_b: Optional[torch.Tensor] = None,
             variant: int = 0) -> torch.Tensor:
    return fp8_gemm_bf16(a, b_t, scale_a, scale_b, variant=variant)


@fp8_gemm.register_fake
def _fp8_gemm_fake(a, b_t, scale_a=None, scale_b=None, variant=0):
    _check_shapes(a, b_t)
    return a.new_empty((a.shape[0], b_t.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op("hipgemm::fp8_gemm_rowcol", mutates_args=())
def fp8_gemm_rowcol(a: torch.Tensor, b_t: torch.Tensor,
                    scale_rows: Optional[torch.Tensor] = None,
                    scale_cols: Optional[torch.Tensor] = None,
                    variant: int = 0) -> torch.Tensor:
    return fp8_gemm_bf16_rowcol(a, b_t, scale_rows, scale_cols,
                                variant=variant)


@fp8_gemm_rowcol.register_fake
def _fp8_gemm_rowcol_fake(a, b_t, scale_rows=None, scale_cols=None,
                          variant=0):
    _check_shapes(a, b_t)
    if scale_rows is not None and tuple(scale_rows.shape) != (a.shape[0],):
        raise HipGemmError("scale_rows must have M elements")
    if scale_cols is not None and tuple(scale_cols.shape) != (b_t.shape[0],):
        raise HipGemmError("scale_cols must have N elements")
    return a.new_empty((a.shape[0], b_t.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op("hipgemm::gemm", mutates_args=())
def gemm(a: torch.Tensor, b_t: torch.Tensor,
         scale_a: Optional[torch.Tensor] = None,
         scale_b: Optional[torch.Tensor] = None,
         scale_rows: Optional[torch.Tensor] = None,
         scale_cols: Optional[torch.Tensor] = None,
         bias: Optional[torch.Tensor] = None, activation: str = "none",
         out_f16: bool = False, variant: int = 0,
         out_dtype: Optional[torch.dtype] = None,
         scale_out: Optional[torch.Tensor] = None,
         mx_scale_a: Optional[torch.Tensor] = None,
         mx_scale_b: Optional[torch.Tensor] = None) -> torch.Tensor:
    return _gemm(a, b_t, out_dtype=_out_dtype(out_f16, out_dtype),
                 scale_a=scale_a, scale_b=scale_b, scale_rows=scale_rows,
                 scale_cols=scale_cols, bias=bias, activation=activation,
                 variant=variant, scale_out=scale_out, mx_scale_a=mx_scale_a,
                 mx_scale_b=mx_scale_b)


def _out_dtype(out_f16, out_dtype):
    if out_dtype is not None:
        if out_dtype not in (torch.bfloat16, torch.float16, torch.float32,
                             torch.float8_e4m3fn):
            raise HipGemmError(f"unsupported out_dtype {out_dtype}")
        return out_dtype
    return torch.float16 if out_f16 else torch.bfloat16


@gemm.register_fake
def _gemm_fake(a, b_t, scale_a=None, scale_b=None, scale_rows=None,
               scale_cols=None, bias=None, activation="none", out_f16=False,
               variant=0, out_dtype=None, scale_out=None, mx_scale_a=None,
               mx_scale_b=None):
    _check_shapes(a, b_t)
    if activation not in ACTIVATIONS:
        raise HipGemmError(f"unknown activation {activation!r}")
    for v, n, name in ((scale_rows, a.shape[0], "scale_rows"),
                       (scale_cols, b_t.shape[0], "scale_cols"),
                       (bias, b_t.shape[0], "bias")):
        if v is not None and tuple(v.shape) != (n,):
            raise HipGemmError(f"{name} must have {n} elements")
    return a.new_empty((a.shape[0], b_t.shape[0]),
                       dtype=_out_dtype(out_f16, out_dtype))


def _check_shapes(a, b_t):
    if a.dim() != 2 or b_t.dim() != 2 or a.shape[1] != b_t.shape[1]:
        raise HipGemmError(f"expected a (M, K) and b_t (N, K), got "
                           f"{tuple(a.shape)} and {tuple(b_t.shape)}")


def quantize_rows(x: torch.Tensor):
    """Per-row e4m3 quantisation: returns (q, s) with q = x / s rounded to
    e4m3 (saturated to +-448) and s = amax(|row|) / 448 (float32, one per
    row; rows of zeros get s = 1).  x ~= q * s[:, None]."""
    xf = x.float()
    amax = xf.abs().amax(dim=1)
    s = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    q = (xf / s[:, None]).clamp_(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q, s


class Fp8Linear(torch.nn.Module):
    """y = act(x W^T + b) with W (out x in) held as e4m3 rows and one
    float32 scale per output feature; x is quantised per token (row) to e4m3
    with its own scale, and the product runs through hipgemm's general
    entry point with the scales, the bias and the activation fused:
    y[t, o] = bf16(act(fma(acc[t, o], sx[t] * sw[o], b[o]))).
    in_features must be a multiple of 16.  activation: None, "relu", "silu"
    or "gelu_tanh"."""

    def __init__(self, weight_e4m3: torch.Tensor, weight_scale: torch.Tensor,
                 bias: Optional[torch.Tensor] = None, variant: int = 0,
                 activation: Optional[str] = None):
        super().__init__()
        if weight_e4m3.dtype != torch.float8_e4m3fn or weight_e4m3.dim() != 2:
            raise HipGemmError("weight must be a 2-D float8_e4m3fn tensor")
        if weight_e4m3.shape[1] % 16 != 0:
            raise HipGemmError("in_features must be a multiple of 16")
        if tuple(weight_scale.shape) != (weight_e4m3.shape[0],):
            raise HipGemmError("weight_scale must have out_features elements")
        self.register_buffer("weight", weight_e4m3.contiguous())
        self.register_buffer("weight_scale",
                             weight_scale.to(torch.float32).contiguous())
        self.register_buffer("bias", None if bias is None else
                             bias.to(torch.float32).contiguous())
        if activation not in ACTIVATIONS:
            raise HipGemmError(f"unknown activation {activation!r}")
        self.activation = activation or "none"
        self.variant = variant

    @property
    def in_features(self) -> int:
        return self.weight.shape[1]

    @property
    def out_features(self) -> int:
        return self.weight.shape[0]

    @classmethod
    def from_linear(cls, linear: torch.nn.Linear, variant: int = 0,
                    activation: Optional[str] = None):
        """Quantise a Linear's weight per output channel (amax / 448)."""
        w, s = quantize_rows(linear.weight.detach())
        return cls(w, s, linear.bias.detach() if linear.bias is not None
                   else None, variant, activation)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        q, s = quantize_rows(x2)
        y = torch.ops.hipgemm.gemm(q, self.weight, scale_rows=s,
                                   scale_cols=self.weight_scale, bias=self.bias,
                                   activation=self.activation,
                                   variant=self.variant)
        return y.reshape(*lead, self.out_features)
