"""(d) The wide edge GEMM on CDNA4 MFMA (HIP kernels).

Reference signatures (fastmd/engine/kernels/triton_wide_gemm.py:482-553):
  ``linear(x, weight, bias=None, precision=None, parts=())`` = ``F.linear`` (y = x W^T + b),
  ``linear_into(out, x, weight, bias=None, rows=None)`` (no autograd),
  ``matmul(grad, weight, c=None, rows=None, accumulate=False, enabled=None)`` = ``grad @ weight (+ c)``.
The reference's 3xTF32 kernels decline K % 16 != 0 (:235), i.e. the configs' K = 2F + 8, and fall
back to cuBLAS SGEMM; here every shape runs the fp32 MFMA kernel (v_mfma_f32_32x32x2_f32), and
``edge_gemm(a, w, dtype=torch.bfloat16)`` the bf16 one (v_mfma_f32_32x32x16_bf16, fp32 out).
``epilogue="silu"`` fuses SiLU into the store.
"""
from __future__ import annotations

import torch
from torch import Tensor
from torch.autograd import Function

from fastmd_amd import _abi
from fastmd_amd._device import require_cuda, rows_view, stream

_EPILOGUES = {None: 0, "none": 0, "silu": 1}


def gemm(a: Tensor, b: Tensor, *, b_layout: int, bias: Tensor | None = None, out: Tensor | None = None,
         accumulate: bool = False, epilogue: str | None = None) -> Tensor:
    """``a @ op(b) (+ bias) (+ out)``: op(b) = b^T for b_layout 0 (b [N, K]), b for 1 (b [K, N])."""
    require_cuda(a, b, bias, out)
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError("gemm takes 2-D operands")
    m, k = a.shape
    n = b.shape[0] if b_layout == 0 else b.shape[1]
    kb = b.shape[1] if b_layout == 0 else b.shape[0]
    if kb != k:
        raise ValueError(f"gemm shape mismatch: {tuple(a.shape)} x {tuple(b.shape)} (layout {b_layout})")
    if bias is not None and (bias.shape != (n,) or bias.dtype != torch.float32):
        raise ValueError("bias must be float32 [N]")
    if bias is not None:
        bias = bias.contiguous()
    if out is None:
        out = (torch.zeros if accumulate else torch.empty)((m, n), dtype=torch.float32, device=a.device)
    elif out.shape != (m, n) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError("out must be float32 [M, N] with unit column stride")
    if a.dtype == torch.float32 and b.dtype == torch.float32:
        name = "fmd_gemm_f32"
    elif a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16:
        name = "fmd_gemm_bf16"
    else:
        raise ValueError(f"gemm operands must both be float32 or bfloat16, got {a.dtype}, {b.dtype}")
    a, lda = rows_view(a)
    b, ldb = rows_view(b)
    if m == 0 or n == 0:
        return out
    _abi.call(name, a.data_ptr(), lda, b.data_ptr(), ldb, b_layout, _abi.ptr(bias), out.data_ptr(),
              out.stride(0) if m > 1 else n, m, n, k, 1 if accumulate else 0, _EPILOGUES[epilogue], stream())
    return out


class _Linear(Function):
    @staticmethod
    def forward(ctx, x, weight, bias):
        y = gemm(x, weight, b_layout=0, bias=bias)
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return y

    @staticmethod
    def backward(ctx, gy):
        x, weight = ctx.saved_tensors
        gy = gy.contiguous()
        gx = gemm(gy, weight, b_layout=1) if ctx.needs_input_grad[0] else None
        # trainable weights are outside the MD path (the reference declines them too,
        # triton_wide_gemm.py:242-243): their gradient is formed by torch
        gw = gy.t().mm(x) if ctx.needs_input_grad[1] else None
        gb = gy.sum(0) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return gx, gw, gb


def linear(x: Tensor, weight: Tensor, bias: Tensor | None = None, precision=None, parts=()) -> Tensor:
    """``F.linear(x, weight, bias)`` on the fp32 MFMA kernel (x 2-D float32). ``precision`` and
    ``parts`` are accepted for signature parity; there is one precision (IEEE-rounded fp32
    products, fp32 accumulation)."""
    if x.dim() != 2:
        shape = x.shape
        return linear(x.reshape(-1, shape[-1]), weight, bias).reshape(*shape[:-1], weight.shape[0])
    return _Linear.apply(x, weight, bias)


def linear_into(out: Tensor, x: Tensor, weight: Tensor, bias: Tensor | None = None, rows: int | None = None):
    """``out[:] = x @ weight^T (+ bias)`` (no autograd); ``rows`` is accepted for parity (a row chunk
    takes the same kernel as the whole GEMM, so the rows are equal either way)."""
    with torch.no_grad():
        return gemm(x, weight, b_layout=0, bias=bias, out=out)


def matmul(grad: Tensor, weight: Tensor, c: Tensor | None = None, rows: int | None = None, accumulate: bool = False,
           enabled: bool | None = None) -> Tensor:
    """``grad @ weight (+ c)``; ``accumulate`` writes into ``c``."""
    with torch.no_grad():
        if c is None:
            return gemm(grad, weight, b_layout=1)
        if accumulate:
            return gemm(grad, weight, b_layout=1, out=c, accumulate=True)
        out = c.clone()
        return gemm(grad, weight, b_layout=1, out=out, accumulate=True)


def edge_gemm(a: Tensor, w: Tensor, dtype: torch.dtype = torch.float32, *, bias: Tensor | None = None,
              epilogue: str | None = None) -> Tensor:
    """The configs' wide edge GEMM ``[E, 2F+8] x [2F+8, 4F]`` with ``w`` stored ``[2F+8, 4F]``
    (b_layout 1); ``dtype`` float32 or bfloat16 operands, float32 output. No autograd."""
    with torch.no_grad():
        if dtype == torch.bfloat16:
            return gemm(a.to(torch.bfloat16), w.to(torch.bfloat16), b_layout=1, bias=bias, epilogue=epilogue)
        if dtype != torch.float32:
            raise ValueError(f"edge_gemm dtype must be float32 or bfloat16, got {dtype}")
        return gemm(a, w, b_layout=1, bias=bias, epilogue=epilogue)
