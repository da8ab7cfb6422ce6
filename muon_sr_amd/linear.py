"""SR gradient accumulation fused with the weight-gradient GEMM of linear layers.

``TritonSRAccumulator`` (muon_sr/triton_adamw.py:232-280) accumulates
``p.grad`` into ``p.acc_grad`` after autograd's weight-gradient GEMM has
written ``p.grad``.  For a linear layer ``y = x W^T + b``, ``SRLinear``
computes ``dW = dy^T x`` inside the accumulation kernel
(``msr_linear_wgrad_sr_accum``) and never writes ``W.grad``: the bf16 rounding
of dW, the fp32 sum with the accumulator, the SR noise (one
``random.getrandbits(32)`` seed per micro-batch, offset = element index) and
the zero first buffer are those of the hook (:252-265).  The input gradient
and the bias go through autograd as usual (the bias through the hook, if one
is assigned).  Shapes or dtypes the fused kernel does not take (features not
multiples of 256, token counts not multiples of 128, non-bf16 tensors) return
``dW`` to autograd instead, so the hook accumulates it as for ``nn.Linear``;
so do operands the kernel cannot address (misaligned views, or an operand of
2 GiB or more, e.g. an LM head's dy at 8,372 tokens or more).
"""
import random

import torch

from . import _lib

__all__ = ["linear_wgrad_sr_accum", "SRLinear"]


def wgrad_shape_fits(out_f: int, in_f: int, tokens: int, ldx: int, ldy: int, x_ptr: int, dy_ptr: int) -> bool:
    """Every precondition msr_linear_wgrad_sr_accum checks on its operands (host-only):
    features multiples of 256 and tokens a multiple of 128 (each below 2^30); x and dy
    16-byte aligned with row strides that are multiples of 8 elements and at least the
    row length; and each operand spanning less than 2 GiB, since its loads address it
    with 32-bit byte offsets ((tokens - 1) * ld + features elements)."""
    if not (0 < tokens < (1 << 30) and 0 < in_f < (1 << 30) and 0 < out_f < (1 << 30)):
        return False
    if in_f % 256 or out_f % 256 or tokens % 128:
        return False
    if ldx < in_f or ldy < out_f or ldx % 8 or ldy % 8 or x_ptr % 16 or dy_ptr % 16:
        return False
    return ((tokens - 1) * ldx + in_f) * 2 < (1 << 31) and ((tokens - 1) * ldy + out_f) * 2 < (1 << 31)


def _fits(weight: torch.Tensor, x2: torch.Tensor, dy2: torch.Tensor) -> bool:
    out_f, in_f = weight.shape
    return (weight.dtype == x2.dtype == dy2.dtype == torch.bfloat16 and x2.is_cuda and
            x2.stride(1) == 1 and dy2.stride(1) == 1 and x2.shape[0] == dy2.shape[0] and
            wgrad_shape_fits(out_f, in_f, x2.shape[0], x2.stride(0), dy2.stride(0), x2.data_ptr(), dy2.data_ptr()))


def linear_wgrad_sr_accum(weight: torch.Tensor, x2: torch.Tensor, dy2: torch.Tensor, seed: int = None) -> bool:
    """``weight.acc_grad <- SR(weight.acc_grad + bf16(dy2^T x2))`` in one kernel.

    x2: bf16 [tokens, in], dy2: bf16 [tokens, out] (unit column stride), weight:
    [out, in].  The buffer is created (as zeros) on the first call.  Returns
    False, with nothing done, when the shapes or dtypes do not fit the fused
    kernel.
    """
    if not _fits(weight, x2, dy2):
        return False
    if seed is None:
        seed = random.getrandbits(32)
    first = not hasattr(weight, "acc_grad")
    if first:
        weight.acc_grad = torch.empty_like(weight, dtype=torch.bfloat16, memory_format=torch.contiguous_format)
    acc = weight.acc_grad
    out_f, in_f = weight.shape
    rc = _lib.lib().msr_linear_wgrad_sr_accum(acc.data_ptr(), x2.data_ptr(), x2.stride(0), dy2.data_ptr(),
                                              dy2.stride(0), x2.shape[0], in_f, out_f, seed, int(first),
                                              _lib.noise_mode(), None, _lib.stream_of(acc))
    _lib.check(rc, "msr_linear_wgrad_sr_accum")
    return True


class _SRLinearFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias):
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return torch.nn.functional.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = dy @ weight
        x2 = x.reshape(-1, x.shape[-1])
        dy2 = dy.reshape(-1, dy.shape[-1])
        if ctx.needs_input_grad[1]:
            if x2.stride(1) != 1:
                x2 = x2.contiguous()
            if dy2.stride(1) != 1:
                dy2 = dy2.contiguous()
            if not linear_wgrad_sr_accum(weight, x2, dy2):
                dw = dy2.t() @ x2
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = dy2.sum(0)
        return dx, dw, db


class SRLinear(torch.nn.Linear):
    """``nn.Linear`` whose weight gradient is accumulated into ``weight.acc_grad``
    with stochastic rounding inside the weight-gradient GEMM (for training with
    ``TritonSRAccumulator``: ``reassign_grad_buffer`` then moves ``acc_grad`` to
    ``grad`` as for every other parameter)."""

    def forward(self, x):
        return _SRLinearFunction.apply(x, self.weight, self.bias)
