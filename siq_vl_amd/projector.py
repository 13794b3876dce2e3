"""Pixel-shuffle projector on MI355X: host side.

Replaces ``SiQ_VLProjector.forward`` (siq_vl/model/modeling.py:100-105): the
pixel shuffle of ``_pixel_shuffle`` (:74-98) followed by the bias-free
``nn.Linear`` ``mlp`` (:59) -- and autograd's backward of both -- with the
HIP kernels behind ``siq_proj_fwd`` / ``siq_proj_bwd``, which fold the
shuffle into the GEMMs' operand loads (no shuffled copy of the features in
either direction).

* ``pixel_shuffle_linear(x, weight, factor)`` -- the autograd op:
  ``x [B, L, Dv]`` bf16 (L a perfect square), ``weight [N, Dv r^2]`` ->
  ``[B, L / r^2, N]``.  fp32 inputs are cast to bf16 first (the reference
  trains the projector under bf16 autocast); gradients flow back through the
  casts.
* ``fused_projector_forward(self, x)`` -- ``SiQ_VLProjector.forward`` with the
  reference's checks and error messages; ``enable_fused_projector(model)``
  installs it on ``model.projector`` (or on ``model`` itself if it is the
  projector).
"""

from __future__ import annotations

import math
import types

import torch

from . import _lib


def _check_shape(seq: int, factor: int) -> int:
    """The reference's two checks (modeling.py:76-90); returns the side length."""
    side = math.isqrt(seq)
    if side * side != seq:
        raise ValueError(
            f"Sequence length {seq} is not a perfect square (sqrt={side}). "
            f"Cannot apply pixel shuffle. Please check your vision model configuration."
        )
    if side % factor != 0:
        valid = [f for f in range(1, side + 1) if side % f == 0]
        raise ValueError(
            f"seq_root {side} is not divisible by scale factor {factor}. "
            f"Valid factors for seq_root {side} are: {valid}. "
            f"Please set pixel_shuffle_factor to one of these values."
        )
    return side


def _workspace(batch: int, side: int, dv: int, factor: int, n: int, device) -> torch.Tensor:
    nbytes = int(_lib.lib().siq_proj_workspace_bytes(batch, side, dv, factor, n))
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def proj_fwd(x: torch.Tensor, weight: torch.Tensor, factor: int) -> torch.Tensor:
    """Raw forward: bf16 contiguous ``x [B, side^2, Dv]``, ``weight [N, Dv r^2]`` -> ``[B, (side/r)^2, N]``."""
    b, seq, dv = x.shape
    side = _check_shape(seq, factor)
    n = weight.shape[0]
    if weight.shape[1] != dv * factor * factor:
        raise ValueError(f"weight is {tuple(weight.shape)}, expected [N, {dv * factor * factor}]")
    t = (side // factor) ** 2
    y = torch.empty(b, t, n, dtype=torch.bfloat16, device=x.device)
    ws = _workspace(b, side, dv, factor, n, x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = _lib.lib().siq_proj_fwd(x.data_ptr(), weight.data_ptr(), y.data_ptr(), b, side, dv, factor, n,
                                 ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "siq_proj_fwd")
    return y


def proj_bwd(x: torch.Tensor, weight: torch.Tensor, dy: torch.Tensor, factor: int, need_dx: bool = True,
             need_dweight: bool = True):
    """Raw backward: returns ``(dx | None, dweight | None)``."""
    b, seq, dv = x.shape
    side = _check_shape(seq, factor)
    n = weight.shape[0]
    dx = torch.empty_like(x) if need_dx else None
    dw = torch.empty_like(weight) if need_dweight else None
    ws = _workspace(b, side, dv, factor, n, x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = _lib.lib().siq_proj_bwd(x.data_ptr(), weight.data_ptr(), dy.data_ptr(),
                                 dx.data_ptr() if dx is not None else None,
                                 dw.data_ptr() if dw is not None else None, b, side, dv, factor, n,
                                 ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "siq_proj_bwd")
    return dx, dw


def _prep(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on the GPU, got {t.device}")
    t = t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16)
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


class _PixelShuffleLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, factor):
        xb, wb = _prep(x, "x"), _prep(weight, "weight")
        ctx.save_for_backward(xb, wb)
        ctx.factor = factor
        return proj_fwd(xb, wb, factor)

    @staticmethod
    def backward(ctx, dy):
        xb, wb = ctx.saved_tensors
        need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (need_dx or need_dw):
            return None, None, None
        dx, dw = proj_bwd(xb, wb, _prep(dy, "dy"), ctx.factor, need_dx, need_dw)
        return dx, dw, None


def pixel_shuffle_linear(x: torch.Tensor, weight: torch.Tensor, factor: int) -> torch.Tensor:
    """``nn.functional.linear(pixel_shuffle(x, factor), weight)`` without the shuffled copy."""
    if x.dim() != 3 or weight.dim() != 2:
        raise ValueError("x must be [batch, seq, dim] and weight [out_features, dim * factor^2]")
    return _PixelShuffleLinear.apply(x, weight, int(factor))


def fused_projector_forward(self, x: torch.Tensor) -> torch.Tensor:
    """``SiQ_VLProjector.forward`` (modeling.py:100-105) on the fused kernels."""
    if getattr(self.mlp, "bias", None) is not None:
        raise ValueError("the SiQ-VL projector's mlp has no bias (modeling.py:59)")
    return pixel_shuffle_linear(x, self.mlp.weight, self.vision_pixel_shuffle_factor)


def enable_fused_projector(model: torch.nn.Module) -> torch.nn.Module:
    """Installs ``fused_projector_forward`` on the model's projector (SiQ_VLForCausalLM
    keeps it as ``model.projector``, modeling.py:243) or on a projector passed directly."""
    proj = model if hasattr(model, "vision_pixel_shuffle_factor") else getattr(model, "projector", None)
    if proj is None or not hasattr(proj, "mlp") or not hasattr(proj, "vision_pixel_shuffle_factor"):
        raise ValueError("no SiQ-VL projector (an 'mlp' Linear and 'vision_pixel_shuffle_factor') found")
    proj.forward = types.MethodType(fused_projector_forward, proj)
    return model


def projector_flops(tokens_out: int, in_features: int, out_features: int, backward: bool = True) -> float:
    """2 m k n per GEMM: the forward, and dX plus dW for the backward."""
    return (6.0 if backward else 2.0) * tokens_out * in_features * out_features
