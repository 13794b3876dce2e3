"""Fused lm_head linear + cross-entropy on MI355X: host side.

Replaces, in the reference path, ``logits = lm_head(h)``
(transformers models/qwen2/modeling_qwen2.py:465) followed by
``ForCausalLMLoss`` / ``fixed_cross_entropy`` (transformers
loss/loss_utils.py:32-71: fp32 upcast, ``F.cross_entropy`` with
``ignore_index=-100``, ``"mean"`` or ``"sum" / num_items_in_batch``) and
their autograd backward, by one call of ``siq_flce_fwd_bwd`` that never
holds more than one token chunk of (exp-normalised) logits.

The forward computes the loss and both gradients at once; the backward only
rescales them by the upstream gradient (a device scalar, no host sync).
"""

from __future__ import annotations

import torch

from . import _lib

# Token rows per logits chunk.  One chunk's softmax numerators are chunk x vocab
# bf16 (5.0 GB at 16384 x 151936); a whole 16384-token batch in one chunk runs
# 3% faster on MI355X than two chunks of 8192 and needs no fp32 dW accumulator.
DEFAULT_CHUNK_TOKENS = 16384
IGNORE_INDEX = -100


def flce_workspace_bytes(n: int, hdim: int, vocab: int, chunk_tokens: int, need_dweight: bool) -> int:
    return int(_lib.lib().siq_flce_workspace_bytes(n, hdim, vocab, chunk_tokens, int(bool(need_dweight))))


def flce_fwd_bwd(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, ignore_index: int = IGNORE_INDEX,
                 divisor: torch.Tensor | None = None, need_dweight: bool = True,
                 chunk_tokens: int = DEFAULT_CHUNK_TOKENS):
    """Raw operator.

    ``hidden [n, hdim]`` bf16, ``weight [vocab, hdim]`` bf16, ``labels [n]`` int64
    (already shifted).  ``divisor`` None -> mean over valid rows; else a
    device scalar: loss = sum / divisor.  Returns
    ``(loss fp32 [], count int64 [], bad_labels int64 [], dhidden, dweight | None)``.
    """
    if hidden.dim() != 2 or weight.dim() != 2:
        raise ValueError("hidden must be [n, hdim] and weight [vocab, hdim]")
    n, hdim = hidden.shape
    vocab = weight.shape[0]
    if weight.shape[1] != hdim:
        raise ValueError(f"weight hdim {weight.shape[1]} != hidden hdim {hdim}")
    for name, t in (("hidden", hidden), ("weight", weight)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
        if t.device.type != "cuda":
            raise ValueError(f"{name} must live on the GPU")
    if labels.dim() != 1 or labels.shape[0] != n:
        raise ValueError(f"labels must be [n] = [{n}], got {tuple(labels.shape)}")
    if labels.dtype != torch.int64:
        raise ValueError(f"labels must be int64, got {labels.dtype}")
    if chunk_tokens <= 0:
        raise ValueError("chunk_tokens must be positive")
    dev = hidden.device
    hidden = hidden.contiguous()
    weight = weight.contiguous()
    labels = labels.to(dev).contiguous()
    loss = torch.empty((), dtype=torch.float32, device=dev)
    count = torch.empty((), dtype=torch.int64, device=dev)
    bad = torch.empty((), dtype=torch.int64, device=dev)
    dh = torch.empty_like(hidden)
    dw = torch.empty_like(weight) if need_dweight else None
    reduction = 0
    div_ptr = None
    if divisor is not None:
        divisor = divisor.to(device=dev, dtype=torch.float32).reshape(())
        reduction = 1
        div_ptr = divisor.data_ptr()
    L = _lib.lib()
    ws_bytes = L.siq_flce_workspace_bytes(n, hdim, vocab, chunk_tokens, int(need_dweight))
    ws = torch.empty((max(ws_bytes, 16),), dtype=torch.uint8, device=dev)
    rc = L.siq_flce_fwd_bwd(hidden.data_ptr(), weight.data_ptr(), labels.data_ptr(), n, hdim, vocab,
                            int(ignore_index), reduction, div_ptr, loss.data_ptr(), count.data_ptr(), bad.data_ptr(),
                            dh.data_ptr(), dw.data_ptr() if dw is not None else None, int(chunk_tokens),
                            ws.data_ptr(), ws.numel(), torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(rc, "siq_flce_fwd_bwd")
    return loss, count, bad, dh, dw


def _scale_(t: torch.Tensor | None, g: torch.Tensor) -> None:
    if t is None:
        return
    rc = _lib.lib().siq_scale_bf16_inplace(t.data_ptr(), t.numel(), g.data_ptr(),
                                           torch.cuda.current_stream(t.device).cuda_stream)
    _lib.check(rc, "siq_scale_bf16_inplace")


class _FusedLinearCE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, weight, labels, ignore_index, divisor, chunk_tokens):
        shape = hidden.shape
        h2 = hidden.reshape(-1, shape[-1])
        loss, _, _, dh, dw = flce_fwd_bwd(h2, weight, labels.reshape(-1), ignore_index, divisor,
                                          need_dweight=weight.requires_grad, chunk_tokens=chunk_tokens)
        ctx.shape = shape
        ctx.save_for_backward(dh, dw if dw is not None else torch.empty(0, device=hidden.device))
        ctx.has_dw = dw is not None
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        dh, dw = ctx.saved_tensors
        g = grad_loss.detach().to(torch.float32).reshape(()).contiguous()
        _scale_(dh, g)
        if ctx.has_dw:
            _scale_(dw, g)
        return dh.reshape(ctx.shape), (dw if ctx.has_dw else None), None, None, None, None


def fused_linear_cross_entropy(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor,
                               ignore_index: int = IGNORE_INDEX, num_items_in_batch=None,
                               chunk_tokens: int = DEFAULT_CHUNK_TOKENS) -> torch.Tensor:
    """``F.cross_entropy(hidden @ weight.T, labels, ignore_index)`` without logits.

    ``labels`` are the already-shifted targets (same shape as ``hidden[..., 0]``).
    With ``num_items_in_batch`` the loss is ``sum / num_items_in_batch`` as in
    ``fixed_cross_entropy``; otherwise the mean over non-ignored rows (NaN if
    every row is ignored, like ``F.cross_entropy``).
    """
    divisor = None
    if num_items_in_batch is not None:
        if torch.is_tensor(num_items_in_batch):
            divisor = num_items_in_batch.to(device=hidden.device, dtype=torch.float32)
        else:
            divisor = torch.tensor(float(num_items_in_batch), dtype=torch.float32, device=hidden.device)
    h = hidden if hidden.dtype == torch.bfloat16 else hidden.to(torch.bfloat16)
    w = weight if weight.dtype == torch.bfloat16 else weight.to(torch.bfloat16)
    return _FusedLinearCE.apply(h, w, labels, int(ignore_index), divisor, int(chunk_tokens))


def shift_labels(labels: torch.Tensor, ignore_index: int = IGNORE_INDEX) -> torch.Tensor:
    """The left shift of ForCausalLMLoss (transformers loss/loss_utils.py:63-64):
    pad one ``ignore_index`` on the right, drop the first column."""
    return torch.nn.functional.pad(labels, (0, 1), value=ignore_index)[..., 1:].contiguous()


def ce_flops(n: int, hdim: int, vocab: int) -> float:
    """Algorithmic FLOPs of forward + backward: 6 * n * hdim * vocab (recompute not counted)."""
    return 6.0 * n * hdim * vocab


__all__ = [
    "DEFAULT_CHUNK_TOKENS",
    "IGNORE_INDEX",
    "ce_flops",
    "flce_fwd_bwd",
    "flce_workspace_bytes",
    "fused_linear_cross_entropy",
    "shift_labels",
]
