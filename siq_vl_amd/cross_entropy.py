"""Fused lm_head linear + cross-entropy on MI355X: host side.

Replaces, in the reference path, ``logits = lm_head(h)``
(transformers models/qwen2/modeling_qwen2.py:465) followed by
``ForCausalLMLoss`` / ``fixed_cross_entropy`` (transformers
loss/loss_utils.py:32-71: fp32 upcast, ``F.cross_entropy`` with
``ignore_index=-100``, ``"mean"`` or ``"sum" / num_items_in_batch``) and
their autograd backward, by one call of ``siq_flce_fwd_bwd`` that never
holds more than one token chunk of (exp-normalised) logits, bounded at
``DEFAULT_E_BUDGET_BYTES``.

The forward computes the loss and both gradients at once; the backward only
rescales them by the upstream gradient (a device scalar, no host sync), in
place unless the graph is retained.
Without gradients (evaluation) the loss-only ``siq_flce_loss`` runs.
"""

from __future__ import annotations

import torch

from . import _lib
from ._deferred import DeferredChecks

IGNORE_INDEX = -100
# Bound on the one logits-sized buffer, a token chunk's softmax numerators
# (chunk x vocab bf16).  At vocab 151,936 this is 6,912 rows (2.1 GB, against
# 5.0 GB for the bf16 logits of a 16,384-token batch and 10 GB for the fp32
# logits the reference's ForCausalLMLoss upcasts to).
DEFAULT_E_BUDGET_BYTES = 2 << 30


def default_chunk_tokens(vocab: int, budget_bytes: int = DEFAULT_E_BUDGET_BYTES) -> int:
    """Token rows per logits chunk: the most 256-row tiles whose numerators
    (rows x vocab bf16) fit in ``budget_bytes`` (at least one tile)."""
    rows = budget_bytes // (2 * max(int(vocab), 1))
    return max(256, (rows // 256) * 256)


def flce_workspace_bytes(n: int, hdim: int, vocab: int, chunk_tokens: int | None, need_dweight: bool) -> int:
    chunk = default_chunk_tokens(vocab) if chunk_tokens is None else int(chunk_tokens)
    return int(_lib.lib().siq_flce_workspace_bytes(n, hdim, vocab, chunk, int(bool(need_dweight))))


def _check_operands(hidden, weight, labels):
    if hidden.dim() != 2 or weight.dim() != 2:
        raise ValueError("hidden must be [n, hdim] and weight [vocab, hdim]")
    n, hdim = hidden.shape
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


def _divisor(divisor, dev):
    if divisor is None:
        return None, 0, None
    divisor = divisor.to(device=dev, dtype=torch.float32).reshape(())
    return divisor, 1, divisor.data_ptr()


def flce_fwd_bwd(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, ignore_index: int = IGNORE_INDEX,
                 divisor: torch.Tensor | None = None, need_dweight: bool = True,
                 chunk_tokens: int | None = None):
    """Raw operator.

    ``hidden [n, hdim]`` bf16, ``weight [vocab, hdim]`` bf16, ``labels [n]`` int64
    (already shifted).  ``divisor`` None -> mean over valid rows; else a
    device scalar: loss = sum / divisor.  ``chunk_tokens`` None -> the
    default bound (``default_chunk_tokens``).  Returns
    ``(loss fp32 [], count int64 [], bad_labels int64 [], dhidden, dweight | None)``.
    """
    _check_operands(hidden, weight, labels)
    n, hdim = hidden.shape
    vocab = weight.shape[0]
    chunk = default_chunk_tokens(vocab) if chunk_tokens is None else int(chunk_tokens)
    if chunk <= 0:
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
    divisor, reduction, div_ptr = _divisor(divisor, dev)
    L = _lib.lib()
    ws_bytes = L.siq_flce_workspace_bytes(n, hdim, vocab, chunk, int(need_dweight))
    ws = torch.empty((max(ws_bytes, 16),), dtype=torch.uint8, device=dev)
    rc = L.siq_flce_fwd_bwd(hidden.data_ptr(), weight.data_ptr(), labels.data_ptr(), n, hdim, vocab,
                            int(ignore_index), reduction, div_ptr, loss.data_ptr(), count.data_ptr(), bad.data_ptr(),
                            dh.data_ptr(), dw.data_ptr() if dw is not None else None, chunk,
                            ws.data_ptr(), ws.numel(), torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(rc, "siq_flce_fwd_bwd")
    return loss, count, bad, dh, dw


def flce_loss(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, ignore_index: int = IGNORE_INDEX,
              divisor: torch.Tensor | None = None):
    """Loss only (``siq_flce_loss``): the logits GEMM and the chunked
    logsumexp, no gradient work.  Returns ``(loss, count, bad_labels)``,
    bitwise those of ``flce_fwd_bwd`` on the same inputs."""
    _check_operands(hidden, weight, labels)
    n, hdim = hidden.shape
    vocab = weight.shape[0]
    dev = hidden.device
    hidden = hidden.contiguous()
    weight = weight.contiguous()
    labels = labels.to(dev).contiguous()
    loss = torch.empty((), dtype=torch.float32, device=dev)
    count = torch.empty((), dtype=torch.int64, device=dev)
    bad = torch.empty((), dtype=torch.int64, device=dev)
    divisor, reduction, div_ptr = _divisor(divisor, dev)
    L = _lib.lib()
    ws_bytes = L.siq_flce_loss_workspace_bytes(n, hdim, vocab)
    ws = torch.empty((max(ws_bytes, 16),), dtype=torch.uint8, device=dev)
    rc = L.siq_flce_loss(hidden.data_ptr(), weight.data_ptr(), labels.data_ptr(), n, hdim, vocab, int(ignore_index),
                         reduction, div_ptr, loss.data_ptr(), count.data_ptr(), bad.data_ptr(), ws.data_ptr(),
                         ws.numel(), torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(rc, "siq_flce_loss")
    return loss, count, bad


class LabelError(ValueError):
    """A label outside [0, vocab) that is not ignore_index (F.cross_entropy
    rejects those too)."""


# Out-of-range labels are counted on the device.  Reading that count at once
# would stall the host on every step, so by default it is copied to pinned
# host memory without blocking and checked when the copy has landed: at the
# next call, or when check_pending_labels() is called.  validate="sync" reads it
# at once (one device-to-host sync), validate=False never checks.
_LABEL_CHECKS = DeferredChecks()


def _raise_bad(nbad: int, vocab: int, ignore_index: int) -> None:
    raise LabelError(f"fused cross-entropy: {nbad} label(s) outside [0, {vocab}) that are not ignore_index "
                     f"({ignore_index}); F.cross_entropy rejects such targets")


def check_pending_labels(block: bool = False) -> None:
    """Raises LabelError for any earlier call whose bad-label count has landed
    and is non-zero (all of them when ``block``)."""
    _LABEL_CHECKS.check(block)


def _track_bad(bad: torch.Tensor, vocab: int, ignore_index: int, validate) -> None:
    if validate is False or validate is None:
        return
    if torch.cuda.is_current_stream_capturing():
        # Inside HIP graph capture neither a host read nor an event query of
        # earlier work is allowed: the labels of a captured call are not
        # validated (check them once outside the graph, with validate="sync").
        return
    if validate == "sync":
        nbad = int(bad)
        if nbad > 0:
            _raise_bad(nbad, vocab, ignore_index)
        return

    def judge(vals):
        if vals[0] > 0:
            _raise_bad(int(vals[0]), vocab, ignore_index)

    _LABEL_CHECKS.add(bad, judge)


def _keeps_graph() -> bool:
    """True inside a backward that retains the graph (``retain_graph=True``):
    the saved gradients must then survive it.  Unknown (a torch without the
    query) counts as True, the safe side."""
    try:
        return bool(torch._C._autograd._get_current_graph_task_keep_graph())
    except (AttributeError, RuntimeError):
        return True


def _scaled(t: torch.Tensor, g: torch.Tensor, inplace: bool) -> torch.Tensor:
    """t * g in bf16: in place (the saved gradient becomes the returned one,
    no second [vocab, hdim] buffer at the backward's peak), or into a new
    tensor when the graph is retained, so that a second backward sees the
    saved gradients unscaled."""
    out = t if inplace else torch.empty_like(t)
    rc = _lib.lib().siq_scale_bf16(t.data_ptr(), out.data_ptr(), t.numel(), g.data_ptr(),
                                   torch.cuda.current_stream(t.device).cuda_stream)
    _lib.check(rc, "siq_scale_bf16")
    return out


class _FusedLinearCE(torch.autograd.Function):
    """Loss forward; its backward returns the gradients the forward already
    computed, times the upstream gradient."""

    @staticmethod
    def forward(ctx, hidden, weight, labels, ignore_index, divisor, chunk_tokens, validate):
        shape = hidden.shape
        h2 = hidden.reshape(-1, shape[-1])
        loss, _, bad, dh, dw = flce_fwd_bwd(h2, weight, labels.reshape(-1), ignore_index, divisor,
                                            need_dweight=weight.requires_grad, chunk_tokens=chunk_tokens)
        _track_bad(bad, weight.shape[0], ignore_index, validate)
        ctx.shape = shape
        ctx.save_for_backward(dh, dw if dw is not None else torch.empty(0, device=hidden.device))
        ctx.has_dw = dw is not None
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        dh, dw = ctx.saved_tensors
        g = grad_loss.detach().to(torch.float32).reshape(()).contiguous()
        inplace = not _keeps_graph()
        gh = _scaled(dh, g, inplace).reshape(ctx.shape) if ctx.needs_input_grad[0] else None
        gw = _scaled(dw, g, inplace) if ctx.has_dw and ctx.needs_input_grad[1] else None
        return gh, gw, None, None, None, None, None


def fused_linear_cross_entropy(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor,
                               ignore_index: int = IGNORE_INDEX, num_items_in_batch=None,
                               chunk_tokens: int | None = None, validate="lazy") -> torch.Tensor:
    """``F.cross_entropy(hidden @ weight.T, labels, ignore_index)`` without logits.

    ``labels`` are the already-shifted targets (same shape as ``hidden[..., 0]``).
    With ``num_items_in_batch`` the loss is ``sum / num_items_in_batch`` as in
    ``fixed_cross_entropy``; otherwise the mean over non-ignored rows (NaN if
    every row is ignored, like ``F.cross_entropy``).

    When no gradient can flow (grad mode off, or neither ``hidden`` nor
    ``weight`` requires grad) only the loss is computed (``flce_loss``).
    Labels outside ``[0, vocab)`` other than ``ignore_index`` raise
    ``LabelError``: ``validate="lazy"`` (default) without a host sync, at the
    next call or ``check_pending_labels()``; ``"sync"`` at once; ``False``
    never.  A lazy check of the last call surfaces only at a later call, so a
    training or evaluation loop ends with ``check_pending_labels(block=True)``.
    Calls captured in a HIP graph are not validated (no host work is allowed
    there).

    ``weight`` that does not require grad (a frozen ``lm_head``: the
    reference's stage 1, and stage 2's LoRA, which leaves ``lm_head`` out of
    its targets) gives the dH-only call: no dW GEMM and no dW buffer.
    """
    divisor = None
    if num_items_in_batch is not None:
        if torch.is_tensor(num_items_in_batch):
            divisor = num_items_in_batch.to(device=hidden.device, dtype=torch.float32)
        else:
            divisor = torch.tensor(float(num_items_in_batch), dtype=torch.float32, device=hidden.device)
    h = hidden if hidden.dtype == torch.bfloat16 else hidden.to(torch.bfloat16)
    w = weight if weight.dtype == torch.bfloat16 else weight.to(torch.bfloat16)
    if not torch.is_grad_enabled() or not (h.requires_grad or w.requires_grad):
        loss, _, bad = flce_loss(h.reshape(-1, h.shape[-1]), w, labels.reshape(-1), int(ignore_index), divisor)
        _track_bad(bad, w.shape[0], int(ignore_index), validate)
        return loss
    return _FusedLinearCE.apply(h, w, labels, int(ignore_index), divisor, chunk_tokens, validate)


def shift_labels(labels: torch.Tensor, ignore_index: int = IGNORE_INDEX) -> torch.Tensor:
    """The left shift of ForCausalLMLoss (transformers loss/loss_utils.py:63-64):
    pad one ``ignore_index`` on the right, drop the first column."""
    return torch.nn.functional.pad(labels, (0, 1), value=ignore_index)[..., 1:].contiguous()


def ce_flops(n: int, hdim: int, vocab: int) -> float:
    """Algorithmic FLOPs of forward + backward: 6 * n * hdim * vocab (recompute not counted)."""
    return 6.0 * n * hdim * vocab


__all__ = [
    "DEFAULT_E_BUDGET_BYTES",
    "IGNORE_INDEX",
    "LabelError",
    "ce_flops",
    "check_pending_labels",
    "default_chunk_tokens",
    "flce_fwd_bwd",
    "flce_loss",
    "flce_workspace_bytes",
    "fused_linear_cross_entropy",
    "shift_labels",
]
