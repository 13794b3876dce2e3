"""Varlen (cu_seqlens-packed) flash attention on MI355X: host side.

Three layers, all ending in the HIP kernels behind ``include/siq_kernels.h``:

* ``varlen_attn_fwd`` / ``varlen_attn_bwd`` -- raw operators (validation,
  workspace, stream) over ``siq_attn_varlen_fwd_plan`` /
  ``siq_attn_varlen_bwd_plan``, with the batch's schedule (``AttnPlan``,
  ``siq_attn_build_plan``) built once per ``cu_seqlens`` tensor and reused by
  every layer's forward and backward.
* ``flash_attn_varlen_func`` -- the autograd op with the varlen call
  convention transformers uses for packed batches
  (transformers modeling_flash_attention_utils.py:796-822:
  ``(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
  softmax_scale=..., causal=...)`` on ``[total, heads, dim]`` tensors).
* ``siq_varlen_attention_forward`` -- the ``AttentionInterface`` function
  (signature of transformers integrations/flash_attention.py:26-102), which the
  reference's attention modules call at models/qwen2/modeling_qwen2.py:216-230
  (causal GQA) and models/siglip/modeling_siglip.py:288-300 (bidirectional)
  once ``config._attn_implementation == "siq_varlen"``.

Semantics are those of the reference's eager/SDPA path
(modeling_qwen2.py:138-172): fp32 softmax of ``scale * Q K^T`` plus the
causal / padding mask, GQA with q-head ``h`` reading kv-head
``h // (Hq // Hkv)``, output ``[B, S, Hq, D]``.
"""

from __future__ import annotations

import weakref
from typing import Any

import torch

from . import _lib

ATTN_IMPLEMENTATION = "siq_varlen"
SUPPORTED_HEAD_DIMS = (64, 128)


# --------------------------------------------------------------------------- validation
def _check_token_major(name: str, t: torch.Tensor, heads: int | None = None, dim: int | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dim() != 3:
        raise ValueError(f"{name} must be [total_tokens, heads, head_dim], got shape {tuple(t.shape)}")
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on the GPU, got device {t.device}")
    if heads is not None and t.shape[1] != heads:
        raise ValueError(f"{name} has {t.shape[1]} heads, expected {heads}")
    if dim is not None and t.shape[2] != dim:
        raise ValueError(f"{name} head_dim {t.shape[2]} != {dim}")
    if t.stride(2) != 1:
        raise ValueError(f"{name} must have a contiguous head_dim (stride(2) == 1)")
    if t.shape[0] > 0 and (t.stride(0) % 8 or t.stride(1) % 8 or t.data_ptr() % 16):
        raise ValueError(f"{name} rows must be 16-byte aligned (strides multiple of 8, aligned base)")


def _ensure_token_major(t: torch.Tensor) -> torch.Tensor:
    """Returns ``t`` if the kernels can read it in place, else a contiguous copy."""
    if t.stride(2) == 1 and t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0 and t.data_ptr() % 16 == 0:
        return t
    return t.contiguous()


def validate_cu_seqlens(cu: torch.Tensor, total: int, name: str = "cu_seqlens") -> None:
    """Host-side checks on a CPU copy of cu_seqlens (the collator keeps one).

    Rejects what the device path would silently clamp: wrong dtype or rank,
    cu[0] != 0, decreasing offsets, cu[-1] != total.
    """
    if cu.dim() != 1 or cu.numel() < 1:
        raise ValueError(f"{name} must be a 1-D tensor of batch+1 offsets")
    if cu.dtype != torch.int32:
        raise ValueError(f"{name} must be int32, got {cu.dtype}")
    if cu.device.type != "cpu":
        return
    vals = cu.tolist()
    if vals[0] != 0:
        raise ValueError(f"{name}[0] must be 0, got {vals[0]}")
    for a, b in zip(vals, vals[1:]):
        if b < a:
            raise ValueError(f"{name} must be non-decreasing ({a} then {b})")
    if vals[-1] != total:
        raise ValueError(f"{name}[-1] ({vals[-1]}) must equal the number of packed tokens ({total})")


def _norm_device(device) -> torch.device:
    """``cuda`` -> ``cuda:<current index>`` (so that equal devices compare equal)."""
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        return torch.device("cuda", torch.cuda.current_device())
    return device


def _device_cu(cu: torch.Tensor, device: torch.device, total: int, name: str) -> torch.Tensor:
    validate_cu_seqlens(cu, total, name)
    device = _norm_device(device)
    if cu.device.type == "cpu":
        cu = cu.to(device, non_blocking=False)
    elif cu.device != device:
        raise ValueError(f"{name} is on {cu.device}, expected {device} or the CPU")
    return cu.contiguous()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check_common(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> tuple[int, int, int]:
    _check_token_major("q", q)
    hq, d = q.shape[1], q.shape[2]
    _check_token_major("k", k, dim=d)
    hkv = k.shape[1]
    _check_token_major("v", v, heads=hkv, dim=d)
    if v.shape[0] != k.shape[0]:
        raise ValueError(f"k and v token counts differ ({k.shape[0]} vs {v.shape[0]})")
    if d not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim {d} unsupported (supported: {SUPPORTED_HEAD_DIMS})")
    if hq % hkv:
        raise ValueError(f"num q heads ({hq}) must be a multiple of num kv heads ({hkv})")
    if not (q.device == k.device == v.device):
        raise ValueError("q, k, v must be on the same device")
    return hq, hkv, d


# --------------------------------------------------------------------------- plans
class AttnPlan:
    """The kernels' schedule of one packed batch (``siq_attn_build_plan``):
    per-sequence extents, the q-tile list of the forward / dQ kernels and the
    dK/dV work items, ordered by decreasing work.  It depends only on the
    sequences, the head counts and causality, so one plan serves the forward
    and backward of every layer of a packed batch (the reference forwards the
    same ``cu_seq_lens_*`` kwargs to each decoder layer,
    siq_vl/model/modeling.py:278-288).

    ``cu_q`` / ``cu_k`` are the plan's own device copies of the offsets it was
    built from (nothing else holds them, so they cannot change under it);
    ``src`` remembers the caller's tensors and their versions, so that handing
    the same unchanged tensors back with the plan needs no comparison."""

    __slots__ = ("buf", "batch", "total_q", "total_k", "hq", "hkv", "causal", "cu_q", "cu_k", "src", "__weakref__")

    def __init__(self, buf, batch, total_q, total_k, hq, hkv, causal, cu_q, cu_k, src=()):
        self.buf, self.batch, self.total_q, self.total_k = buf, batch, total_q, total_k
        self.hq, self.hkv, self.causal, self.cu_q, self.cu_k = hq, hkv, causal, cu_q, cu_k
        self.src = src

    def matches(self, batch: int, total_q: int, total_k: int, hq: int, hkv: int, causal: bool) -> bool:
        return (self.batch, self.total_q, self.total_k, self.hq // self.hkv, self.hkv, self.causal) == (
            batch, total_q, total_k, hq // hkv, hkv, bool(causal))

    def describes(self, cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor) -> bool:
        """True when the plan was built from these offsets: the plan's own
        copies, the unchanged tensors it was built from, or tensors holding
        the same values (compared on the device: one device-to-host read)."""
        for given, own, i in ((cu_seqlens_q, self.cu_q, 0), (cu_seqlens_k, self.cu_k, 1)):
            if given is own:
                continue
            if len(self.src) == 2:
                ref, ver = self.src[i]
                if ref() is given and given._version == ver:
                    continue
            if given.dim() != 1 or given.numel() != own.numel():
                return False
            if not torch.equal(given.to(device=own.device, dtype=torch.int32), own):
                return False
        return True

    def status(self) -> dict:
        """The plan header's status words (one device-to-host read; for tests
        and debugging): overflow bits of the scheduler, mismatch bits of the
        kernels that were handed this plan."""
        words = self.buf[:64].view(torch.int32).cpu().tolist()
        return {"magic": words[4], "status_q": words[10], "status_kv": words[11], "status_use": words[12]}


def _own_copy(src: torch.Tensor, dev_copy: torch.Tensor) -> torch.Tensor:
    """A device copy of offsets that no caller holds (``dev_copy`` itself when
    it was made from a host tensor, else a clone)."""
    return dev_copy if dev_copy is not src else dev_copy.clone()


def build_attn_plan(cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, total_q: int, total_k: int, hq: int,
                    hkv: int, causal: bool, device: torch.device | None = None) -> AttnPlan:
    """Builds a plan on the device (one small kernel, no host sync)."""
    device = _norm_device(device or (cu_seqlens_q.device if cu_seqlens_q.device.type == "cuda" else "cuda"))
    cu_q = _own_copy(cu_seqlens_q, _device_cu(cu_seqlens_q, device, total_q, "cu_seqlens_q"))
    if cu_seqlens_k is cu_seqlens_q:
        cu_k = cu_q
    else:
        cu_k = _own_copy(cu_seqlens_k, _device_cu(cu_seqlens_k, device, total_k, "cu_seqlens_k"))
    if cu_q.numel() != cu_k.numel():
        raise ValueError("cu_seqlens_q and cu_seqlens_k must describe the same number of sequences")
    if hq <= 0 or hkv <= 0 or hq % hkv:
        raise ValueError(f"num q heads ({hq}) must be a positive multiple of num kv heads ({hkv})")
    batch = cu_q.numel() - 1
    L = _lib.lib()
    nbytes = L.siq_attn_plan_bytes(batch, total_q, total_k)
    buf = torch.empty((max(nbytes, 256),), dtype=torch.uint8, device=device)
    if batch > 0:
        rc = L.siq_attn_build_plan(cu_q.data_ptr(), cu_k.data_ptr(), batch, total_q, total_k, hq, hkv,
                                   int(bool(causal)), buf.data_ptr(), buf.numel(), _stream(device))
        _lib.check(rc, "siq_attn_build_plan")
    src = tuple((weakref.ref(t), t._version) for t in (cu_seqlens_q, cu_seqlens_k))
    return AttnPlan(buf, batch, int(total_q), int(total_k), int(hq), int(hkv), bool(causal), cu_q, cu_k, src)


_PLAN_ATTR = "_siq_attn_plans"


def cached_attn_plan(cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, total_q: int, total_k: int, hq: int,
                     hkv: int, causal: bool, device: torch.device) -> AttnPlan:
    """The plan for these offsets, built on first use and kept on the
    ``cu_seqlens_q`` tensor object itself (so it lives exactly as long as
    that tensor); an in-place change of either offsets tensor (its
    ``_version``) or other totals / heads / causality build a new one."""
    device = _norm_device(device)
    key = (cu_seqlens_q._version, cu_seqlens_k._version, int(total_q), int(total_k), int(hq) // int(hkv), int(hkv),
           bool(causal), str(device))
    cache = getattr(cu_seqlens_q, _PLAN_ATTR, None)
    if cache is not None:
        hit = cache.get(key)
        if hit is not None and hit[0]() is cu_seqlens_k:
            return hit[1]
    plan = build_attn_plan(cu_seqlens_q, cu_seqlens_k, total_q, total_k, hq, hkv, causal, device)
    try:
        new = dict(cache) if cache is not None else {}
        if len(new) >= 4:
            new.clear()
        new[key] = (weakref.ref(cu_seqlens_k), plan)
        setattr(cu_seqlens_q, _PLAN_ATTR, new)
    except (AttributeError, TypeError, RuntimeError):  # tensors that refuse attributes are simply not cached
        pass
    return plan


def _resolve_plan(plan, cu_seqlens_q, cu_seqlens_k, total_q, total_k, hq, hkv, causal, device) -> AttnPlan:
    if plan is None:
        return cached_attn_plan(cu_seqlens_q, cu_seqlens_k, total_q, total_k, hq, hkv, causal, device)
    batch = cu_seqlens_q.numel() - 1
    if not plan.matches(batch, total_q, total_k, hq, hkv, causal) or plan.buf.device != _norm_device(device):
        raise ValueError("the attention plan was built for other sequences, heads or causality")
    if not plan.describes(cu_seqlens_q, cu_seqlens_k):
        raise ValueError("the attention plan was built for other sequences (cu_seqlens differ from the plan's)")
    return plan


# --------------------------------------------------------------------------- raw operators
def varlen_attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                    cu_seqlens_k: torch.Tensor, max_seqlen_q: int, max_seqlen_k: int, softmax_scale: float,
                    causal: bool, plan: AttnPlan | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns ``(out [total_q, hq, d] bf16, lse [hq, total_q] fp32, natural log)``.
    ``plan`` None: the cached plan of ``cu_seqlens_q`` (built on first use)."""
    hq, hkv, d = _check_common(q, k, v)
    total_q, total_k = q.shape[0], k.shape[0]
    pl = _resolve_plan(plan, cu_seqlens_q, cu_seqlens_k, total_q, total_k, hq, hkv, causal, q.device)
    out = torch.empty((total_q, hq, d), dtype=q.dtype, device=q.device)
    lse = torch.empty((hq, total_q), dtype=torch.float32, device=q.device)
    L = _lib.lib()
    strides = _lib.int64_array([q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                                out.stride(0), out.stride(1)])
    rc = L.siq_attn_varlen_fwd_plan(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                    pl.batch, total_q, total_k, hq, hkv, d, strides, float(softmax_scale),
                                    int(bool(causal)), pl.buf.data_ptr(), pl.buf.numel(), _stream(q.device))
    _lib.check(rc, "siq_attn_varlen_fwd_plan")
    return out, lse


# Backward used when a call does not choose (``deterministic=None``): True is
# the bitwise-reproducible backward (dQ in a kernel of its own), False the one
# that forms dQ in the dK/dV kernel and sums it with fp32 atomics.
DETERMINISTIC_DEFAULT = True

# flash-attention's ``deterministic=False`` (what transformers passes unless
# FLASH_ATTENTION_DETERMINISTIC=1) permits a non-deterministic backward; it
# does not ask for one.  On MI355X the deterministic backward is also the
# faster one (2.0-3.1x over the atomic-dQ backward at the BASELINE shapes), so
# ``flash_attn_varlen_func(..., deterministic=False)`` takes it too unless this
# is set.  ``varlen_attn_bwd(deterministic=False)`` and the C ABI's
# deterministic = 0 always run the atomic-dQ backward.
ATOMIC_BACKWARD_ON_FALSE = False


def varlen_attn_bwd(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                    lse: torch.Tensor, cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, max_seqlen_q: int,
                    max_seqlen_k: int, softmax_scale: float, causal: bool, plan: AttnPlan | None = None,
                    deterministic: bool | None = None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns ``(dq, dk, dv)``: bitwise reproducible when ``deterministic``
    (None: ``DETERMINISTIC_DEFAULT``), else dQ summed with fp32 atomics (its
    bits may vary from run to run; dk and dv never do)."""
    det = DETERMINISTIC_DEFAULT if deterministic is None else bool(deterministic)
    hq, hkv, d = _check_common(q, k, v)
    total_q, total_k = q.shape[0], k.shape[0]
    _check_token_major("out", out, heads=hq, dim=d)
    _check_token_major("dout", dout, heads=hq, dim=d)
    if out.shape[0] != total_q or dout.shape[0] != total_q:
        raise ValueError("out / dout must have total_q rows")
    if lse.shape != (hq, total_q) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError(f"lse must be a contiguous fp32 [{hq}, {total_q}] tensor")
    pl = _resolve_plan(plan, cu_seqlens_q, cu_seqlens_k, total_q, total_k, hq, hkv, causal, q.device)
    dq = torch.empty((total_q, hq, d), dtype=q.dtype, device=q.device)
    dk = torch.empty((total_k, hkv, d), dtype=q.dtype, device=q.device)
    dv = torch.empty((total_k, hkv, d), dtype=q.dtype, device=q.device)
    L = _lib.lib()
    ws_bytes = L.siq_attn_bwd_plan_workspace_bytes(pl.batch, total_q, total_k, hq, hkv, d, int(det))
    ws = torch.empty((max(ws_bytes, 16),), dtype=torch.uint8, device=q.device)
    strides = _lib.int64_array([q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                                out.stride(0), out.stride(1), dout.stride(0), dout.stride(1), dq.stride(0),
                                dq.stride(1), dk.stride(0), dk.stride(1), dv.stride(0), dv.stride(1)])
    rc = L.siq_attn_varlen_bwd_plan(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                    dout.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), pl.batch, total_q,
                                    total_k, hq, hkv, d, strides, float(softmax_scale), int(bool(causal)), int(det),
                                    pl.buf.data_ptr(), pl.buf.numel(), ws.data_ptr(), ws.numel(), _stream(q.device))
    _lib.check(rc, "siq_attn_varlen_bwd_plan")
    return dq, dk, dv


class _VarlenAttnFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cu_q, cu_k, max_q, max_k, scale, causal, deterministic=None):
        q, k, v = (_ensure_token_major(t) for t in (q, k, v))
        hq, hkv = q.shape[1], k.shape[1]
        plan = cached_attn_plan(cu_q, cu_k, q.shape[0], k.shape[0], hq, hkv, causal, q.device)
        out, lse = varlen_attn_fwd(q, k, v, cu_q, cu_k, max_q, max_k, scale, causal, plan=plan)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.plan = plan
        ctx.args = (max_q, max_k, scale, causal, deterministic)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        max_q, max_k, scale, causal, deterministic = ctx.args
        plan = ctx.plan
        dout = _ensure_token_major(dout)
        dq, dk, dv = varlen_attn_bwd(dout, q, k, v, out, lse, plan.cu_q, plan.cu_k, max_q, max_k, scale, causal,
                                     plan=plan, deterministic=deterministic)
        return dq, dk, dv, None, None, None, None, None, None, None


def _check_rope_rows(cos: torch.Tensor, sin: torch.Tensor, total_q: int, d: int) -> None:
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dim() != 2 or t.shape[0] != total_q or t.shape[1] != d:
            raise ValueError(f"{name} must be [total_q, head_dim] = [{total_q}, {d}], got {tuple(t.shape)}")
        if t.dtype != torch.bfloat16 or t.device.type != "cuda":
            raise ValueError(f"{name} must be a bf16 GPU tensor")
        if t.stride(1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16:
            raise ValueError(f"{name} rows must be contiguous and 16-byte aligned")


def varlen_attn_rope_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                         cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, max_seqlen_q: int,
                         max_seqlen_k: int, softmax_scale: float, causal: bool,
                         plan: AttnPlan | None = None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Attention with the decoder's rotary embedding of q fused in
    (``siq_attn_rope_fwd_plan``): ``q`` is the query BEFORE rotation, ``k`` the
    key after it, ``cos`` / ``sin`` ``[total_q, d]`` rows per token.  Returns
    ``(out, lse, q_embed)``; ``q_embed`` (the rotated q, bitwise
    ``rope_fwd``'s) is what the backward reads."""
    hq, hkv, d = _check_common(q, k, v)
    total_q, total_k = q.shape[0], k.shape[0]
    _check_rope_rows(cos, sin, total_q, d)
    pl = _resolve_plan(plan, cu_seqlens_q, cu_seqlens_k, total_q, total_k, hq, hkv, causal, q.device)
    out = torch.empty((total_q, hq, d), dtype=q.dtype, device=q.device)
    lse = torch.empty((hq, total_q), dtype=torch.float32, device=q.device)
    qe = torch.empty((total_q, hq, d), dtype=q.dtype, device=q.device)
    strides = _lib.int64_array([q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                                out.stride(0), out.stride(1), qe.stride(0), qe.stride(1), cos.stride(0),
                                sin.stride(0)])
    rc = _lib.lib().siq_attn_rope_fwd_plan(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                           qe.data_ptr(), cos.data_ptr(), sin.data_ptr(), pl.batch, total_q, total_k,
                                           hq, hkv, d, strides, float(softmax_scale), int(bool(causal)),
                                           pl.buf.data_ptr(), pl.buf.numel(), _stream(q.device))
    _lib.check(rc, "siq_attn_rope_fwd_plan")
    return out, lse, qe


def varlen_attn_rope_bwd(dout: torch.Tensor, q_embed: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         out: torch.Tensor, lse: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                         cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, max_seqlen_q: int,
                         max_seqlen_k: int, softmax_scale: float, causal: bool,
                         plan: AttnPlan | None = None) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Backward of ``varlen_attn_rope_fwd`` (``siq_attn_rope_bwd_plan``):
    ``(dq, dk, dv)`` with dq for the q BEFORE rotation (bitwise ``rope_bwd``
    of the unfused dq), dk for the rotated k."""
    hq, hkv, d = _check_common(q_embed, k, v)
    total_q, total_k = q_embed.shape[0], k.shape[0]
    _check_token_major("out", out, heads=hq, dim=d)
    _check_token_major("dout", dout, heads=hq, dim=d)
    if out.shape[0] != total_q or dout.shape[0] != total_q:
        raise ValueError("out / dout must have total_q rows")
    if lse.shape != (hq, total_q) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError(f"lse must be a contiguous fp32 [{hq}, {total_q}] tensor")
    _check_rope_rows(cos, sin, total_q, d)
    pl = _resolve_plan(plan, cu_seqlens_q, cu_seqlens_k, total_q, total_k, hq, hkv, causal, q_embed.device)
    dq = torch.empty((total_q, hq, d), dtype=q_embed.dtype, device=q_embed.device)
    dk = torch.empty((total_k, hkv, d), dtype=q_embed.dtype, device=q_embed.device)
    dv = torch.empty((total_k, hkv, d), dtype=q_embed.dtype, device=q_embed.device)
    L = _lib.lib()
    ws_bytes = L.siq_attn_bwd_plan_workspace_bytes(pl.batch, total_q, total_k, hq, hkv, d, 1)
    ws = torch.empty((max(ws_bytes, 16),), dtype=torch.uint8, device=q_embed.device)
    q = q_embed
    strides = _lib.int64_array([q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                                out.stride(0), out.stride(1), dout.stride(0), dout.stride(1), dq.stride(0),
                                dq.stride(1), dk.stride(0), dk.stride(1), dv.stride(0), dv.stride(1), cos.stride(0),
                                sin.stride(0)])
    rc = L.siq_attn_rope_bwd_plan(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                  dout.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), cos.data_ptr(),
                                  sin.data_ptr(), pl.batch, total_q, total_k, hq, hkv, d, strides,
                                  float(softmax_scale), int(bool(causal)), pl.buf.data_ptr(), pl.buf.numel(),
                                  ws.data_ptr(), ws.numel(), _stream(q.device))
    _lib.check(rc, "siq_attn_rope_bwd_plan")
    return dq, dk, dv


class _VarlenRopeAttnFn(torch.autograd.Function):
    """apply_rotary_pos_emb(q, k) followed by attention, as one autograd node.

    Forward: one RoPE pass over q and k (its q_embed is what the backward's
    dK/dV kernel stages from memory anyway), then the attention forward.
    Backward: the rotation's backward of dq is fused into the dQ kernel's
    store epilogue (dq of the q before rotation leaves the kernel directly;
    dq_embed never reaches memory) and k's goes through a k-only RoPE pass.
    Measured on MI355X at the config-2 shape this split beats both the
    unfused pair and rotating q inside the attention forward as well
    (``varlen_attn_rope_fwd``), whose extra q_embed stores and rotation sit
    on every workgroup's critical path."""

    @staticmethod
    def forward(ctx, q, k, v, cos, sin, cu_q, cu_k, max_q, max_k, scale, causal):
        from . import rope as _rope

        cos, sin = cos.contiguous(), sin.contiguous()
        qe, ke = _rope.rope_fwd(q[None], k[None], cos[None], sin[None])
        qe, ke = qe[0], ke[0]
        v = _ensure_token_major(v)
        hq, hkv = qe.shape[1], ke.shape[1]
        plan = cached_attn_plan(cu_q, cu_k, qe.shape[0], ke.shape[0], hq, hkv, causal, qe.device)
        out, lse = varlen_attn_fwd(qe, ke, v, cu_q, cu_k, max_q, max_k, scale, causal, plan=plan)
        ctx.save_for_backward(qe, ke, v, out, lse, cos, sin)
        ctx.plan = plan
        ctx.args = (max_q, max_k, scale, causal)
        return out

    @staticmethod
    def backward(ctx, dout):
        from . import rope as _rope

        qe, ke, v, out, lse, cos, sin = ctx.saved_tensors
        max_q, max_k, scale, causal = ctx.args
        plan = ctx.plan
        dq, dke, dv = varlen_attn_rope_bwd(_ensure_token_major(dout), qe, ke, v, out, lse, cos, sin, plan.cu_q,
                                           plan.cu_k, max_q, max_k, scale, causal, plan=plan)
        dk = _rope.rotate_k_backward(dke, cos, sin)
        return dq, dk, dv, None, None, None, None, None, None, None, None


class _VarlenRopeF32Attn(torch.autograd.Function):
    """The same pair with fp32 cos / sin rows (bf16 autocast over fp32 master
    weights): one RoPE pass writes the bf16 q_embed / k_embed that the
    reference's promoted fp32 rotation gives after the attention's cast
    (``siq_rope_fwd_ex``), the attention runs on them, and one RoPE pass takes
    the attention's dq_embed / dk_embed back through the rotation
    (``siq_rope_bwd_ex``), as the reference's autograd does through the cast
    and the promoted ops.  Bitwise the unfused path under autocast."""

    @staticmethod
    def forward(ctx, q, k, v, cos, sin, cu_q, cu_k, max_q, max_k, scale, causal):
        from . import rope as _rope

        cos, sin = cos.contiguous(), sin.contiguous()
        qe, ke = _rope.rope_fwd(q[None], k[None], cos[None], sin[None])
        qe, ke = qe[0], ke[0]
        v = _ensure_token_major(v)
        plan = cached_attn_plan(cu_q, cu_k, qe.shape[0], ke.shape[0], qe.shape[1], ke.shape[1], causal, qe.device)
        out, lse = varlen_attn_fwd(qe, ke, v, cu_q, cu_k, max_q, max_k, scale, causal, plan=plan)
        ctx.save_for_backward(qe, ke, v, out, lse, cos, sin)
        ctx.plan = plan
        ctx.args = (max_q, max_k, scale, causal)
        return out

    @staticmethod
    def backward(ctx, dout):
        from . import rope as _rope

        qe, ke, v, out, lse, cos, sin = ctx.saved_tensors
        max_q, max_k, scale, causal = ctx.args
        plan = ctx.plan
        dqe, dke, dv = varlen_attn_bwd(_ensure_token_major(dout), qe, ke, v, out, lse, plan.cu_q, plan.cu_k, max_q,
                                       max_k, scale, causal, plan=plan)
        dq, dk = _rope.rope_bwd(dqe[None], dke[None], cos[None], sin[None])
        return dq[0], dk[0], dv, None, None, None, None, None, None, None, None


def flash_attn_varlen_rope_func(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                                sin: torch.Tensor, cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
                                max_seqlen_q: int, max_seqlen_k: int, softmax_scale: float | None = None,
                                causal: bool = False) -> torch.Tensor:
    """``flash_attn_varlen_func(*apply_rotary_pos_emb(q, k, cos, sin), v)`` as
    one op: ``q [total, hq, d]`` and ``k [total, hkv, d]`` BEFORE rotation
    (self-attention: q and k rows are the same tokens), ``cos`` / ``sin
    [total, d]`` the rows of each packed token, bf16 or fp32 (the latter under
    bf16 autocast over fp32 master weights, where the reference rotates in
    fp32 and the attention casts the result to bf16).  Output and gradients
    are bitwise those of the two separate ops."""
    if cos.requires_grad or sin.requires_grad:
        raise ValueError("gradients with respect to cos / sin are not supported")
    if q.shape[0] != k.shape[0]:
        raise ValueError("the fused rotary attention needs q and k rows of the same tokens")
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    fn = _VarlenRopeF32Attn if cos.dtype == torch.float32 else _VarlenRopeAttnFn
    return fn.apply(q, k, v, cos, sin, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q), int(max_seqlen_k),
                    float(softmax_scale), bool(causal))


def flash_attn_varlen_func(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                           cu_seqlens_k: torch.Tensor, max_seqlen_q: int, max_seqlen_k: int, dropout_p: float = 0.0,
                           softmax_scale: float | None = None, causal: bool = False,
                           window_size: tuple[int, int] = (-1, -1), softcap: float = 0.0,
                           alibi_slopes: torch.Tensor | None = None, deterministic: bool | None = None,
                           return_attn_probs: bool = False, **kwargs: Any) -> torch.Tensor:
    """Varlen attention with the flash-attention varlen call convention.

    ``q [total_q, hq, d]``, ``k/v [total_k, hkv, d]`` (bf16); returns ``[total_q, hq, d]``.
    ``deterministic`` picks the backward (None: ``DETERMINISTIC_DEFAULT``;
    False: the deterministic one as well, the faster here, unless
    ``ATOMIC_BACKWARD_ON_FALSE``).  Features outside the reference path (dropout, sliding window, softcap,
    ALiBi, returning probabilities) are rejected, not approximated.
    """
    if dropout_p:
        raise ValueError("siq_varlen attention does not implement dropout (the reference trains with dropout 0)")
    if tuple(window_size) != (-1, -1):
        raise ValueError("sliding-window attention is not supported")
    if softcap:
        raise ValueError("logit softcapping is not supported")
    if alibi_slopes is not None:
        raise ValueError("ALiBi is not supported")
    if return_attn_probs:
        raise ValueError("attention probabilities are never materialised")
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    det = None if deterministic is None else (bool(deterministic) or not ATOMIC_BACKWARD_ON_FALSE)
    return _VarlenAttnFn.apply(q, k, v, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q), int(max_seqlen_k),
                               float(softmax_scale), bool(causal), det)


# --------------------------------------------------------------------------- transformers plug-in
_DERIVED_ATTR = "_siq_attn_derived"


def _cached_derived(t: torch.Tensor, tag: str, make):
    """``make()``'s result kept on tensor ``t`` (keyed by ``tag`` and ``t``'s
    version): the offsets derived from one batch's position_ids or padding
    mask are computed -- with their one device-to-host read -- by the first
    decoder layer and reused by the others, which receive the same tensor."""
    key = (tag, t._version)
    cache = getattr(t, _DERIVED_ATTR, None)
    if cache is not None and key in cache:
        return cache[key]
    val = make()
    try:
        setattr(t, _DERIVED_ATTR, {key: val})
    except (AttributeError, TypeError, RuntimeError):
        pass
    return val


def _cu_from_position_ids(position_ids: torch.Tensor) -> tuple[torch.Tensor, int]:
    """Packed position_ids restart at 0 for each sequence (transformers
    modeling_flash_attention_utils.py:458-495): offsets are where they do.
    Computed once per position_ids tensor (one host read of the longest
    sequence), then reused."""

    def make():
        pos = position_ids.reshape(-1)
        starts = torch.nonzero(pos == 0, as_tuple=False).reshape(-1).to(torch.int32)
        if starts.numel() == 0 or int(starts[0]) != 0:
            starts = torch.cat([torch.zeros(1, dtype=torch.int32, device=pos.device), starts])
        total = torch.tensor([pos.numel()], dtype=torch.int32, device=pos.device)
        cu = torch.cat([starts, total])
        max_len = int((cu[1:] - cu[:-1]).max().item())
        return cu, max_len

    return _cached_derived(position_ids, "pos", make)


def _unpad_from_mask(mask2d: torch.Tensor, s_k: int) -> tuple[torch.Tensor, torch.Tensor, int]:
    """(cu_seqlens, kept token indices, longest row) of a 2-D padding mask,
    computed once per mask tensor."""

    def make():
        mask = mask2d[:, -s_k:].to(torch.bool)
        seqlens = mask.sum(dim=-1, dtype=torch.int32)
        cu = torch.nn.functional.pad(torch.cumsum(seqlens, 0, dtype=torch.int32), (1, 0))
        idx = torch.nonzero(mask.reshape(-1), as_tuple=False).reshape(-1)
        return cu, idx, int(seqlens.max().item())

    return _cached_derived(mask2d, f"mask{s_k}", make)


def _attend_packed(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attention_mask: torch.Tensor | None,
                   is_causal: bool, scaling: float, kwargs: dict, rope=None) -> torch.Tensor:
    """q ``[B, S_q, Hq, D]``, k / v ``[B, S_k, Hkv, D]`` (bf16 token-major views)
    -> out ``[B, S_q, Hq, D]``.  Packing is read, in order, from
    ``cu_seq_lens_q/k`` + ``max_length_q/k`` kwargs, from a 2-D padding
    ``attention_mask`` (rows are unpadded), from restarting ``position_ids``
    (B == 1); otherwise every batch row is one sequence.  ``rope`` = (cos, sin)
    ``[B or 1, S_q, D]``: q and k arrive before rotation and are rotated by
    the attention op (``flash_attn_varlen_rope_func``)."""
    bsz, s_q, hq, d = q.shape
    s_k, hkv = k.shape[1], k.shape[2]
    cos_t = sin_t = None
    if rope is not None:
        cos, sin = rope
        cos_t = cos.expand(bsz, s_q, d).reshape(bsz * s_q, d).contiguous()
        sin_t = sin.expand(bsz, s_q, d).reshape(bsz * s_q, d).contiguous()

    def attend(qf, kf, vf, cu_q, cu_k, mq, mk, cs=None, sn=None):
        if cs is None:
            return flash_attn_varlen_func(qf, kf, vf, cu_q, cu_k, mq, mk, softmax_scale=scaling, causal=is_causal)
        return flash_attn_varlen_rope_func(qf, kf, vf, cs, sn, cu_q, cu_k, mq, mk, softmax_scale=scaling,
                                           causal=is_causal)

    cu_q = kwargs.get("cu_seq_lens_q")
    cu_k = kwargs.get("cu_seq_lens_k")
    max_q = kwargs.get("max_length_q")
    max_k = kwargs.get("max_length_k")
    position_ids = kwargs.get("position_ids")
    if cu_q is not None and cu_k is not None and max_q is not None and max_k is not None:
        out = attend(q.reshape(-1, hq, d), k.reshape(-1, hkv, d), v.reshape(-1, hkv, d), cu_q.to(torch.int32),
                     cu_k.to(torch.int32), int(max_q), int(max_k), cos_t, sin_t)
        return out.reshape(bsz, s_q, hq, d)
    if attention_mask is not None and attention_mask.dim() == 2:
        cu, idx, maxlen = _unpad_from_mask(attention_mask, s_k)
        if s_q != s_k:
            raise ValueError("padded (unpacked) inputs need equal query and key lengths")
        qu = q.reshape(-1, hq, d).index_select(0, idx)
        ku = k.reshape(-1, hkv, d).index_select(0, idx)
        vu = v.reshape(-1, hkv, d).index_select(0, idx)
        cu_cs = None if cos_t is None else cos_t.index_select(0, idx)
        cu_sn = None if sin_t is None else sin_t.index_select(0, idx)
        ou = attend(qu, ku, vu, cu, cu, maxlen, maxlen, cu_cs, cu_sn)
        out = torch.zeros((bsz * s_q, hq, d), dtype=ou.dtype, device=ou.device)
        return out.index_copy(0, idx, ou).reshape(bsz, s_q, hq, d)
    if position_ids is not None and bsz == 1 and s_q == s_k:
        cu, maxlen = _cu_from_position_ids(position_ids)
        out = attend(q.reshape(-1, hq, d), k.reshape(-1, hkv, d), v.reshape(-1, hkv, d), cu, cu, maxlen, maxlen,
                     cos_t, sin_t)
        return out.reshape(bsz, s_q, hq, d)
    if attention_mask is not None:
        raise ValueError("siq_varlen expects a 2-D padding mask or None (register its mask interface)")
    cu_q = torch.arange(0, (bsz + 1) * s_q, s_q, dtype=torch.int32, device=q.device)
    cu_k = cu_q if s_k == s_q else torch.arange(0, (bsz + 1) * s_k, s_k, dtype=torch.int32, device=q.device)
    out = attend(q.reshape(-1, hq, d), k.reshape(-1, hkv, d), v.reshape(-1, hkv, d), cu_q, cu_k, s_q, s_k, cos_t,
                 sin_t)
    return out.reshape(bsz, s_q, hq, d)


def siq_varlen_attention_forward(module: torch.nn.Module, query: torch.Tensor, key: torch.Tensor,
                                 value: torch.Tensor, attention_mask: torch.Tensor | None, dropout: float = 0.0,
                                 scaling: float | None = None, sliding_window: int | None = None,
                                 softcap: float | None = None, is_causal: bool | None = None,
                                 **kwargs: Any) -> tuple[torch.Tensor, None]:
    """``AttentionInterface`` entry: ``query [B, Hq, S, D]``, ``key/value [B, Hkv, S, D]``
    -> ``(out [B, S, Hq, D] contiguous, None)``.

    Packing is read, in order, from ``cu_seq_lens_q/k`` + ``max_length_q/k``
    kwargs, from a 2-D padding ``attention_mask`` (rows are unpadded), or from
    restarting ``position_ids`` (B == 1); otherwise every batch row is one
    sequence.  Unknown kwargs (e.g. the collator's raw ``questions``) are
    ignored.
    """
    if dropout:
        raise ValueError("siq_varlen attention does not implement dropout")
    if softcap:
        raise ValueError("logit softcapping is not supported")
    if sliding_window is not None:
        raise ValueError("sliding-window attention is not supported")
    if is_causal is None:
        is_causal = bool(getattr(module, "is_causal", False))
    d = query.shape[-1]
    if scaling is None:
        scaling = d**-0.5
    target = torch.bfloat16
    q = query.transpose(1, 2).to(target)
    k = key.transpose(1, 2).to(target)
    v = value.transpose(1, 2).to(target)
    out = _attend_packed(q, k, v, attention_mask, is_causal, scaling, kwargs)
    return out.to(_output_dtype(query)).contiguous(), None


def _output_dtype(query: torch.Tensor) -> torch.dtype:
    """The dtype the stock backends hand back: under bf16 autocast an fp32
    query (the RoPE's output over fp32 master weights) gives bf16, as
    ``F.scaled_dot_product_attention`` (an autocast lower-precision op) and
    flash-attention's ``get_target_dtype`` (transformers
    integrations/flash_attention.py:12-23) do, so no fp32 copy of the output
    is made only to be cast back by ``o_proj``; otherwise the query's dtype."""
    dev = query.device.type
    if query.dtype == torch.float32 and torch.is_autocast_enabled(dev) and \
            torch.get_autocast_dtype(dev) == torch.bfloat16:
        return torch.bfloat16
    return query.dtype


def register(name: str = ATTN_IMPLEMENTATION) -> str:
    """Registers the kernels as a transformers attention backend.

    After this, ``from_pretrained(..., attn_implementation="siq_varlen")`` (the
    reference's model builders at siq_vl/model/modeling.py:326-327,363) or
    ``config._attn_implementation = "siq_varlen"`` routes every Qwen2 / SigLIP
    attention call here.  The mask interface is the flash-attention one: the
    function receives ``None`` or a 2-D padding mask, never a 4-D bias.
    """
    from transformers import AttentionInterface

    AttentionInterface.register(name, siq_varlen_attention_forward)
    try:
        from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, flash_attention_mask

        ALL_MASK_ATTENTION_FUNCTIONS.register(name, flash_attention_mask)
    except ImportError:  # older transformers: masks are resolved by name
        pass
    return name


def attention_flops(cu_seqlens: torch.Tensor, hq: int, d: int, causal: bool, backward: bool = True) -> float:
    """Algorithmic FLOPs: 4*D*P*Hq forward (+ 8*D*P*Hq backward), P = allowed
    (q, k) pairs of the realised cu_seqlens; recompute is not counted."""
    lens = (cu_seqlens[1:] - cu_seqlens[:-1]).to(torch.float64).cpu()
    pairs = float((lens * (lens + 1) / 2).sum()) if causal else float((lens * lens).sum())
    return (12.0 if backward else 4.0) * d * pairs * hq


__all__ = [
    "ATTN_IMPLEMENTATION",
    "flash_attn_varlen_rope_func",
    "varlen_attn_rope_bwd",
    "varlen_attn_rope_fwd",
    "AttnPlan",
    "build_attn_plan",
    "cached_attn_plan",
    "attention_flops",
    "flash_attn_varlen_func",
    "register",
    "siq_varlen_attention_forward",
    "validate_cu_seqlens",
    "varlen_attn_bwd",
    "varlen_attn_fwd",
]
