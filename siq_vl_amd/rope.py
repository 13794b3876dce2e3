"""Fused rotary position embedding of q and k on MI355X: host side.

Replaces, in the reference's Qwen2 decoder, ``apply_rotary_pos_emb``
(transformers models/qwen2/modeling_qwen2.py:105-135 with ``rotate_half``;
called from ``Qwen2Attention.forward`` at :206-211) by one launch of
``siq_rope_fwd`` over q and k, and its autograd backward by one launch of
``siq_rope_bwd``.  Results are bitwise those of the reference's bf16 torch ops
``q * cos + rotate_half(q) * sin`` (each op rounds to bf16; the kernel repeats
those roundings), forward and backward.

Layers:

* ``rope_fwd`` / ``rope_bwd`` -- raw operators on ``[batch, seqlen, heads, D]``
  views (any strides with a contiguous ``D``).
* ``apply_rotary_pos_emb`` -- the reference's signature (``q, k, cos, sin,
  position_ids=None, unsqueeze_dim=1``), autograd-aware; bf16 CUDA inputs run
  the HIP kernels, anything else (fp32 evaluation, CPU generation) takes the
  original transformers function.
* ``enable_fused_rope()`` -- installs it as
  ``transformers.models.qwen2.modeling_qwen2.apply_rotary_pos_emb``, the name
  ``Qwen2Attention.forward`` looks up at call time.
* ``enable_fused_rope_attention(model)`` -- goes one step further on a model
  using the ``siq_varlen`` attention backend: rotation and attention become
  one op (``flash_attn_varlen_rope_func``) whose backward rotates dq inside
  the dQ kernel, leaving a k-only rotation pass; bitwise the same results.
"""

from __future__ import annotations

import torch

from . import _lib

_ORIGINAL = None  # transformers' apply_rotary_pos_emb, once enable_fused_rope() has run


def _usable(t: torch.Tensor, rank: int) -> bool:
    if t.dim() != rank or t.stride(-1) != 1 or t.data_ptr() % 16:
        return False
    return all(s % 8 == 0 and s >= 0 for s in t.stride()[:-1])


def _bshd(t: torch.Tensor, unsqueeze_dim: int) -> torch.Tensor:
    """[batch, seqlen, heads, D] view of a q/k tensor laid out as apply_rotary_pos_emb receives it."""
    if t.dim() != 4:
        raise ValueError(f"q / k must be 4-D, got shape {tuple(t.shape)}")
    if unsqueeze_dim == 1:
        return t.transpose(1, 2)  # [B, H, S, D] -> [B, S, H, D]
    if unsqueeze_dim == 2:
        return t
    raise ValueError(f"unsqueeze_dim must be 1 ([B, H, S, D]) or 2 ([B, S, H, D]), got {unsqueeze_dim}")


def _prep(t: torch.Tensor, rank: int) -> torch.Tensor:
    return t if _usable(t, rank) else t.contiguous()


_CS_DTYPE = {torch.bfloat16: 0, torch.float32: 1}  # SIQ_DTYPE_BF16 / SIQ_DTYPE_FP32


def _launch(fn_name: str, x0, x1, cos, sin, y0, y1) -> None:
    b, s, hq, d = x0.shape
    hkv = x1.shape[2]
    strides = [*x0.stride()[:3], *x1.stride()[:3], *cos.stride()[:2], *sin.stride()[:2], *y0.stride()[:3],
               *y1.stride()[:3]]
    stream = torch.cuda.current_stream(x0.device).cuda_stream
    rc = getattr(_lib.lib(), fn_name + "_ex")(x0.data_ptr(), x1.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                              y0.data_ptr(), y1.data_ptr(), b, s, hq, hkv, d,
                                              _lib.int64_array(strides), _CS_DTYPE[cos.dtype], stream)
    _lib.check(rc, fn_name)


def _check(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> None:
    """q / k bf16; cos / sin bf16, or both fp32 (bf16 autocast over fp32
    master weights: the outputs are then the bf16 rounding of torch's
    promoted fp32 result)."""
    for name, t in (("q", q), ("k", k), ("cos", cos), ("sin", sin)):
        ok = t.dtype == torch.bfloat16 or (name in ("cos", "sin") and t.dtype == torch.float32)
        if not ok:
            raise ValueError(f"{name} must be bfloat16{' or float32' if name in ('cos', 'sin') else ''}, "
                             f"got {t.dtype}")
        if t.device.type != "cuda":
            raise ValueError(f"{name} must live on the GPU, got {t.device}")
    if cos.dtype != sin.dtype:
        raise ValueError(f"cos and sin must have one dtype, got {cos.dtype} and {sin.dtype}")
    b, s, _, d = q.shape
    if k.shape[0] != b or k.shape[1] != s or k.shape[3] != d:
        raise ValueError(f"k {tuple(k.shape)} does not match q {tuple(q.shape)} in batch / seqlen / head_dim")
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dim() != 3 or t.shape[1] != s or t.shape[2] != d or t.shape[0] not in (1, b):
            raise ValueError(f"{name} must be [batch or 1, seqlen, head_dim] = [{b}, {s}, {d}], got {tuple(t.shape)}")


def _expand_cs(t: torch.Tensor, b: int) -> torch.Tensor:
    return t.expand(b, -1, -1) if t.shape[0] != b else t


def rope_fwd(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """Raw forward on ``[B, S, H, D]`` views; returns ``(q_embed, k_embed)``
    (bf16) laid out like q and k.  With fp32 cos / sin: the bf16 rounding of
    the fp32 result torch's promotion gives (``siq_rope_fwd_ex``)."""
    _check(q, k, cos, sin)
    q, k = _prep(q, 4), _prep(k, 4)
    cos, sin = _prep(_expand_cs(cos, q.shape[0]), 3), _prep(_expand_cs(sin, q.shape[0]), 3)
    qe, ke = torch.empty_like(q), torch.empty_like(k)
    if q.numel() and k.numel():
        _launch("siq_rope_fwd", q, k, cos, sin, qe, ke)
    return qe, ke


def rope_bwd(dq_embed: torch.Tensor, dk_embed: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """Raw backward on ``[B, S, H, D]`` views; returns ``(dq, dk)``."""
    _check(dq_embed, dk_embed, cos, sin)
    g0, g1 = _prep(dq_embed, 4), _prep(dk_embed, 4)
    cos, sin = _prep(_expand_cs(cos, g0.shape[0]), 3), _prep(_expand_cs(sin, g0.shape[0]), 3)
    dq, dk = torch.empty_like(g0), torch.empty_like(g1)
    if g0.numel() and g1.numel():
        _launch("siq_rope_bwd", g0, g1, cos, sin, dq, dk)
    return dq, dk


class _Rope(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, cos, sin, unsqueeze_dim):
        if cos.requires_grad or sin.requires_grad:
            raise ValueError("gradients with respect to cos / sin are not supported")
        qe, ke = rope_fwd(_bshd(q, unsqueeze_dim), _bshd(k, unsqueeze_dim), cos, sin)
        ctx.save_for_backward(cos, sin)
        ctx.unsqueeze_dim = unsqueeze_dim
        return _bshd(qe, unsqueeze_dim), _bshd(ke, unsqueeze_dim)

    @staticmethod
    def backward(ctx, dqe, dke):
        cos, sin = ctx.saved_tensors
        u = ctx.unsqueeze_dim
        dq, dk = rope_bwd(_bshd(dqe, u), _bshd(dke, u), cos, sin)
        return _bshd(dq, u), _bshd(dk, u), None, None, None


def apply_rotary_pos_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, position_ids=None,
                         unsqueeze_dim: int = 1):
    """Signature of transformers' ``apply_rotary_pos_emb`` (``position_ids`` is unused there too)."""
    del position_ids
    if all(t.is_cuda and t.dtype == torch.bfloat16 for t in (q, k, cos, sin)):
        return _Rope.apply(q, k, cos, sin, unsqueeze_dim)
    if _ORIGINAL is None:
        raise ValueError("the fused RoPE takes bf16 CUDA tensors (enable_fused_rope() keeps the original for others)")
    return _ORIGINAL(q, k, cos, sin, unsqueeze_dim=unsqueeze_dim)


def enable_fused_rope() -> None:
    """Makes every Qwen2 attention layer call the fused RoPE (idempotent)."""
    global _ORIGINAL
    from transformers.models.qwen2 import modeling_qwen2 as m

    if m.apply_rotary_pos_emb is apply_rotary_pos_emb:
        return
    _ORIGINAL = m.apply_rotary_pos_emb
    m.apply_rotary_pos_emb = apply_rotary_pos_emb


def disable_fused_rope() -> None:
    """Restores transformers' own apply_rotary_pos_emb."""
    global _ORIGINAL
    from transformers.models.qwen2 import modeling_qwen2 as m

    if _ORIGINAL is not None and m.apply_rotary_pos_emb is apply_rotary_pos_emb:
        m.apply_rotary_pos_emb = _ORIGINAL
    _ORIGINAL = None


# --------------------------------------------------------------------------- rotation fused into attention
def _launch_k(fn_name: str, x1, cos, sin, y1) -> None:
    """k-only pass (hq = 0): q and its output are not touched."""
    b, s, hkv, d = x1.shape
    strides = [0, 0, 0, *x1.stride()[:3], *cos.stride()[:2], *sin.stride()[:2], 0, 0, 0, *y1.stride()[:3]]
    stream = torch.cuda.current_stream(x1.device).cuda_stream
    rc = getattr(_lib.lib(), fn_name + "_ex")(None, x1.data_ptr(), cos.data_ptr(), sin.data_ptr(), None,
                                              y1.data_ptr(), b, s, 0, hkv, d, _lib.int64_array(strides),
                                              _CS_DTYPE[cos.dtype], stream)
    _lib.check(rc, fn_name)


def _k_only(fn_name: str, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    _check(k, k, cos, sin)
    k = _prep(k, 4)
    cos, sin = _prep(_expand_cs(cos, k.shape[0]), 3), _prep(_expand_cs(sin, k.shape[0]), 3)
    out = torch.empty_like(k)
    if k.numel():
        _launch_k(fn_name, k, cos, sin, out)
    return out


class _RopeK(torch.autograd.Function):
    @staticmethod
    def forward(ctx, k, cos, sin):
        ctx.save_for_backward(cos, sin)
        return _k_only("siq_rope_fwd", k, cos, sin)

    @staticmethod
    def backward(ctx, dke):
        cos, sin = ctx.saved_tensors
        return _k_only("siq_rope_bwd", dke, cos, sin), None, None


def rotate_k_backward(dk_embed: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """The rotation's backward for k alone on token-major ``[T, Hkv, D]`` with
    ``cos`` / ``sin [T, D]`` (one k-only pass of ``siq_rope_bwd``)."""
    return _k_only("siq_rope_bwd", dk_embed[None], cos[None], sin[None])[0]


def rotate_k(k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """k half of ``apply_rotary_pos_emb`` on ``[B, S, Hkv, D]`` (autograd-aware,
    bitwise ``rope_fwd``'s k_embed); the q half is done inside the attention
    kernels by ``flash_attn_varlen_rope_func``."""
    if cos.requires_grad or sin.requires_grad:
        raise ValueError("gradients with respect to cos / sin are not supported")
    return _RopeK.apply(k, cos, sin)


def fused_qwen2_attention_forward(self, hidden_states: torch.Tensor, position_embeddings, attention_mask,
                                  past_key_values=None, **kwargs):
    """``Qwen2Attention.forward`` (transformers models/qwen2/modeling_qwen2.py:
    176-234; the reference's decoder attention via SiQ_VLTextModel,
    siq_vl/model/modeling.py:139-153) with the rotary embedding and the
    attention as one op (``flash_attn_varlen_rope_func``): the rotation's
    backward of q runs inside the attention backward's dQ kernel.  Same
    signature and return; bitwise the outputs and gradients of the unfused
    path (``enable_fused_rope`` + ``siq_varlen``), for a bf16 model and under
    bf16 autocast over fp32 master weights (fp32 cos / sin: the rotation in
    fp32, rounded once to bf16 as the attention's cast rounds the reference's
    fp32 q_embed / k_embed).  Calls it cannot serve (a KV cache, another
    attention backend, fp32 projections or CPU tensors) take the stock
    forward."""
    from .attention import ATTN_IMPLEMENTATION, _attend_packed

    cos, sin = position_embeddings
    # bf16 projections: a bf16 model, or bf16 autocast over fp32 master weights (the reference's bf16=True
    # training, scripts/train.py:712), where the rotary embedding hands over fp32 cos / sin
    bf16_proj = hidden_states.dtype == torch.bfloat16 or (
        hidden_states.is_cuda and torch.is_autocast_enabled("cuda")
        and torch.get_autocast_dtype("cuda") == torch.bfloat16)
    usable = (past_key_values is None and getattr(self.config, "_attn_implementation", None) == ATTN_IMPLEMENTATION
              and hidden_states.is_cuda and bf16_proj and cos.dtype == sin.dtype
              and cos.dtype in (torch.bfloat16, torch.float32)
              and getattr(self, "sliding_window", None) is None and self.head_dim in (64, 128))
    if not usable:
        return type(self).forward(self, hidden_states, position_embeddings, attention_mask,
                                  past_key_values=past_key_values, **kwargs)
    dropout = 0.0 if not self.training else self.attention_dropout
    if dropout:
        raise ValueError("siq_varlen attention does not implement dropout")
    input_shape = hidden_states.shape[:-1]
    hidden_shape = (*input_shape, -1, self.head_dim)
    q = self.q_proj(hidden_states).view(hidden_shape)  # [B, S, Hq, D]: the token-major layout the kernels read
    k = self.k_proj(hidden_states).view(hidden_shape)
    v = self.v_proj(hidden_states).view(hidden_shape)
    if not (q.dtype == k.dtype == v.dtype == torch.bfloat16):
        raise ValueError("the fused rotary attention expects bf16 projections")
    out = _attend_packed(q, k, v, attention_mask, bool(self.is_causal), self.scaling, kwargs, rope=(cos, sin))
    attn_output = out.reshape(*input_shape, -1).contiguous()
    return self.o_proj(attn_output), None


def enable_fused_rope_attention(model: torch.nn.Module) -> int:
    """Installs ``fused_qwen2_attention_forward`` on every Qwen2 attention
    layer of ``model`` (the model must use ``attn_implementation="siq_varlen"``
    for the fusion to apply); returns the number of layers patched."""
    import types

    from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention

    n = 0
    for mod in model.modules():
        if isinstance(mod, Qwen2Attention):
            mod.forward = types.MethodType(fused_qwen2_attention_forward, mod)
            n += 1
    return n


def rope_bytes(tokens: int, hq: int, hkv: int, d: int) -> int:
    """Algorithmic HBM bytes of one pass (forward or backward): q and k read and
    written once, plus one cos and one sin row per token."""
    return tokens * (2 * (hq + hkv) * d * 2 + 2 * d * 2)
