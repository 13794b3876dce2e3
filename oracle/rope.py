"""CPU oracle of the fused RoPE -- TEST INFRASTRUCTURE ONLY.

Restates transformers models/qwen2/modeling_qwen2.py:105-135 (``rotate_half``
and ``apply_rotary_pos_emb``, the reference's pin transformers 4.57.3; called
at :206-211) on bf16 values held as float32, with the reference's rounding:
each torch op on bf16 tensors computes in fp32 and rounds its result to bf16
(round to nearest even), so

    q_embed = rb(rb(q * cos) + rb(rotate_half(q) * sin)),
    rotate_half(x) = cat(-x[..., D/2:], x[..., :D/2]).

The backward restates the autograd graph of those ops: MulBackward gives
rb(g * cos) and rb(g * sin); the cat / neg / narrow backwards route the second
product's gradient to the other half with the sign of rotate_half; the two
contributions to x are added once, in bf16.

Parity pinning (tests/test_oracle_rope.py): bitwise against torch's own bf16
ops and autograd on the same inputs (the library the reference runs, here on
the CPU), plus closed forms -- cos = 1, sin = 0 is the identity; cos = 0,
sin = 1 is rotate_half exactly; the fp32 rotation is norm preserving per
frequency pair when cos^2 + sin^2 = 1; the backward of the fp32 map is its
transpose (adjoint identity <R x, g> = <x, R^T g>).
"""

from __future__ import annotations

import numpy as np


def round_bf16(x) -> np.ndarray:
    """fp32 -> nearest-even bf16, returned as float32 (finite inputs)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).reshape(x.shape)


def _halves(x: np.ndarray):
    d = x.shape[-1]
    return x[..., : d // 2], x[..., d // 2:]


def rotate_half(x: np.ndarray) -> np.ndarray:
    """cat(-x2, x1) along the last axis (exact)."""
    x1, x2 = _halves(x)
    return np.concatenate([-x2, x1], axis=-1)


def rope_fwd(x, cos, sin) -> np.ndarray:
    """x [..., S, H, D] (or any layout whose cos/sin broadcast), bf16 values as float32."""
    x = np.asarray(x, dtype=np.float32)
    cos = np.asarray(cos, dtype=np.float32)
    sin = np.asarray(sin, dtype=np.float32)
    return round_bf16(round_bf16(x * cos) + round_bf16(rotate_half(x) * sin))


def rope_bwd(g, cos, sin) -> np.ndarray:
    """Gradient w.r.t. x of rope_fwd's output, given its upstream gradient g."""
    g = np.asarray(g, dtype=np.float32)
    cos = np.asarray(cos, dtype=np.float32)
    sin = np.asarray(sin, dtype=np.float32)
    a = round_bf16(g * cos)           # through x * cos
    r = round_bf16(g * sin)           # gradient of rotate_half(x)
    r1, r2 = _halves(r)
    through_rot = np.concatenate([r2, -r1], axis=-1)  # rotate_half^T
    return round_bf16(a + through_rot)


def rope_fwd_f64(x, cos, sin) -> np.ndarray:
    """The same map in float64 without rounding (for the closed-form checks)."""
    x = np.asarray(x, dtype=np.float64)
    return x * np.asarray(cos, np.float64) + rotate_half(x) * np.asarray(sin, np.float64)


def rope_bwd_f64(g, cos, sin) -> np.ndarray:
    g = np.asarray(g, dtype=np.float64)
    r = g * np.asarray(sin, np.float64)
    r1, r2 = _halves(r)
    return g * np.asarray(cos, np.float64) + np.concatenate([r2, -r1], axis=-1)


def qwen2_cos_sin(position_ids, head_dim: int, theta: float = 1000000.0):
    """cos / sin as Qwen2RotaryEmbedding builds them for the default rope type
    (inv_freq = theta^(-2i/D), emb = cat(freqs, freqs), fp32 then cast to
    bf16), returned as bf16 values in float32.  [B, S] -> [B, S, D]."""
    pos = np.asarray(position_ids, dtype=np.float32)
    inv = (1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float32) / head_dim))).astype(np.float32)
    freqs = pos[..., None] * inv
    emb = np.concatenate([freqs, freqs], axis=-1)
    return round_bf16(np.cos(emb)), round_bf16(np.sin(emb))
