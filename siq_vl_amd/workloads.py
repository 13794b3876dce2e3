"""Seeded synthetic workloads of the five hot-path configurations.

Every generator uses ``torch.Generator().manual_seed(seed)`` (42 by default,
the reference's training seed, scripts/train.py:426-429) so the bench, the GPU
parity tests and the CPU baseline see the same sequence lengths and values.
Tensors are drawn in fp32 and rounded to bf16; the CPU baseline up-casts the
same bf16 values.

Config index follows the order of the configs list of the build's baseline:
  1  causal GQA forward, Qwen2.5-0.5B heads (14 q / 2 kv, d 64), 8 seqs, 4096 tokens
  2  causal GQA fwd+bwd, Qwen2.5-1.5B heads (12 / 2, d 128), 32 lognormal seqs, 16384 tokens
  3  bidirectional fwd+bwd, SigLIP2-large-512 (16 / 16, d 64), 16 x 1024 tokens
  4  fused linear CE fwd+bwd, h [16384, 1536], W [151936, 1536], 30% span mask
  5  skewed causal fwd+bwd (12 / 2, d 128): 16384 + 8192 + sequences of 81..600
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

SEED = 42
LOGNORMAL_SIGMA = 0.75  # sigma of config 2's lognormal lengths (median 400)
QWEN_VOCAB = 151936
IGNORE_INDEX = -100


@dataclass(frozen=True)
class AttnConfig:
    name: str
    hq: int
    hkv: int
    d: int
    causal: bool
    backward: bool
    lengths: tuple[int, ...]

    @property
    def total(self) -> int:
        return sum(self.lengths)

    def cu_seqlens(self) -> torch.Tensor:
        cu = [0]
        for n in self.lengths:
            cu.append(cu[-1] + n)
        return torch.tensor(cu, dtype=torch.int32)

    @property
    def max_seqlen(self) -> int:
        return max(self.lengths) if self.lengths else 0

    def pairs(self) -> int:
        """Allowed (q, k) pairs: sum L(L+1)/2 causal, sum L^2 bidirectional."""
        return sum(n * (n + 1) // 2 for n in self.lengths) if self.causal else sum(n * n for n in self.lengths)

    def flops(self) -> float:
        return (12.0 if self.backward else 4.0) * self.d * self.pairs() * self.hq


def _fix_total(lengths: list[int], total: int, lo: int, hi: int) -> list[int]:
    """Integer fix-up so the lengths sum to ``total`` while staying in [lo, hi]:
    the difference goes to the last length first, then to earlier ones."""
    out = [min(max(int(x), lo), hi) for x in lengths]
    diff = total - sum(out)
    i = len(out) - 1
    while diff != 0 and i >= 0:
        room = (hi - out[i]) if diff > 0 else (lo - out[i])
        step = min(diff, room) if diff > 0 else max(diff, room)
        out[i] += step
        diff -= step
        i -= 1
    if diff != 0:
        raise ValueError("cannot fit the lengths into the requested total")
    return out


def _rescale(raw: torch.Tensor, total: int, lo: int, hi: int) -> list[int]:
    raw = raw.to(torch.float64)
    scaled = torch.floor(raw * (total / float(raw.sum()))).tolist()
    return _fix_total([int(x) for x in scaled], total, lo, hi)


def config1_lengths(seed: int = SEED) -> list[int]:
    g = torch.Generator().manual_seed(seed)
    raw = torch.randint(64, 1025, (8,), generator=g)
    return _rescale(raw, 4096, 1, 4096)


def config2_lengths(seed: int = SEED) -> list[int]:
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(32, generator=g, dtype=torch.float64)
    raw = torch.exp(torch.log(torch.tensor(400.0, dtype=torch.float64)) + LOGNORMAL_SIGMA * z).clamp(16, 4096)
    return _rescale(raw, 16384, 16, 4096)


def config3_lengths() -> list[int]:
    return [1024] * 16


def config5_lengths(seed: int = SEED) -> list[int]:
    g = torch.Generator().manual_seed(seed)
    rest = 32768 - 16384 - 8192
    out: list[int] = []
    left = rest
    while left > 0:
        n = int(torch.randint(81, 601, (1,), generator=g))
        if left - n < 81:  # last one takes what is left (fix-up)
            n = left
        out.append(n)
        left -= n
    return [16384, 8192] + out


def attn_config(idx: int, seed: int = SEED) -> AttnConfig:
    if idx == 1:
        return AttnConfig("qwen2.5-0.5b-causal-fwd", 14, 2, 64, True, False, tuple(config1_lengths(seed)))
    if idx == 2:
        return AttnConfig("qwen2.5-1.5b-causal-fwdbwd", 12, 2, 128, True, True, tuple(config2_lengths(seed)))
    if idx == 3:
        return AttnConfig("siglip2-large-512-bidir-fwdbwd", 16, 16, 64, False, True, tuple(config3_lengths()))
    if idx == 5:
        return AttnConfig("qwen2.5-1.5b-skewed-fwdbwd", 12, 2, 128, True, True, tuple(config5_lengths(seed)))
    if idx == 6:
        # not one of the BASELINE configs: four equal 4096-token causal sequences at the config-2 heads, the
        # long-sequence reference point for the kernels' inner loops
        return AttnConfig("qwen2.5-1.5b-4x4096-causal-fwdbwd", 12, 2, 128, True, True, (4096,) * 4)
    raise ValueError(f"no attention config {idx}")


def attn_inputs(cfg: AttnConfig, seed: int = SEED, device: str | torch.device = "cpu",
                total: int | None = None) -> dict[str, torch.Tensor]:
    """q, k, v, dout ~ N(0, 1) rounded to bf16 (drawn on ``device``)."""
    t = cfg.total if total is None else total
    g = torch.Generator(device=device).manual_seed(seed)

    def draw(*shape):
        return torch.randn(*shape, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)

    return {
        "q": draw(t, cfg.hq, cfg.d),
        "k": draw(t, cfg.hkv, cfg.d),
        "v": draw(t, cfg.hkv, cfg.d),
        "dout": draw(t, cfg.hq, cfg.d),
    }


@dataclass(frozen=True)
class CEConfig:
    name: str
    n: int
    hdim: int
    vocab: int
    mask_frac: float = 0.3

    def flops(self) -> float:
        return 6.0 * self.n * self.hdim * self.vocab


CONFIG4 = CEConfig("qwen2.5-1.5b-lm-head-ce", 16384, 1536, QWEN_VOCAB)


def span_masked_labels(n: int, vocab: int, mask_frac: float, g: torch.Generator,
                       device: str | torch.device = "cpu") -> torch.Tensor:
    """Uniform labels with a contiguous ``ignore`` span at the head of each
    pseudo-sequence (prompt + image block, as the reference's label masking
    leaves only the assistant answer, siq_vl/model/processing.py:450-479).
    Pseudo-sequence lengths follow config 2's lognormal."""
    labels = torch.randint(0, vocab, (n,), generator=g, device=device, dtype=torch.int64)
    gl = torch.Generator().manual_seed(int(torch.randint(0, 2**31 - 1, (1,), generator=g, device=device)))
    start = 0
    while start < n:
        z = float(torch.randn(1, generator=gl, dtype=torch.float64))
        ln = int(min(max(400.0 * float(torch.exp(torch.tensor(LOGNORMAL_SIGMA * z))), 16), 4096))
        ln = min(ln, n - start)
        span = int(round(mask_frac * ln))
        labels[start:start + span] = IGNORE_INDEX
        start += ln
    return labels


def ce_inputs(cfg: CEConfig, seed: int = SEED, device: str | torch.device = "cpu") -> dict[str, torch.Tensor]:
    g = torch.Generator(device=device).manual_seed(seed)
    h = torch.randn(cfg.n, cfg.hdim, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    w = (0.02 * torch.randn(cfg.vocab, cfg.hdim, generator=g, device=device, dtype=torch.float32)).to(torch.bfloat16)
    y = span_masked_labels(cfg.n, cfg.vocab, cfg.mask_frac, g, device)
    return {"hidden": h, "weight": w, "labels": y}
