"""Benchmark of the SiQ-VL hot path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

One step = one forward + backward of varlen packed attention over the config-2
batch (Qwen2.5-1.5B heads: 12 q / 2 kv, d 128, 32 lognormal sequences, 16384
tokens, causal), inputs already resident in HBM, including the build of the
batch's schedule (the plan every layer of a packed batch shares; built once
per step here, so its cost is charged in full to one layer).  The headline
``value`` is its algorithmic TFLOP/s (12 * d * P * Hq per step, P = allowed
(q, k) pairs of the realised cu_seqlens; recompute not counted), from the
median step time.

Every other BASELINE configuration is timed the same way and reported beside
it: config 3 (SigLIP bidirectional) and config 5 (skewed packing) fwd+bwd,
config 1 forward (also timed on the host CPU: the reference path's fp32 SDPA
with a block-diagonal mask), and config 4, the fused lm_head cross-entropy
(tokens/s over all rows, and TFLOP/s at 6 * n * hdim * vocab over all rows and
over the rows whose label counts).  "Config 6" (four 4096-token causal
sequences at the config-2 heads) is not a BASELINE configuration: it is the
long-sequence reference point of the attention kernels.  Each attention
config also reports its backward in both modes (deterministic, atomic dQ),
and the RoPE, projector and splice legs run after the CE.

Timing: four consecutive attention steps are captured once as a HIP graph and
replayed (the same kernels and arguments as eager steps, without the host
launch gaps between them); HIP events on the replay stream bracket every
replay (step time = replay time / 4), W warm-up replays first, device
synchronisation on both sides; the median over K >= 20 replays is reported.
Eager per-call medians are reported beside it.  The shader clock is probed
right after the timed steps (``gpu_clock_mhz``).  The CPU baseline times the
reference path's own library calls (oracle/cpu_path.py) on bounded samples of
the same inputs.  ``--leg NAME`` runs one leg only (a profiling aid).
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import torch

from siq_vl_amd import _lib
from siq_vl_amd import attention as A
from siq_vl_amd import cross_entropy as C
from siq_vl_amd import projector as PJ
from siq_vl_amd import rope as R
from siq_vl_amd import splice as SP
from siq_vl_amd import workloads as W

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA (256 CUs x 2.4 GHz)
PEAK_HBM_GBS = 8000.0
PEAK_CLOCK_MHZ = 2400.0
COPY_BYTES = 256 << 20
MIN_STEPS = 20
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")


CSRC_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "siq_vl_amd", "csrc")


def kernel_sources_digest() -> str:
    """sha256 (first 16 hex digits) over the kernel sources (file names and
    contents, in name order): what profiles/traffic.json is stamped with when
    the rocprofv3 passes are summarised, so that a traffic figure measured on
    other kernels is recognised as stale."""
    import hashlib

    h = hashlib.sha256()
    for name in sorted(os.listdir(CSRC_DIR)):
        path = os.path.join(CSRC_DIR, name)
        if os.path.isfile(path) and name.endswith((".hip", ".h", ".cpp")):
            h.update(name.encode())
            with open(path, "rb") as fh:
                h.update(fh.read())
    return h.hexdigest()[:16]


def measured_traffic(key: str) -> dict:
    """HBM bytes per call of ``key`` from the last rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes (scaled by a plain copy's readings), with the commit and kernel
    sources they were measured on.  ``bytes`` is None when never measured or
    when the kernel sources changed since (``stale``)."""
    out = {"bytes": None, "measured_at_commit": None, "stale": None}
    try:
        with open(TRAFFIC_FILE) as fh:
            ent = json.load(fh)[key]
    except (OSError, KeyError, ValueError):
        return out
    cur = kernel_sources_digest()
    stale = ent.get("sources_sha16") != cur
    out.update({"measured_at_commit": ent.get("commit"), "sources_sha16": ent.get("sources_sha16"),
                "current_sources_sha16": cur, "stale": stale})
    if stale:
        out["stale_bytes"] = int(ent["bytes_per_call"])
    else:
        out["bytes"] = int(ent["bytes_per_call"])
    return out


METRIC = "packed varlen attn fwd+bwd TFLOP/s (% bf16 MFMA peak); fused-CE tokens/s"


def _events(n):
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def _median(a):
    a = sorted(a)
    n = len(a)
    return a[n // 2] if n % 2 else 0.5 * (a[n // 2 - 1] + a[n // 2])


def probe_clock_mhz() -> float | None:
    """Shader clock right now (MHz), from the library's clock probe (~200 us of spinning)."""
    out = torch.zeros(2, dtype=torch.int64, device="cuda")
    rc = _lib.lib().siq_probe_clock(out.data_ptr(), 20000, torch.cuda.current_stream().cuda_stream)
    if rc != 0:
        return None
    cyc, ticks = (int(x) for x in out.cpu().tolist())
    return 100.0 * cyc / ticks if ticks > 0 else None


def timed_steps(parts, steps: int, warmup: int) -> dict:
    """Runs ``parts`` (list of (name, fn)) in order as one step, ``warmup`` times
    untimed, then ``steps`` times with events on the launch stream around every
    part.  Returns median / mean step ms and median ms per part."""
    for _ in range(warmup):
        for _, fn in parts:
            fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    np_ = len(parts)
    ev = _events(steps * np_ + 1)
    ev[0].record(stream)
    for i in range(steps):
        for j, (_, fn) in enumerate(parts):
            fn()
            ev[i * np_ + j + 1].record(stream)
    torch.cuda.synchronize()
    per_step = [ev[i * np_].elapsed_time(ev[(i + 1) * np_]) for i in range(steps)]
    res = {"median_ms": _median(per_step), "mean_ms": ev[0].elapsed_time(ev[-1]) / steps, "steps": steps}
    for j, (name, _) in enumerate(parts):
        res[name + "_ms"] = _median([ev[i * np_ + j].elapsed_time(ev[i * np_ + j + 1]) for i in range(steps)])
    return res


def host_ahead_ms(fn, steps: int, warmup: int) -> float:
    """Median GPU time per call of ``fn`` with the host running ahead, as in a
    training step: a spin kernel holds the stream while the calls are enqueued
    behind it, so the events between calls time the GPU's work, not the
    host's launch overhead."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = _events(steps + 1)
    torch.cuda._sleep(100_000_000)
    ev[0].record(stream)
    for i in range(steps):
        fn()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    return _median([ev[i].elapsed_time(ev[i + 1]) for i in range(steps)])


GRAPH_STEPS_PER_REPLAY = 4


def graphed_steps(parts, steps: int, warmup: int, per_replay: int = GRAPH_STEPS_PER_REPLAY) -> dict:
    """One step = ``parts`` in order.  ``per_replay`` consecutive steps are
    captured once as a HIP graph; the graph is replayed ``warmup`` times
    untimed, then ``steps`` times with an event after each replay on the
    replay stream.  Returns the median / mean ms per step (replay time /
    ``per_replay``).  The kernels and their arguments are exactly those of
    eager steps; the graph removes the host-side launch gaps between them, and
    several steps per replay amortise the gap between two replays (10-20 us on
    this runtime, as much as a short kernel)."""
    for _ in range(2):
        for _, fn in parts:
            fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_replay):
            for _, fn in parts:
                fn()
    for _ in range(max(warmup, 1)):
        g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = _events(steps + 1)
    ev[0].record(stream)
    for i in range(steps):
        g.replay()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) / per_replay for i in range(steps)]
    return {"median_ms": _median(per), "mean_ms": ev[0].elapsed_time(ev[-1]) / (steps * per_replay),
            "steps": steps, "per_replay": per_replay}


def bench_attention(idx: int, steps: int, warmup: int) -> dict:
    """Config ``idx``: plan + forward (+ backward when the config has one) per
    step, timed as graph-replayed steps (headline) and as eager calls (per
    call medians)."""
    cfg = W.attn_config(idx)
    dev = torch.device("cuda")
    x = W.attn_inputs(cfg, device=dev)
    cu = cfg.cu_seqlens().to(dev)
    scale = cfg.d**-0.5
    mx = cfg.max_seqlen
    st = {}

    def plan():
        st["plan"] = A.build_attn_plan(cu, cu, cfg.total, cfg.total, cfg.hq, cfg.hkv, cfg.causal, dev)

    def fwd():
        st["out"], st["lse"] = A.varlen_attn_fwd(x["q"], x["k"], x["v"], cu, cu, mx, mx, scale, cfg.causal,
                                                 plan=st["plan"])

    def bwd():
        A.varlen_attn_bwd(x["dout"], x["q"], x["k"], x["v"], st["out"], st["lse"], cu, cu, mx, mx, scale,
                          cfg.causal, plan=st["plan"])

    parts = [("plan", plan), ("fwd", fwd)] + ([("bwd", bwd)] if cfg.backward else [])
    r = timed_steps(parts, steps, warmup)
    gr = graphed_steps(parts, steps, warmup)
    pairs = cfg.pairs()
    flops_fwd = 4.0 * cfg.d * pairs * cfg.hq
    flops_bwd = 8.0 * cfg.d * pairs * cfg.hq if cfg.backward else 0.0
    t, hq, hkv, d = cfg.total, cfg.hq, cfg.hkv, cfg.d
    qb, kvb, lseb = t * hq * d * 2, t * hkv * d * 2, t * hq * 4
    # algorithmic bytes: read q,k,v (fwd) + q,k,v,o,do,lse (bwd); write o,lse (fwd) + dq,dk,dv (bwd)
    bytes_fwd = qb + 2 * kvb + qb + lseb
    bytes_bwd = 3 * qb + 2 * kvb + lseb + qb + 2 * kvb
    ms = gr["median_ms"]
    out = {
        "cfg": cfg, "pairs": pairs, "ms_per_step": ms, "mean_ms_per_step": gr["mean_ms"],
        "eager_ms_per_step": r["median_ms"],
        "plan_ms": r["plan_ms"], "fwd_ms": r["fwd_ms"],
        "tflops": (flops_fwd + flops_bwd) / (ms * 1e-3) / 1e12,
        "fwd_tflops": flops_fwd / (r["fwd_ms"] * 1e-3) / 1e12,
        "flops_fwd": flops_fwd, "flops_bwd": flops_bwd, "bytes_fwd": bytes_fwd, "bytes_bwd": bytes_bwd,
    }
    if cfg.backward:
        out["bwd_ms"] = r["bwd_ms"]
        out["bwd_tflops"] = flops_bwd / (r["bwd_ms"] * 1e-3) / 1e12
        # the two backward modes, graph-replayed over a plan built once (the choice of the default)
        plan_once = A.build_attn_plan(cu, cu, cfg.total, cfg.total, cfg.hq, cfg.hkv, cfg.causal, dev)
        o1, l1 = A.varlen_attn_fwd(x["q"], x["k"], x["v"], cu, cu, mx, mx, scale, cfg.causal, plan=plan_once)
        for det in (True, False):
            out["bwd_graph_ms_" + ("deterministic" if det else "atomic")] = graphed_ms(
                lambda: A.varlen_attn_bwd(x["dout"], x["q"], x["k"], x["v"], o1, l1, cu, cu, mx, mx, scale,
                                          cfg.causal, plan=plan_once, deterministic=det), 5, steps, warmup)
    return out


def attn_block(a: dict) -> dict:
    """The JSON block of one attention config."""
    cfg = a["cfg"]
    blk = {"workload": cfg.name, "total_tokens": cfg.total, "sequences": len(cfg.lengths),
           "max_seqlen": cfg.max_seqlen, "heads": f"{cfg.hq}/{cfg.hkv}", "head_dim": cfg.d, "causal": cfg.causal,
           "pairs": a["pairs"], "ms_per_step": round(a["ms_per_step"], 4),
           "mean_ms_per_step": round(a["mean_ms_per_step"], 4),
           "eager_ms_per_step": round(a["eager_ms_per_step"], 4), "plan_us": round(a["plan_ms"] * 1e3, 2),
           "fwd_ms": round(a["fwd_ms"], 4), "fwd_tflops": round(a["fwd_tflops"], 2),
           "tflops": round(a["tflops"], 2), "pct_bf16_peak": round(100.0 * a["tflops"] / PEAK_BF16_TFLOPS, 2)}
    if cfg.backward:
        blk["bwd_ms"] = round(a["bwd_ms"], 4)
        blk["bwd_tflops"] = round(a["bwd_tflops"], 2)
        blk["bwd_modes_us"] = {"timing": "backward call over a prebuilt plan, 5 per HIP graph, replayed",
                               "deterministic": round(a["bwd_graph_ms_deterministic"] * 1e3, 1),
                               "atomic_dq": round(a["bwd_graph_ms_atomic"] * 1e3, 1),
                               "default": "deterministic" if A.DETERMINISTIC_DEFAULT else "atomic_dq"}
        ach = (a["flops_fwd"] + a["flops_bwd"]) / ((a["fwd_ms"] + a["bwd_ms"]) * 1e-3) / 1e12
        blk["roofline"] = {"bound": "mfma", "kernel": "forward + backward calls", "achieved": round(ach, 2),
                           "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(ach / PEAK_BF16_TFLOPS, 4)}
    else:
        blk["roofline"] = {"bound": "mfma", "kernel": "forward call", "achieved": round(a["fwd_tflops"], 2),
                           "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                           "frac": round(a["fwd_tflops"] / PEAK_BF16_TFLOPS, 4)}
    return blk


def _rope_inputs(cfg, dev):
    """Config-2 q / k as Qwen2Attention hands them to apply_rotary_pos_emb ([1, H, T, D]
    views of the [1, T, H*D] projections), position ids restarting per sequence."""
    g = torch.Generator().manual_seed(W.SEED)
    t, d = cfg.total, cfg.d
    proj = lambda h: torch.randn(1, t, h * d, generator=g).to(torch.bfloat16).to(dev).view(1, t, h, d).transpose(1, 2)
    q, k = proj(cfg.hq), proj(cfg.hkv)
    cu = cfg.cu_seqlens().tolist()
    pos = torch.cat([torch.arange(cu[i + 1] - cu[i]) for i in range(len(cu) - 1)]).float()
    inv = 1.0 / (1000000.0 ** (torch.arange(0, d, 2).float() / d))
    emb = torch.cat([pos[:, None] * inv, pos[:, None] * inv], dim=-1)[None]
    cos, sin = emb.cos().to(torch.bfloat16).to(dev), emb.sin().to(torch.bfloat16).to(dev)
    dq = torch.randn(q.shape, generator=g).to(torch.bfloat16).to(dev)
    dk = torch.randn(k.shape, generator=g).to(torch.bfloat16).to(dev)
    return q, k, cos, sin, dq, dk


def bench_rope(steps: int, warmup: int) -> dict:
    """Fused RoPE forward and backward at the config-2 shape; the reference's own
    torch ops (modeling_qwen2.py:105-135 and their autograd) timed beside it."""
    cfg = W.attn_config(2)
    dev = torch.device("cuda")
    q, k, cos, sin, gq, gk = _rope_inputs(cfg, dev)
    bq, bk = R._bshd(q, 1), R._bshd(k, 1)
    bgq, bgk = R._bshd(gq, 1), R._bshd(gk, 1)
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ev = _events(steps + 1)
        ev[0].record(stream)
        for i in range(steps):
            fn()
            ev[i + 1].record(stream)
        torch.cuda.synchronize()
        per = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
        return per[len(per) // 2]

    def graphed(fn, reps=20):
        # one call is a few microseconds of GPU work, less than its host-side cost: capture
        # `reps` back-to-back launches in a HIP graph so the events time the kernels, not Python
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                fn()
        per = timed(g.replay)
        return per / reps

    fwd_ms = graphed(lambda: R.rope_fwd(bq, bk, cos, sin))
    bwd_ms = graphed(lambda: R.rope_bwd(bgq, bgk, cos, sin))
    eager_fwd_ms = timed(lambda: R.rope_fwd(bq, bk, cos, sin))

    def rh(x):
        return torch.cat((-x[..., x.shape[-1] // 2:], x[..., : x.shape[-1] // 2]), dim=-1)

    qr, kr = q.detach().requires_grad_(), k.detach().requires_grad_()
    c1, s1 = cos.unsqueeze(1), sin.unsqueeze(1)

    def ref_step():
        qe = qr * c1 + rh(qr) * s1
        ke = kr * c1 + rh(kr) * s1
        torch.autograd.backward((qe, ke), (gq, gk))
        qr.grad = None
        kr.grad = None

    ref_ms = timed(ref_step)
    nbytes = R.rope_bytes(cfg.total, cfg.hq, cfg.hkv, cfg.d)
    return {"fwd_ms": fwd_ms, "bwd_ms": bwd_ms, "ref_ms": ref_ms, "bytes": nbytes, "eager_fwd_ms": eager_fwd_ms,
            "fwd_gbs": nbytes / (fwd_ms * 1e-3) / 1e9, "bwd_gbs": nbytes / (bwd_ms * 1e-3) / 1e9}


def graphed_ms(fn, reps: int, steps: int, warmup: int) -> float:
    """Median ms of one ``fn()`` call: ``reps`` calls captured in a HIP graph,
    replayed ``steps`` times after ``warmup`` replays (events on the launch
    stream).  For steps made of short kernels whose host launch cost would
    otherwise be timed."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    for _ in range(max(warmup, 1)):
        g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = _events(steps + 1)
    ev[0].record(stream)
    for i in range(steps):
        g.replay()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    return _median([ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]) / reps


def bench_rope_attention(steps: int, warmup: int) -> dict:
    """Config 2 with the decoder's RoPE in the step (plan built once per batch,
    outside): the unfused pipeline (RoPE of q and k, attention fwd + bwd, RoPE
    backward), the drop-in (the rotation's backward of dq inside the dQ
    kernel, k-only RoPE backward) and the fully fused variant (q also rotated
    inside the attention forward); all bitwise the same results.  Each step
    is graph-replayed: several of its kernels are shorter than their launch."""
    cfg = W.attn_config(2)
    dev = torch.device("cuda")
    x = W.attn_inputs(cfg, device=dev)
    cu = cfg.cu_seqlens().to(dev)
    t, d = cfg.total, cfg.d
    pos = torch.cat([torch.arange(n) for n in cfg.lengths]).float()
    inv = 1.0 / (1000000.0 ** (torch.arange(0, d, 2).float() / d))
    emb = torch.cat([pos[:, None] * inv, pos[:, None] * inv], dim=-1)
    cos, sin = emb.cos().to(torch.bfloat16).to(dev), emb.sin().to(torch.bfloat16).to(dev)
    scale = d**-0.5
    plan = A.build_attn_plan(cu, cu, t, t, cfg.hq, cfg.hkv, True, dev)
    q, k, v, do = x["q"], x["k"], x["v"], x["dout"]

    def unfused():
        qe, ke = R.rope_fwd(q[None], k[None], cos[None], sin[None])
        out, lse = A.varlen_attn_fwd(qe[0], ke[0], v, cu, cu, 0, 0, scale, True, plan=plan)
        dqe, dke, _ = A.varlen_attn_bwd(do, qe[0], ke[0], v, out, lse, cu, cu, 0, 0, scale, True, plan=plan)
        R.rope_bwd(dqe[None], dke[None], cos[None], sin[None])

    def dropin():
        qe, ke = R.rope_fwd(q[None], k[None], cos[None], sin[None])
        out, lse = A.varlen_attn_fwd(qe[0], ke[0], v, cu, cu, 0, 0, scale, True, plan=plan)
        _, dke, _ = A.varlen_attn_rope_bwd(do, qe[0], ke[0], v, out, lse, cos, sin, cu, cu, 0, 0, scale, True,
                                           plan=plan)
        R.rotate_k_backward(dke, cos, sin)

    def fused_fwd():
        ke = R.rotate_k(k[None], cos[None], sin[None])[0]
        out, lse, qe = A.varlen_attn_rope_fwd(q, ke, v, cos, sin, cu, cu, 0, 0, scale, True, plan=plan)
        _, dke, _ = A.varlen_attn_rope_bwd(do, qe, ke, v, out, lse, cos, sin, cu, cu, 0, 0, scale, True,
                                           plan=plan)
        R.rotate_k_backward(dke, cos, sin)

    def attention_only():
        out, lse = A.varlen_attn_fwd(q, k, v, cu, cu, 0, 0, scale, True, plan=plan)
        A.varlen_attn_bwd(do, q, k, v, out, lse, cu, cu, 0, 0, scale, True, plan=plan)

    # bf16 autocast over fp32 master weights (the reference's bf16=True training): fp32 cos / sin.  The stock
    # path rotates in fp32 (torch's promoted ops and their autograd) and casts q_embed / k_embed to bf16 for
    # the attention; the fused path writes the bf16 cast directly (siq_rope_fwd_ex / siq_rope_bwd_ex)
    cos32, sin32 = emb.cos().to(dev), emb.sin().to(dev)
    qg, kg = q.detach().clone().requires_grad_(), k.detach().clone().requires_grad_()

    def rotate_half(x):
        return torch.cat((-x[..., d // 2:], x[..., : d // 2]), dim=-1)

    def autocast_stock():
        qe = (qg * cos32[:, None]) + (rotate_half(qg) * sin32[:, None])
        ke = (kg * cos32[:, None]) + (rotate_half(kg) * sin32[:, None])
        out = A.flash_attn_varlen_func(qe.to(torch.bfloat16), ke.to(torch.bfloat16), v, cu, cu, 0, 0,
                                       softmax_scale=scale, causal=True)
        out.backward(do)

    def autocast_fused():
        out = A.flash_attn_varlen_rope_func(qg, kg, v, cos32, sin32, cu, cu, 0, 0, softmax_scale=scale,
                                            causal=True)
        out.backward(do)

    res = {}
    for name, fn in (("attention_only", attention_only), ("unfused", unfused), ("dropin", dropin),
                     ("fused_fwd", fused_fwd)):
        res[name + "_ms"] = graphed_ms(fn, 5, steps, warmup)
    # autograd steps, timed with the host running ahead (the stock path's many small ops cost GPU time, not
    # only launches); the attention's plan is cached on cu after the first call
    res["autocast_stock_ms"] = host_ahead_ms(autocast_stock, steps, warmup)
    res["autocast_fused_ms"] = host_ahead_ms(autocast_fused, steps, warmup)
    return res


def bench_projector(steps: int, warmup: int) -> dict:
    """Pixel-shuffle projector forward + backward (dx and dweight) at the production
    shape: 16 SigLIP2-large-512 tiles (32 x 32 patches x 1024) -> Qwen2.5-1.5B (1536),
    r = 2; the reference's torch ops (modeling.py:74-105 and their autograd) beside it."""
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(W.SEED)
    batch, side, dv, r, n = 16, 32, 1024, 2, 1536
    x = torch.randn(batch, side * side, dv, generator=g).to(torch.bfloat16).to(dev)
    w = (0.02 * torch.randn(n, dv * r * r, generator=g)).to(torch.bfloat16).to(dev)
    dy = torch.randn(batch, (side // r) ** 2, n, generator=g).to(torch.bfloat16).to(dev)
    stream = torch.cuda.current_stream(dev)

    def timed(fn, reps):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ev = _events(steps + 1)
        ev[0].record(stream)
        for i in range(steps):
            fn()
            ev[i + 1].record(stream)
        torch.cuda.synchronize()
        per = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
        return per[len(per) // 2] / reps

    def graphed(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(reps):
                fn()
        return timed(gr.replay, reps)

    fwd_ms = graphed(lambda: PJ.proj_fwd(x, w, r))
    bwd_ms = graphed(lambda: PJ.proj_bwd(x, w, dy, r))
    xr, wr = x.detach().requires_grad_(), w.detach().requires_grad_()

    def ref_step():
        xs = xr.view(batch, side, side, dv).reshape(batch, side // r, r, side // r, r, dv)
        xs = xs.permute(0, 1, 3, 2, 4, 5).contiguous().reshape(batch, (side // r) ** 2, dv * r * r)
        torch.nn.functional.linear(xs, wr).backward(dy)
        xr.grad = None
        wr.grad = None

    ref_ms = timed(ref_step, 1)
    m, k = batch * (side // r) ** 2, dv * r * r
    fl_f, fl_b = PJ.projector_flops(m, k, n, backward=False), PJ.projector_flops(m, k, n) - PJ.projector_flops(
        m, k, n, backward=False)
    return {"fwd_ms": fwd_ms, "bwd_ms": bwd_ms, "ref_ms": ref_ms, "m": m, "k": k, "n": n,
            "tflops": (fl_f + fl_b) / ((fwd_ms + bwd_ms) * 1e-3) / 1e12,
            "fwd_tflops": fl_f / (fwd_ms * 1e-3) / 1e12, "bwd_tflops": fl_b / (bwd_ms * 1e-3) / 1e12}


def bench_splice(steps: int, warmup: int) -> dict:
    """Vision-token splice forward at config-4 scale: 16384 tokens of Qwen2.5-1.5B (1536
    features, 151936-row table) of which 4096 are image tokens (16 tiles x 256); the
    reference's torch ops (embedding, nonzero, index assignment) beside it."""
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(W.SEED)
    n, hidden, vocab, nimg, img = 16384, 1536, 151936, 4096, 151655
    ids = torch.randint(0, vocab, (1, n), generator=g)
    ids[ids == img] = 0
    ids[0, torch.randperm(n, generator=g)[:nimg]] = img
    ids = ids.to(dev)
    weight = (0.02 * torch.randn(vocab, hidden, generator=g)).to(torch.bfloat16).to(dev)
    vis = torch.randn(nimg, hidden, generator=g).to(torch.bfloat16).to(dev)
    emb = torch.nn.Embedding(vocab, hidden).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        emb.weight.copy_(weight)
    stream = torch.cuda.current_stream(dev)
    flat = ids.view(-1)

    def timed(fn, reps):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ev = _events(steps + 1)
        ev[0].record(stream)
        for i in range(steps):
            fn()
            ev[i + 1].record(stream)
        torch.cuda.synchronize()
        per = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
        return per[len(per) // 2] / reps

    def graphed(fn, reps=10):
        fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(reps):
                fn()
        return timed(gr.replay, reps)

    # the kernels alone; the op adds the count check: lazy (a pinned copy and an event, judged at the next call)
    # or sync (one device-to-host read, as the reference's nonzero makes)
    fwd_ms = graphed(lambda: SP.splice_fwd(flat, weight, vis, img))

    def ref_step():
        te = emb(ids)
        positions = (ids == img).nonzero(as_tuple=True)
        te[positions] = vis

    ref_ms = timed(ref_step, 1)
    op_ms = timed(lambda: SP.splice_vision_tokens(ids, weight, vis, img), 1)
    op_sync_ms = timed(lambda: SP.splice_vision_tokens(ids, weight, vis, img, validate="sync"), 1)
    op_queued_ms = host_ahead_ms(lambda: SP.splice_vision_tokens(ids, weight, vis, img), steps, warmup)
    SP.check_pending_splices(block=True)
    # the embedding table's gradient (full fine-tune): the HIP per-id sum against torch's embedding backward
    gout = torch.randn(n, hidden, generator=g).to(torch.bfloat16).to(dev)
    table_ms = graphed(lambda: SP.embedding_bwd(gout, flat, vocab, (img,)), reps=5)
    table_ref_ms = timed(lambda: torch.ops.aten.embedding_dense_backward(gout, flat, vocab, img, False), 1)
    nbytes = SP.splice_bytes(n, hidden)
    table_bytes = n * (hidden * 2 + 8) + vocab * hidden * 2
    return {"fwd_ms": fwd_ms, "op_ms": op_ms, "op_sync_ms": op_sync_ms, "op_queued_ms": op_queued_ms,
            "ref_ms": ref_ms, "bytes": nbytes,
            "gbs": nbytes / (fwd_ms * 1e-3) / 1e9, "table_ms": table_ms, "table_ref_ms": table_ref_ms,
            "table_bytes": table_bytes, "table_gbs": table_bytes / (table_ms * 1e-3) / 1e9}


def bench_ce(steps: int, warmup: int, chunk: int | None, modes=("full", "dh_only")) -> dict:
    cfg = W.CONFIG4
    dev = torch.device("cuda")
    x = W.ce_inputs(cfg, device=dev)
    chunk = C.default_chunk_tokens(cfg.vocab) if chunk is None else chunk

    def step():
        return C.flce_fwd_bwd(x["hidden"], x["weight"], x["labels"], chunk_tokens=chunk)

    def step_dh():
        # a frozen lm_head (the reference's stage 1, and stage 2's LoRA, which leaves lm_head out of its
        # targets): loss and dHidden only, no dW GEMM
        return C.flce_fwd_bwd(x["hidden"], x["weight"], x["labels"], need_dweight=False, chunk_tokens=chunk)

    r = timed_steps([("ce", step)], steps, warmup) if "full" in modes else None
    r_dh = timed_steps([("ce_dh", step_dh)], steps, warmup) if "dh_only" in modes else None
    if r is None:  # the dH-only leg alone (a profiling aid)
        return {"dh_only_ms": r_dh["median_ms"], "chunk": chunk}
    ms = r["median_ms"]
    # tokens/s counts every row of the batch (the metric); the executed TFLOP/s counts the work the
    # kernels run: rows whose label is ignored are compacted out before the logits GEMM
    n_valid = int(((x["labels"] != C.IGNORE_INDEX) & (x["labels"] >= 0) & (x["labels"] < cfg.vocab)).sum())
    ws = C.flce_workspace_bytes(cfg.n, cfg.hdim, cfg.vocab, chunk, True)
    return {
        "cfg": cfg, "ms_per_step": ms, "mean_ms_per_step": r["mean_ms"],
        "tokens_per_s": cfg.n / (ms * 1e-3), "n_valid": n_valid,
        "tflops_all_rows": 6.0 * cfg.n * cfg.hdim * cfg.vocab / (ms * 1e-3) / 1e12,
        "tflops_executed": 6.0 * n_valid * cfg.hdim * cfg.vocab / (ms * 1e-3) / 1e12,
        "chunk": chunk, "workspace_bytes": ws,
        "dh_only_ms": r_dh["median_ms"] if r_dh else None, "dh_only_workspace_bytes": C.flce_workspace_bytes(cfg.n, cfg.hdim, cfg.vocab, chunk, False),
        "e_bytes": 2 * chunk * cfg.vocab,
        "algorithmic_bytes": 2 * (2 * cfg.n * cfg.hdim + 2 * cfg.vocab * cfg.hdim) + 8 * cfg.n,
    }


def _cpu_threads() -> int:
    # the host share this GPU's job may use (OMP_NUM_THREADS on the GPU box), never above the core count
    cores = os.cpu_count() or 1
    return min(cores, int(os.environ.get("OMP_NUM_THREADS") or cores))


def _cpu_attention_sample(cfg, lens: list[int], budget_s: float, max_reps: int = 50):
    """fwd+bwd of the reference path (fp32 SDPA, block-diagonal mask,
    repeat_kv, autograd) over ``lens``, each a prefix of the config's
    sequences (the first len tokens of a causal sequence are themselves a
    causal sequence).  Returns (TFLOP/s at 12 * d * P * Hq, reps)."""
    from oracle import cpu_path

    x = W.attn_inputs(cfg, device="cpu")
    starts = cfg.cu_seqlens().tolist()
    rows = torch.cat([torch.arange(starts[i], starts[i] + n) for i, n in lens])
    q, k, v, do = (x[n][rows].float().requires_grad_(n != "dout") for n in ("q", "k", "v", "dout"))
    cu = [0]
    for _, n in lens:
        cu.append(cu[-1] + n)
    pairs = sum(n * (n + 1) // 2 for _, n in lens) if cfg.causal else sum(n * n for _, n in lens)
    flops = 12.0 * cfg.d * pairs * cfg.hq
    t0 = time.perf_counter()
    reps = 0
    while True:
        out = cpu_path.sdpa_attention(q, k, v, cu, cfg.d**-0.5, cfg.causal)
        out.backward(do)
        reps += 1
        if time.perf_counter() - t0 > budget_s or reps >= max_reps:
            break
    return flops / ((time.perf_counter() - t0) / reps) / 1e12, reps


def cpu_baseline(budget_s: float = 24.0) -> dict:
    """Reference path (oracle/cpu_path.py) on the host cores, bounded samples."""
    from oracle import cpu_path

    torch.set_num_threads(_cpu_threads())
    res = {}
    # config 2 (headline): the first sequences of the batch, ~2048 tokens, fwd+bwd
    cfg = W.attn_config(2)
    lens = []
    for i, n in enumerate(cfg.lengths):
        if sum(m for _, m in lens) + n > 2048 and lens:
            break
        lens.append((i, n))
    tf, reps = _cpu_attention_sample(cfg, lens, budget_s * 0.25)
    res["attn"] = {"value": tf, "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
                   "sample": f"config-2 first {len(lens)} sequences ({sum(n for _, n in lens)} tokens), fp32 SDPA + "
                             f"block-diagonal mask + repeat_kv, fwd+bwd autograd, {reps} reps"}
    # config 3: two whole 1024-token images (16 heads, d 64, bidirectional)
    c3 = W.attn_config(3)
    tf, reps = _cpu_attention_sample(c3, [(0, 1024), (1, 1024)], budget_s * 0.15)
    res["attn_config3"] = {"value": tf, "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
                           "sample": f"config 3, 2 of the 16 images (2 x 1024 tokens, 16/16 heads, d 64), fp32 SDPA "
                                     f"+ block-diagonal bidirectional mask, fwd+bwd autograd, {reps} reps"}
    # config 5: the first 2048 tokens of the 16384-token sequence (a causal prefix) plus the first short
    # sequences (81..600 tokens) up to ~1024 tokens
    c5 = W.attn_config(5)
    short = []
    for i, n in enumerate(c5.lengths):
        if n <= 600:
            if sum(m for _, m in short) + n > 1024 and short:
                break
            short.append((i, n))
    big = max(range(len(c5.lengths)), key=lambda i: c5.lengths[i])
    lens5 = [(big, 2048)] + short
    tf, reps = _cpu_attention_sample(c5, lens5, budget_s * 0.15)
    res["attn_config5"] = {"value": tf, "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
                           "sample": f"config 5, the first 2048 tokens of its 16384-token sequence plus {len(short)} "
                                     f"of its short sequences ({sum(n for _, n in short)} tokens, 81..600 each), "
                                     f"12/2 heads, d 128, fp32 SDPA + block-diagonal causal mask + repeat_kv, "
                                     f"fwd+bwd autograd, {reps} reps"}
    # config 1 (CPU-reported in the baseline): the whole batch, forward only
    c1 = W.attn_config(1)
    x1 = W.attn_inputs(c1, device="cpu")
    cu1 = c1.cu_seqlens().tolist()
    q1, k1, v1 = (x1[n].float() for n in ("q", "k", "v"))
    flops1 = 4.0 * c1.d * c1.pairs() * c1.hq
    t0 = time.perf_counter()
    reps = 0
    with torch.no_grad():
        while True:
            cpu_path.sdpa_attention(q1, k1, v1, cu1, c1.d**-0.5, True)
            reps += 1
            if time.perf_counter() - t0 > budget_s * 0.2 or reps >= 20:
                break
    dt1 = (time.perf_counter() - t0) / reps
    res["attn_config1"] = {"value": flops1 / dt1 / 1e12, "unit": "TFLOP/s", "ms": dt1 * 1e3,
                           "cores": torch.get_num_threads(), "kind": "port",
                           "sample": f"config 1 whole batch ({c1.total} tokens, 8 sequences, 14/2 heads, d 64), fp32 "
                                     f"SDPA + block-diagonal causal mask + repeat_kv, forward, {reps} reps"}
    # CE: 256 rows of config 4 against the full vocabulary
    c4 = W.CONFIG4
    g = torch.Generator().manual_seed(W.SEED)
    n = 256
    h = torch.randn(n, c4.hdim, generator=g).to(torch.bfloat16).float().requires_grad_(True)
    w = (0.02 * torch.randn(c4.vocab, c4.hdim, generator=g)).to(torch.bfloat16).float().requires_grad_(True)
    y = W.span_masked_labels(n, c4.vocab, c4.mask_frac, g)
    t0 = time.perf_counter()
    reps = 0
    while True:
        loss = cpu_path.cross_entropy(h, w, y)
        loss.backward()
        reps += 1
        if time.perf_counter() - t0 > budget_s * 0.2 or reps >= 20:
            break
    dt = (time.perf_counter() - t0) / reps
    res["ce"] = {"value": n / dt, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
                 "sample": f"{n} rows of config 4 (hdim 1536, vocab 151936), F.linear + fp32 F.cross_entropy, "
                           f"fwd+bwd autograd, {reps} reps"}
    res["host"] = {"cpu_count": os.cpu_count(), "threads": torch.get_num_threads(), "cpu": platform.processor()}
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ce-chunk", type=int, default=None,
                    help="CE token rows per logits chunk (default: the 2 GiB bound on the chunk's numerators)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-ce", action="store_true")
    ap.add_argument("--skip-rope", action="store_true")
    ap.add_argument("--skip-projector", action="store_true")
    ap.add_argument("--skip-splice", action="store_true")
    ap.add_argument("--attn-only", action="store_true", help="attention configs only (no CE / widening legs)")
    ap.add_argument("--leg", choices=["attn1", "attn2", "attn3", "attn5", "attn6", "ce", "ce_dh", "rope", "rope_attn",
                                      "proj", "splice"],
                    default=None,
                    help="run one leg only and print its timings (a profiling aid: one rocprofv3 counter pass per "
                         "leg attributes every dispatch to its workload); no contract JSON line")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device copy (3 times): the known-size reference that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2

    if args.calibrate_copy:
        src = torch.ones(COPY_BYTES, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[bench] copied {COPY_BYTES} bytes 3 times", file=sys.stderr, flush=True)
        return 0
    if args.attn_only:
        args.skip_ce = args.skip_rope = args.skip_projector = args.skip_splice = True
    if args.leg is not None:
        steps = max(args.steps, 1)
        fns = {"attn1": lambda: bench_attention(1, steps, args.warmup),
               "attn2": lambda: bench_attention(2, steps, args.warmup),
               "attn3": lambda: bench_attention(3, steps, args.warmup),
               "attn5": lambda: bench_attention(5, steps, args.warmup),
               "attn6": lambda: bench_attention(6, steps, args.warmup),
               "ce": lambda: bench_ce(steps, args.warmup, args.ce_chunk, modes=("full",)),
               "ce_dh": lambda: bench_ce(steps, args.warmup, args.ce_chunk, modes=("dh_only",)),
               "rope": lambda: bench_rope(steps, args.warmup),
               "rope_attn": lambda: bench_rope_attention(steps, args.warmup),
               "proj": lambda: bench_projector(steps, args.warmup),
               "splice": lambda: bench_splice(steps, args.warmup)}
        res = fns[args.leg]()
        torch.cuda.synchronize()
        out = {k: (round(v, 6) if isinstance(v, float) else v) for k, v in res.items()
               if isinstance(v, (int, float, str))}
        print(json.dumps({"leg": args.leg, "steps": steps, **out}), flush=True)
        return 0

    # the headline leg first, then the other configurations (all >= MIN_STEPS timed steps)
    steps = max(args.steps, 1)
    leg_steps = max(steps, MIN_STEPS)
    att = bench_attention(2, steps, args.warmup)
    clock = probe_clock_mhz()
    print(f"[bench] config 2 attention fwd+bwd {att['ms_per_step']:.4f} ms/step (median, graph-replayed; eager "
          f"{att['eager_ms_per_step']:.4f}), {att['tflops']:.1f} TFLOP/s (eager per call: plan "
          f"{att['plan_ms'] * 1e3:.1f} us, fwd {att['fwd_ms'] * 1e3:.1f} us, bwd {att['bwd_ms'] * 1e3:.1f} us); "
          f"shader clock after {clock} MHz", file=sys.stderr, flush=True)
    print(f"[bench] config 2 backward modes (graph-replayed): deterministic "
          f"{att['bwd_graph_ms_deterministic'] * 1e3:.1f} us, atomic dQ {att['bwd_graph_ms_atomic'] * 1e3:.1f} us",
          file=sys.stderr, flush=True)
    others = {}
    for idx in (3, 5, 1, 6):
        others[idx] = bench_attention(idx, leg_steps, args.warmup)
        o = others[idx]
        extra = ""
        if "bwd_ms" in o:
            extra = (f", bwd {o['bwd_ms'] * 1e3:.1f} us; graph-replayed backward deterministic "
                     f"{o['bwd_graph_ms_deterministic'] * 1e3:.1f} us, atomic dQ {o['bwd_graph_ms_atomic'] * 1e3:.1f} us")
        print(f"[bench] config {idx} attention {o['ms_per_step']:.4f} ms/step, {o['tflops']:.1f} TFLOP/s (fwd "
              f"{o['fwd_ms'] * 1e3:.1f} us{extra})", file=sys.stderr, flush=True)
    ce = None
    if not args.skip_ce:
        ce = bench_ce(leg_steps, args.warmup, args.ce_chunk)
        print(f"[bench] config 4 fused CE {ce['ms_per_step']:.3f} ms/step (median), {ce['tokens_per_s']:.3e} tokens/s, "
              f"{ce['tflops_all_rows']:.1f} TFLOP/s over all rows, {ce['tflops_executed']:.1f} executed "
              f"(chunk {ce['chunk']} rows); dH only (frozen lm_head) {ce['dh_only_ms']:.3f} ms/step",
              file=sys.stderr, flush=True)
    rope = None
    if not args.skip_rope:
        rope = bench_rope(leg_steps, args.warmup)
        print(f"[bench] fused RoPE fwd {rope['fwd_ms'] * 1e3:.1f} us ({rope['fwd_gbs']:.0f} GB/s), bwd "
              f"{rope['bwd_ms'] * 1e3:.1f} us ({rope['bwd_gbs']:.0f} GB/s) in a graph; one eager call "
              f"{rope['eager_fwd_ms'] * 1e3:.1f} us; reference torch ops fwd+bwd {rope['ref_ms'] * 1e3:.1f} us",
              file=sys.stderr, flush=True)
    ropeattn = None
    if not args.skip_rope:
        ropeattn = bench_rope_attention(leg_steps, args.warmup)
        print(f"[bench] config 2 with RoPE (graph-replayed): attention alone {ropeattn['attention_only_ms'] * 1e3:.1f} "
              f"us, unfused {ropeattn['unfused_ms'] * 1e3:.1f} us, drop-in (dq rotation in the dQ kernel) "
              f"{ropeattn['dropin_ms'] * 1e3:.1f} us, q also rotated in the forward {ropeattn['fused_fwd_ms'] * 1e3:.1f} "
              f"us; under autocast over fp32 weights: stock {ropeattn['autocast_stock_ms'] * 1e3:.1f} us, fused "
              f"{ropeattn['autocast_fused_ms'] * 1e3:.1f} us", file=sys.stderr, flush=True)
    proj = None
    if not args.skip_projector:
        proj = bench_projector(leg_steps, args.warmup)
        print(f"[bench] projector fwd {proj['fwd_ms'] * 1e3:.1f} us ({proj['fwd_tflops']:.0f} TFLOP/s), bwd "
              f"{proj['bwd_ms'] * 1e3:.1f} us ({proj['bwd_tflops']:.0f} TFLOP/s); reference torch ops fwd+bwd "
              f"{proj['ref_ms'] * 1e3:.1f} us", file=sys.stderr, flush=True)
    spl = None
    if not args.skip_splice:
        spl = bench_splice(leg_steps, args.warmup)
        print(f"[bench] splice kernels {spl['fwd_ms'] * 1e3:.1f} us ({spl['gbs']:.0f} GB/s), whole op with its lazy "
              f"count check {spl['op_ms'] * 1e3:.1f} us (host ahead {spl['op_queued_ms'] * 1e3:.1f} us, sync {spl['op_sync_ms'] * 1e3:.1f} us); reference torch ops "
              f"{spl['ref_ms'] * 1e3:.1f} us; table gradient {spl['table_ms'] * 1e3:.1f} us "
              f"({spl['table_gbs']:.0f} GB/s; torch {spl['table_ref_ms'] * 1e3:.1f} us)", file=sys.stderr, flush=True)
    clock_end = probe_clock_mhz()
    cpu = None if args.no_cpu_baseline else cpu_baseline()

    cfg = att["cfg"]
    # the dominant kernel's launch duration: the backward call over a prebuilt plan, graph-replayed (its three
    # kernels back to back, as rocprofv3 times them), in the default (deterministic) mode
    bwd_graph_ms = att["bwd_graph_ms_deterministic" if A.DETERMINISTIC_DEFAULT else "bwd_graph_ms_atomic"]
    bwd_achieved = att["flops_bwd"] / (bwd_graph_ms * 1e-3) / 1e12
    traffic_bwd = measured_traffic("attention_bwd_config2")
    line = {
        "metric": METRIC,
        "value": round(att["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(att["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16, lognormal lengths; no checkpoint)",
        "config": {"workload": "config 2: varlen causal GQA attention fwd+bwd, Qwen2.5-1.5B heads "
                               "(12 q / 2 kv, d 128), 32 lognormal(400, 0.75) sequences, 16384 tokens; "
                               "step = plan build + forward + backward",
                   "timing": f"{GRAPH_STEPS_PER_REPLAY} consecutive steps captured once as a HIP graph and "
                             "replayed; median of the timed replays / steps per replay, events on the replay "
                             "stream (eager_ms_per_step: the same step launched eagerly)",
                   "eager_ms_per_step": round(att["eager_ms_per_step"], 4),
                   "total_tokens": cfg.total, "max_seqlen": cfg.max_seqlen, "pairs": att["pairs"],
                   "pct_bf16_peak": round(100.0 * att["tflops"] / PEAK_BF16_TFLOPS, 2),
                   "mean_ms_per_step": round(att["mean_ms_per_step"], 4),
                   "plan_us": round(att["plan_ms"] * 1e3, 2),
                   "fwd_ms": round(att["fwd_ms"], 4), "bwd_ms": round(att["bwd_ms"], 4),
                   "fwd_tflops": round(att["fwd_tflops"], 2), "bwd_tflops": round(att["bwd_tflops"], 2)},
        "roofline": {"bound": "mfma", "kernel": "attention backward call (dQ + dK/dV + split-tile sum kernels) "
                                               "over the batch's plan, 5 calls per HIP graph, replayed",
                     "duration_us": round(bwd_graph_ms * 1e3, 1),
                     "achieved": round(bwd_achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(bwd_achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic_bwd["bytes"], "traffic_source": traffic_bwd,
                     "algorithmic_bytes": att["bytes_bwd"]},
        "cpu_baseline": cpu["attn"] if cpu else None,
        "gpu_clock_mhz": {"after_headline": None if clock is None else round(clock, 1),
                          "at_end": None if clock_end is None else round(clock_end, 1),
                          "peak_quoted_at": PEAK_CLOCK_MHZ,
                          "method": "siq_probe_clock: shader-clock counter over the 100 MHz counter, one wave per CU"},
        "attention_configs": {str(i): attn_block(o) for i, o in [(2, att)] + sorted(others.items())},
    }
    if cpu:
        line["attention_configs"]["1"]["cpu_baseline"] = cpu["attn_config1"]
        line["attention_configs"]["3"]["cpu_baseline"] = cpu["attn_config3"]
        line["attention_configs"]["5"]["cpu_baseline"] = cpu["attn_config5"]
    if ce is not None:
        traffic_ce = measured_traffic("ce_config4")
        cfg4_n = W.CONFIG4.n
        line["ce"] = {"workload": "config 4: fused linear CE fwd+bwd, h [16384,1536], W [151936,1536], 30% span mask",
                      "tokens_per_s": round(ce["tokens_per_s"], 1), "ms_per_step": round(ce["ms_per_step"], 4),
                      "mean_ms_per_step": round(ce["mean_ms_per_step"], 4),
                      "tflops_all_rows": round(ce["tflops_all_rows"], 2),
                      "pct_bf16_peak_all_rows": round(100.0 * ce["tflops_all_rows"] / PEAK_BF16_TFLOPS, 2),
                      "tflops_executed": round(ce["tflops_executed"], 2), "rows_with_label": ce["n_valid"],
                      "chunk_tokens": ce["chunk"], "numerator_buffer_bytes": ce["e_bytes"],
                      "workspace_bytes": ce["workspace_bytes"],
                      "roofline": {"bound": "mfma", "kernel": "siq_flce_fwd_bwd call (all kernels)",
                                   "achieved": round(ce["tflops_executed"], 2), "peak": PEAK_BF16_TFLOPS,
                                   "unit": "TFLOP/s", "frac": round(ce["tflops_executed"] / PEAK_BF16_TFLOPS, 4),
                                   "work": "6 * rows_with_label * hdim * vocab",
                                   "traffic": traffic_ce["bytes"], "traffic_source": traffic_ce,
                                   "algorithmic_bytes": ce["algorithmic_bytes"]},
                      "cpu_baseline": cpu["ce"] if cpu else None,
                      "dh_only": {"workload": "the same call with a frozen lm_head (dweight = NULL): loss and dHidden "
                                              "only, as the reference trains in stage 1 and stage 2 with LoRA",
                                  "ms_per_step": round(ce["dh_only_ms"], 4),
                                  "tokens_per_s": round(cfg4_n / (ce["dh_only_ms"] * 1e-3), 1),
                                  "tflops_executed": round(4.0 * ce["n_valid"] * W.CONFIG4.hdim * W.CONFIG4.vocab
                                                           / (ce["dh_only_ms"] * 1e-3) / 1e12, 2),
                                  "work": "4 * rows_with_label * hdim * vocab (logits and dH GEMMs)",
                                  "workspace_bytes": ce["dh_only_workspace_bytes"]}}
    if rope is not None:
        line["rope"] = {"workload": "config-2 shape: RoPE of q [16384,12,128] and k [16384,2,128] (Qwen2 layout, "
                                    "packed position ids), forward and backward",
                        "fwd_us": round(rope["fwd_ms"] * 1e3, 2), "bwd_us": round(rope["bwd_ms"] * 1e3, 2),
                        "timing": "20 launches captured in a HIP graph, replayed; events on the launch stream",
                        "eager_call_fwd_us": round(rope["eager_fwd_ms"] * 1e3, 2),
                        "roofline": {"bound": "hbm", "achieved": round(rope["fwd_gbs"], 1), "peak": PEAK_HBM_GBS,
                                     "unit": "GB/s", "frac": round(rope["fwd_gbs"] / PEAK_HBM_GBS, 4),
                                     "algorithmic_bytes": rope["bytes"]},
                        "bwd_gbs": round(rope["bwd_gbs"], 1),
                        "reference_torch_ops_fwd_bwd_us": round(rope["ref_ms"] * 1e3, 2)}
    if ropeattn is not None:
        line["rope_attention"] = {
            "workload": "config 2 step with the decoder's RoPE, plan built outside, graph-replayed: unfused = "
                        "RoPE(q, k) + attention fwd + bwd + RoPE bwd; dropin = the same with the rotation's backward "
                        "of dq inside the dQ kernel and a k-only RoPE bwd; fused_fwd = q also rotated inside the "
                        "attention forward (k-only RoPE fwd); all bitwise the same outputs",
            "attention_only_us": round(ropeattn["attention_only_ms"] * 1e3, 2),
            "unfused_us": round(ropeattn["unfused_ms"] * 1e3, 2), "dropin_us": round(ropeattn["dropin_ms"] * 1e3, 2),
            "fused_fwd_us": round(ropeattn["fused_fwd_ms"] * 1e3, 2),
            "rope_round_trip_unfused_us": round((ropeattn["unfused_ms"] - ropeattn["attention_only_ms"]) * 1e3, 2),
            "rope_cost_dropin_us": round((ropeattn["dropin_ms"] - ropeattn["attention_only_ms"]) * 1e3, 2),
            "autocast": {
                "workload": "the same step under bf16 autocast over fp32 master weights (fp32 cos / sin): stock = "
                            "torch's promoted fp32 rotation + casts to bf16 + attention + autograd; fused = "
                            "flash_attn_varlen_rope_func (siq_rope_fwd_ex / _bwd_ex around the attention); "
                            "bitwise the same gradients",
                "timing": "eager autograd steps queued behind a spin kernel (GPU time per step)",
                "stock_us": round(ropeattn["autocast_stock_ms"] * 1e3, 2),
                "fused_us": round(ropeattn["autocast_fused_ms"] * 1e3, 2)}}
    if proj is not None:
        line["projector"] = {
            "workload": "pixel-shuffle projector fwd+bwd (dx, dweight): 16 tiles x 32x32 patches x 1024 -> r 2 -> "
                        "[4096 tokens, 4096] x [1536, 4096]^T",
            "fwd_us": round(proj["fwd_ms"] * 1e3, 2), "bwd_us": round(proj["bwd_ms"] * 1e3, 2),
            "timing": "5 launches captured in a HIP graph, replayed; events on the launch stream",
            "roofline": {"bound": "mfma", "achieved": round(proj["tflops"], 1), "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(proj["tflops"] / PEAK_BF16_TFLOPS, 4)},
            "reference_torch_ops_fwd_bwd_us": round(proj["ref_ms"] * 1e3, 2)}
    if spl is not None:
        line["splice"] = {
            "workload": "vision-token splice: 16384 tokens x 1536 (4096 image tokens), 151936-row embedding table",
            "kernels_us": round(spl["fwd_ms"] * 1e3, 2),
            "timing": "10 launches captured in a HIP graph, replayed; events on the launch stream",
            "roofline": {"bound": "hbm", "achieved": round(spl["gbs"], 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(spl["gbs"] / PEAK_HBM_GBS, 4), "algorithmic_bytes": spl["bytes"]},
            "op_with_count_check_us": round(spl["op_ms"] * 1e3, 2),
            "op_with_count_check_host_ahead_us": round(spl["op_queued_ms"] * 1e3, 2),
            "op_with_sync_count_check_us": round(spl["op_sync_ms"] * 1e3, 2),
            "op_timing": "eager calls back to back (the host's launch work is on the clock); host_ahead: the calls "
                         "queued behind a spin kernel, so the GPU's own time per call",
            "reference_torch_ops_us": round(spl["ref_ms"] * 1e3, 2),
            "table_gradient": {
                "workload": "embedding-table gradient of the same 16384 tokens into [151936, 1536] bf16 (image "
                            "token skipped)",
                "us": round(spl["table_ms"] * 1e3, 2), "timing": "5 launches in a HIP graph, replayed",
                "roofline": {"bound": "hbm", "achieved": round(spl["table_gbs"], 1), "peak": PEAK_HBM_GBS,
                             "unit": "GB/s", "frac": round(spl["table_gbs"] / PEAK_HBM_GBS, 4),
                             "algorithmic_bytes": spl["table_bytes"]},
                "torch_embedding_dense_backward_us": round(spl["table_ref_ms"] * 1e3, 2)}}
    if cpu:
        line["host"] = cpu["host"]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
