"""GPU parity of the pixel-shuffle projector (through the C ABI).

Small and medium shapes against the fp64 CPU oracle (oracle/projector.py),
the production shape (16 SigLIP2-512 tiles -> Qwen2.5-1.5B) against the
reference's own torch ops in fp32.  Tolerance: relative Frobenius error
<= 2e-2 on y, dx and dweight (bf16 inputs, fp32 accumulation); repeat calls
are bitwise identical (split-K partial sums are added in a fixed order).
"""

import numpy as np
import pytest
import torch

from oracle import projector as op
from siq_vl_amd import projector as P

pytestmark = pytest.mark.gpu

TOL = 2e-2
DEV = "cuda"


def rel(x, ref) -> float:
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(x - ref) / max(np.linalg.norm(ref), 1e-30))


def make(batch, side, dv, r, n, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, side * side, dv, generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(n, dv * r * r, generator=g)).to(torch.bfloat16)
    dy = torch.randn(batch, (side // r) ** 2, n, generator=g).to(torch.bfloat16)
    return x, w, dy


def reference_torch(x, w, r):
    """SiQ_VLProjector.forward (modeling.py:74-105) as torch runs it, in fp32."""
    b, seq, d = x.shape
    side = int(seq**0.5)
    xs = x.view(b, side, side, d).reshape(b, side // r, r, side // r, r, d).permute(0, 1, 3, 2, 4, 5).contiguous()
    return torch.nn.functional.linear(xs.reshape(b, (side // r) ** 2, d * r * r), w)


# (batch, side, dv, r, n): tails in every GEMM dimension, r = 3 (the 81-token grid), split-K in the
# forward (few tiles, long k) and in dweight (1024 tokens)
CASES = [(2, 4, 64, 2, 40), (3, 6, 128, 3, 72), (1, 32, 64, 2, 264), (2, 9, 64, 3, 8), (2, 32, 1024, 2, 1536),
         (16, 16, 256, 2, 512), (1, 27, 64, 3, 136)]


@pytest.mark.parametrize("case", CASES)
def test_vs_oracle(case):
    batch, side, dv, r, n = case
    print(f"projector {case}", flush=True)
    x, w, dy = make(batch, side, dv, r, n)
    y = P.proj_fwd(x.to(DEV), w.to(DEV), r)
    dx, dw = P.proj_bwd(x.to(DEV), w.to(DEV), dy.to(DEV), r)
    torch.cuda.synchronize()
    xf, wf, gf = x.double().numpy(), w.double().numpy(), dy.double().numpy()
    ref_y = op.projector_fwd(xf, wf, r)
    ref_dx, ref_dw = op.projector_bwd(xf, wf, gf, r)
    assert y.shape == ref_y.shape and dx.shape == x.shape and dw.shape == w.shape
    ry, rdx, rdw = rel(y.float().cpu(), ref_y), rel(dx.float().cpu(), ref_dx), rel(dw.float().cpu(), ref_dw)
    print(f"  y {ry:.2e} dx {rdx:.2e} dw {rdw:.2e}", flush=True)
    assert ry <= TOL and rdx <= TOL and rdw <= TOL


def test_repeat_is_bitwise():
    x, w, dy = (t.to(DEV) for t in make(16, 16, 256, 2, 512, seed=1))
    a = (P.proj_fwd(x, w, 2), *P.proj_bwd(x, w, dy, 2))
    b = (P.proj_fwd(x, w, 2), *P.proj_bwd(x, w, dy, 2))
    for u, v in zip(a, b):
        assert torch.equal(u.view(torch.int16), v.view(torch.int16))


def test_autograd_casts_and_needs_input_grad():
    print("projector autograd", flush=True)
    x, w, dy = make(2, 8, 64, 2, 24, seed=2)
    xg = x.float().to(DEV).requires_grad_()
    wg = w.float().to(DEV).requires_grad_()  # fp32 master weight, as under autocast
    y = P.pixel_shuffle_linear(xg, wg, 2)
    assert y.dtype == torch.bfloat16
    y.backward(dy.to(DEV))
    ref_dx, ref_dw = op.projector_bwd(x.double().numpy(), w.double().numpy(), dy.double().numpy(), 2)
    assert xg.grad.dtype == torch.float32 and wg.grad.dtype == torch.float32
    assert rel(xg.grad.cpu(), ref_dx) <= TOL and rel(wg.grad.cpu(), ref_dw) <= TOL
    # a frozen vision tower: no dx
    w2 = w.to(DEV).requires_grad_()
    P.pixel_shuffle_linear(x.to(DEV), w2, 2).backward(dy.to(DEV))
    assert rel(w2.grad.float().cpu(), ref_dw) <= TOL


def test_dropin_projector_module():
    print("projector drop-in", flush=True)

    class Projector(torch.nn.Module):  # the reference module's attributes (modeling.py:53-60)
        def __init__(self, dv, n, r):
            super().__init__()
            self.vision_pixel_shuffle_factor = r
            self.mlp = torch.nn.Linear(dv * r * r, n, bias=False)

        def forward(self, x):
            return self.mlp(reference_torch_bf16(x, self.vision_pixel_shuffle_factor))

    def reference_torch_bf16(x, r):
        b, seq, d = x.shape
        side = int(seq**0.5)
        xs = x.view(b, side, side, d).reshape(b, side // r, r, side // r, r, d).permute(0, 1, 3, 2, 4, 5).contiguous()
        return xs.reshape(b, (side // r) ** 2, d * r * r)

    torch.manual_seed(0)
    ref = Projector(128, 96, 2).to(DEV).to(torch.bfloat16)
    ours = Projector(128, 96, 2).to(DEV).to(torch.bfloat16)
    ours.load_state_dict(ref.state_dict())
    P.enable_fused_projector(ours)
    x, _, dy = make(3, 16, 128, 2, 96, seed=3)
    x1 = x.to(DEV).requires_grad_()
    x2 = x.to(DEV).requires_grad_()
    y1 = ref.float()(x1.float())
    y1.backward(dy.to(DEV).float())
    y2 = ours(x2)
    y2.backward(dy.to(DEV))
    assert rel(y2.float().detach().cpu(), y1.detach().cpu()) <= TOL
    assert rel(x2.grad.float().cpu(), x1.grad.float().cpu()) <= TOL
    assert rel(ours.mlp.weight.grad.float().cpu(), ref.mlp.weight.grad.float().cpu()) <= TOL


def test_reference_errors_and_empty_batch():
    w = torch.zeros(8, 64 * 4, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="not a perfect square"):
        P.pixel_shuffle_linear(torch.zeros(1, 15, 64, dtype=torch.bfloat16, device=DEV), w, 2)
    with pytest.raises(ValueError, match="not divisible by scale factor"):
        P.pixel_shuffle_linear(torch.zeros(1, 9, 64, dtype=torch.bfloat16, device=DEV), w, 2)
    x0 = torch.zeros(0, 16, 64, dtype=torch.bfloat16, device=DEV)
    y = P.proj_fwd(x0, w, 2)
    assert y.shape == (0, 4, 8)
    dy0 = torch.zeros(0, 4, 8, dtype=torch.bfloat16, device=DEV)
    _, dw = P.proj_bwd(x0, torch.ones_like(w), dy0, 2)
    torch.cuda.synchronize()
    assert bool((dw == 0).all())


@pytest.mark.slow
def test_production_shape_vs_torch_fp32():
    # 16 SigLIP2-large-512 tiles (32 x 32 patches, 1024 features) -> Qwen2.5-1.5B (1536), r = 2
    print("projector production shape", flush=True)
    x, w, dy = (t.to(DEV) for t in make(16, 32, 1024, 2, 1536, seed=4))
    y = P.proj_fwd(x, w, 2)
    dx, dw = P.proj_bwd(x, w, dy, 2)
    xf = x.float().requires_grad_()
    wf = w.float().requires_grad_()
    yf = reference_torch(xf, wf, 2)
    yf.backward(dy.float())
    ry = float((y.float() - yf).norm() / yf.norm())
    rdx = float((dx.float() - xf.grad).norm() / xf.grad.norm())
    rdw = float((dw.float() - wf.grad).norm() / wf.grad.norm())
    print(f"  y {ry:.2e} dx {rdx:.2e} dw {rdw:.2e}", flush=True)
    assert ry <= TOL and rdx <= TOL and rdw <= TOL
