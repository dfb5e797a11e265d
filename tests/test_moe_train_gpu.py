"""MoE training kernels (moe_dispatch.rs:244-384, fused_swiglu.rs:106-150)
against torch.autograd (float64, CPU) of the forward expressions: an
independent derivation of each backward. bf16 variants against the f32
kernels at bf16 resolution."""
import numpy as np
import pytest
import torch

from summa_amd import ops

pytestmark = pytest.mark.gpu


def _plan(dev, T, k, E, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    return ops.moe_route_plan(idx.to(dev), E)


@pytest.mark.parametrize("T,k,E,d", [(37, 2, 8, 96), (128, 2, 32, 2048), (5, 1, 3, 130)])
def test_gather_forward_and_backward_match_autograd(dev, T, k, E, d):
    plan = _plan(dev, T, k, E, T)
    order = plan.order.cpu().long()
    x = torch.randn(T, d, dtype=torch.float64)
    xg = x.clone().requires_grad_(True)
    routed_ref = xg[order // k]
    routed = ops.moe_gather(x.float().to(dev), plan)
    np.testing.assert_array_equal(routed.cpu().numpy(), routed_ref.detach().float().numpy())
    g = torch.randn(T * k, d, dtype=torch.float64)
    routed_ref.backward(g)
    got = ops.moe_gather_backward(g.float().to(dev), plan).cpu().double()
    torch.testing.assert_close(got, xg.grad, rtol=1e-6, atol=1e-6)
    # adjoint: <gather(x), g> == <x, gather^T(g)>
    lhs = float((routed.double().cpu() * g).sum())
    rhs = float((x * got).sum())
    assert abs(lhs - rhs) <= 1e-5 * (abs(lhs) + 1)


@pytest.mark.parametrize("T,k,E,d", [(37, 2, 8, 96), (128, 2, 32, 2048)])
def test_combine_backward_matches_autograd(dev, T, k, E, d):
    plan = _plan(dev, T, k, E, T + 1)
    inv = plan.inverse.cpu().long()
    routed = torch.randn(T * k, d, dtype=torch.float64, requires_grad=True)
    w = torch.rand(T, k, dtype=torch.float64, requires_grad=True)
    out = (routed[inv].view(T, k, d) * w.unsqueeze(-1)).sum(1)
    g = torch.randn(T, d, dtype=torch.float64)
    out.backward(g)
    gr, gw = ops.moe_combine_backward(g.float().to(dev), routed.detach().float().to(dev),
                                      w.detach().float().to(dev), plan)
    torch.testing.assert_close(gr.cpu().double(), routed.grad, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(gw.cpu().double(), w.grad, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("rows,F", [(64, 1408), (7, 100)])
def test_swiglu_forward_and_backward_match_autograd(dev, rows, F):
    gv = (torch.randn(rows, 2 * F, dtype=torch.float64) * 3).requires_grad_(True)
    g, v = gv[:, :F], gv[:, F:]
    out = torch.nn.functional.silu(g) * v
    dy = torch.randn(rows, F, dtype=torch.float64)
    out.backward(dy)
    y = ops.swiglu(gv.detach().float().to(dev))
    torch.testing.assert_close(y.cpu().double(), out.detach(), rtol=1e-5, atol=1e-6)
    dgv = ops.swiglu_backward(gv.detach().float().to(dev), dy.float().to(dev))
    torch.testing.assert_close(dgv.cpu().double(), gv.grad, rtol=1e-5, atol=1e-5)


def test_bf16_variants_follow_f32_at_bf16_resolution(dev):
    T, k, E, d, F = 64, 2, 8, 256, 128
    plan = _plan(dev, T, k, E, 3)
    x = torch.randn(T, d, device=dev)
    xb = x.bfloat16()
    assert torch.equal(ops.moe_gather(xb, plan), ops.moe_gather(xb.float(), plan).bfloat16())
    g = torch.randn(T * k, d, device=dev).bfloat16()
    a = ops.moe_gather_backward(g, plan).float()
    b = ops.moe_gather_backward(g.float(), plan)
    torch.testing.assert_close(a, b, rtol=2 ** -8, atol=1e-6)
    gv = torch.randn(T, 2 * F, device=dev).bfloat16()
    dy = torch.randn(T, F, device=dev).bfloat16()
    torch.testing.assert_close(ops.swiglu_backward(gv, dy).float(),
                               ops.swiglu_backward(gv.float(), dy.float()), rtol=2 ** -7, atol=1e-6)
