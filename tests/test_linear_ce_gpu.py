"""Fused linear head + cross-entropy through the C ABI
(sm_linear_cross_entropy / _backward) against float64 autograd of the
materialised computation, on the reference's own test cases
(summa-llm/src/model/linear_cross_entropy/tests.rs:19-126 and :141-216) and
at a 65536-entry vocabulary."""
import math

import numpy as np
import pytest
import torch

from summa_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _expected(hidden, weight, bias, targets, lv, grad_output=1.0):
    """f64 autograd of CE(hidden W[:lv]^T + b[:lv], targets) (mean over
    tokens): loss, dhidden, dweight (rows >= lv zero), dbias."""
    h = hidden.double().cpu().requires_grad_()
    w = weight.double().cpu().requires_grad_()
    b = bias.double().cpu().requires_grad_() if bias is not None else None
    logits = h @ w[:lv].T
    if b is not None:
        logits = logits + b[:lv]
    loss = torch.nn.functional.cross_entropy(logits, targets.long().cpu())
    (loss * grad_output).backward()
    return loss.detach(), h.grad, w.grad, (b.grad if b is not None else None)


def _check(dev, hidden, weight, bias, targets, lv, chunk, grad_output=1.0, tol=1e-6, rtol=0.0):
    hd, wd = hidden.to(dev), weight.to(dev)
    bd = bias.to(dev) if bias is not None else None
    td = targets.to(dev)
    loss, lp = ops.linear_cross_entropy(hd, wd, bd, td, lv, chunk, want_logprob=True)
    go = torch.tensor([grad_output], dtype=torch.float32, device=dev)
    gh, gw, gb = ops.linear_cross_entropy_backward(hd, wd, bd, td, go, lv, chunk)
    torch.cuda.synchronize()
    e_loss, e_h, e_w, e_b = _expected(hidden, weight, bias, targets, lv, grad_output)
    assert abs(float(loss.cpu()[0]) - float(e_loss)) <= tol + rtol * abs(float(e_loss))
    # per-token log-probs sum to -tokens * loss
    assert abs(float(lp.double().sum()) + float(e_loss) * len(targets)) <= \
        (tol + rtol * abs(float(e_loss))) * len(targets)
    stored = weight.shape[0]
    gw_c = gw.cpu()
    if stored > lv:
        assert torch.all(gw_c[lv:] == 0), "padded weight rows must get exactly zero gradient"
        if gb is not None:
            assert torch.all(gb.cpu()[lv:] == 0), "padded bias entries must get exactly zero"
    for got, want, name in ((gh.cpu(), e_h, "hidden"), (gw_c, e_w, "weight"),
                            (None if gb is None else gb.cpu(), e_b, "bias")):
        if want is None:
            assert got is None
            continue
        scale = float(want.abs().max())
        err = float((got.double() - want).abs().max())
        print(f"grad {name}: max |err| {err:.2e} (max |g| {scale:.2e})", flush=True)
        assert err <= tol + rtol * scale, name


@pytest.mark.parametrize("stored", [11, 16])
@pytest.mark.parametrize("use_bias", [False, True])
def test_reference_chunked_case(dev, stored, use_bias):
    """tests.rs:19-126: 7 tokens, hidden 5, logical vocab 11 stored as 11 or
    16, chunk 3, sin / cos generators, bias 0.01 i; every output within 1e-6
    of the materialised cross-entropy, padded gradients exactly 0."""
    print(f"case reference chunked stored={stored} bias={use_bias}", flush=True)
    T, d, lv = 7, 5, 11
    i = torch.arange(T * d, dtype=torch.float32)
    hidden = (torch.sin(i * 0.071) * 0.2).reshape(T, d)
    j = torch.arange(stored * d, dtype=torch.float32)
    weight = (torch.cos(j * 0.113) * 0.3).reshape(stored, d)
    bias = torch.arange(stored, dtype=torch.float32) * 0.01 if use_bias else None
    targets = torch.tensor([0, 3, 7, 2, 10, 4, 1], dtype=torch.int32)
    _check(dev, hidden, weight, bias, targets, lv, 3, tol=1e-6)


@pytest.mark.parametrize("use_bias", [False, True])
def test_reference_gpu_case(dev, use_bias):
    """tests.rs:141-216: (tokens 7, hidden 8, stored 64, logical 50, chunk 3)
    with the integer-modular generators; the reference allows 1e-2 for its
    bf16 tensor cores, this f32-grade path is held to 1e-5."""
    print(f"case reference gpu bias={use_bias}", flush=True)
    T, d, stored, lv, chunk = 7, 8, 64, 50, 3
    hidden = torch.tensor([((i * 37 + 11) % 23) * 0.11 - 1.2 for i in range(T * d)],
                          dtype=torch.float32).reshape(T, d)
    weight = torch.tensor([((i * 29 + 5) % 19) * 0.07 - 0.6 for i in range(stored * d)],
                          dtype=torch.float32).reshape(stored, d)
    bias = torch.tensor([((i * 13 + 3) % 17) * 0.05 - 0.4 for i in range(stored)],
                        dtype=torch.float32) if use_bias else None
    targets = torch.tensor([(i * 7 + 2) % lv for i in range(T)], dtype=torch.int32)
    _check(dev, hidden, weight, bias, targets, lv, chunk, tol=1e-5)


@pytest.mark.parametrize("tokens,chunk", [(300, 128), (97, 512)])
def test_large_vocab(dev, tokens, chunk):
    """V = 65536 stored, 65500 logical, d 256 (the matrix-core GEMM path),
    bias, grad_output 0.37, chunks that do not divide the tokens (or exceed
    them): loss within 1e-5 relative, gradients within 1e-4 of their largest
    entry against f64 autograd."""
    print(f"case large vocab tokens={tokens} chunk={chunk}", flush=True)
    g = torch.Generator().manual_seed(tokens)
    d, stored, lv = 256, 65536, 65500
    hidden = torch.randn(tokens, d, generator=g)
    weight = torch.randn(stored, d, generator=g) * 0.05
    bias = torch.randn(stored, generator=g) * 0.1
    targets = torch.randint(0, lv, (tokens,), generator=g, dtype=torch.int32)
    _check(dev, hidden, weight, bias, targets, lv, chunk, grad_output=0.37, tol=0.0, rtol=1e-4)


def test_errors_follow_the_reference(dev):
    h = torch.zeros(4, 8, device=dev)
    w = torch.zeros(16, 8, device=dev)
    t = torch.zeros(4, dtype=torch.int32, device=dev)
    with pytest.raises(_lib.SummaError, match="chunk size must be positive"):
        ops.linear_cross_entropy(h, w, None, t, 16, 0)
    with pytest.raises(_lib.SummaError, match="logical vocabulary 17 must be in 1..=16"):
        ops.linear_cross_entropy(h, w, None, t, 17, 2)
    loss = ops.linear_cross_entropy(h, w, None, t, 16, 3)
    assert math.isclose(float(loss.cpu()[0]), math.log(16), rel_tol=1e-6)
    assert np.isfinite(loss.cpu().numpy()).all()
