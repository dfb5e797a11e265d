"""The float-weight grouped expert projections and the route permutation at the
reference's dispatch seam (sm_grouped_linear / _backward,
sm_grouped_swiglu_mlp / _backward: GroupedLinearBackend,
summa-llm/src/model/grouped_linear.rs:23-111, 779-826; sm_row_permute:
RowPermutationBackend, row_permute.rs:33-41) against float64 on the host:
the reference's own test case (grouped_linear.rs tests: counts [2, 0, 5],
input 7 x 4, weight [3, 4, 5]), ragged shapes on the matrix-core GEMM path,
the SwiGLU MLP against autograd, and the permutation bit for bit."""
import math

import numpy as np
import pytest
import torch

from summa_amd import _lib
from summa_amd._lib import call

pytestmark = pytest.mark.gpu


def _st():
    return torch.cuda.current_stream().cuda_stream


def _counts(c):
    return np.ascontiguousarray(c, dtype=np.int64)


def _grouped(x, w, counts):
    """f64 restatement: each expert's consecutive rows times its matrix."""
    out, off = [], 0
    for e, c in enumerate(counts):
        out.append(x[off:off + c] @ w[e])
        off += c
    return np.concatenate(out) if out else np.zeros((0, w.shape[2]))


def _run_linear(x, w, counts, grad):
    dev = torch.device("cuda:0")
    xd = torch.from_numpy(x.astype(np.float32)).to(dev)
    wd = torch.from_numpy(w.astype(np.float32)).to(dev)
    gd = torch.from_numpy(grad.astype(np.float32)).to(dev)
    R, din = x.shape
    E, _, dout = w.shape
    c = _counts(counts)
    y = torch.full((R, dout), float("nan"), device=dev)
    call("sm_grouped_linear", xd.data_ptr(), wd.data_ptr(), c.ctypes.data, E, R, din, dout,
         y.data_ptr(), _st())
    gx = torch.full_like(xd, float("nan"))
    gw = torch.full_like(wd, float("nan"))
    call("sm_grouped_linear_backward", xd.data_ptr(), wd.data_ptr(), gd.data_ptr(), c.ctypes.data,
         E, R, din, dout, gx.data_ptr(), gw.data_ptr(), _st())
    return y.cpu().double().numpy(), gx.cpu().double().numpy(), gw.cpu().double().numpy()


def test_grouped_linear_reference_case(dev):
    """The reference's grouped-linear test data (grouped_linear.rs tests:
    input[i] = 0.4 sin(0.19 i) over [7, 4], weight[i] = 0.3 cos(0.13 i) over
    [3, 4, 5], counts [2, 0, 5], loss = sum(output * factors) with
    factors[i] = 0.2 + sin(0.07 i) over [7, 5]): output and both gradients
    against float64, the empty expert's weight gradient exactly 0."""
    counts = [2, 0, 5]
    x = np.array([math.sin(i * 0.19) * 0.4 for i in range(28)]).reshape(7, 4)
    w = np.array([math.cos(i * 0.13) * 0.3 for i in range(60)]).reshape(3, 4, 5)
    f = np.array([0.2 + math.sin(i * 0.07) for i in range(35)]).reshape(7, 5)
    x32 = x.astype(np.float32).astype(np.float64)
    w32 = w.astype(np.float32).astype(np.float64)
    f32 = f.astype(np.float32).astype(np.float64)
    y, gx, gw = _run_linear(x, w, counts, f)
    np.testing.assert_allclose(y, _grouped(x32, w32, counts), rtol=1e-6, atol=1e-7)
    # d/dx sum(y * f) = f W_e^T; d/dW_e = x_e^T f_e
    want_gx = np.concatenate([f32[0:2] @ w32[0].T, f32[2:7] @ w32[2].T])
    np.testing.assert_allclose(gx, want_gx, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(gw[0], x32[0:2].T @ f32[0:2], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(gw[2], x32[2:7].T @ f32[2:7], rtol=1e-6, atol=1e-7)
    assert np.all(gw[1] == 0.0)


@pytest.mark.parametrize("counts,din,dout", [([700, 0, 513, 1200], 512, 640),
                                             ([3, 17, 0, 1, 64], 96, 40)])
def test_grouped_linear_ragged_against_f64(dev, counts, din, dout):
    """Ragged expert groups (an empty expert, single rows, and groups large
    enough for the matrix-core GEMM path): output, grad_input and
    grad_weight within f32-grade error of float64."""
    print(f"case grouped linear counts={counts} din={din} dout={dout}", flush=True)
    rng = np.random.default_rng(sum(counts) + din)
    R, E = sum(counts), len(counts)
    x = rng.normal(0, 1, (R, din)).astype(np.float32).astype(np.float64)
    w = rng.normal(0, 0.05, (E, din, dout)).astype(np.float32).astype(np.float64)
    g = rng.normal(0, 1, (R, dout)).astype(np.float32).astype(np.float64)
    y, gx, gw = _run_linear(x, w, counts, g)
    want_y = _grouped(x, w, counts)
    want_gx = _grouped(g, np.transpose(w, (0, 2, 1)), counts)
    offs = np.concatenate([[0], np.cumsum(counts)])
    want_gw = np.stack([x[offs[e]:offs[e + 1]].T @ g[offs[e]:offs[e + 1]] for e in range(E)])
    for got, want in ((y, want_y), (gx, want_gx), (gw, want_gw)):
        scale = np.abs(want).max() + 1e-30
        assert np.abs(got - want).max() <= 2e-6 * scale, float(np.abs(got - want).max() / scale)


def test_grouped_swiglu_mlp_against_autograd(dev):
    """sm_grouped_swiglu_mlp (projected = [gate | value], hidden = silu(gate)
    value, output) and its backward against torch autograd in float64."""
    counts = [300, 0, 257, 41]
    E, R, d, I, dout = len(counts), sum(counts), 256, 160, 192
    rng = np.random.default_rng(9)
    x = torch.from_numpy(rng.normal(0, 1, (R, d)).astype(np.float32)).double()
    wi = torch.from_numpy(rng.normal(0, 0.06, (E, d, 2 * I)).astype(np.float32)).double()
    wd = torch.from_numpy(rng.normal(0, 0.06, (E, I, dout)).astype(np.float32)).double()
    g = torch.from_numpy(rng.normal(0, 1, (R, dout)).astype(np.float32)).double()
    x.requires_grad_(True)
    wi.requires_grad_(True)
    wd.requires_grad_(True)
    outs, projs, hids, off = [], [], [], 0
    for e, c in enumerate(counts):
        p = x[off:off + c] @ wi[e]
        h = torch.nn.functional.silu(p[:, :I]) * p[:, I:]
        outs.append(h @ wd[e])
        projs.append(p)
        hids.append(h)
        off += c
    out_t, proj_t, hid_t = torch.cat(outs), torch.cat(projs), torch.cat(hids)
    (out_t * g).sum().backward()
    dv = torch.device("cuda:0")
    xd, wid, wdd, gd = (t.detach().float().contiguous().to(dv) for t in (x, wi, wd, g))
    c = _counts(counts)
    out = torch.empty(R, dout, device=dv)
    proj = torch.empty(R, 2 * I, device=dv)
    hid = torch.empty(R, I, device=dv)
    call("sm_grouped_swiglu_mlp", xd.data_ptr(), wid.data_ptr(), wdd.data_ptr(), c.ctypes.data, E,
         R, d, I, dout, out.data_ptr(), proj.data_ptr(), hid.data_ptr(), _st())
    gx, gwi, gwd = torch.empty_like(xd), torch.empty_like(wid), torch.empty_like(wdd)
    scratch = torch.empty(R * 3 * I, device=dv)
    call("sm_grouped_swiglu_mlp_backward", xd.data_ptr(), wid.data_ptr(), wdd.data_ptr(),
         c.ctypes.data, E, R, d, I, dout, proj.data_ptr(), hid.data_ptr(), gd.data_ptr(),
         gx.data_ptr(), gwi.data_ptr(), gwd.data_ptr(), scratch.data_ptr(), _st())
    for got, want in ((out, out_t), (proj, proj_t), (hid, hid_t), (gx, x.grad), (gwi, wi.grad),
                      (gwd, wd.grad)):
        want = want.detach()
        err = float((got.cpu().double() - want).abs().max() / (want.abs().max() + 1e-30))
        assert err <= 5e-6, err
    assert torch.count_nonzero(gwi[1]) == 0 and torch.count_nonzero(gwd[1]) == 0


@pytest.mark.parametrize("dtype,cols", [(_lib.SM_F32, 768), (_lib.SM_F32, 777), (_lib.SM_BF16, 333),
                                        (_lib.SM_BF16, 2048), (_lib.SM_F16, 5)])
def test_row_permute_bit_exact_and_inverse(dev, dtype, cols):
    """out[i] = input[order[i]] bit for bit (16-byte, 4-byte and 2-byte row
    copies), the inverse permutation restores the input (the backward of
    row_permute_inner), and an out-of-range order entry gives a zero row."""
    print(f"case row permute dtype={dtype} cols={cols}", flush=True)
    rows = 1000
    tdt = {_lib.SM_F32: torch.float32, _lib.SM_BF16: torch.bfloat16, _lib.SM_F16: torch.float16}[dtype]
    g = torch.Generator(device=dev).manual_seed(cols)
    x = torch.randn(rows, cols, generator=g, device=dev).to(tdt)
    order = torch.randperm(rows, generator=g, device=dev).to(torch.int32)
    inv = torch.empty_like(order)
    inv[order.long()] = torch.arange(rows, dtype=torch.int32, device=dev)
    y = torch.empty_like(x)
    call("sm_row_permute", x.data_ptr(), dtype, rows, cols, order.data_ptr(), y.data_ptr(), _st())
    assert torch.equal(y.view(torch.int16) if tdt != torch.float32 else y.view(torch.int32),
                       (x.index_select(0, order.long())).view(
                           torch.int16 if tdt != torch.float32 else torch.int32))
    z = torch.empty_like(x)
    call("sm_row_permute", y.data_ptr(), dtype, rows, cols, inv.data_ptr(), z.data_ptr(), _st())
    assert torch.equal(z, x)
    bad = order.clone()
    bad[7] = rows + 3
    call("sm_row_permute", x.data_ptr(), dtype, rows, cols, bad.data_ptr(), y.data_ptr(), _st())
    assert torch.count_nonzero(y[7]) == 0


def test_grouped_linear_rejects_bad_counts(dev):
    x = torch.zeros(6, 4, device=dev)
    w = torch.zeros(2, 4, 3, device=dev)
    y = torch.zeros(6, 3, device=dev)
    for bad, msg in (([2, 3], "cover the input"), ([7, -1], "negative count")):
        c = _counts(bad)
        with pytest.raises(_lib.SummaError, match=msg):
            call("sm_grouped_linear", x.data_ptr(), w.data_ptr(), c.ctypes.data, 2, 6, 4, 3,
                 y.data_ptr(), _st())


def test_python_mirrors_equal_the_abi_calls(dev):
    """summa_amd.ops' grouped_linear / _backward, grouped_swiglu_mlp / _backward
    and row_permute (the reference's function names and argument order) give
    the C-ABI calls' bits and reject counts that do not cover the input."""
    from summa_amd import ops
    counts = [3, 0, 6, 2]
    E, R, d, I, dout = 4, 11, 32, 24, 16
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(R, d, generator=g, device=dev)
    w = torch.randn(E, d, dout, generator=g, device=dev) * 0.1
    grad = torch.randn(R, dout, generator=g, device=dev)
    c = _counts(counts)
    y = torch.empty(R, dout, device=dev)
    call("sm_grouped_linear", x.data_ptr(), w.data_ptr(), c.ctypes.data, E, R, d, dout,
         y.data_ptr(), _st())
    assert torch.equal(ops.grouped_linear(x, w, counts), y)
    gx, gw = ops.grouped_linear_backward(x, w, grad, counts)
    gx2, gw2 = torch.empty_like(x), torch.empty_like(w)
    call("sm_grouped_linear_backward", x.data_ptr(), w.data_ptr(), grad.data_ptr(), c.ctypes.data,
         E, R, d, dout, gx2.data_ptr(), gw2.data_ptr(), _st())
    assert torch.equal(gx, gx2) and torch.equal(gw, gw2)
    wi = torch.randn(E, d, 2 * I, generator=g, device=dev) * 0.1
    wd = torch.randn(E, I, dout, generator=g, device=dev) * 0.1
    out, proj, hid = ops.grouped_swiglu_mlp(x, wi, wd, counts, I)
    assert torch.equal(proj, ops.grouped_linear(x, wi, counts))
    assert torch.equal(hid, ops.swiglu(proj))
    assert torch.equal(out, ops.grouped_linear(hid, wd, counts))
    gxm, gwi, gwd = ops.grouped_swiglu_mlp_backward(x, wi, wd, counts, proj, hid, grad, I)
    gh, gwd2 = ops.grouped_linear_backward(hid, wd, grad, counts)
    gxm2, gwi2 = ops.grouped_linear_backward(x, wi, ops.swiglu_backward(proj, gh), counts)
    assert torch.equal(gwd, gwd2) and torch.equal(gxm, gxm2) and torch.equal(gwi, gwi2)
    order = torch.randperm(R, generator=g, device=dev).to(torch.int32)
    assert torch.equal(ops.row_permute(x, order), x.index_select(0, order.long()))
    with pytest.raises(ValueError, match="cover the input"):
        ops.grouped_linear(x, w, [3, 0, 6, 1])
