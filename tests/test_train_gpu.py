"""Policy-update path for fp32 models (summa_amd/train.py over the train.hip
kernels) against torch.autograd in float64 on the CPU: each backward kernel,
the whole policy gradient of sum(dlp * lp) through an independent torch
restatement of the decoder, AdamW against torch.optim.AdamW, and Muon's
Newton-Schulz against its formula and the orthogonality it aims for."""
import math

import numpy as np
import pytest
import torch

import oracle
from summa_amd import _lib, ops, train
from summa_amd._lib import call
from summa_amd.model import Model, ModelConfig

pytestmark = pytest.mark.gpu


def _st():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_ex_transposes(dev, ta, tb):
    M, N, K = 77, 130, 45
    rng = np.random.default_rng(ta * 2 + tb)
    A = rng.normal(0, 1, (K, M) if ta else (M, K))
    B = rng.normal(0, 1, (N, K) if tb else (K, N))
    C = rng.normal(0, 1, (M, N))
    ref = 0.5 * ((A.T if ta else A) @ (B.T if tb else B)) + 2.0 * C
    out = torch.from_numpy(C.astype(np.float32)).to(dev)
    train.gemm(torch.from_numpy(A.astype(np.float32)).to(dev), torch.from_numpy(B.astype(np.float32)).to(dev),
               ta=bool(ta), tb=bool(tb), out=out, alpha=0.5, beta=2.0)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-4)


def _gemm_case(rng, ta, tb, M, N, K, pad):
    """A, B (f64) in the stored layouts, as f32 device views whose leading
    dimension is padded by `pad` (pad 1: odd strides, no 16-byte rows)."""
    def dev_view(x):
        r, c = x.shape
        buf = torch.zeros(r, c + pad, dtype=torch.float32)
        buf[:, :c] = torch.from_numpy(x.astype(np.float32))
        return buf.cuda()[:, :c]
    A = rng.normal(0, 1, (K, M) if ta else (M, K))
    B = rng.normal(0, 1, (N, K) if tb else (K, N))
    A32, B32 = A.astype(np.float32).astype(np.float64), B.astype(np.float32).astype(np.float64)
    ref = (A32.T if ta else A32) @ (B32.T if tb else B32)
    return dev_view(A), dev_view(B), ref, A32, B32


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K,pad", [(77, 130, 45, 0), (300, 260, 333, 0), (256, 384, 512, 0),
                                       (129, 257, 100, 1), (1, 5, 1, 0)])
def test_gemm_mfma_f32_grade(dev, ta, tb, M, N, K, pad):
    """The three-plane bf16 matrix-core GEMM against f64: its error stays
    within 4x that of torch's own f32 matmul of the same f32 inputs (a kernel
    that dropped the third plane, or the cross terms, would be ~2^-17 or
    ~2^-9 relative, far outside), for every transpose pair, ragged tiles and
    unaligned leading dimensions; beta = 0 never reads C (NaN there)."""
    print(f"case gemm_mfma ta={ta} tb={tb} M={M} N={N} K={K} pad={pad}", flush=True)
    rng = np.random.default_rng(1000 + 4 * ta + 2 * tb + M)
    a, b, ref, A32, B32 = _gemm_case(rng, ta, tb, M, N, K, pad)
    out = torch.full((M, N), float("nan"), device=dev)
    train.gemm(a, b, ta=bool(ta), tb=bool(tb), out=out, alpha=1.0, beta=0.0, entry="sm_gemm_mfma")
    t32 = ((torch.from_numpy(A32).float().T if ta else torch.from_numpy(A32).float())
           @ (torch.from_numpy(B32).float().T if tb else torch.from_numpy(B32).float()))
    err = float(np.abs(out.cpu().double().numpy() - ref).max())
    err32 = float(np.abs(t32.double().numpy() - ref).max())
    print(f"  max |err| {err:.3g} vs torch f32 {err32:.3g}", flush=True)
    assert err <= 4 * err32 + 1e-6
    # alpha / beta
    C = rng.normal(0, 1, (M, N))
    out2 = torch.from_numpy(C.astype(np.float32)).to(dev)
    train.gemm(a, b, ta=bool(ta), tb=bool(tb), out=out2, alpha=0.5, beta=2.0, entry="sm_gemm_mfma")
    np.testing.assert_allclose(out2.cpu().numpy(), 0.5 * ref + 2.0 * C.astype(np.float32),
                               rtol=1e-5, atol=1e-4)


def _bf16_rne(x):
    """f32 -> the nearest bf16 (ties to even), as f64 (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("planes", [1, 2])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K,pad", [(300, 260, 333, 0), (129, 257, 100, 1)])
def test_gemm_planes_reduced(dev, planes, ta, tb, M, N, K, pad):
    """sm_gemm_planes with one or two bf16 planes against the same plane
    arithmetic done in f64 on the host: planes 1 = bf16(a) bf16(b) (round to
    nearest even), planes 2 = a0 b0 + a0 b1 + a1 b0 with a1 = bf16(a - a0).
    The kernel's only other error is its f32 accumulation, so it stays within
    4x torch's f32 matmul error of that f64 value; a truncating rounding, a
    dropped or extra cross term, or the third plane would be off by ~2^-9 or
    ~2^-17 relative per product, far outside."""
    print(f"case gemm_planes planes={planes} ta={ta} tb={tb} M={M} N={N} K={K} pad={pad}",
          flush=True)
    rng = np.random.default_rng(2000 + 8 * planes + 4 * ta + 2 * tb + M)
    a, b, ref, A32, B32 = _gemm_case(rng, ta, tb, M, N, K, pad)
    A0, B0 = _bf16_rne(A32), _bf16_rne(B32)
    opA = lambda x: x.T if ta else x  # noqa: E731
    opB = lambda x: x.T if tb else x  # noqa: E731
    if planes == 1:
        want = opA(A0) @ opB(B0)
    else:
        A1, B1 = _bf16_rne(A32 - A0), _bf16_rne(B32 - B0)
        want = opA(A0) @ opB(B0) + opA(A0) @ opB(B1) + opA(A1) @ opB(B0)
    out = torch.full((M, N), float("nan"), device=dev)
    call("sm_gemm_planes", planes, ta, tb, M, N, K, 1.0, a.data_ptr(), a.stride(0), b.data_ptr(),
         b.stride(0), 0.0, out.data_ptr(), out.stride(0), torch.cuda.current_stream().cuda_stream)
    t32 = (torch.from_numpy(opA(A32)).float() @ torch.from_numpy(opB(B32)).float())
    err = float(np.abs(out.cpu().double().numpy() - want).max())
    err32 = float(np.abs(t32.double().numpy() - ref).max())
    dist = float(np.abs(want - ref).max())
    print(f"  max |err| vs plane model {err:.3g} (torch f32 {err32:.3g}; plane model vs exact "
          f"{dist:.3g})", flush=True)
    assert err <= 4 * err32 + 1e-6
    assert dist > 3 * err  # the kernel follows the plane model, not the exact product


@pytest.mark.parametrize("planes", [1, 2, 3])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(300, 260, 333), (513, 130, 1030)])
def test_gemm_planes_scratch_is_bit_exact(dev, planes, ta, tb, M, N, K):
    """sm_gemm_planes_ws equals sm_gemm_planes (the kernel's own plane split
    and transposed loads) bit for bit, with alpha and beta, on each of its
    paths: a scratch of sm_gemm_planes_scratch_bytes (one plane: both operands
    converted once into zero-padded bf16 copies, transposed where k is not
    contiguous; more planes: the transposes below); one only big enough for
    the transposes of the operands whose k is not contiguous (rows padded to
    4 floats); none."""
    print(f"case gemm_planes_ws planes={planes} ta={ta} tb={tb} M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=dev).manual_seed(M + N + K + 4 * ta + 2 * tb)
    a = torch.randn((K, M) if ta else (M, K), generator=g, device=dev)
    b = torch.randn((N, K) if tb else (K, N), generator=g, device=dev)
    c0 = torch.randn(M, N, generator=g, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    need = int(_lib.lib().sm_gemm_planes_scratch_bytes(ta, tb, M, N, K))
    kp4 = (K + 3) // 4 * 4
    trans = 4 * ((M * kp4 if ta else 0) + (0 if tb else N * kp4))
    mp, np_, kp = -(-M // 128) * 128, -(-N // 128) * 128, -(-K // 64) * 64
    assert need == max(4 * ((mp * kp + np_ * kp + 1) // 2), trans)
    ref = c0.clone()
    call("sm_gemm_planes", planes, ta, tb, M, N, K, 0.75, a.data_ptr(), a.stride(0), b.data_ptr(),
         b.stride(0), 0.5, ref.data_ptr(), N, st)
    for nbytes in (need, trans, 0):
        scratch = torch.full((max(need, 16) // 4,), float("nan"), device=dev)
        out = c0.clone()
        call("sm_gemm_planes_ws", planes, 0, ta, tb, M, N, K, 0.75, a.data_ptr(), a.stride(0),
             b.data_ptr(), b.stride(0), 0.5, out.data_ptr(), N, scratch.data_ptr(), nbytes, st)
        assert torch.equal(out, ref), (nbytes, float((out - ref).abs().max()))


@pytest.mark.parametrize("ta,tb", [(0, 1), (0, 0), (1, 1)])
def test_gemm_planes_two_plane_b_is_bit_exact(dev, ta, tb):
    """b_planes 2 (B exact in two bf16 planes, as the policy's fake-quantized
    weights are: bf16 scales times 4-bit codes) gives three-plane GEMMs the
    same bits with five plane products as with six; B values that are not
    two-plane exact (a plain f32 B) do differ, so the flag does change the
    arithmetic. Bad b_planes values are rejected."""
    M, N, K = 300, 260, 1030
    print(f"case gemm_planes two-plane B ta={ta} tb={tb}", flush=True)
    g = torch.Generator(device=dev).manual_seed(5 + ta + 2 * tb)
    a = torch.randn((K, M) if ta else (M, K), generator=g, device=dev)
    bshape = (N, K) if tb else (K, N)
    codes = torch.randint(-7, 8, bshape, generator=g, device=dev).float()
    scale = (torch.rand(bshape, generator=g, device=dev) * 0.05 + 0.01).bfloat16().float()
    bq = codes * scale  # a bf16 scale times a 4-bit code, exact in f32
    bf = torch.randn(bshape, generator=g, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    need = int(_lib.lib().sm_gemm_planes_scratch_bytes(ta, tb, M, N, K))
    scratch = torch.empty(max(need, 16) // 4, device=dev)

    def run(b, bp, nbytes=need):
        out = torch.zeros(M, N, device=dev)
        call("sm_gemm_planes_ws", 3, bp, ta, tb, M, N, K, 1.0, a.data_ptr(), a.stride(0),
             b.data_ptr(), b.stride(0), 0.0, out.data_ptr(), N, scratch.data_ptr(), nbytes, st)
        return out
    ref = run(bq, 3)
    assert torch.equal(run(bq, 2), ref)  # pre-split planes
    assert torch.equal(run(bq, 2, 0), ref)  # the kernel's own split
    assert not torch.equal(run(bf, 2), run(bf, 3))
    with pytest.raises(_lib.SummaError, match="b_planes must be"):
        run(bq, 1)


def test_gemm_planes_rejects_bad_count(dev):
    x = torch.zeros(4, 4, device=dev)
    for planes in (0, 4):
        with pytest.raises(_lib.SummaError, match="planes must be 1, 2 or 3"):
            call("sm_gemm_planes", planes, 0, 0, 4, 4, 4, 1.0, x.data_ptr(), 4, x.data_ptr(), 4,
                 0.0, x.data_ptr(), 4, 0)


def test_gemm_ex_large_runs_on_matrix_cores(dev):
    """Above its size threshold sm_gemm_ex is the matrix-core kernel (same
    bits as sm_gemm_mfma); below it, the f32 FMA kernel (within f32 rounding)."""
    rng = np.random.default_rng(7)
    for (M, N, K) in [(512, 512, 512), (64, 96, 80)]:
        print(f"case gemm_ex dispatch M={M} N={N} K={K}", flush=True)
        a, b, ref, _, _ = _gemm_case(rng, 0, 1, M, N, K, 0)
        o1 = train.gemm(a, b, tb=True)
        o2 = train.gemm(a, b, tb=True, entry="sm_gemm_mfma")
        if M * N * K >= 1 << 27:
            assert torch.equal(o1, o2)
        np.testing.assert_allclose(o1.cpu().numpy(), ref, rtol=1e-5, atol=1e-4)


def test_rmsnorm_backward_matches_autograd(dev):
    rows, d, eps = 33, 300, 1e-5
    x = torch.randn(rows, d, dtype=torch.float64, requires_grad=True)
    g = torch.rand(d, dtype=torch.float64, requires_grad=True)
    y = x / torch.sqrt((x * x).mean(1, keepdim=True) + eps) * g
    dy = torch.randn(rows, d, dtype=torch.float64)
    y.backward(dy)
    dx = torch.full((rows, d), 0.5, device=dev)
    dg = torch.zeros(d, device=dev)
    rinv = torch.empty(rows, device=dev)
    xd, gd, dyd = (t.detach().float().to(dev) for t in (x, g, dy))
    call("sm_rmsnorm_backward", xd.data_ptr(), gd.data_ptr(), dyd.data_ptr(), rows, d, eps, 1,
         dx.data_ptr(), dg.data_ptr(), rinv.data_ptr(), _st())
    torch.testing.assert_close(dx.cpu().double(), x.grad + 0.5, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(dg.cpu().double(), g.grad, rtol=1e-4, atol=1e-4)


def _rope_t(x, tab, pos):
    """adjacent-pair rotation of x [.., L, heads, hd] at positions pos [L] (f64)."""
    c = tab[pos][:, None, :, 0]
    s = tab[pos][:, None, :, 1]
    a, b = x[..., 0::2], x[..., 1::2]
    out = torch.stack([a * c - b * s, b * c + a * s], -1)
    return out.flatten(-2)


def test_rope_qk_forward_and_backward(dev):
    cfg = ModelConfig(layers=1, d_model=128, heads=4, kv_heads=2, head_dim=64, ffn=128,
                      vocab=10, max_seq=32, quantized=False)
    S, L, H, KVH, hd = 2, 9, 4, 2, 64
    tab = train.rope_table(cfg, dev)
    pos0 = torch.tensor([0, 5], dtype=torch.int32, device=dev)
    qkv = torch.randn(S * L, (H + 2 * KVH) * hd, dtype=torch.float64)
    x = qkv.clone().requires_grad_(True)
    t64 = tab.cpu().double()
    parts = []
    for s in range(S):
        pos = torch.arange(L) + int(pos0[s])
        row = x[s * L:(s + 1) * L]
        q = _rope_t(row[:, :H * hd].view(L, H, hd), t64, pos).reshape(L, -1)
        k = _rope_t(row[:, H * hd:(H + KVH) * hd].view(L, KVH, hd), t64, pos).reshape(L, -1)
        parts.append(torch.cat([q, k, row[:, (H + KVH) * hd:]], 1))
    y = torch.cat(parts)
    dy = torch.randn_like(y)
    y.backward(dy)
    d = qkv.float().to(dev)
    call("sm_rope_qk", d.data_ptr(), tab.data_ptr(), pos0.data_ptr(), S, L, H, KVH, hd, 0, _st())
    torch.testing.assert_close(d.cpu().double(), y.detach(), rtol=1e-5, atol=1e-5)
    g = dy.float().to(dev)
    call("sm_rope_qk", g.data_ptr(), tab.data_ptr(), pos0.data_ptr(), S, L, H, KVH, hd, 1, _st())
    torch.testing.assert_close(g.cpu().double(), x.grad, rtol=1e-5, atol=1e-5)


def _attn_t(q, k, v, H, KVH):
    """causal GQA attention, q [S, L, H, hd], k/v [S, KVH, L, hd] (f64)."""
    S, L, _, hd = q.shape
    kk = k.repeat_interleave(H // KVH, dim=1)
    vv = v.repeat_interleave(H // KVH, dim=1)
    sc = torch.einsum("slhd,shtd->shlt", q, kk) / math.sqrt(hd)
    mask = torch.ones(L, L, dtype=torch.bool).triu(1)
    sc = sc.masked_fill(mask, float("-inf"))
    p = torch.softmax(sc, -1)
    return torch.einsum("shlt,shtd->slhd", p, vv), torch.logsumexp(sc, -1)


@pytest.mark.parametrize("hd,H,KVH,L", [(64, 4, 2, 21), (128, 4, 4, 21), (128, 8, 2, 100),
                                        (64, 4, 1, 70), (128, 2, 2, 64)])
def test_attention_backward_matches_autograd(dev, hd, H, KVH, L):
    """Causal GQA backward (32 x 32 tiles: one partial tile, several tiles with
    a partial last one, exact tiles) against float64 autograd."""
    print(f"case attention backward hd={hd} H={H} KVH={KVH} L={L}", flush=True)
    S = 2
    q = torch.randn(S, L, H, hd, dtype=torch.float64, requires_grad=True)
    k = torch.randn(S, KVH, L, hd, dtype=torch.float64, requires_grad=True)
    v = torch.randn(S, KVH, L, hd, dtype=torch.float64, requires_grad=True)
    o, lse = _attn_t(q, k, v, H, KVH)
    do = torch.randn_like(o)
    o.backward(do)
    qd, kd, vd, od, dod = (t.detach().float().contiguous().to(dev) for t in (q, k, v, o, do))
    lsed = lse.detach().float().contiguous().to(dev)
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    delta = torch.empty(S * H * L, device=dev)
    call("sm_attn_backward_f32", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), od.data_ptr(),
         dod.data_ptr(), lsed.data_ptr(), S, L, H, KVH, hd, dq.data_ptr(), dk.data_ptr(),
         dv.data_ptr(), delta.data_ptr(), _st())
    for got, want in ((dq, q.grad), (dk, k.grad), (dv, v.grad)):
        torch.testing.assert_close(got.cpu().double(), want, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("hd,H,KVH,L", [(64, 4, 2, 21), (128, 8, 2, 100), (64, 4, 1, 70),
                                        (128, 2, 2, 64), (128, 16, 4, 160)])
def test_attention_bf16ops_forward_and_backward(dev, hd, H, KVH, L):
    """sm_attn_prefill_lse_bf16ops / sm_attn_backward_bf16ops (the one-plane
    policy's attention: bf16 operands, f32 accumulation) against float64
    autograd: every output within bf16-operand error (relative Frobenius error
    <= 1e-2, worst element <= 5 % of the largest), and measurably different
    from the f32 kernels on the same inputs, so the bf16 path is the one that
    ran; the f32 kernels stay within 1e-5 there. Rows shorter than 32 keep the
    f32 forward (L 21: bit-equal to sm_attn_prefill_lse)."""
    print(f"case attention bf16ops hd={hd} H={H} KVH={KVH} L={L}", flush=True)
    S = 2
    q = torch.randn(S, L, H, hd, dtype=torch.float64, requires_grad=True)
    k = torch.randn(S, KVH, L, hd, dtype=torch.float64, requires_grad=True)
    v = torch.randn(S, KVH, L, hd, dtype=torch.float64, requires_grad=True)
    o, lse = _attn_t(q, k, v, H, KVH)
    do = torch.randn_like(o)
    o.backward(do)
    qd, kd, vd, dod = (t.detach().float().contiguous().to(dev) for t in (q, k, v, do))
    pos0 = torch.zeros(S, dtype=torch.int32, device=dev)

    def fwd(name, *dt):
        out = torch.empty_like(qd)
        ls = torch.empty(S * H, L, device=dev)
        call(name, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), pos0.data_ptr(), out.data_ptr(),
             ls.data_ptr(), *dt, S, L, H, KVH, L, hd, _st())
        return out, ls

    def bwd(name, od, lsed):
        dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
        delta = torch.empty(S * H * L, device=dev)
        call(name, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), od.data_ptr(), dod.data_ptr(),
             lsed.data_ptr(), S, L, H, KVH, hd, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
             delta.data_ptr(), _st())
        return dq, dk, dv

    def rel(got, want):
        got = got.cpu().double().reshape(want.shape)
        return float((got - want).norm() / want.norm()), float(
            (got - want).abs().max() / want.abs().max())

    o16, l16 = fwd("sm_attn_prefill_lse_bf16ops")
    o32, l32 = fwd("sm_attn_prefill_lse", _lib.SM_F32, _lib.SM_F32)
    if L < 32:
        assert torch.equal(o16, o32) and torch.equal(l16, l32)
    else:
        fr, mx = rel(o16, o.detach())
        assert fr <= 1e-2 and mx <= 5e-2, (fr, mx)
        assert rel(o32, o.detach())[0] <= 1e-5
        assert rel(o16, o32.cpu().double())[0] > 1e-5  # the bf16 operands were used
    lse_want = lse.detach().reshape(S * H, L)
    assert float((l16.cpu().double() - lse_want).abs().max()) <= 5e-2
    # both backwards from the exact forward, so only the backward's operands differ
    od = o.detach().float().contiguous().to(dev)
    lsed = lse.detach().float().contiguous().to(dev)
    g16 = bwd("sm_attn_backward_bf16ops", od, lsed)
    g32 = bwd("sm_attn_backward_f32", od, lsed)
    for got, ref, want in zip(g16, g32, (q.grad, k.grad, v.grad)):
        fr, mx = rel(got, want)
        assert fr <= 1e-2 and mx <= 5e-2, (fr, mx)
        assert rel(ref, want)[0] <= 1e-5
        assert rel(got, ref.cpu().double())[0] > 1e-5


CFG = ModelConfig(layers=2, d_model=256, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=1000,
                  max_seq=32, quantized=False)


def _torch_lp(w, cfg, prompts, tokens):
    """Independent float64 restatement of the decoder's recompute."""
    S, P = prompts.shape
    N = tokens.shape[1]
    L = P + N - 1
    H, KVH, hd, F, eps = cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.ffn, cfg.norm_eps
    ids = torch.cat([prompts, tokens[:, :N - 1]], 1).long()
    rms = lambda x, g: x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * g
    half = hd // 2
    freq = float(cfg.rope_theta) ** (-2.0 * torch.arange(half, dtype=torch.float64) / hd)
    ang = torch.arange(L, dtype=torch.float64)[:, None] * freq[None, :]
    tab = torch.stack([torch.cos(ang), torch.sin(ang)], -1).float().double()
    pos = torch.arange(L)
    x = w["embed"][ids]
    for i in range(cfg.layers):
        h = rms(x, w["attn_norm"][i])
        qkv = h @ w["qkv"][i].T
        q = _rope_t(qkv[..., :H * hd].reshape(S, L, H, hd), tab, pos)
        k = _rope_t(qkv[..., H * hd:(H + KVH) * hd].reshape(S, L, KVH, hd), tab, pos)
        v = qkv[..., (H + KVH) * hd:].reshape(S, L, KVH, hd)
        o, _ = _attn_t(q, k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3), H, KVH)
        x = x + o.reshape(S, L, H * hd) @ w["o"][i].T
        u = rms(x, w["ffn_norm"][i]) @ w["in"][i].T
        x = x + (torch.nn.functional.silu(u[..., :F]) * u[..., F:]) @ w["down"][i].T
    hf = rms(x, w["final_norm"])[:, P - 1:P - 1 + N]
    logits = hf @ w["lm_head"].T
    return torch.log_softmax(logits, -1).gather(-1, tokens.long()[..., None])[..., 0]


def test_policy_gradient_matches_autograd(dev):
    cfg = CFG.oracle_cfg()
    w = oracle.random_weights(cfg, seed=11, std=0.05)
    rng = np.random.default_rng(2)
    prompts = torch.from_numpy(rng.integers(0, CFG.vocab, (4, 8)).astype(np.int32))
    tokens = torch.from_numpy(rng.integers(0, CFG.vocab, (4, 6)).astype(np.int32))
    pol = train.Fp32Policy(CFG, w, dev)
    lp = pol.forward(prompts.to(dev), tokens.to(dev))
    m = Model(CFG)
    m.load_host_weights(w, dev)
    np.testing.assert_allclose(lp.cpu().numpy(), m.logprobs(prompts.to(dev), tokens.to(dev)).cpu().numpy(),
                               atol=1e-5)
    dlp = torch.randn(4, 6, dtype=torch.float64)
    grads = pol.backward(dlp.float().to(dev))
    wt = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)).requires_grad_(True) for k, v in w.items()}
    lp_t = _torch_lp(wt, CFG, prompts, tokens)
    np.testing.assert_allclose(lp.cpu().numpy(), lp_t.detach().numpy(), atol=2e-5)
    (dlp * lp_t).sum().backward()
    for k, t in wt.items():
        got = grads[k].cpu().double()
        scale = t.grad.abs().max().item() + 1e-12
        err = (got - t.grad).abs().max().item() / scale
        assert err < 2e-4, (k, err)


def test_adamw_matches_torch(dev):
    rng = np.random.default_rng(3)
    p0 = rng.normal(0, 1, 1000)
    tp = torch.tensor(p0, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.AdamW([tp], lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    p = torch.tensor(p0, dtype=torch.float32, device=dev)
    m, v = torch.zeros_like(p), torch.zeros_like(p)
    for step in range(1, 6):
        gr = rng.normal(0, 1, 1000)
        tp.grad = torch.tensor(gr)
        opt.step()
        gd = torch.tensor(gr, dtype=torch.float32, device=dev)
        call("sm_adamw_step", p.data_ptr(), gd.data_ptr(), m.data_ptr(), v.data_ptr(), 1000,
             1e-2, 0.9, 0.95, 1e-8, 0.1, step, _st())
    np.testing.assert_allclose(p.cpu().numpy(), tp.detach().numpy(), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("shape", [(96, 256), (256, 96)])
def test_newton_schulz_formula_and_orthogonality(dev, shape):
    g = torch.randn(*shape, dtype=torch.float64)
    got = train.newton_schulz(g.float().to(dev)).cpu().double()
    # muon.rs:257-285 in float64, on the Burn orientation of this [out, in] matrix
    x = g.t()
    tr = x.shape[0] > x.shape[1]
    if tr:
        x = x.t()
    x = x / x.norm().clamp_min(1e-7)
    a, b, c = train.NS_COEFFICIENTS
    for _ in range(train.NS_STEPS):
        gram = x @ x.t()
        x = a * x + (b * gram + c * gram @ gram) @ x
    want = (x.t() if tr else x).t()
    torch.testing.assert_close(got, want, rtol=1e-3, atol=1e-4)
    sv = torch.linalg.svdvals(got)
    assert sv.min() > 0.5 and sv.max() < 1.3, sv  # near-orthogonal: the point of the iteration


def test_grpo_update_lowers_the_surrogate_loss(dev):
    """One GRPO step end to end: rollouts from the inference model, the
    device loss and its dlp, the policy gradient, an AdamW step on every
    weight, and the updated weights back in the model: the same batch's loss
    drops."""
    cfg = CFG.oracle_cfg()
    w = oracle.random_weights(cfg, seed=12, std=0.05)
    m = Model(CFG)
    m.load_host_weights(w, dev)
    G, B = 8, 2
    prompts = torch.from_numpy(np.random.default_rng(4).integers(0, CFG.vocab, (B * G, 8)).astype(np.int32)).to(dev)
    tok, beh = m.generate(prompts, 6, temperature=1.0, seed=9)
    rewards = torch.from_numpy(np.random.default_rng(5).random((B, G)).astype(np.float32)).to(dev)
    pol = train.Fp32Policy(CFG, w, dev)

    def loss_and_dlp():
        lp = pol.forward(prompts, tok)
        out = ops.grpo_loss_batched(rewards, lp.view(B, G, 6), beh.view(B, G, 6), None, None,
                                    kl_coefficient=0.0)
        return float(out["stats"][:, 0].sum()), out["dlp"].view(B * G, 6)

    l0, dlp = loss_and_dlp()
    grads = pol.backward(dlp)
    pol.adamw_step(grads, list(pol.p))  # the trainer's AdamW settings
    l1, _ = loss_and_dlp()
    assert l1 < l0, (l0, l1)
    pol.to_model(m)
    lp_m = m.logprobs(prompts, tok).cpu().numpy()
    lp_p = pol.forward(prompts, tok).cpu().numpy()
    np.testing.assert_allclose(lp_m, lp_p, atol=1e-5)
