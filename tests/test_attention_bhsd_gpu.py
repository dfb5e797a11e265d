"""sm_attention / sm_attention_backward: the reference's AttentionBackend pair
(summa-llm/src/model/fused_attention.rs:37-74) in its [B, H, S, hd] layout,
against float64 restatements of reference_attention (:177-217, with
attention_log_sum_exp :166-172) and of its backward (autograd of the same
expression, as reference_attention_backward :219-261 computes it)."""
import numpy as np
import pytest
import torch

from summa_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _reference(q, k, v, causal):
    """f64 reference_attention on CPU tensors: (out, lse [B*H, S])."""
    B, H, S, hd = q.shape
    rep = H // k.shape[1]
    k = k.repeat_interleave(rep, dim=1)  # repeat_kv: head h uses KV head h // rep
    v = v.repeat_interleave(rep, dim=1)
    scores = q @ k.transpose(-1, -2) / np.sqrt(hd)
    if causal:
        mask = torch.triu(torch.ones(S, S, dtype=torch.bool), 1)
        scores = scores.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(scores, -1).reshape(B * H, S)
    return torch.softmax(scores, -1) @ v, lse


CASES = [(1, 4, 4, 1, 64), (2, 4, 4, 63, 64), (3, 8, 2, 130, 128), (2, 16, 4, 257, 128),
         (1, 12, 12, 200, 64)]


@pytest.mark.parametrize("B,H,KVH,S,hd", CASES)
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_attention_matches_reference(dev, B, H, KVH, S, hd, causal, dtype):
    print(f"case attention B={B} H={H} KVH={KVH} S={S} hd={hd} causal={causal} {dtype}",
          flush=True)
    g = torch.Generator().manual_seed(B * 1000 + S)
    q, k, v = (torch.randn(B, h_, S, hd, generator=g) for h_ in (H, KVH, KVH))
    qd, kd, vd = (t.to(dtype).to(dev) for t in (q, k, v))
    out, lse = ops.attention(qd, kd, vd, causal=causal, want_lse=True)
    # the reference on the values the kernel consumed
    ref, ref_lse = _reference(*(t.cpu().double() for t in (qd, kd, vd)), causal)
    got = out.cpu().double()
    if dtype == torch.float32:
        tol = 2e-6 + 2e-6 * ref.abs()
    else:  # one rounding of the f32-accumulated output to the 16-bit dtype
        ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
        tol = ulp * ref.abs() + 1e-4
    assert bool(((got - ref).abs() <= tol).all()), float((got - ref).abs().max())
    np.testing.assert_allclose(lse.cpu().double().numpy(), ref_lse.numpy(), atol=2e-5, rtol=1e-6)
    # without lse the output is the same
    assert torch.equal(ops.attention(qd, kd, vd, causal=causal), out)


@pytest.mark.parametrize("dtype,dt_id", [(torch.bfloat16, _lib.SM_BF16), (torch.float16, _lib.SM_F16),
                                         (torch.float32, _lib.SM_F32)])
def test_layout_entry_equals_cache_entry(dev, dtype, dt_id):
    """Causal [B, H, S, hd] attention is the model's prefill attention over a
    cache of capacity S with the query rows transposed to [B, S, H, hd]: the
    two entry points give identical bits."""
    B, H, KVH, S, hd = 2, 8, 2, 150, 128
    g = torch.Generator().manual_seed(9)
    q, k, v = (torch.randn(B, h_, S, hd, generator=g).to(dtype).to(dev) for h_ in (H, KVH, KVH))
    out, lse = ops.attention(q, k, v, causal=True, want_lse=True)
    q_rows = q.transpose(1, 2).contiguous()  # [B, S, H, hd]
    o_rows = torch.empty_like(q_rows)
    lse2 = torch.empty_like(lse)
    pos0 = torch.zeros(B, dtype=torch.int32, device=dev)
    _lib.call("sm_attn_prefill_lse", q_rows.data_ptr(), k.data_ptr(), v.data_ptr(),
              pos0.data_ptr(), o_rows.data_ptr(), lse2.data_ptr(), dt_id, dt_id, B, S, H, KVH, S,
              hd, torch.cuda.current_stream().cuda_stream)
    assert torch.equal(o_rows.transpose(1, 2).contiguous(), out)
    assert torch.equal(lse2, lse)


@pytest.mark.parametrize("B,H,KVH,S,hd", [(2, 4, 4, 33, 64), (1, 8, 2, 70, 128)])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_backward_matches_autograd(dev, B, H, KVH, S, hd, causal):
    print(f"case attention backward B={B} H={H} KVH={KVH} S={S} hd={hd} causal={causal}",
          flush=True)
    g = torch.Generator().manual_seed(S)
    q, k, v = (torch.randn(B, h_, S, hd, generator=g) for h_ in (H, KVH, KVH))
    dout = torch.randn(B, H, S, hd, generator=g)
    qd, kd, vd, gd = (t.to(dev) for t in (q, k, v, dout))
    out, lse = ops.attention(qd, kd, vd, causal=causal, want_lse=True)
    dq, dk, dv = ops.attention_backward(qd, kd, vd, out, gd, lse, causal=causal)
    q64, k64, v64 = (t.double().requires_grad_() for t in (q, k, v))
    ref, _ = _reference(q64, k64, v64, causal)
    ref.backward(dout.double())
    for name, got, want in (("dq", dq, q64.grad), ("dk", dk, k64.grad), ("dv", dv, v64.grad)):
        err = float((got.cpu().double() - want).abs().max())
        scale = float(want.abs().max())
        assert err <= 1e-5 * max(scale, 1.0), (name, err, scale)


def test_attention_rejects_bad_shapes(dev):
    q = torch.zeros(1, 6, 8, 64, device=dev)
    k = torch.zeros(1, 4, 8, 64, device=dev)
    with pytest.raises(_lib.SummaError, match="multiple of key/value heads"):
        ops.attention(q, k, k.clone())
    q = torch.zeros(1, 4, 8, 96, device=dev)
    with pytest.raises(_lib.SummaError, match="head_dim must be 64 or 128"):
        ops.attention(q, q.clone(), q.clone())
