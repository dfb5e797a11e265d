"""sm_q4_matmul_noalloc (no counterpart in the reference: the Q4 matmul for
callers that cannot allocate) against sm_q4_matmul_ws with a caller workspace
of the queried size: bit-identical results on two calls in a row, the second
with a smaller input, and a clear rejection of a call whose split-K workspace
exceeds the static scratch."""
import numpy as np
import pytest
import torch

from summa_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _call(name, qw, xd, xdt, out, epi, *extra):
    M = xd.shape[0]
    _lib.call(name, qw.tcodes.data_ptr(), qw.tscales.data_ptr(), qw.n, qw.k, xd.data_ptr(), xdt,
              M, xd.stride(0), out.data_ptr(), out.stride(0), epi, *extra,
              torch.cuda.current_stream().cuda_stream)


# (M, N, K, epilogue, activation dtype): decode-batch shapes that split K
# (the LDS-staged kernel over K ranges, and the batch kernel's split)
CASES = [(256, 2048, 5632, _lib.SM_EPI_ADD_F32, _lib.SM_F16X2),
         (128, 4096, 4096, _lib.SM_EPI_STORE_F32, _lib.SM_BF16)]


def test_noalloc_equals_workspace_entry_on_two_calls(dev):
    assert _lib.lib().sm_q4_noalloc_scratch_bytes() == 96 * 1024 * 1024
    for M, N, K, epi, xdt in CASES:  # the second call is the smaller one
        print(f"case noalloc M={M} N={N} K={K} epi={epi} x={xdt}", flush=True)
        w = torch.empty(N, K, device=dev)
        ops.fill_normal(w, 0.0, 0.02, seed=N + K)
        qw = ops.Q4Weight.quantize(w)
        x = torch.randn(M, K, device=dev)
        xd = ops.f16_pair(x) if xdt == _lib.SM_F16X2 else x.to(torch.bfloat16)
        need = _lib.lib().sm_q4_matmul_workspace_bytes(M, N, K, epi)
        assert 0 < need <= _lib.lib().sm_q4_noalloc_scratch_bytes()
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        base = torch.randn(M, N, device=dev)
        ref, got = base.clone(), base.clone()
        _call("sm_q4_matmul_ws", qw, xd, xdt, ref, epi, ws.data_ptr(), need)
        _call("sm_q4_matmul_noalloc", qw, xd, xdt, got, epi)
        torch.cuda.synchronize()
        assert int(ws.int().abs().sum().item()) != 0  # the split really ran
        assert torch.equal(got, ref)


def test_noalloc_rejects_oversized_call(dev):
    M, N, K = 256, 65536, 2048
    need = _lib.lib().sm_q4_matmul_workspace_bytes(M, N, K, _lib.SM_EPI_STORE_F32)
    assert need > _lib.lib().sm_q4_noalloc_scratch_bytes()
    w = ops.Q4Weight.quantize(torch.zeros(N, K, device=dev))
    x = torch.zeros(M, K, dtype=torch.float16, device=dev)
    y = torch.full((M, N), 3.0, device=dev)
    with pytest.raises(_lib.SummaError, match="static scratch holds 100663296"):
        _call("sm_q4_matmul_noalloc", w, x, _lib.SM_F16, y, _lib.SM_EPI_STORE_F32)
    torch.cuda.synchronize()
    assert bool((y == 3.0).all())  # nothing was launched
