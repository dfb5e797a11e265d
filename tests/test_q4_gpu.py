"""Q4G128 quantizer and quantized matmul (sm_q4_quantize / sm_q4_matmul) vs the oracle."""
import numpy as np
import pytest
import torch

import oracle
from summa_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _weights(n, k, seed):
    return np.random.default_rng(seed).normal(0, 0.02, (n, k)).astype(np.float32)


def _bf16_dev(a, dev):
    return torch.from_numpy(oracle.bf16_bits(a).view(np.int16)).to(dev).view(torch.bfloat16)


def _oracle_matmul(codes, scales, n, k, xr):
    return np.stack([oracle.q4_matvec(codes, scales, n, k, xr[m]) for m in range(xr.shape[0])])


def _bound(codes, scales, n, k, xr):
    dense = oracle.q4_decode(codes, scales, n * k).reshape(n, k).astype(np.float64)
    return np.abs(xr.astype(np.float64)) @ np.abs(dense).T


@pytest.mark.parametrize("n,k", [(96, 256), (2304, 768), (5, 1000)])
def test_quantizer_bit_exact(dev, n, k):
    w = _weights(n, k, 1)
    w[0, :128] = 0.0  # all-zero group -> scale 0, codes 0
    codes, scales = oracle.q4_quantize(w)
    q = ops.Q4Weight.quantize(torch.from_numpy(w).to(dev))
    np.testing.assert_array_equal(q.codes.cpu().numpy(), codes)
    np.testing.assert_array_equal(q.scales.cpu().numpy().view(np.uint16), scales)
    # bf16 input path
    wb = oracle.bf16_bits(w)
    codes_b, scales_b = oracle.q4_quantize(oracle.bf16_to_f32(wb))
    qb = ops.Q4Weight.quantize(_bf16_dev(w, dev))
    np.testing.assert_array_equal(qb.codes.cpu().numpy(), codes_b)
    np.testing.assert_array_equal(qb.scales.cpu().numpy().view(np.uint16), scales_b)


@pytest.mark.parametrize("n,k", [(96, 256), (2304, 768), (768, 768), (130, 5632), (32768, 768)])
@pytest.mark.parametrize("m", [1, 3, 16, 17, 64, 128, 200])
def test_matmul_matches_oracle(dev, n, k, m):
    """bf16 activations against the oracle's sequential-f32 matrix_vector per
    row; the largest cases (where that costs seconds per row block) against
    float64 on the decoded weights instead, within the same bound."""
    print(f"case n={n} k={k} m={m}", flush=True)
    w = _weights(n, k, n + k)
    codes, scales = oracle.q4_quantize(w)
    x = np.random.default_rng(m).normal(0, 1, (m, k)).astype(np.float32)
    xr = oracle.round_bf16(x)
    qw = ops.Q4Weight.from_host(codes, scales, n, k, dev)
    y = ops.q4_matmul(qw, _bf16_dev(x, dev)).cpu().numpy()
    if n * k * m > 2304 * 768 * 128 and m > 17:
        dense = oracle.q4_decode(codes, scales, n * k).reshape(n, k).astype(np.float64)
        y_ref = xr.astype(np.float64) @ dense.T
    else:
        y_ref = _oracle_matmul(codes, scales, n, k, xr)
    tol = 2e-6 * _bound(codes, scales, n, k, xr) + 1e-7
    assert np.all(np.abs(y - y_ref) <= tol), float(np.abs(y - y_ref).max())


def test_epilogues(dev):
    n, k, m = 512, 768, 9
    w = _weights(n, k, 7)
    codes, scales = oracle.q4_quantize(w)
    qw = ops.Q4Weight.from_host(codes, scales, n, k, dev)
    x = np.random.default_rng(0).normal(0, 1, (m, k)).astype(np.float32)
    xr = oracle.round_bf16(x)
    xd = _bf16_dev(x, dev)
    y_ref = _oracle_matmul(codes, scales, n, k, xr)
    tol = 2e-6 * _bound(codes, scales, n, k, xr) + 1e-7
    # bf16 store: one rounding of the f32 result
    yb = ops.q4_matmul(qw, xd, epilogue=_lib.SM_EPI_STORE_BF16).float().cpu().numpy()
    assert np.all(np.abs(yb - y_ref) <= np.abs(y_ref) * 2 ** -8 + tol)
    # residual add into f32
    base = np.random.default_rng(1).normal(0, 1, (m, n)).astype(np.float32)
    acc = torch.from_numpy(base.copy()).to(dev)
    ops.q4_matmul(qw, xd, out=acc, epilogue=_lib.SM_EPI_ADD_F32)
    assert np.all(np.abs(acc.cpu().numpy() - (base + y_ref)) <= tol + 1e-6)
    # SwiGLU over [gate | value]: h = silu(gate) * value, bf16
    F = n // 2
    h = ops.q4_matmul(qw, xd, epilogue=_lib.SM_EPI_SWIGLU_BF16).float().cpu().numpy()
    g, v = y_ref[:, :F], y_ref[:, F:]
    h_ref = g / (1 + np.exp(-g)) * v
    assert h.shape == (m, F)
    np.testing.assert_allclose(h, h_ref, rtol=2 ** -7, atol=1e-6)


def test_rejects_bad_shapes(dev):
    w = ops.Q4Weight.quantize(torch.zeros(64, 256, device=dev))
    with pytest.raises(ValueError, match="K % 128"):
        bad = ops.Q4Weight(w.codes, w.scales, 64, 200)
        ops.q4_matmul(bad, torch.zeros(2, 200, dtype=torch.bfloat16, device=dev))
    # the C ABI rejects it too (no kernel launch)
    from summa_amd._lib import lib
    st = lib().sm_q4_matmul(w.tcodes.data_ptr(), w.tscales.data_ptr(), 64, 200,
                            w.tcodes.data_ptr(), 1, 2, 200, w.tcodes.data_ptr(), 64, 0, None)
    assert st == -1 and b"multiple of 128" in lib().sm_last_error()


@pytest.mark.parametrize("m", [1, 7, 128])
def test_matmul_f16_activations_and_swiglu_f16(dev, m):
    n, k = 768, 3072
    w = _weights(n, k, 3)
    codes, scales = oracle.q4_quantize(w)
    qw = ops.Q4Weight.from_host(codes, scales, n, k, dev)
    x = np.random.default_rng(m).normal(0, 1, (m, k)).astype(np.float32)
    xh = x.astype(np.float16)
    xr = xh.astype(np.float32)  # f16 values are what the kernel consumes
    y = ops.q4_matmul(qw, torch.from_numpy(xh).to(dev)).cpu().numpy()
    y_ref = _oracle_matmul(codes, scales, n, k, xr)
    tol = 2e-6 * _bound(codes, scales, n, k, xr) + 1e-7
    assert np.all(np.abs(y - y_ref) <= tol)
    F = n // 2
    h = ops.q4_matmul(qw, torch.from_numpy(xh).to(dev),
                      epilogue=_lib.SM_EPI_SWIGLU_F16).float().cpu().numpy()
    g, v = y_ref[:, :F], y_ref[:, F:]
    np.testing.assert_allclose(h, g / (1 + np.exp(-g)) * v, rtol=2 ** -10, atol=1e-6)


@pytest.mark.parametrize("m,n,k", [(33, 768, 768), (257, 768, 768), (600, 130, 1024),
                                   (1000, 2304, 768), (2100, 64, 256), (1100, 11264, 256)])
@pytest.mark.parametrize("xdt", ["bf16", "f16"])
def test_large_m_lds_kernel(dev, m, n, k, xdt):
    """M > 32 runs the batch kernel (weights dequantised once per workgroup into
    LDS; XCD-ordered row tiles with padding once there are >= 8 row tiles)."""
    print(f"case m={m} n={n} k={k} x={xdt}", flush=True)
    w = _weights(n, k, m + n)
    codes, scales = oracle.q4_quantize(w)
    qw = ops.Q4Weight.from_host(codes, scales, n, k, dev)
    x = np.random.default_rng(k).normal(0, 1, (m, k)).astype(np.float32)
    if xdt == "f16":
        xr = x.astype(np.float16).astype(np.float32)
        xd = torch.from_numpy(x.astype(np.float16)).to(dev)
    else:
        xr = oracle.round_bf16(x)
        xd = _bf16_dev(x, dev)
    y_ref = _oracle_matmul(codes, scales, n, k, xr)
    tol = 2e-6 * _bound(codes, scales, n, k, xr) + 1e-7
    y = ops.q4_matmul(qw, xd).cpu().numpy()
    assert np.all(np.abs(y - y_ref) <= tol), float(np.abs(y - y_ref).max())
    base = np.random.default_rng(2).normal(0, 1, (m, n)).astype(np.float32)
    acc = torch.from_numpy(base.copy()).to(dev)
    ops.q4_matmul(qw, xd, out=acc, epilogue=_lib.SM_EPI_ADD_F32)
    assert np.all(np.abs(acc.cpu().numpy() - (base + y_ref)) <= tol + 1e-6)
    if n % 2 == 0:
        F = n // 2
        h = ops.q4_matmul(qw, xd, epilogue=_lib.SM_EPI_SWIGLU_F16).float().cpu().numpy()
        g, v = y_ref[:, :F], y_ref[:, F:]
        np.testing.assert_allclose(h, g / (1 + np.exp(-g)) * v, rtol=2 ** -10, atol=1e-5)


def _pair_host(x):
    """fp32 -> SM_F16X2 rows (hi | lo) and the exact value they carry."""
    hi = x.astype(np.float16)
    lo = (x - hi.astype(np.float32)).astype(np.float16)
    return np.concatenate([hi, lo], 1), hi.astype(np.float32) + lo.astype(np.float32)


@pytest.mark.parametrize("m,n,k", [(1, 768, 3072), (7, 2304, 768), (128, 11264, 2048),
                                   (600, 768, 768), (1000, 256, 1024)])
def test_matmul_f16_pair_activations(dev, m, n, k):
    """SM_F16X2 input (two MFMAs per step on the same codes) and the SwiGLU
    f16-pair epilogue: fp32-grade activations through the f16 MFMA path.
    m > 32 runs the batch kernel (two MFMAs per weight fragment)."""
    print(f"case pair m={m} n={n} k={k}", flush=True)
    w = _weights(n, k, m + 7)
    codes, scales = oracle.q4_quantize(w)
    qw = ops.Q4Weight.from_host(codes, scales, n, k, dev)
    x = np.random.default_rng(m + 1).normal(0, 1, (m, k)).astype(np.float32)
    xp, xr = _pair_host(x)
    assert np.abs(xr - x).max() <= 2.0 ** -21 * np.abs(x).max()
    xd = torch.from_numpy(xp).to(dev)
    y = ops.q4_matmul(qw, xd, pair=True).cpu().numpy()
    dense = oracle.q4_decode(codes, scales, n * k).reshape(n, k).astype(np.float64)
    y_ref = xr.astype(np.float64) @ dense.T
    tol = 2e-6 * _bound(codes, scales, n, k, xr) + 1e-7
    assert np.all(np.abs(y - y_ref) <= tol), float(np.abs(y - y_ref).max())
    # device split of an f32 activation gives the same result
    y2 = ops.q4_matmul(qw, ops.f16_pair(torch.from_numpy(x).to(dev)), pair=True).cpu().numpy()
    np.testing.assert_array_equal(y2, y)
    F = n // 2
    h = ops.unpair(ops.q4_matmul(qw, xd, epilogue=_lib.SM_EPI_SWIGLU_F16X2, pair=True))
    g, v = y_ref[:, :F], y_ref[:, F:]
    ref_h = g / (1 + np.exp(-g)) * v
    hb = (np.abs(g) + 1) * (tol[:, F:] + tol[:, :F]) * (np.abs(v) + 1)  # propagated matmul error
    assert np.all(np.abs(h.cpu().numpy() - ref_h) <= hb + 1e-6 * np.abs(ref_h) + 1e-7)


def test_pair_rejects_short_rows(dev):
    w = _weights(64, 256, 1)
    codes, scales = oracle.q4_quantize(w)
    qw = ops.Q4Weight.from_host(codes, scales, 64, 256, dev)
    x = torch.zeros((2, 256), dtype=torch.float16, device=dev)  # pair rows need 2K
    y = torch.empty((2, 64), device=dev)
    with pytest.raises(_lib.SummaError, match="ldx must be >= 512"):
        _lib.call("sm_q4_matmul", qw.tcodes.data_ptr(), qw.tscales.data_ptr(), 64, 256,
                  x.data_ptr(), _lib.SM_F16X2, 2, 256, y.data_ptr(), 64, 0,
                  torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("m,n,k,epi", [(256, 1024, 2048, "add"), (256, 2048, 5632, "add"),
                                       (200, 1024, 2048, "swiglu"), (256, 1024, 4096, "store")])
@pytest.mark.parametrize("xdt", ["pair", "bf16"])
def test_split_k_workspace(dev, m, n, k, epi, xdt):
    """sm_q4_matmul_ws: with a workspace, batch calls that would underfill the
    GPU split K and reduce fp32 partials in a fixed order (run-to-run exact).
    f16 pairs run the LDS-staged decode kernel over K ranges, bf16 the batch
    kernel's split."""
    print(f"case split-k m={m} n={n} k={k} {epi} {xdt}", flush=True)
    w = _weights(n, k, m + n + 3)
    codes, scales = oracle.q4_quantize(w)
    qw = ops.Q4Weight.from_host(codes, scales, n, k, dev)
    x = np.random.default_rng(m + 5).normal(0, 1, (m, k)).astype(np.float32)
    pair = xdt == "pair"
    if pair:
        xp, xr = _pair_host(x)
        xd = torch.from_numpy(xp).to(dev)
    else:
        xd = torch.from_numpy(x).to(dev).to(torch.bfloat16)
        xr = xd.float().cpu().numpy()
    dense = oracle.q4_decode(codes, scales, n * k).reshape(n, k).astype(np.float64)
    y_ref = xr.astype(np.float64) @ dense.T
    tol = 2e-6 * _bound(codes, scales, n, k, xr) + 1e-7
    e = {"add": _lib.SM_EPI_ADD_F32, "store": _lib.SM_EPI_STORE_F32,
         "swiglu": _lib.SM_EPI_SWIGLU_F16X2}[epi]
    ws = ops.q4_workspace(m, n, k, e, dev)
    ws.zero_()
    if epi == "swiglu":
        outs = [ops.unpair(ops.q4_matmul(qw, xd, epilogue=e, pair=pair, workspace=ws))
                for _ in range(2)]
        torch.testing.assert_close(outs[0], outs[1], rtol=0, atol=0)
        F = n // 2
        g, v = y_ref[:, :F], y_ref[:, F:]
        np.testing.assert_allclose(outs[0].cpu().numpy(), g / (1 + np.exp(-g)) * v,
                                   rtol=1e-5, atol=2e-6)
        return
    base = np.random.default_rng(9).normal(0, 1, (m, n)).astype(np.float32)
    outs = []
    for _ in range(2):
        acc = torch.from_numpy(base.copy()).to(dev)
        ops.q4_matmul(qw, xd, out=acc, epilogue=e, pair=pair, workspace=ws)
        outs.append(acc.cpu().numpy())
    np.testing.assert_array_equal(outs[0], outs[1])
    # a call of another shape on the same workspace leaves nothing behind that
    # changes the next result
    other = torch.zeros((m, 128), device=dev)
    w2 = ops.Q4Weight.from_host(*oracle.q4_quantize(_weights(128, k, 1)), 128, k, dev)
    ops.q4_matmul(w2, xd, out=other, pair=pair, workspace=ws)
    acc = torch.from_numpy(base.copy()).to(dev)
    ops.q4_matmul(qw, xd, out=acc, epilogue=e, pair=pair, workspace=ws)
    np.testing.assert_array_equal(acc.cpu().numpy(), outs[0])
    assert int(ws.int().abs().sum().item()) != 0  # the split really ran
    expect = (base + y_ref) if epi == "add" else y_ref
    assert np.all(np.abs(outs[0] - expect) <= tol + 1e-6), float(np.abs(outs[0] - expect).max())


@pytest.mark.parametrize("n,k,pair", [(16400, 2048, False), (16400, 1024, True), (1000, 640, False),
                                      (1000, 640, True), (300, 256, False), (65536, 2048, False),
                                      (2048, 5632, True), (4096, 4096, False), (40000, 4096, True),
                                      (1000, 2048, True), (1003, 5632, False), (65533, 2048, True)])
def test_gemv_m1_equals_tile_kernel(dev, n, k, pair):
    """M = 1 runs the single-row GEMV (activation row in LDS, double-buffered
    weight groups; K split across waves for small N and for K >= 2048). Where
    the 16-row tile kernel splits K the same way (fewer than 512 of its
    64-column workgroups) the arithmetic and summation order are the same, so
    row 0 of an M = 2 call matches bit for bit; otherwise (the 65536 x 2048 LM
    head) only the order of the four K-quarter partial sums differs. The
    store-bf16 and add epilogues follow the same value."""
    print(f"case gemv1 n={n} k={k} pair={pair}", flush=True)
    w = torch.empty(n, k, device=dev)
    ops.fill_normal(w, 0.0, 0.02, seed=n + k)
    qw = ops.Q4Weight.quantize(w)
    x = torch.randn(2, k, device=dev)
    xd = ops.f16_pair(x) if pair else x.to(torch.float16)
    y1 = ops.q4_matmul(qw, xd[:1], pair=pair)
    y2 = ops.q4_matmul(qw, xd, pair=pair)
    tile_split = (n + 63) // 64 < 512
    if tile_split or k < 2048:
        assert torch.equal(y1[0], y2[0])
    else:
        # |x| ~ 0.8, |w| ~ 0.016: the sum of |x_k w_k| is ~0.013 k, and
        # reordering four f32 partial sums moves the result by a few ulps of it
        bound = 1e-6 * 0.013 * k
        assert float((y1[0] - y2[0]).abs().max()) <= bound
    yb = ops.q4_matmul(qw, xd[:1], pair=pair, epilogue=_lib.SM_EPI_STORE_BF16)
    assert torch.equal(yb.float(), y1.to(torch.bfloat16).float())
    base = torch.randn(1, n, device=dev)
    acc = base.clone()
    ops.q4_matmul(qw, xd[:1], out=acc, pair=pair, epilogue=_lib.SM_EPI_ADD_F32)
    assert torch.equal(acc, base + y1)
    if n * k <= 1000 * 640:  # against the decoded weights in f64
        codes = qw.codes.cpu().numpy()
        scales = qw.scales.cpu().numpy().view(np.uint16)
        dense = oracle.q4_decode(codes, scales, n * k).reshape(n, k).astype(np.float64)
        xr = (ops.unpair(xd[:1]) if pair else xd[:1].float()).cpu().numpy().astype(np.float64)
        y_ref = xr @ dense.T
        tol = 2e-6 * (np.abs(xr) @ np.abs(dense).T) + 1e-7
        assert np.all(np.abs(y1.cpu().numpy() - y_ref) <= tol)


WIDE_EPI = [("store", _lib.SM_EPI_STORE_F32), ("bf16", _lib.SM_EPI_STORE_BF16),
            ("add", _lib.SM_EPI_ADD_F32), ("swiglu_bf16", _lib.SM_EPI_SWIGLU_BF16),
            ("swiglu_f16", _lib.SM_EPI_SWIGLU_F16), ("swiglu_pair", _lib.SM_EPI_SWIGLU_F16X2)]


@pytest.mark.parametrize("m,n,k", [(2048, 4096, 512), (2000, 4000, 384)])
@pytest.mark.parametrize("pair", [False, True])
@pytest.mark.parametrize("epi", [e for e, _ in WIDE_EPI])
def test_wide_kernel_equals_tile_kernel(dev, m, n, k, pair, epi):
    """Large dense problems (>= 128 workgroups of 256 x 256) run the wide-tile
    kernel; its accumulation order is the 128 x 128 kernel's, which row chunks
    of 512 rows (32 workgroups of 256 x 256, too few for the wide kernel; above
    the decode sizes that take the LDS-staged kernel) still run: results agree
    bit for bit, for every epilogue, f16 and f16-pair inputs, and ragged M / N
    edges."""
    print(f"case wide m={m} n={n} k={k} pair={pair} epi={epi}", flush=True)
    e = dict(WIDE_EPI)[epi]
    w = torch.empty(n, k, device=dev)
    ops.fill_normal(w, 0.0, 0.05, seed=n + k)
    qw = ops.Q4Weight.quantize(w)
    x = torch.randn(m, k, device=dev)
    xd = ops.f16_pair(x) if pair else x.to(torch.float16)
    if e == _lib.SM_EPI_ADD_F32:
        base = torch.randn(m, n, device=dev)
        big = base.clone()
        ops.q4_matmul(qw, xd, out=big, epilogue=e, pair=pair)
        ref = base.clone()
        for r0 in range(0, m, 512):
            ops.q4_matmul(qw, xd[r0:r0 + 512], out=ref[r0:r0 + 512], epilogue=e, pair=pair)
    else:
        big = ops.q4_matmul(qw, xd, epilogue=e, pair=pair)
        ref = torch.cat([ops.q4_matmul(qw, xd[r0:r0 + 512], epilogue=e, pair=pair)
                         for r0 in range(0, m, 512)])
    assert big.shape == ref.shape
    assert torch.equal(big.view(torch.int16) if big.dtype != torch.float32 else big,
                       ref.view(torch.int16) if ref.dtype != torch.float32 else ref)


@pytest.mark.parametrize("S,L,H,KVH", [(8, 320, 32, 16), (10, 300, 32, 8)])
def test_wide_kernel_qkv_rope_equals_tile_kernel(dev, S, L, H, KVH):
    """sm_q4_qkv_rope over a prefill-sized batch (the wide kernel) writes the
    same q / K / V cache bits as one sequence at a time (the 128 x 128 kernel)."""
    from summa_amd._lib import SM_F16, SM_F16X2, call
    print(f"case wide qkv-rope S={S} L={L} H={H} KVH={KVH}", flush=True)
    hd, K, p0 = 64, 512, 3
    N = (H + 2 * KVH) * hd
    w = torch.empty(N, K, device=dev)
    ops.fill_normal(w, 0.0, 0.05, seed=N)
    qw = ops.Q4Weight.quantize(w)
    xp = ops.f16_pair(torch.randn(S * L, K, device=dev))
    cap = p0 + L + 1
    half = hd // 2
    inv = 1.0 / (10000.0 ** (np.arange(half) * 2.0 / hd))
    ang = np.arange(cap)[:, None] * inv[None, :]
    tab = torch.from_numpy(np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)).to(dev)
    pos0 = torch.tensor([p0 + s for s in range(S)], dtype=torch.int32, device=dev) % 2
    st = torch.cuda.current_stream().cuda_stream
    outs = []
    for chunked in (False, True):
        q = torch.zeros(S * L, H, hd, dtype=torch.float16, device=dev)
        kc = torch.zeros(S, KVH, cap, hd, dtype=torch.float16, device=dev)
        vc = torch.zeros(S, KVH, cap, hd, dtype=torch.float16, device=dev)
        spans = [(s, 1) for s in range(S)] if chunked else [(0, S)]
        for s0, ns in spans:
            call("sm_q4_qkv_rope", qw.tcodes.data_ptr(), qw.tscales.data_ptr(), H, KVH, hd, K,
                 xp[s0 * L:].data_ptr(), SM_F16X2, ns, L, xp.stride(0), tab.data_ptr(),
                 pos0[s0:].data_ptr(), cap, q[s0 * L:].data_ptr(), kc[s0:].data_ptr(),
                 vc[s0:].data_ptr(), SM_F16, st)
        outs.append((q, kc, vc))
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("m,n,k", [(128, 2304, 768), (256, 2048, 2048), (256, 3072, 2048),
                                   (200, 6144, 768), (33, 4096, 1024), (64, 8192, 256)])
@pytest.mark.parametrize("pair", [True, False])
def test_dense_decode_lds_kernel(dev, m, n, k, pair):
    """Decode-batch shapes (32 < M <= 256, K <= 2048, 2k-8k columns) run the
    kernel that stages each 16-row activation tile once per workgroup in LDS
    (dense mode of the grouped decode kernel): store, bf16, residual add and
    SwiGLU epilogues against float64 on the decoded weights."""
    print(f"case dense-lds m={m} n={n} k={k} pair={pair}", flush=True)
    w = _weights(n, k, m + n)
    codes, scales = oracle.q4_quantize(w)
    qw = ops.Q4Weight.from_host(codes, scales, n, k, dev)
    x = np.random.default_rng(m + 2).normal(0, 1, (m, k)).astype(np.float32)
    if pair:
        xp, xr = _pair_host(x)
        xd = torch.from_numpy(xp).to(dev)
    else:
        xd = torch.from_numpy(x).to(dev).to(torch.float16)
        xr = xd.float().cpu().numpy()
    dense = oracle.q4_decode(codes, scales, n * k).reshape(n, k).astype(np.float64)
    y_ref = xr.astype(np.float64) @ dense.T
    tol = 2e-6 * _bound(codes, scales, n, k, xr) + 1e-7
    y = ops.q4_matmul(qw, xd, pair=pair).cpu().numpy()
    assert np.all(np.abs(y - y_ref) <= tol), float(np.abs(y - y_ref).max())
    yb = ops.q4_matmul(qw, xd, pair=pair, epilogue=_lib.SM_EPI_STORE_BF16)
    assert torch.equal(yb.float().cpu(), torch.from_numpy(y).to(torch.bfloat16).float())
    base = np.random.default_rng(4).normal(0, 1, (m, n)).astype(np.float32)
    acc = torch.from_numpy(base.copy()).to(dev)
    ops.q4_matmul(qw, xd, out=acc, pair=pair, epilogue=_lib.SM_EPI_ADD_F32)
    np.testing.assert_array_equal(acc.cpu().numpy(), base + y)
    F = n // 2
    h = ops.q4_matmul(qw, xd, pair=pair,
                      epilogue=_lib.SM_EPI_SWIGLU_F16X2 if pair else _lib.SM_EPI_SWIGLU_F16)
    h = (ops.unpair(h) if pair else h.float()).cpu().numpy()
    g, v = y_ref[:, :F], y_ref[:, F:]
    ref_h = g / (1 + np.exp(-g)) * v
    hb = (np.abs(g) + 1) * (tol[:, F:] + tol[:, :F]) * (np.abs(v) + 1)
    rel = 1e-6 if pair else 2.0 ** -11
    assert np.all(np.abs(h - ref_h) <= hb + rel * np.abs(ref_h) + 1e-7)


@pytest.mark.parametrize("m,n,k", [(256, 11264, 2048), (200, 8320, 512), (129, 8448, 256)])
@pytest.mark.parametrize("pair", [True, False])
def test_decode_ffn_in_thick_kernel(dev, m, n, k, pair):
    """The decode FFN-in shapes (128 < M <= 256, more than 8192 gate + value
    columns: config[2]'s 256 x 2 x 5632) run the 32 x 128-tile thick-wave
    kernel: its SwiGLU epilogues (f16 pair, f16, bf16) against float64 on the
    decoded weights, ragged row tiles included."""
    print(f"case thick ffn-in m={m} n={n} k={k} pair={pair}", flush=True)
    w = _weights(n, k, m + 3 * n)
    codes, scales = oracle.q4_quantize(w)
    qw = ops.Q4Weight.from_host(codes, scales, n, k, dev)
    x = np.random.default_rng(m + 5).normal(0, 1, (m, k)).astype(np.float32)
    if pair:
        xp, xr = _pair_host(x)
        xd = torch.from_numpy(xp).to(dev)
    else:
        xd = torch.from_numpy(x).to(dev).to(torch.float16)
        xr = xd.float().cpu().numpy()
    dense = oracle.q4_decode(codes, scales, n * k).reshape(n, k).astype(np.float64)
    y_ref = xr.astype(np.float64) @ dense.T
    tol = 2e-6 * _bound(codes, scales, n, k, xr) + 1e-7
    F = n // 2
    g, v = y_ref[:, :F], y_ref[:, F:]
    ref_h = g / (1 + np.exp(-g)) * v
    hb = (np.abs(g) + 1) * (tol[:, F:] + tol[:, :F]) * (np.abs(v) + 1)
    epis = ([(_lib.SM_EPI_SWIGLU_F16X2, ops.unpair, 1e-6)] if pair else
            [(_lib.SM_EPI_SWIGLU_F16, lambda t: t.float(), 2.0 ** -11),
             (_lib.SM_EPI_SWIGLU_BF16, lambda t: t.float(), 2.0 ** -8)])
    for e, conv, rel in epis:
        h = conv(ops.q4_matmul(qw, xd, pair=pair, epilogue=e)).cpu().numpy()
        assert h.shape == (m, F)
        assert np.all(np.abs(h - ref_h) <= hb + rel * np.abs(ref_h) + 1e-7), e


@pytest.mark.parametrize("S,H,KVH,hd,K", [(128, 12, 12, 64, 768), (256, 16, 4, 128, 2048),
                                          (40, 16, 16, 128, 2048)])
def test_dense_decode_lds_qkv_rope(dev, S, H, KVH, hd, K):
    """sm_q4_qkv_rope at decode size (one new token per sequence, the LDS
    kernel's RoPE epilogue): q and the appended K/V rows against the f32
    matmul of the same weights with RoPE applied on the host; every other
    cache slot stays untouched."""
    from summa_amd._lib import SM_F16, SM_F16X2, call
    print(f"case dense-lds qkv-rope S={S} H={H} KVH={KVH} hd={hd} K={K}", flush=True)
    N = (H + 2 * KVH) * hd
    w = torch.empty(N, K, device=dev)
    ops.fill_normal(w, 0.0, 0.05, seed=N + K)
    qw = ops.Q4Weight.quantize(w)
    xp = ops.f16_pair(torch.randn(S, K, device=dev))
    cap = 64
    pos0 = torch.from_numpy(np.random.default_rng(S).integers(0, cap, S).astype(np.int32)).to(dev)
    half = hd // 2
    inv = 1.0 / (10000.0 ** (np.arange(half) * 2.0 / hd))
    ang = np.arange(cap)[:, None] * inv[None, :]
    tab = torch.from_numpy(np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)).to(dev)
    q = torch.zeros(S, H, hd, dtype=torch.float16, device=dev)
    kc = torch.full((S, KVH, cap, hd), 7.0, dtype=torch.float16, device=dev)
    vc = torch.full((S, KVH, cap, hd), 7.0, dtype=torch.float16, device=dev)
    call("sm_q4_qkv_rope", qw.tcodes.data_ptr(), qw.tscales.data_ptr(), H, KVH, hd, K,
         xp.data_ptr(), SM_F16X2, S, 1, xp.stride(0), tab.data_ptr(), pos0.data_ptr(), cap,
         q.data_ptr(), kc.data_ptr(), vc.data_ptr(), SM_F16, torch.cuda.current_stream().cuda_stream)
    y = ops.q4_matmul(qw, xp, pair=True).cpu().numpy().astype(np.float64).reshape(S, H + 2 * KVH, hd)
    p = pos0.cpu().numpy()
    c, s_ = np.cos(ang[p])[:, None, :], np.sin(ang[p])[:, None, :]
    def rope(t):
        a, b = t[..., 0::2], t[..., 1::2]
        out = np.empty_like(t)
        out[..., 0::2], out[..., 1::2] = a * c - b * s_, b * c + a * s_
        return out
    q_ref, k_ref, v_ref = rope(y[:, :H]), rope(y[:, H:H + KVH]), y[:, H + KVH:]
    tol = lambda r: 2.0 ** -10 * np.abs(r) + 1e-4
    qn = q.float().cpu().numpy()
    assert np.all(np.abs(qn - q_ref) <= tol(q_ref)), float(np.abs(qn - q_ref).max())
    kn, vn = kc.float().cpu().numpy(), vc.float().cpu().numpy()
    rows = np.arange(S)
    kg, vg = kn[rows, :, p], vn[rows, :, p]
    assert np.all(np.abs(kg - k_ref) <= tol(k_ref)), float(np.abs(kg - k_ref).max())
    assert np.all(np.abs(vg - v_ref) <= tol(v_ref)), float(np.abs(vg - v_ref).max())
    mask = np.ones((S, cap), bool)
    mask[rows, p] = False
    assert np.all(kn.transpose(0, 2, 1, 3)[mask] == 7.0) and np.all(vn.transpose(0, 2, 1, 3)[mask] == 7.0)


# Recompute / prefill GEMM shapes of configs [1] and [2] (tokens x out x in):
# qkv, o, FFN-in and down. At M >= 256 with >= 128 workgroups of 256 x 256
# and f16 / f16-pair inputs these run the wide-tile kernel.
RECOMPUTE_SHAPES = [(16384, 3072, 2048), (16384, 2048, 2048), (16384, 11264, 2048),
                    (16384, 2048, 5632), (8192, 2304, 768), (8192, 6144, 768), (8192, 768, 3072)]


@pytest.mark.parametrize("m,n,k", RECOMPUTE_SHAPES)
@pytest.mark.parametrize("pair", [True, False])
def test_wide_kernel_recompute_shapes_vs_f64(dev, m, n, k, pair):
    """The wide-tile kernel at the log-prob recompute shapes against float64
    on the decoded weights (PackedTensor::decode . x, quantization.rs:445-497,
    630-654), for every epilogue, on a sample of rows (the first and last of
    each 256-row tile band edge and random ones) over all columns."""
    print(f"case wide-f64 m={m} n={n} k={k} pair={pair}", flush=True)
    w = torch.empty(n, k, device=dev)
    ops.fill_normal(w, 0.0, 0.02, seed=m + n + k)
    qw = ops.Q4Weight.quantize(w)
    del w
    x = torch.randn(m, k, device=dev, generator=torch.Generator(device=dev).manual_seed(k))
    xd = ops.f16_pair(x) if pair else x.to(torch.float16)
    xv = ops.unpair(xd) if pair else xd.float()  # the values the kernel consumes
    rng = np.random.default_rng(n)
    rows = np.unique(np.concatenate([[0, 255, 256, m // 2 - 1, m - 256, m - 1],
                                     rng.integers(0, m, 42)]))
    ridx = torch.from_numpy(rows).to(dev)
    codes = qw.codes.cpu().numpy()
    scales = qw.scales.cpu().numpy().view(np.uint16)
    dense = oracle.q4_decode(codes, scales, n * k).reshape(n, k).astype(np.float64)
    xr = xv[ridx].cpu().numpy().astype(np.float64)
    y_ref = xr @ dense.T
    tol = 2e-6 * (np.abs(xr) @ np.abs(dense).T) + 1e-7
    y = ops.q4_matmul(qw, xd, pair=pair)
    yr = y[ridx].cpu().numpy()
    assert np.all(np.abs(yr - y_ref) <= tol), float(np.abs(yr - y_ref).max())
    yb = ops.q4_matmul(qw, xd, pair=pair, epilogue=_lib.SM_EPI_STORE_BF16)[ridx]
    assert torch.equal(yb.float().cpu(), torch.from_numpy(yr).to(torch.bfloat16).float())
    base = torch.randn(m, n, device=dev)
    acc = base.clone()
    ops.q4_matmul(qw, xd, out=acc, pair=pair, epilogue=_lib.SM_EPI_ADD_F32)
    np.testing.assert_array_equal(acc[ridx].cpu().numpy(), base[ridx].cpu().numpy() + yr)
    del acc, base, y
    F = n // 2
    g, v = y_ref[:, :F], y_ref[:, F:]
    ref_h = g / (1 + np.exp(-g)) * v
    hb = (np.abs(g) + 1) * (tol[:, F:] + tol[:, :F]) * (np.abs(v) + 1)
    for e, conv, rel in ((_lib.SM_EPI_SWIGLU_F16X2, ops.unpair, 1e-6),
                         (_lib.SM_EPI_SWIGLU_F16, lambda t: t.float(), 2.0 ** -10),
                         (_lib.SM_EPI_SWIGLU_BF16, lambda t: t.float(), 2.0 ** -8)):
        h = conv(ops.q4_matmul(qw, xd, pair=pair, epilogue=e)[ridx]).cpu().numpy()
        assert np.all(np.abs(h - ref_h) <= hb + rel * np.abs(ref_h) + 1e-7), \
            (e, float(np.abs(h - ref_h).max()))


GEMV_JOBS = [(3072, 2048), (2048, 2048), (11264, 2048), (2048, 5632), (2304, 768), (768, 3072),
             (1000, 640), (65536, 2048)]


@pytest.mark.parametrize("pair", [False, True])
def test_gemv_multi_equals_single_launches(dev, pair):
    """sm_q4_gemv_multi over jobs of different N, K and epilogues (ragged N,
    K from 640 to 5632, the LM head) gives each job's sm_q4_matmul M = 1
    result bit for bit, and a second launch of the same plan repeats it."""
    print(f"case gemv-multi pair={pair}", flush=True)
    g = torch.Generator().manual_seed(3)
    epis = [_lib.SM_EPI_STORE_F32, _lib.SM_EPI_ADD_F32, _lib.SM_EPI_STORE_BF16]
    jobs, refs = [], []
    for i, (n, k) in enumerate(GEMV_JOBS):
        w = torch.empty(n, k, device=dev)
        ops.fill_normal(w, 0.0, 0.05, seed=10 + i)
        qw = ops.Q4Weight.quantize(w)
        x = torch.randn(1, k, generator=g).to(dev)
        xd = ops.f16_pair(x) if pair else x.to(torch.float16)
        epi = epis[i % 3]
        dt = torch.bfloat16 if epi == _lib.SM_EPI_STORE_BF16 else torch.float32
        base = torch.randn(1, n, generator=g).to(dev).to(dt)
        y, ref = base.clone(), base.clone()
        ops.q4_matmul(qw, xd, out=ref, epilogue=epi, pair=pair)
        jobs.append((qw, xd, y, epi))
        refs.append((base, ref))
    batch = ops.GemvBatch(jobs, pair=pair)
    assert batch.nblocks == sum((n + 15) // 16 for n, _ in GEMV_JOBS)
    batch.launch()
    for (qw, xd, y, epi), (base, ref) in zip(jobs, refs):
        assert torch.equal(y.view(torch.int16) if y.dtype != torch.float32 else y,
                           ref.view(torch.int16) if ref.dtype != torch.float32 else ref), qw.n
        y.copy_(base)
    batch.launch()
    for (qw, xd, y, epi), (base, ref) in zip(jobs, refs):
        assert torch.equal(y.float(), ref.float()), qw.n


@pytest.mark.parametrize("m,n,k,exact", [(256, 2048, 2048, False), (256, 2048, 5632, True),
                                         (128, 2048, 2048, False), (200, 1024, 2048, True),
                                         (128, 768, 768, False), (128, 768, 3072, False),
                                         (1024, 2048, 2048, True)])
def test_matmul_add_rmsnorm(dev, m, n, k, exact):
    """sm_q4_matmul_add_rmsnorm (a residual projection and the RMSNorm after
    it in one call) against the two-step form (sm_q4_matmul_ws + sm_rmsnorm):
    the normalised rows are always sm_rmsnorm's bits of the returned residual;
    the residual equals the two-step one bit for bit where the matmul splits K
    itself or the fused form does not apply (exact), and is within the split
    tolerance of base + x.W^T in f64 everywhere. Shapes: config[2]'s decode o
    (forced split) and down projections, config[4]'s o at 128 rows, a narrow
    N, config[1]'s decode o and down (768 columns, where the plain matmul
    takes the in-workgroup K-split kernel), and a prefill shape that falls
    back to the two steps."""
    print(f"case add+rmsnorm m={m} n={n} k={k}", flush=True)
    st = torch.cuda.current_stream().cuda_stream
    w = _weights(n, k, m + n + k)
    codes, scales = oracle.q4_quantize(w)
    qw = ops.Q4Weight.from_host(codes, scales, n, k, dev)
    x = np.random.default_rng(m + 11).normal(0, 1, (m, k)).astype(np.float32)
    xp, xr = _pair_host(x)
    xd = torch.from_numpy(xp).to(dev)
    rng = np.random.default_rng(n)
    base = rng.normal(0, 1, (m, n)).astype(np.float32)
    gamma = torch.from_numpy(rng.uniform(0.5, 1.5, n).astype(np.float32)).to(dev)
    eps = 1e-5
    ws = ops.q4_workspace(m, n, k, _lib.SM_EPI_ADD_F32, dev)

    def fused():
        r = torch.from_numpy(base.copy()).to(dev)
        h = torch.empty((m, 2 * n), dtype=torch.float16, device=dev)
        _lib.call("sm_q4_matmul_add_rmsnorm", qw.tcodes.data_ptr(), qw.tscales.data_ptr(), n, k,
                  xd.data_ptr(), _lib.SM_F16X2, m, 2 * k, r.data_ptr(), gamma.data_ptr(), eps,
                  h.data_ptr(), ws.data_ptr(), ws.numel(), st)
        return r, h

    def norm(r):
        h = torch.empty((m, 2 * n), dtype=torch.float16, device=dev)
        _lib.call("sm_rmsnorm", r.data_ptr(), gamma.data_ptr(), m, n, eps, h.data_ptr(),
                  _lib.SM_F16X2, st)
        return h

    r1, h1 = fused()
    r1b, h1b = fused()
    torch.testing.assert_close(r1, r1b, rtol=0, atol=0)  # run to run
    torch.testing.assert_close(h1, h1b, rtol=0, atol=0)
    torch.testing.assert_close(h1, norm(r1), rtol=0, atol=0)
    r2 = torch.from_numpy(base.copy()).to(dev)
    ops.q4_matmul(qw, xd, out=r2, epilogue=_lib.SM_EPI_ADD_F32, pair=True, workspace=ws)
    if exact:
        torch.testing.assert_close(r1, r2, rtol=0, atol=0)
        torch.testing.assert_close(h1, norm(r2), rtol=0, atol=0)
    dense = oracle.q4_decode(codes, scales, n * k).reshape(n, k).astype(np.float64)
    expect = base + xr.astype(np.float64) @ dense.T
    tol = 2e-6 * _bound(codes, scales, n, k, xr) + 1e-6
    got = r1.cpu().numpy()
    assert np.all(np.abs(got - expect) <= tol), float(np.abs(got - expect).max())
