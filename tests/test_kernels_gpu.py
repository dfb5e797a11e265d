"""Per-kernel GPU checks: attention (decode / prefill), RoPE + KV append, RMSNorm,
embedding and token selection, each against a CPU restatement."""
import numpy as np
import pytest
import torch

import oracle
from summa_amd import _lib
from summa_amd._lib import SM_BF16, SM_F16, SM_F16X2, SM_F32, call

pytestmark = pytest.mark.gpu


def _s():
    return torch.cuda.current_stream().cuda_stream


def _bf16(a, dev):
    return torch.from_numpy(oracle.bf16_bits(a).view(np.int16)).to(dev).view(torch.bfloat16)


def _f16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float16)).to(dev)


def _unpair(t, width):
    """SM_F16X2 rows (hi[width] | lo[width]) -> f64 values hi + lo."""
    a = t.cpu().numpy().astype(np.float64).reshape(-1, 2 * width)
    return a[:, :width] + a[:, width:]


def _attn_ref(q, k, v, lens):
    """q [S, H, hd], k/v [S, KVH, T, hd] -> [S, H, hd] in f64 (repeat_kv GQA)."""
    S, H, hd = q.shape
    KVH = k.shape[1]
    out = np.zeros((S, H, hd))
    for s in range(S):
        for h in range(H):
            kv = h // (H // KVH)
            n = lens[s]
            sc = k[s, kv, :n].astype(np.float64) @ q[s, h].astype(np.float64) / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            out[s, h] = (p / p.sum()) @ v[s, kv, :n].astype(np.float64)
    return out


@pytest.mark.parametrize("S,H,KVH,hd,cap", [(3, 12, 12, 64, 300), (4, 16, 4, 128, 1100),
                                            (2, 4, 4, 64, 70), (5, 8, 1, 128, 257),
                                            (3, 12, 4, 64, 200), (2, 16, 8, 128, 300),
                                            (2, 32, 2, 128, 400)])
def test_attn_decode_bf16(dev, S, H, KVH, hd, cap):
    print(f"case S={S} H={H} KVH={KVH} hd={hd} cap={cap}", flush=True)
    rng = np.random.default_rng(S * H + cap)
    q = oracle.round_bf16(rng.normal(0, 1, (S, H, hd)).astype(np.float32))
    k = oracle.round_bf16(rng.normal(0, 1, (S, KVH, cap, hd)).astype(np.float32))
    v = oracle.round_bf16(rng.normal(0, 1, (S, KVH, cap, hd)).astype(np.float32))
    lens = rng.integers(1, cap + 1, S).astype(np.int32)
    lens[0] = cap
    out = torch.empty(S, H, hd, dtype=torch.bfloat16, device=dev)
    L = torch.from_numpy(lens).to(dev)
    qd, kd, vd = _bf16(q, dev), _bf16(k, dev), _bf16(v, dev)
    call("sm_attn_decode", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), L.data_ptr(),
         out.data_ptr(), SM_BF16, SM_BF16, S, H, KVH, cap, hd, _s())
    ref = _attn_ref(q, k, v, lens)
    # bf16 output: one rounding (2^-8 relative) on top of fp32 accumulation
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, rtol=2 ** -7, atol=2e-3)


@pytest.mark.parametrize("S,H,KVH,hd,cap", [(3, 12, 12, 64, 300), (4, 16, 4, 128, 1100),
                                            (5, 8, 1, 128, 257), (3, 12, 4, 64, 200),
                                            (2, 16, 8, 128, 300), (2, 32, 2, 128, 400)])
def test_attn_decode_f16_cache_pair_out(dev, S, H, KVH, hd, cap):
    """f16 q / cache (the quantized models' KV dtype), f16-pair output: only the
    fp32 accumulation separates the result from the exact attention."""
    print(f"case f16 S={S} H={H} KVH={KVH} hd={hd} cap={cap}", flush=True)
    rng = np.random.default_rng(S * H + cap + 1)
    q, k, v = (rng.normal(0, 1, sh).astype(np.float16)
               for sh in ((S, H, hd), (S, KVH, cap, hd), (S, KVH, cap, hd)))
    lens = rng.integers(1, cap + 1, S).astype(np.int32)
    lens[0] = cap
    out = torch.empty(S, 2 * H * hd, dtype=torch.float16, device=dev)
    L = torch.from_numpy(lens).to(dev)
    qd, kd, vd = _f16(q, dev), _f16(k, dev), _f16(v, dev)
    call("sm_attn_decode", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), L.data_ptr(),
         out.data_ptr(), SM_F16, SM_F16X2, S, H, KVH, cap, hd, _s())
    ref = _attn_ref(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), lens)
    np.testing.assert_allclose(_unpair(out, H * hd).reshape(S, H, hd), ref, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("H,KVH,hd", [(16, 4, 128), (12, 12, 64), (8, 1, 128)])
def test_attn_decode_tile_edges(dev, H, KVH, hd):
    """Lengths around the 32-key tile and the 4-wave stride (1, 31-33, 127-129,
    255-257 keys): the clamped loads past the end and the masked keys of a
    partial tile must not reach the result."""
    lens = np.array([1, 31, 32, 33, 127, 128, 129, 255, 256, 257], dtype=np.int32)
    S, cap = len(lens), 300
    print(f"case tile edges H={H} KVH={KVH} hd={hd} lens={lens.tolist()}", flush=True)
    rng = np.random.default_rng(hd + H)
    q, k, v = (rng.normal(0, 1, sh).astype(np.float16)
               for sh in ((S, H, hd), (S, KVH, cap, hd), (S, KVH, cap, hd)))
    # poison the rows past each length: a read of them would show in the result
    for s_, n in enumerate(lens):
        k[s_, :, n:] = 60.0
        v[s_, :, n:] = 1000.0
    out = torch.empty(S, 2 * H * hd, dtype=torch.float16, device=dev)
    L = torch.from_numpy(lens).to(dev)
    qd, kd, vd = _f16(q, dev), _f16(k, dev), _f16(v, dev)
    call("sm_attn_decode", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), L.data_ptr(),
         out.data_ptr(), SM_F16, SM_F16X2, S, H, KVH, cap, hd, _s())
    ref = _attn_ref(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), lens)
    np.testing.assert_allclose(_unpair(out, H * hd).reshape(S, H, hd), ref, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("G,S,H,KVH,hd,P,cap,kf16",
                         [(8, 16, 16, 4, 128, 512, 700, True), (8, 16, 12, 12, 64, 128, 300, True),
                          (4, 8, 8, 2, 128, 40, 100, True), (2, 6, 16, 1, 64, 600, 700, True),
                          (8, 16, 16, 4, 128, 300, 400, False), (1, 3, 4, 4, 64, 33, 90, True)])
def test_attn_decode_prefix(dev, G, S, H, KVH, hd, P, cap, kf16):
    """Shared-prompt decode attention (sm_attn_decode_prefix): rollout s attends
    its group's prompt keys 0..P-1 (stored once per group) and its own keys
    P..lens[s]-1, against f64 attention over the concatenation, and against
    sm_attn_decode over per-rollout copies of the prompt (same keys, other
    f32 order). Prompt lengths off the 32-key tiles, empty continuations
    (lens = P), one and two 16-query blocks, one and two key splits. The
    per-rollout cache rows below P and past each length are poisoned."""
    print(f"case prefix G={G} S={S} H={H} KVH={KVH} hd={hd} P={P} cap={cap} f16={kf16}",
          flush=True)
    rng = np.random.default_rng(G * 1000 + P + hd)
    groups = S // G
    q = rng.normal(0, 1, (S, H, hd)).astype(np.float32)
    pk = rng.normal(0, 1, (groups, KVH, P, hd)).astype(np.float32)
    pv = rng.normal(0, 1, (groups, KVH, P, hd)).astype(np.float32)
    k = rng.normal(0, 1, (S, KVH, cap, hd)).astype(np.float32)
    v = rng.normal(0, 1, (S, KVH, cap, hd)).astype(np.float32)
    rnd = (lambda a: a.astype(np.float16).astype(np.float32)) if kf16 else oracle.round_bf16
    q, pk, pv, k, v = (rnd(a) for a in (q, pk, pv, k, v))
    lens = rng.integers(P, cap + 1, S).astype(np.int32)
    lens[0], lens[-1] = P, P + 1
    full_k, full_v = k.copy(), v.copy()  # the per-rollout cache with the prompt copied in
    for s_ in range(S):
        full_k[s_, :, :P], full_v[s_, :, :P] = pk[s_ // G], pv[s_ // G]
        k[s_, :, :P], v[s_, :, :P] = 60.0, 1000.0  # never read: the prompt comes from pk / pv
        k[s_, :, lens[s_]:], v[s_, :, lens[s_]:] = 60.0, 1000.0
        full_k[s_, :, lens[s_]:], full_v[s_, :, lens[s_]:] = 60.0, 1000.0
    to = (lambda a: _f16(a, dev)) if kf16 else (lambda a: _bf16(a, dev))
    dt = SM_F16 if kf16 else SM_BF16
    qd, pkd, pvd, kd, vd = (to(a) for a in (q, pk, pv, k, v))
    L = torch.from_numpy(lens).to(dev)
    nws = int(_lib.lib().sm_attn_decode_prefix_workspace_bytes(S, G, P, H, KVH, hd))
    assert nws > 0
    ws = torch.empty(nws // 4, dtype=torch.float32, device=dev)
    out = torch.empty(S, 2 * H * hd, dtype=torch.float16, device=dev)
    call("sm_attn_decode_prefix", qd.data_ptr(), pkd.data_ptr(), pvd.data_ptr(), kd.data_ptr(),
         vd.data_ptr(), L.data_ptr(), out.data_ptr(), ws.data_ptr(), nws, dt, SM_F16X2, S, G, P,
         H, KVH, cap, hd, _s())
    got = _unpair(out, H * hd).reshape(S, H, hd)
    ref = _attn_ref(q, full_k, full_v, lens)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-6)
    fk, fv = to(full_k), to(full_v)
    out2 = torch.empty_like(out)
    call("sm_attn_decode", qd.data_ptr(), fk.data_ptr(), fv.data_ptr(), L.data_ptr(),
         out2.data_ptr(), dt, SM_F16X2, S, H, KVH, cap, hd, _s())
    np.testing.assert_allclose(got, _unpair(out2, H * hd).reshape(S, H, hd), rtol=2e-5, atol=2e-6)


def test_attn_decode_prefix_rejects(dev):
    """Bad shapes and a short workspace are refused before any launch."""
    ws = torch.empty(16, dtype=torch.float32, device=dev)
    x = torch.empty(16, dtype=torch.float16, device=dev)
    L = torch.full((4,), 8, dtype=torch.int32, device=dev)
    p = [x.data_ptr()] * 5 + [L.data_ptr(), x.data_ptr(), ws.data_ptr()]
    with pytest.raises(RuntimeError, match="workspace"):
        call("sm_attn_decode_prefix", *p, 64, SM_F16, SM_F16X2, 4, 2, 8, 4, 4, 16, 64, _s())
    with pytest.raises(RuntimeError, match="whole groups"):
        call("sm_attn_decode_prefix", *p, 1 << 20, SM_F16, SM_F16X2, 5, 2, 8, 4, 4, 16, 64, _s())
    with pytest.raises(RuntimeError, match="32 per group"):
        call("sm_attn_decode_prefix", *p, 1 << 20, SM_F16, SM_F16X2, 4, 4, 8, 16, 1, 16, 64, _s())
    with pytest.raises(RuntimeError, match="P <= cap"):
        call("sm_attn_decode_prefix", *p, 1 << 20, SM_F16, SM_F16X2, 4, 2, 20, 4, 4, 16, 64, _s())


@pytest.mark.parametrize("S,L,p0,H,KVH,hd", [(2, 100, 0, 4, 4, 64), (2, 64, 0, 16, 4, 128),
                                             (1, 130, 3, 8, 2, 128)])
def test_attn_prefill_f16_cache_pair_out(dev, S, L, p0, H, KVH, hd):
    print(f"case f16 prefill S={S} L={L} p0={p0} H={H} KVH={KVH} hd={hd}", flush=True)
    rng = np.random.default_rng(L + hd + 1)
    cap = p0 + L
    q, k, v = (rng.normal(0, 1, sh).astype(np.float16)
               for sh in ((S, L, H, hd), (S, KVH, cap, hd), (S, KVH, cap, hd)))
    out = torch.empty(S * L, 2 * H * hd, dtype=torch.float16, device=dev)
    pos0 = torch.full((S,), p0, dtype=torch.int32, device=dev)
    qd, kd, vd = _f16(q, dev), _f16(k, dev), _f16(v, dev)
    call("sm_attn_prefill", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), pos0.data_ptr(),
         out.data_ptr(), SM_F16, SM_F16X2, S, L, H, KVH, cap, hd, _s())
    got = _unpair(out, H * hd).reshape(S, L, H, hd)
    qf, kf, vf = (a.astype(np.float32) for a in (q, k, v))
    for r in range(L):
        ref = _attn_ref(qf[:, r], kf, vf, np.full(S, p0 + r + 1))
        # P as an f16 hi + lo pair (~21 bits) and exact f16 V in the P.V MFMA
        np.testing.assert_allclose(got[:, r], ref, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("S,L,p0,H,KVH,hd", [(2, 100, 0, 4, 4, 64), (2, 64, 0, 16, 4, 128),
                                             (3, 37, 5, 12, 12, 64), (1, 130, 3, 8, 2, 128)])
@pytest.mark.parametrize("dtype", [SM_BF16, SM_F32])
def test_attn_prefill(dev, S, L, p0, H, KVH, hd, dtype):
    print(f"case S={S} L={L} p0={p0} H={H} KVH={KVH} hd={hd} dtype={dtype}", flush=True)
    rng = np.random.default_rng(L + hd)
    cap = p0 + L
    q = rng.normal(0, 1, (S, L, H, hd)).astype(np.float32)
    k = rng.normal(0, 1, (S, KVH, cap, hd)).astype(np.float32)
    v = rng.normal(0, 1, (S, KVH, cap, hd)).astype(np.float32)
    if dtype == SM_BF16:
        q, k, v = oracle.round_bf16(q), oracle.round_bf16(k), oracle.round_bf16(v)
        qd, kd, vd = _bf16(q, dev), _bf16(k, dev), _bf16(v, dev)
        out = torch.empty(S, L, H, hd, dtype=torch.bfloat16, device=dev)
    else:
        qd, kd, vd = (torch.from_numpy(a).to(dev) for a in (q, k, v))
        out = torch.empty(S, L, H, hd, dtype=torch.float32, device=dev)
    pos0 = torch.full((S,), p0, dtype=torch.int32, device=dev)
    call("sm_attn_prefill", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), pos0.data_ptr(),
         out.data_ptr(), dtype, dtype, S, L, H, KVH, cap, hd, _s())
    got = out.float().cpu().numpy()
    for r in range(L):
        ref = _attn_ref(q[:, r], k, v, np.full(S, p0 + r + 1))
        if dtype == SM_BF16:
            # P and V enter the P.V MFMA as f16; output rounded to bf16
            np.testing.assert_allclose(got[:, r], ref, rtol=2 ** -7, atol=3e-3)
        else:
            np.testing.assert_allclose(got[:, r], ref, rtol=1e-5, atol=1e-5)


def _rope_table(max_pos, hd, theta=1e4):
    half = hd // 2
    p = np.arange(half)
    freq = theta ** (-2.0 * p / hd)
    ang = np.arange(max_pos)[:, None] * freq[None, :]
    return np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)


def test_rope_append_adjacent_pairs(dev):
    S, L, H, KVH, hd, cap = 2, 5, 4, 2, 64, 16
    rng = np.random.default_rng(0)
    qkv = rng.normal(0, 1, (S * L, (H + 2 * KVH) * hd)).astype(np.float32)
    tab = _rope_table(cap, hd)
    pos0 = np.array([0, 7], np.int32)
    q = torch.empty(S * L, H, hd, device=dev)
    kc = torch.zeros(S, KVH, cap, hd, device=dev)
    vc = torch.zeros(S, KVH, cap, hd, device=dev)
    qkv_d, tab_d, pos_d = (torch.from_numpy(a).to(dev) for a in (qkv, tab, pos0))
    call("sm_rope_append", qkv_d.data_ptr(), tab_d.data_ptr(), pos_d.data_ptr(), S, L, H, KVH,
         hd, cap, q.data_ptr(), SM_F32, kc.data_ptr(), vc.data_ptr(), SM_F32, _s())
    x = qkv.reshape(S, L, H + 2 * KVH, hd)
    for s in range(S):
        for i in range(L):
            pos = pos0[s] + i
            c, sn = tab[pos, :, 0], tab[pos, :, 1]
            a, b = x[s, i, :, 0::2], x[s, i, :, 1::2]
            rot = np.empty_like(x[s, i])
            rot[:, 0::2] = a * c - b * sn
            rot[:, 1::2] = b * c + a * sn
            np.testing.assert_allclose(q.cpu().numpy()[s * L + i], rot[:H], rtol=1e-6, atol=1e-6)
            np.testing.assert_allclose(kc.cpu().numpy()[s, :, pos], rot[H:H + KVH], rtol=1e-6, atol=1e-6)
            np.testing.assert_array_equal(vc.cpu().numpy()[s, :, pos], x[s, i, H + KVH:])
    # untouched cache slots stay zero
    assert np.all(kc.cpu().numpy()[0, :, L:] == 0)
    # f16 q / cache (quantized models): the same values rounded once to f16
    q16 = torch.empty(S * L, H, hd, dtype=torch.float16, device=dev)
    kc16 = torch.zeros(S, KVH, cap, hd, dtype=torch.float16, device=dev)
    vc16 = torch.zeros(S, KVH, cap, hd, dtype=torch.float16, device=dev)
    call("sm_rope_append", qkv_d.data_ptr(), tab_d.data_ptr(), pos_d.data_ptr(), S, L, H, KVH,
         hd, cap, q16.data_ptr(), SM_F16, kc16.data_ptr(), vc16.data_ptr(), SM_F16, _s())
    np.testing.assert_array_equal(q16.cpu().numpy(), q.cpu().numpy().astype(np.float16))
    np.testing.assert_array_equal(kc16.cpu().numpy(), kc.cpu().numpy().astype(np.float16))
    np.testing.assert_array_equal(vc16.cpu().numpy(), vc.cpu().numpy().astype(np.float16))


def test_rmsnorm_and_embed(dev):
    rows, d, V = 5, 768, 100
    rng = np.random.default_rng(1)
    table = rng.normal(0, 0.02, (V, d)).astype(np.float32)
    ids = np.array([3, 0, 99, 42, 3], np.int32)
    x = torch.empty(rows, d, device=dev)
    table_d, ids_d = torch.from_numpy(table).to(dev), torch.from_numpy(ids).to(dev)
    call("sm_embed", table_d.data_ptr(), SM_F32, ids_d.data_ptr(), rows, d, V, 1.0,
         x.data_ptr(), _s())
    np.testing.assert_array_equal(x.cpu().numpy(), table[ids])
    g = rng.uniform(0.5, 1.5, d).astype(np.float32)
    y = torch.empty(rows, d, dtype=torch.bfloat16, device=dev)
    g_d = torch.from_numpy(g).to(dev)
    call("sm_rmsnorm", x.data_ptr(), g_d.data_ptr(), rows, d, 1e-5, y.data_ptr(), SM_BF16, _s())
    xr = table[ids].astype(np.float64)
    ref = xr / np.sqrt((xr ** 2).mean(1, keepdims=True) + 1e-5) * g
    np.testing.assert_allclose(y.float().cpu().numpy(), ref, rtol=2 ** -8, atol=1e-6)
    # f16-pair output: hi = f16(y), lo = f16(y - hi); fp32-level precision
    yp = torch.empty(rows, 2 * d, dtype=torch.float16, device=dev)
    call("sm_rmsnorm", x.data_ptr(), g_d.data_ptr(), rows, d, 1e-5, yp.data_ptr(), SM_F16X2, _s())
    hi = yp.cpu().numpy()[:, :d].astype(np.float64)
    assert np.all(np.abs(hi - ref) <= np.abs(ref) * 2.0 ** -11 + 2.0 ** -24)  # hi = f16(y)
    np.testing.assert_allclose(_unpair(yp, d), ref, rtol=1e-6, atol=1e-7)
    assert np.all(np.abs(yp.cpu().numpy()[:, d:].astype(np.float64))
                  <= np.abs(hi) * 2.0 ** -11 + 2.0 ** -24)


@pytest.mark.parametrize("d", [768, 1024, 2048, 3072, 4096, 320, 1000])
def test_rmsnorm_widths_and_dtypes(dev, d):
    """Wave-per-row kernel (d = 256 * {3, 4, 8, 12, 16}) and the generic
    kernel (other widths) against float64, every output dtype, a row count
    that leaves a partial workgroup."""
    rows = 7
    rng = np.random.default_rng(d)
    x = rng.normal(0, 1.5, (rows, d)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, d).astype(np.float32)
    xd, gd = torch.from_numpy(x).to(dev), torch.from_numpy(g).to(dev)
    xr = x.astype(np.float64)
    ref = xr / np.sqrt((xr ** 2).mean(1, keepdims=True) + 1e-5) * g
    for dt, tdt, rtol in ((SM_F32, torch.float32, 2e-6), (SM_BF16, torch.bfloat16, 2 ** -8),
                          (SM_F16, torch.float16, 2 ** -11)):
        y = torch.full((rows, d), float("nan"), dtype=tdt, device=dev)
        call("sm_rmsnorm", xd.data_ptr(), gd.data_ptr(), rows, d, 1e-5, y.data_ptr(), dt, _s())
        np.testing.assert_allclose(y.float().cpu().numpy(), ref, rtol=rtol, atol=1e-6)
    yp = torch.full((rows, 2 * d), float("nan"), dtype=torch.float16, device=dev)
    call("sm_rmsnorm", xd.data_ptr(), gd.data_ptr(), rows, d, 1e-5, yp.data_ptr(), SM_F16X2, _s())
    np.testing.assert_allclose(_unpair(yp, d), ref, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("temperature", [0.0, 1.0, 0.7])
def test_sample_matches_oracle(dev, temperature):
    rows, V = 16, 32768
    rng = np.random.default_rng(2)
    logits = rng.normal(0, 1, (rows, V)).astype(np.float32)
    logits[3, 100] = logits[3, 200] = 50.0  # exact tie: lowest index wins under greedy
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    lp = torch.empty(rows, device=dev)
    ld = torch.from_numpy(logits).to(dev)
    call("sm_sample", ld.data_ptr(), rows, V, V, float(temperature), 1234, 5, tok.data_ptr(), 1,
         lp.data_ptr(), 1, None, _s())
    rt, rlp = oracle.sample(logits, temperature, 1234, 5)
    np.testing.assert_array_equal(tok.cpu().numpy(), rt)
    np.testing.assert_allclose(lp.cpu().numpy(), rlp, atol=1e-5)
    if temperature == 0.0:
        assert tok.cpu().numpy()[3] == 100


def test_sample_temperature_distribution(dev):
    # Gumbel-max draws follow softmax(l / T): chi-square-style check on a 4-way row
    V, rows, T = 4, 20000, 0.5
    base = np.array([0.0, 0.5, 1.0, -1.0], np.float32)
    logits = torch.from_numpy(np.tile(base, (rows, 1))).to(dev)
    tok = torch.empty(rows, dtype=torch.int32, device=dev)
    call("sm_sample", logits.data_ptr(), rows, V, V, T, 7, 0, tok.data_ptr(), 1, None, 1, None, _s())
    counts = np.bincount(tok.cpu().numpy(), minlength=V) / rows
    p = np.exp(base / T) / np.exp(base / T).sum()
    assert np.all(np.abs(counts - p) < 0.015), (counts, p)


@pytest.mark.parametrize("S,L,p0,H,KVH,hd,K", [(64, 1, 37, 12, 12, 64, 768), (2, 40, 3, 16, 4, 128, 512),
                                               (3, 5, 0, 4, 2, 64, 256), (1, 1, 70, 4, 4, 64, 256)])
def test_qkv_rope_fused_matches_separate(dev, S, L, p0, H, KVH, hd, K):
    """sm_q4_qkv_rope == sm_q4_matmul (f16 pairs) followed by sm_rope_append:
    the same f16 q / cache values up to one f16 rounding step (the two paths
    may accumulate the projection in different kernels)."""
    from summa_amd import ops
    print(f"case qkv-rope S={S} L={L} p0={p0} H={H} KVH={KVH} hd={hd} K={K}", flush=True)
    N = (H + 2 * KVH) * hd
    rng = np.random.default_rng(S + L + K)
    w = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    codes, scales = oracle.q4_quantize(w)
    qw = ops.Q4Weight.from_host(codes, scales, N, K, dev)
    x = torch.from_numpy(rng.normal(0, 1, (S * L, K)).astype(np.float32)).to(dev)
    xp = ops.f16_pair(x)
    cap = p0 + L + 2
    tab = torch.from_numpy(_rope_table(cap, hd)).to(dev)
    pos0 = torch.full((S,), p0, dtype=torch.int32, device=dev)
    outs = []
    for fused in (True, False):
        q = torch.zeros(S * L, H, hd, dtype=torch.float16, device=dev)
        kc = torch.zeros(S, KVH, cap, hd, dtype=torch.float16, device=dev)
        vc = torch.zeros(S, KVH, cap, hd, dtype=torch.float16, device=dev)
        if fused:
            call("sm_q4_qkv_rope", qw.tcodes.data_ptr(), qw.tscales.data_ptr(), H, KVH, hd, K,
                 xp.data_ptr(), SM_F16X2, S, L, xp.stride(0), tab.data_ptr(), pos0.data_ptr(),
                 cap, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), SM_F16, _s())
        else:
            y = ops.q4_matmul(qw, xp, pair=True)
            call("sm_rope_append", y.data_ptr(), tab.data_ptr(), pos0.data_ptr(), S, L, H, KVH,
                 hd, cap, q.data_ptr(), SM_F16, kc.data_ptr(), vc.data_ptr(), SM_F16, _s())
        outs.append([t.float().cpu().numpy() for t in (q, kc, vc)])
    for a, b in zip(*outs):
        np.testing.assert_allclose(a, b, rtol=2 ** -10, atol=1e-6)
    # untouched cache positions stay zero
    assert np.all(outs[0][1][:, :, :p0] == 0) and np.all(outs[0][1][:, :, p0 + L:] == 0)


@pytest.mark.parametrize("dtype", [SM_F16, SM_F32])
def test_attn_prefill_lse(dev, dtype):
    """sm_attn_prefill_lse: log-sum-exp of the scaled, masked scores, [S*H, L]
    (fused_attention.rs:166-172), next to the same output as sm_attn_prefill."""
    S, L, p0, H, KVH, hd = 2, 70, 5, 8, 2, 64
    rng = np.random.default_rng(11)
    cap = p0 + L
    q, k, v = (rng.normal(0, 1, sh).astype(np.float32)
               for sh in ((S, L, H, hd), (S, KVH, cap, hd), (S, KVH, cap, hd)))
    if dtype == SM_F16:
        q, k, v = (a.astype(np.float16).astype(np.float32) for a in (q, k, v))
        qd, kd, vd = (_f16(a, dev) for a in (q, k, v))
        out = torch.empty(S * L, 2 * H * hd, dtype=torch.float16, device=dev)
        od = SM_F16X2
    else:
        qd, kd, vd = (torch.from_numpy(a).to(dev) for a in (q, k, v))
        out = torch.empty(S, L, H, hd, device=dev)
        od = SM_F32
    pos0 = torch.full((S,), p0, dtype=torch.int32, device=dev)
    lse = torch.empty(S * H, L, device=dev)
    call("sm_attn_prefill_lse", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), pos0.data_ptr(),
         out.data_ptr(), lse.data_ptr(), dtype, od, S, L, H, KVH, cap, hd, _s())
    got = lse.cpu().numpy().reshape(S, H, L)
    for s in range(S):
        for h in range(H):
            kv = h // (H // KVH)
            sc = q[s, :, h].astype(np.float64) @ k[s, kv].T.astype(np.float64) / np.sqrt(hd)
            sc[np.arange(cap)[None, :] > (p0 + np.arange(L))[:, None]] = -np.inf
            m = sc.max(1)
            ref = m + np.log(np.exp(sc - m[:, None]).sum(1))
            np.testing.assert_allclose(got[s, h], ref, rtol=1e-5, atol=1e-5)
