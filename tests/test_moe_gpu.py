"""Top-2 MoE on the GPU (router, route plan, grouped Q4 matmuls, combine, and a
quantized MoE decoder end to end) vs numpy and the CPU oracle.

Mirrors the reference's MoE tests: top-2 == general CPU top-k
(moe_topk.rs:143), the route plan is stable and invertible (moe_route.rs:200),
dispatch / combine == the tensor expression (moe_dispatch.rs:660) and grouped
forward == per-expert matmuls (grouped_linear.rs:919).
"""
import numpy as np
import pytest
import torch

import oracle
from summa_amd import _lib, ops
from summa_amd.model import Model, ModelConfig
from test_model_gpu import _gumbel

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------- router ---

@pytest.mark.parametrize("T,d,E", [(1, 128, 2), (37, 256, 8), (256, 2048, 32), (300, 512, 64)])
@pytest.mark.parametrize("hdt", ["f32", "f16"])
def test_top2_matches_cpu_topk(dev, T, d, E, hdt):
    print(f"case router T={T} d={d} E={E} h={hdt}", flush=True)
    rng = np.random.default_rng(T + E)
    h = rng.normal(0, 1, (T, d)).astype(np.float32)
    if hdt == "f16":
        h = h.astype(np.float16)
    wr = rng.normal(0, 1 / np.sqrt(d), (E, d)).astype(np.float32)
    hd = torch.from_numpy(h).to(dev)
    idx, wts, logits = ops.moe_top2_indices(hd, torch.from_numpy(wr).to(dev), want_logits=True)
    idx, wts, logits = idx.cpu().numpy(), wts.cpu().numpy(), logits.cpu().numpy()
    ref = h.astype(np.float64) @ wr.T.astype(np.float64)
    bound = np.abs(h.astype(np.float64)) @ np.abs(wr.T.astype(np.float64))
    assert np.all(np.abs(logits - ref) <= 2e-6 * bound + 1e-7)
    # the kernel's own logits decide: strict '>' scan == stable descending argsort
    top = np.argsort(-logits, axis=1, kind="stable")[:, :2]
    np.testing.assert_array_equal(idx, top)
    l0 = np.take_along_axis(logits, top[:, :1], 1)[:, 0].astype(np.float64)
    l1 = np.take_along_axis(logits, top[:, 1:], 1)[:, 0].astype(np.float64)
    w1 = np.exp(l1 - l0) / (1 + np.exp(l1 - l0))
    np.testing.assert_allclose(wts[:, 1], w1, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(wts[:, 0], 1 - w1, rtol=1e-6, atol=1e-7)
    # against the f64 logits wherever the top-2 set is not a near-tie
    srt = np.sort(ref, 1)[:, ::-1]
    clear = (srt[:, 0] - srt[:, 1] > 1e-4) & (srt[:, 1] - srt[:, 2] > 1e-4) if E > 2 else \
        srt[:, 0] - srt[:, 1] > 1e-4
    np.testing.assert_array_equal(idx[clear], np.argsort(-ref, 1, kind="stable")[clear, :2])


def test_top2_ties_keep_first_index(dev):
    d, E, T = 256, 8, 64
    rng = np.random.default_rng(5)
    r = rng.normal(0, 0.1, d).astype(np.float32)
    # e0 = 3z, e2 = e5 = z, the rest -z: exact ties broken toward the lower index
    wr = np.stack([3 * r, -r, r, -r, -r, r, -r, -r]).astype(np.float32)
    h = rng.normal(0, 1, (T, d)).astype(np.float32)
    idx, wts, _ = ops.moe_top2_indices(torch.from_numpy(h).to(dev), torch.from_numpy(wr).to(dev))
    idx = idx.cpu().numpy()
    z = h.astype(np.float64) @ r.astype(np.float64)
    pos, neg = z > 1e-3, z < -1e-3
    assert pos.any() and neg.any()
    np.testing.assert_array_equal(idx[pos], np.tile([0, 2], (pos.sum(), 1)))
    np.testing.assert_array_equal(idx[neg], np.tile([1, 3], (neg.sum(), 1)))
    np.testing.assert_allclose(wts.cpu().numpy()[neg], 0.5, rtol=0, atol=0)


# ------------------------------------------------------------ route plan ---

def _expected_tiles(counts, rows):
    out = []
    for e, c in enumerate(counts):
        out += [(e, r) for r in range(0, int(c), rows)]
    return out


@pytest.mark.parametrize("T,k,E,used", [(1, 2, 2, 2), (7, 2, 8, 3), (128, 2, 32, 32),
                                        (4096, 2, 32, 20), (8192, 2, 64, 64), (1000, 1, 16, 16),
                                        (0, 2, 8, 8), (512, 2, 64, 40), (300, 2, 64, 64),
                                        (513, 2, 32, 32)])
def test_route_plan_is_stable_and_invertible(dev, T, k, E, used):
    """Up to 1024 routes the one-thread-per-route ballot kernel runs, above it
    the counting-sort kernel; both must give numpy's stable argsort."""
    print(f"case plan T={T} k={k} E={E}", flush=True)
    rng = np.random.default_rng(T + E)
    experts_used = rng.choice(E, used, replace=False)
    idx = experts_used[rng.integers(0, used, (T, k))].astype(np.int32)
    plan = ops.moe_route_plan(torch.from_numpy(idx).to(dev), E)
    R = T * k
    flat = idx.ravel()
    counts = np.bincount(flat, minlength=E)
    order = np.argsort(flat, kind="stable")
    np.testing.assert_array_equal(plan.counts.cpu().numpy(), counts)
    np.testing.assert_array_equal(plan.offsets.cpu().numpy(), np.concatenate([[0], np.cumsum(counts)]))
    if R:
        np.testing.assert_array_equal(plan.order.cpu().numpy(), order)
        inv = plan.inverse.cpu().numpy()
        np.testing.assert_array_equal(inv[order], np.arange(R))
        np.testing.assert_array_equal(plan.src_rows.cpu().numpy(), order // k)
    assert int(plan.error.item()) == 0
    # device tile lists (16- and 128-row tiles per non-empty expert)
    w = plan.words.cpu().numpy()
    o = 2 * E + 1 + 3 * R
    m16 = (R + 15) // 16 + E
    n16 = int(w[o])
    t16 = [tuple(x) for x in w[o + 1:o + 1 + 2 * n16].reshape(-1, 2)]
    assert t16 == _expected_tiles(counts, 16)
    o2 = o + 1 + 2 * m16
    n128 = int(w[o2])
    t128 = [tuple(x) for x in w[o2 + 1:o2 + 1 + 2 * n128].reshape(-1, 2)]
    assert t128 == _expected_tiles(counts, 128)


def test_route_plan_flags_bad_expert_index(dev):
    idx = torch.tensor([[0, 1], [2, 8]], dtype=torch.int32, device=dev)
    plan = ops.moe_route_plan(idx, 8)
    assert int(plan.error.item()) == 1
    with pytest.raises(_lib.SummaError, match="experts must be <= 64"):
        ops.moe_route_plan(idx, 65)


# --------------------------------------------------------- grouped matmul ---

def _bank(E, n, k, seed, dev):
    w = np.random.default_rng(seed).normal(0, 0.02, (E, n, k)).astype(np.float32)
    dense, qs = [], []
    for e in range(E):
        codes, scales = oracle.q4_quantize(w[e])
        dense.append(oracle.q4_decode(codes, scales, n * k).reshape(n, k).astype(np.float64))
        qs.append(ops.Q4Weight.from_host(codes, scales, n, k, dev))
    return ops.ExpertBank(qs), dense


@pytest.mark.parametrize("T,E,used,n,k", [(128, 8, 8, 512, 512), (5, 16, 3, 256, 384),
                                          (2500, 8, 8, 256, 256), (3000, 4, 2, 384, 128)])
@pytest.mark.parametrize("mode", ["swiglu_gather", "store", "pair_swiglu_gather", "pair_store"])
def test_grouped_matmul_matches_per_expert(dev, T, E, used, n, k, mode):
    """Routes <= 4096 run the small-M kernel (16-row tiles), more the batch
    kernel over the plan's 128-row tiles."""
    print(f"case grouped T={T} E={E} n={n} k={k} {mode}", flush=True)
    rng = np.random.default_rng(T * E + n)
    bank, dense = _bank(E, n, k, T + k, dev)
    idx = rng.choice(E, used, replace=False)[rng.integers(0, used, (T, 2))].astype(np.int32)
    plan = ops.moe_route_plan(torch.from_numpy(idx).to(dev), E)
    R = 2 * T
    order = np.argsort(idx.ravel(), kind="stable")
    exp_of = idx.ravel()[order]
    if mode == "swiglu_gather":
        x = rng.normal(0, 1, (T, k)).astype(np.float16)
        rows = x[order // 2].astype(np.float64)
        y = ops.grouped_q4_matmul(bank, torch.from_numpy(x).to(dev), plan, gather=True,
                                  epilogue=_lib.SM_EPI_SWIGLU_F16).float().cpu().numpy()
    elif mode.startswith("pair"):
        gather = mode == "pair_swiglu_gather"
        x = torch.from_numpy(rng.normal(0, 1, (T if gather else R, k)).astype(np.float32)).to(dev)
        xp = ops.f16_pair(x)
        exact = ops.unpair(xp).cpu().numpy().astype(np.float64)
        rows = exact[order // 2] if gather else exact
        if gather:
            y = ops.unpair(ops.grouped_q4_matmul(bank, xp, plan, gather=True, pair=True,
                                                 epilogue=_lib.SM_EPI_SWIGLU_F16X2)).cpu().numpy()
        else:
            y = ops.grouped_q4_matmul(bank, xp, plan, gather=False, pair=True).cpu().numpy()
    else:
        x = rng.normal(0, 1, (R, k)).astype(np.float16)
        rows = x.astype(np.float64)
        y = ops.grouped_q4_matmul(bank, torch.from_numpy(x).to(dev), plan,
                                  gather=False).cpu().numpy()
    ref = np.empty((R, n))
    bound = np.empty((R, n))
    for e in range(E):
        sel = exp_of == e
        ref[sel] = rows[sel] @ dense[e].T
        bound[sel] = np.abs(rows[sel]) @ np.abs(dense[e]).T
    if mode == "swiglu_gather":
        F = n // 2
        g, v = ref[:, :F], ref[:, F:]
        np.testing.assert_allclose(y, g / (1 + np.exp(-g)) * v, rtol=2 ** -10, atol=1e-5)
    elif mode == "pair_swiglu_gather":
        F = n // 2
        g, v = ref[:, :F], ref[:, F:]
        np.testing.assert_allclose(y, g / (1 + np.exp(-g)) * v, rtol=1e-5, atol=2e-6)
    else:
        assert np.all(np.abs(y - ref) <= 2e-6 * bound + 1e-7), float(np.abs(y - ref).max())


def test_grouped_matmul_rejects_bad_shapes(dev):
    bank, _ = _bank(2, 64, 128, 0, dev)
    plan = ops.moe_route_plan(torch.zeros((4, 2), dtype=torch.int32, device=dev), 2)
    x = torch.zeros((4, 128), dtype=torch.float16, device=dev)
    with pytest.raises(_lib.SummaError, match="epilogue"):
        ops.grouped_q4_matmul(bank, x, plan, gather=True, epilogue=_lib.SM_EPI_ADD_F32)
    with pytest.raises(ValueError, match="input width"):
        ops.grouped_q4_matmul(bank, x[:, :64].contiguous(), plan, gather=True)


# ---------------------------------------------------------------- combine ---

@pytest.mark.parametrize("T,E,d", [(1, 2, 64), (128, 32, 2048), (3000, 8, 512)])
def test_combine_matches_tensor_expression(dev, T, E, d):
    rng = np.random.default_rng(T + d)
    idx = rng.integers(0, E, (T, 2)).astype(np.int32)
    plan = ops.moe_route_plan(torch.from_numpy(idx).to(dev), E)
    routed = rng.normal(0, 1, (2 * T, d)).astype(np.float32)
    w = rng.uniform(0, 1, (T, 2)).astype(np.float32)
    x0 = rng.normal(0, 1, (T, d)).astype(np.float32)
    x = ops.moe_route_combine(torch.from_numpy(routed).to(dev), torch.from_numpy(w).to(dev), plan,
                              torch.from_numpy(x0).to(dev)).cpu().numpy()
    inv = np.empty(2 * T, np.int64)
    inv[np.argsort(idx.ravel(), kind="stable")] = np.arange(2 * T)
    r = routed.astype(np.float64)[inv].reshape(T, 2, d)
    ref = x0 + (r * w[:, :, None]).sum(1)
    np.testing.assert_allclose(x, ref, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("T,E,d", [(128, 32, 2048), (33, 8, 768), (5, 4, 4096), (7, 4, 320)])
def test_combine_rmsnorm_equals_two_steps(dev, T, E, d):
    """sm_moe_combine_rmsnorm (the combine and the next RMSNorm in one launch)
    gives sm_moe_combine + sm_rmsnorm's bits for x and for the f16-pair rows,
    for the widths it fuses and for one it hands to the two steps (320)."""
    from summa_amd._lib import SM_F16X2, call
    print(f"case combine+rmsnorm T={T} E={E} d={d}", flush=True)
    st = torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(T * d + E)
    idx = torch.from_numpy(rng.integers(0, E, (T, 2)).astype(np.int32)).to(dev)
    plan = ops.moe_route_plan(idx, E)
    routed = torch.from_numpy(rng.normal(0, 1, (2 * T, d)).astype(np.float32)).to(dev)
    w = torch.from_numpy(rng.uniform(0, 1, (T, 2)).astype(np.float32)).to(dev)
    x0 = rng.normal(0, 1, (T, d)).astype(np.float32)
    gamma = torch.from_numpy(rng.uniform(0.5, 1.5, d).astype(np.float32)).to(dev)
    x1, x2 = torch.from_numpy(x0.copy()).to(dev), torch.from_numpy(x0.copy()).to(dev)
    h1 = torch.empty((T, 2 * d), dtype=torch.float16, device=dev)
    h2 = torch.empty_like(h1)
    call("sm_moe_combine_rmsnorm", routed.data_ptr(), w.data_ptr(), plan.words.data_ptr(), T, 2,
         E, d, x1.data_ptr(), gamma.data_ptr(), 1e-5, h1.data_ptr(), st)
    ops.moe_route_combine(routed, w, plan, x2)
    call("sm_rmsnorm", x2.data_ptr(), gamma.data_ptr(), T, d, 1e-5, h2.data_ptr(), SM_F16X2, st)
    torch.testing.assert_close(x1, x2, rtol=0, atol=0)
    torch.testing.assert_close(h1, h2, rtol=0, atol=0)


# ------------------------------------------------------------ end to end ---

def _first_bad(lp, lp_ref, tol):
    bad = np.abs(lp - lp_ref) > tol
    return np.where(bad.any(1), bad.argmax(1), lp.shape[1])


def test_moe_decoder_matches_oracle(dev):
    """Quantized top-2 MoE decoder: rollout tokens and per-token log-probs vs the
    oracle (2e-3). A sequence may leave the comparison only at a near-tie: a
    sampled-token near-tie (as in the dense tests) or a router near-tie (top-2
    set decided by < 1e-3 in some layer at an earlier or the same position)."""
    mc = ModelConfig(layers=2, d_model=512, heads=4, kv_heads=2, head_dim=128, ffn=256,
                     vocab=4096, max_seq=64, quantized=True, experts=8, expert_ffn=256)
    cfg = mc.oracle_cfg()
    w = oracle.random_weights(cfg, seed=21, std=0.02)
    host = oracle.HostModel(cfg, w, quantized=True)
    m = Model(mc)
    m.load_host_weights(w, dev)
    S, P, N = 8, 20, 8
    prompts = np.random.default_rng(22).integers(0, cfg["V"], (S, P)).astype(np.int32)
    pd = torch.from_numpy(prompts).to(dev)
    tok, lp_beh = m.generate(pd, N, temperature=1.0, seed=5)
    lp_cur = m.logprobs(pd, tok).cpu().numpy()
    tok_np = tok.cpu().numpy()
    lp_or = host.logprobs(prompts, tok_np)
    gaps = host.router_gaps(np.concatenate([prompts, tok_np], 1))  # [layers, S, P+N]
    tie_pos = np.where((gaps < 1e-3).any(0).any(1), (gaps < 1e-3).any(0).argmax(1), P + N)
    tie_tok = np.maximum(tie_pos - (P - 1), 0)  # first generated token a tie can touch
    excused = set()
    for name, lp in (("logprobs", lp_cur), ("behavior", lp_beh.cpu().numpy())):
        first = _first_bad(lp, lp_or, 2e-3)
        for s in range(S):
            if first[s] < N:
                assert tie_tok[s] <= first[s], f"{name} seq {s} token {first[s]}: no router near-tie"
                excused.add(s)
    # rollout tokens: identical to the oracle's own sampling until a near-tie
    tok_or, _ = host.generate(prompts, N, 1.0, 5)
    for s in range(S):
        diff = np.nonzero(tok_np[s] != tok_or[s])[0]
        if diff.size and diff[0] < tie_tok[s]:
            n = int(diff[0])
            ids = np.concatenate([prompts[s], tok_np[s, :n]])[None]
            logits = host.forward_logits(ids)[0, P - 1 + n].astype(np.float64)
            key = logits + _gumbel(5, s, n, cfg["V"])
            a, b = int(tok_np[s, n]), int(tok_or[s, n])
            assert abs(key[a] - key[b]) < 4e-3, f"seq {s} step {n}: not a near-tie"
    print(f"sequences excused by a router near-tie: {len(excused)}, min gap {gaps.min():.2e}",
          flush=True)
    assert len(excused) <= S // 2


# --------------------------------------------- fused decode-step routing ---

@pytest.mark.parametrize("T,E", [(1, 2), (128, 32), (512, 64), (700, 32), (4096, 8)])
def test_route_plan_from_logits_equals_two_steps(dev, T, E):
    """sm_moe_route_plan_logits (the top-2 of router logits and the route plan
    in one launch for up to 512 tokens, a top-2 kernel then the plan kernel
    above) equals sm_moe_router_top2's top-2 of the same logits and
    sm_moe_route_plan of those indices, bit for bit."""
    print(f"case plan from logits T={T} E={E}", flush=True)
    rng = np.random.default_rng(T * 3 + E)
    d = 256
    h = torch.from_numpy(rng.normal(0, 1, (T, d)).astype(np.float32)).to(dev)
    wr = torch.from_numpy(rng.normal(0, 1 / np.sqrt(d), (E, d)).astype(np.float32)).to(dev)
    if T >= 4:  # exact ties: identical router rows
        wr[E // 2] = wr[0]
    idx0, w0, logits = ops.moe_top2_indices(h, wr, want_logits=True)
    plan0 = ops.moe_route_plan(idx0, E)
    idx1, w1, plan1 = ops.moe_route_plan_logits(logits)
    torch.cuda.synchronize()
    assert torch.equal(idx0, idx1)
    assert torch.equal(w0, w1)
    assert _plan_content(plan0) == _plan_content(plan1)
    assert int(plan1.error.cpu()[0]) == 0


def _plan_content(plan):
    """The defined words of a route plan: counts, offsets, order, inverse,
    src_rows and both tile lists up to their lengths (the unused tail of a
    tile list is never written)."""
    R, E = plan.tokens * plan.top_k, plan.experts
    w = plan.words.cpu().numpy()
    at = 2 * E + 1 + 3 * R
    out = [w[:at].tolist()]
    for rows in (16, 128):
        cap = -(-R // rows) + E
        n = int(w[at])
        out.append(w[at + 1:at + 1 + 2 * n].tolist())
        at += 1 + 2 * cap
    return out


@pytest.mark.parametrize("m,n,k,E", [(128, 2048, 2048, 32), (64, 1024, 2048, 8),
                                     (200, 2048, 5632, 64), (600, 2048, 2048, 32)])
def test_add_rmsnorm_router_equals_separate_router(dev, m, n, k, E):
    """sm_q4_matmul_add_rmsnorm_router (config[4]'s decode FFN norm with the
    router and its top-2 in the same launch) against sm_q4_matmul_add_rmsnorm
    followed by sm_moe_router_top2 on its output: residual and normed rows
    bit-identical; logits within f32 summation order of each other and of f64
    over the pair values; the top-2 equal to the strict first-index scan of the
    fused logits (the same scan over the separate router's logits wherever the
    top-2 set is not a near-tie); a prefill-size M (600) falls back to the
    separate router kernel and matches it exactly. Exact ties (two identical
    router rows) keep the lower index."""
    print(f"case add+rmsnorm+router m={m} n={n} k={k} E={E}", flush=True)
    st = torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(m + n + E)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    codes, scales = oracle.q4_quantize(w)
    qw = ops.Q4Weight.from_host(codes, scales, n, k, dev)
    xd = ops.f16_pair(torch.from_numpy(rng.normal(0, 1, (m, k)).astype(np.float32)).to(dev))
    base = rng.normal(0, 1, (m, n)).astype(np.float32)
    gamma = torch.from_numpy(rng.uniform(0.5, 1.5, n).astype(np.float32)).to(dev)
    wr_h = rng.normal(0, 1 / np.sqrt(n), (E, n)).astype(np.float32)
    wr_h[E - 1] = wr_h[1]  # an exact tie between experts 1 and E - 1
    wr = torch.from_numpy(wr_h).to(dev)
    ws = ops.q4_workspace(m, n, k, _lib.SM_EPI_ADD_F32, dev)
    eps = 1e-5

    def run(router):
        r = torch.from_numpy(base.copy()).to(dev)
        h = torch.empty((m, 2 * n), dtype=torch.float16, device=dev)
        if router:
            lg = torch.full((m, E), float("nan"), dtype=torch.float32, device=dev)
            idx = torch.full((m, 2), -7, dtype=torch.int32, device=dev)
            wts = torch.full((m, 2), float("nan"), dtype=torch.float32, device=dev)
            _lib.call("sm_q4_matmul_add_rmsnorm_router", qw.tcodes.data_ptr(),
                      qw.tscales.data_ptr(), n, k, xd.data_ptr(), _lib.SM_F16X2, m, 2 * k,
                      r.data_ptr(), gamma.data_ptr(), eps, h.data_ptr(), wr.data_ptr(), E,
                      lg.data_ptr(), idx.data_ptr(), wts.data_ptr(), ws.data_ptr(), ws.numel(),
                      st)
        else:
            _lib.call("sm_q4_matmul_add_rmsnorm", qw.tcodes.data_ptr(), qw.tscales.data_ptr(), n,
                      k, xd.data_ptr(), _lib.SM_F16X2, m, 2 * k, r.data_ptr(), gamma.data_ptr(),
                      eps, h.data_ptr(), ws.data_ptr(), ws.numel(), st)
            idx, wts, lg = ops.moe_top2_indices(h, wr, want_logits=True, pair=True)
        torch.cuda.synchronize()
        return r, h, lg, idx, wts

    r1, h1, l1, i1, w1 = run(True)
    r0, h0, l0, i0, w0 = run(False)
    assert torch.equal(r1, r0) and torch.equal(h1, h0)
    assert torch.isfinite(l1).all()
    hv = ops.unpair(h1).double().cpu().numpy()
    ref = hv @ wr.double().cpu().numpy().T
    bound = np.abs(hv) @ np.abs(wr.double().cpu().numpy().T)
    for got in (l1, l0):
        assert np.all(np.abs(got.cpu().numpy() - ref) <= 2e-6 * bound + 1e-7)
    lg = l1.cpu().numpy()
    top = np.argsort(-lg, axis=1, kind="stable")[:, :2]  # == the strict '>' first-index scan
    np.testing.assert_array_equal(i1.cpu().numpy(), top)
    v0 = np.take_along_axis(lg, top[:, :1], 1)[:, 0].astype(np.float64)
    v1 = np.take_along_axis(lg, top[:, 1:], 1)[:, 0].astype(np.float64)
    e1 = np.exp(v1 - v0)
    np.testing.assert_allclose(w1.cpu().numpy()[:, 1], e1 / (1 + e1), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(w1.cpu().numpy()[:, 0], 1 / (1 + e1), rtol=1e-6, atol=1e-7)
    # expert E - 1 ties with expert 1: it can only be the second choice, after 1
    ii = i1.cpu().numpy()
    has = (ii == E - 1).any(1)
    assert np.all(ii[has, 0] == 1) and np.all(ii[has, 1] == E - 1)
    srt = np.sort(ref, 1)[:, ::-1]
    clear = (srt[:, 1] - srt[:, 2] > 1e-4) & (srt[:, 0] - srt[:, 1] > 1e-4)
    np.testing.assert_array_equal(i1.cpu().numpy()[clear], i0.cpu().numpy()[clear])
    if m > 512:  # the two-step fallback runs the router kernel itself
        assert torch.equal(l1, l0) and torch.equal(i1, i0) and torch.equal(w1, w0)
