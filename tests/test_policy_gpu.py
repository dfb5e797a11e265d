"""The library's trainable policy (sm_policy_*): prepare_device_batch's
recompute + GRPO loss + staged backward in one C call and optimizer_step in
another (posttrain.rs:1288-1305), checked against float64 autograd of an
independent torch restatement of the decoder, against torch.optim.AdamW, the
global-norm clip of gradient_norm_and_clip (main.rs:667-694), the Python
composition of Muon, and end to end (a GRPO update lowers the loss; a
quantized policy's recompute equals the quantized rollout model's)."""
import numpy as np
import pytest
import torch

import oracle
from summa_amd import _lib, train
from summa_amd.model import Model, ModelConfig, rl_prepare

from _workloads import build_models
from summa_amd.configs import RL_WORKLOADS
from test_train_gpu import CFG, _attn_t, _rope_t, _torch_lp

pytestmark = pytest.mark.gpu


def _batch(cfg, seed, dev, B=2, G=4, P=8, N=6):
    rng = np.random.default_rng(seed)
    prompts = torch.from_numpy(rng.integers(0, cfg.vocab, (B * G, P)).astype(np.int32)).to(dev)
    tokens = torch.from_numpy(rng.integers(0, cfg.vocab, (B * G, N)).astype(np.int32)).to(dev)
    rewards = torch.from_numpy(rng.random((B, G)).astype(np.float32)).to(dev)
    return prompts, tokens, rewards


def test_native_policy_gradient_matches_autograd(dev):
    w = oracle.random_weights(CFG.oracle_cfg(), seed=11, std=0.05)
    pol = train.Policy(CFG, w, dev)
    prompts, tokens, rewards = _batch(CFG, 2, dev)
    beh = torch.full(tokens.shape, -7.0, device=dev)  # off-policy rollouts: rho != 1
    out = pol.prepare(None, prompts, tokens, beh, rewards, kl_coefficient=0.0)
    assert int(out["flags"].abs().sum()) == 0
    lp = out["lp_cur"].cpu()
    dlp = out["dlp"].cpu().double()
    wt = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)).requires_grad_(True)
          for k, v in w.items()}
    lp_t = _torch_lp(wt, CFG, prompts.cpu(), tokens.cpu())
    np.testing.assert_allclose(lp.numpy(), lp_t.detach().numpy(), atol=2e-5)
    # the GRPO loss and dlp are the oracle's on these log-probs
    st_or, _, dlp_or, err = oracle.grpo_loss(rewards.cpu().numpy(),
                                             lp.numpy().reshape(2, 4, 6),
                                             beh.cpu().numpy().reshape(2, 4, 6), None, None,
                                             0.2, 1e-6, 0.0)
    assert err == 0
    np.testing.assert_allclose(dlp.numpy(), dlp_or.reshape(8, 6), rtol=1e-4, atol=1e-9)
    (dlp * lp_t).sum().backward()
    for k, t in wt.items():
        layers = range(CFG.layers) if k in train.LAYER_KEYS else [-1]
        for layer in layers:
            got = pol.tensor(k, layer, gradient=True).cpu().double()
            want = t.grad[layer] if layer >= 0 else t.grad
            scale = want.abs().max().item() + 1e-12
            assert (got - want).abs().max().item() / scale < 2e-4, (k, layer)
    # a second prepare adds the same gradient again (staged accumulation)
    g1 = pol.tensor("qkv", 1, gradient=True)
    pol.prepare(None, prompts, tokens, beh, rewards, kl_coefficient=0.0)
    torch.testing.assert_close(pol.tensor("qkv", 1, gradient=True), 2 * g1, rtol=1e-5, atol=1e-7)


# (max |lp - f64|, max relative gradient error) per GEMM plane count: f32-grade
# for three planes (measured 1.0e-5, 2.2e-6); 16-bit operands for two
# (5.8e-5, 2.1e-5); bf16 operands in the matmuls and in attention, the
# reference's CUDA-path precision, for one (3.6e-2, 1.4e-2; 2.9e-2, 1.2e-2
# with f32 attention: this policy's weights are N(0, 0.05), its logits a few
# units). Every gradient also keeps its direction (cosine >= 0.9999; measured
# 0.99994 at one plane).
PLANE_BOUNDS = {3: (2e-5, 2e-4), 2: (2e-4, 1e-4), 1: (6e-2, 3e-2)}


@pytest.mark.parametrize("planes", [3, 2, 1])
def test_native_policy_gradient_on_matrix_cores(dev, planes):
    """A policy large enough that every linear's forward, data-gradient and
    weight-gradient GEMM crosses sm_gemm_ex's matrix-core threshold (2^27
    multiply-adds, 128 x 128 x 16 outputs) and attention spans several 32 x 32
    backward tiles (127 positions): the staged gradient against float64
    autograd, as for the small policy, with the GEMMs on 3, 2 or 1 bf16 planes
    (PLANE_BOUNDS)."""
    print(f"case matrix-core policy planes={planes}", flush=True)
    cfg = ModelConfig(layers=1, d_model=512, heads=4, kv_heads=2, head_dim=128, ffn=1024,
                      vocab=2048, max_seq=160, quantized=False)
    w = oracle.random_weights(cfg.oracle_cfg(), seed=21, std=0.05)
    pol = train.Policy(cfg, w, dev, matmul_planes=planes)
    lp_bound, grad_bound = PLANE_BOUNDS[planes]
    prompts, tokens, rewards = _batch(cfg, 5, dev, P=64, N=64)
    beh = torch.full(tokens.shape, -9.0, device=dev)
    out = pol.prepare(None, prompts, tokens, beh, rewards, kl_coefficient=0.0)
    assert int(out["flags"].abs().sum()) == 0
    wt = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)).requires_grad_(True)
          for k, v in w.items()}
    lp_t = _torch_lp(wt, cfg, prompts.cpu(), tokens.cpu())
    lp_err = float((out["lp_cur"].cpu().double() - lp_t.detach()).abs().max())
    print(f"matrix-core policy: max |lp - f64| {lp_err:.2e}", flush=True)
    assert lp_err < lp_bound
    (out["dlp"].cpu().double() * lp_t).sum().backward()
    for k, t in wt.items():
        layers = range(cfg.layers) if k in train.LAYER_KEYS else [-1]
        for layer in layers:
            got = pol.tensor(k, layer, gradient=True).cpu().double()
            want = t.grad[layer] if layer >= 0 else t.grad
            err = (got - want).abs().max().item() / (want.abs().max().item() + 1e-12)
            cos = float((got * want).sum() / (got.norm() * want.norm() + 1e-300))
            print(f"  {k}[{layer}] relative gradient error {err:.2e}, cosine {cos:.6f}",
                  flush=True)
            assert err < grad_bound, (k, layer)
            assert cos >= 0.9999, (k, layer)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("cfg_id", [2, 4])
def test_policy_at_full_geometry_against_oracle(dev, cfg_id):
    """The trainable policy at config[2]'s full geometry (24 layers, d 2048,
    16 / 4 heads, F 5632, V 65536: 1.35 G f32 masters, fake-quantized Q4G128
    forward) and at config[4]'s (16 MoE layers of 32 experts, top-2, f32
    routers) on a small batch rolled out by the installed Q4 model: its
    recompute (f32 activations, matrix-core GEMMs at these shapes, tiled
    attention) against the CPU oracle's quantized model with q, k and v kept
    in f32 as the policy keeps them (an f32 computation: 5e-5 after 24
    layers; measured 1e-5), then one optimizer step (finite norm) after which the installed
    model's log-probs move."""
    wl = RL_WORKLOADS[cfg_id]
    mc, (model,), host_w = build_models(wl, dev, seed=3, count=1)
    print(f"case policy at config[{cfg_id}] geometry: layers={mc.layers} d={mc.d_model} "
          f"experts={mc.experts}", flush=True)
    pol = train.Policy(mc, host_w, dev)
    G, P, N = 4, 24, 8
    gen = torch.Generator().manual_seed(11)
    prompts = torch.randint(0, mc.vocab, (G, P), generator=gen, dtype=torch.int32).to(dev)
    tok, beh = model.generate(prompts, N, temperature=1.0, seed=5)
    rewards = torch.rand(1, G, generator=gen).to(dev)
    out = pol.prepare(None, prompts, tok, beh, rewards, kl_coefficient=0.0)
    assert int(out["flags"].abs().sum()) == 0
    host = oracle.HostModel(mc.oracle_cfg(), host_w, quantized=True, kv_f32=True)
    del host_w
    lp_or, _ = host.continuation(prompts.cpu().numpy(), tok.cpu().numpy())
    lp = out["lp_cur"].cpu().numpy()
    err = float(np.abs(lp - lp_or).max())
    gap = float((out["lp_cur"] - beh).abs().max())
    print(f"policy recompute vs oracle (f32 q/k/v) {err:.2e}; vs the Q4 rollout (f16 KV "
          f"cache) {gap:.2e}", flush=True)
    assert err <= 5e-5
    norm = pol.optimizer_step(1.0)
    assert np.isfinite(norm) and norm > 0
    before = model.logprobs(prompts, tok)
    pol.install(model)
    assert float((model.logprobs(prompts, tok) - before).abs().max()) > 0


MOE_CFG = ModelConfig(layers=2, d_model=256, heads=4, kv_heads=2, head_dim=64, ffn=512,
                      vocab=1000, max_seq=32, quantized=False, experts=4, expert_ffn=128)


def _torch_lp_moe(w, cfg, prompts, tokens):
    """Independent float64 restatement of an MoE decoder's recompute: f64
    router, the top two experts by logit (the first index on equal logits),
    weights softmax over the pair, SwiGLU experts, weighted sum
    (SparseMoe::forward, ffn.rs:478-711). Also returns, per layer, the gap
    between each token's second and third largest router logits."""
    S, P = prompts.shape
    N = tokens.shape[1]
    L = P + N - 1
    H, KVH, hd, eps = cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.norm_eps
    E, Fe = cfg.experts, cfg.expert_ffn
    ids = torch.cat([prompts, tokens[:, :N - 1]], 1).long()
    rms = lambda x, g: x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * g  # noqa: E731
    half = hd // 2
    freq = float(cfg.rope_theta) ** (-2.0 * torch.arange(half, dtype=torch.float64) / hd)
    ang = torch.arange(L, dtype=torch.float64)[:, None] * freq[None, :]
    tab = torch.stack([torch.cos(ang), torch.sin(ang)], -1).float().double()
    pos = torch.arange(L)
    x = w["embed"][ids]
    gaps = []
    for i in range(cfg.layers):
        h = rms(x, w["attn_norm"][i])
        qkv = h @ w["qkv"][i].T
        q = _rope_t(qkv[..., :H * hd].reshape(S, L, H, hd), tab, pos)
        k = _rope_t(qkv[..., H * hd:(H + KVH) * hd].reshape(S, L, KVH, hd), tab, pos)
        v = qkv[..., (H + KVH) * hd:].reshape(S, L, KVH, hd)
        o, _ = _attn_t(q, k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3), H, KVH)
        x = x + o.reshape(S, L, H * hd) @ w["o"][i].T
        h2 = rms(x, w["ffn_norm"][i]).reshape(S * L, -1)
        logits = h2 @ w["router"][i].T
        srt = logits.detach().sort(-1, descending=True).values
        gaps.append(float((srt[:, 1] - srt[:, 2]).min()))
        i0 = logits.detach().argmax(-1)
        masked = logits.detach().clone()
        masked[torch.arange(S * L), i0] = -float("inf")
        i1 = masked.argmax(-1)
        pr = torch.softmax(torch.stack([logits.gather(1, i0[:, None])[:, 0],
                                        logits.gather(1, i1[:, None])[:, 0]], 1), -1)
        ys = []
        for e in range(E):
            u = h2 @ w["exp_in"][i][e].T
            ys.append((torch.nn.functional.silu(u[:, :Fe]) * u[:, Fe:]) @ w["exp_down"][i][e].T)
        ys = torch.stack(ys)  # [E, tokens, d]
        t = torch.arange(S * L)
        y = pr[:, :1] * ys[i0, t] + pr[:, 1:] * ys[i1, t]
        x = x + y.reshape(S, L, -1)
    hf = rms(x, w["final_norm"])[:, P - 1:P - 1 + N]
    logits = hf @ w["lm_head"].T
    return torch.log_softmax(logits, -1).gather(-1, tokens.long()[..., None])[..., 0], gaps


@pytest.mark.parametrize("planes", [3])
def test_moe_policy_gradient_matches_autograd(dev, planes):
    """An MoE policy (4 experts, top-2): the recompute and the staged gradient
    of every tensor (router and experts included) against float64 autograd of
    the independent MoE restatement, where every token's routing is
    unambiguous (second and third router logits apart by > 1e-4, checked), at
    the plane counts' bounds (PLANE_BOUNDS); then an optimizer step."""
    print(f"case moe policy planes={planes}", flush=True)
    cfg = MOE_CFG
    w = oracle.random_weights(cfg.oracle_cfg(), seed=31, std=0.05)
    pol = train.Policy(cfg, w, dev, matmul_planes=planes)
    prompts, tokens, rewards = _batch(cfg, 7, dev)
    beh = torch.full(tokens.shape, -7.0, device=dev)
    out = pol.prepare(None, prompts, tokens, beh, rewards, kl_coefficient=0.0)
    assert int(out["flags"].abs().sum()) == 0
    wt = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)).requires_grad_(True)
          for k, v in w.items()}
    lp_t, gaps = _torch_lp_moe(wt, cfg, prompts.cpu(), tokens.cpu())
    print(f"  routing gaps per layer {[f'{g:.2e}' for g in gaps]}", flush=True)
    assert min(gaps) > 1e-4
    lp_bound, grad_bound = PLANE_BOUNDS[planes]
    lp_err = float((out["lp_cur"].cpu().double() - lp_t.detach()).abs().max())
    print(f"  max |lp - f64| {lp_err:.2e}", flush=True)
    assert lp_err < lp_bound
    (out["dlp"].cpu().double() * lp_t).sum().backward()
    for k, t in wt.items():
        layers = range(cfg.layers) if k in train.LAYER_KEYS + train.MOE_LAYER_KEYS else [-1]
        for layer in layers:
            got = pol.tensor(k, layer, gradient=True).cpu().double()
            want = t.grad[layer] if layer >= 0 else t.grad
            err = (got - want).abs().max().item() / (want.abs().max().item() + 1e-12)
            cos = float((got * want).sum() / (got.norm() * want.norm() + 1e-300))
            print(f"  {k}[{layer}] relative gradient error {err:.2e}, cosine {cos:.6f}",
                  flush=True)
            assert err < grad_bound, (k, layer)
            assert cos >= 0.9999, (k, layer)
    before = pol.tensor("exp_in", 1).clone()
    norm = pol.optimizer_step(1.0)
    assert np.isfinite(norm) and norm > 0
    assert float((pol.tensor("exp_in", 1) - before).abs().max()) > 0


def test_native_optimizer_step_adamw_and_clip(dev):
    """AdamW on every tensor after the global-norm clip, against torch in f64
    fed with the policy's own staged gradients."""
    w = oracle.random_weights(CFG.oracle_cfg(), seed=13, std=0.05)
    clip = 1e-3  # well below the batch's gradient norm: the clip engages
    pol = train.Policy(CFG, w, dev, lr=1e-2, weight_decay=0.1, grad_clip=clip)
    prompts, tokens, rewards = _batch(CFG, 3, dev)
    beh = torch.full(tokens.shape, -7.0, device=dev)
    pol.prepare(None, prompts, tokens, beh, rewards, kl_coefficient=0.0)
    names = list(w)
    grads = {}
    for k in names:
        if k in train.LAYER_KEYS:
            grads[k] = torch.stack([pol.tensor(k, i, gradient=True) for i in range(CFG.layers)])
        else:
            grads[k] = pol.tensor(k, gradient=True)
    norm = float(torch.sqrt(sum((g.double() ** 2).sum() for g in grads.values())))
    got_norm = pol.optimizer_step(0.5)  # learning-rate scale 0.5
    assert abs(got_norm - norm) <= 1e-5 * norm
    assert norm > clip
    for k in names:
        tp = torch.tensor(np.asarray(w[k], dtype=np.float64), requires_grad=True)
        opt = torch.optim.AdamW([tp], lr=1e-2 * 0.5, betas=(0.9, 0.95), eps=1e-8,
                                weight_decay=0.1)
        tp.grad = grads[k].cpu().double() * (clip / norm)
        opt.step()
        if k in train.LAYER_KEYS:
            got = torch.stack([pol.tensor(k, i) for i in range(CFG.layers)])
        else:
            got = pol.tensor(k)
        np.testing.assert_allclose(got.cpu().numpy(), tp.detach().numpy(), rtol=1e-5, atol=1e-6)
        assert float(pol.tensor(k, 0 if k in train.LAYER_KEYS else -1,
                                gradient=True).abs().max()) == 0.0  # cleared


def test_native_muon_matches_python_composition(dev):
    w = oracle.random_weights(CFG.oracle_cfg(), seed=14, std=0.05)
    pol = train.Policy(CFG, w, dev, lr=1e-3, muon_lr=0.02, grad_clip=0.0)
    prompts, tokens, rewards = _batch(CFG, 4, dev)
    beh = torch.full(tokens.shape, -7.0, device=dev)
    pol.prepare(None, prompts, tokens, beh, rewards, kl_coefficient=0.0)
    ref = train.Fp32Policy(CFG, w, dev)
    grads = {k: torch.stack([pol.tensor(k, i, gradient=True) for i in range(CFG.layers)])
             for k in ref.muon_keys()}
    pol.optimizer_step(1.0)
    ref.muon_step(grads, ref.muon_keys(), lr=0.02)
    for k in ref.muon_keys():
        for i in range(CFG.layers):
            torch.testing.assert_close(pol.tensor(k, i), ref.p[k][i], rtol=1e-5, atol=1e-6)


def test_native_grpo_update_lowers_the_loss(dev):
    """Rollouts from the inference model, prepare (reference = the frozen
    initial model), an optimizer step, install: the same batch's GRPO loss
    drops and the model now holds the policy's weights."""
    w = oracle.random_weights(CFG.oracle_cfg(), seed=15, std=0.05)
    model, frozen = Model(CFG), Model(CFG)
    model.load_host_weights(w, dev)
    frozen.load_host_weights(w, dev)
    pol = train.Policy(CFG, w, dev)
    G, B = 8, 2
    prompts = torch.from_numpy(np.random.default_rng(4).integers(0, CFG.vocab, (B * G, 8))
                               .astype(np.int32)).to(dev)
    tok, beh = model.generate(prompts, 6, temperature=1.0, seed=9)
    rewards = torch.from_numpy(np.random.default_rng(5).random((B, G)).astype(np.float32)).to(dev)
    out0 = pol.prepare(frozen, prompts, tok, beh, rewards)
    l0 = float(out0["stats"][:, 0].sum())
    np.testing.assert_allclose(out0["lp_cur"].cpu().numpy(), beh.cpu().numpy(), atol=1e-5)
    pol.optimizer_step(1.0)
    pol.install(model)
    out1 = rl_prepare(model, frozen, prompts, tok, beh, rewards)
    l1 = float(out1["stats"][:, 0].sum())
    assert l1 < l0, (l0, l1)
    probe = pol.prepare(frozen, prompts, tok, beh, rewards)
    np.testing.assert_allclose(out1["lp_cur"].cpu().numpy(), probe["lp_cur"].cpu().numpy(),
                               atol=1e-5)


@pytest.mark.parametrize("planes", [3, 1])
def test_prepare_with_given_reference_lp_is_bit_exact(dev, planes):
    """sm_policy_prepare_with_ref (the frozen model's log-probs passed in, as
    grpo_loss_tensor takes reference_token_log_probs) against sm_policy_prepare
    with the frozen model, on two policies with the same weights: lp_cur, the
    group statistics, dlp, the flags and every staged gradient bit for bit,
    with a positive KL coefficient (the embedding gradient up to the order of its
    atomic adds); a positive KL coefficient without reference log-probs fails."""
    print(f"case prepare with given reference lp planes={planes}", flush=True)
    w = oracle.random_weights(CFG.oracle_cfg(), seed=31, std=0.05)
    frozen = Model(CFG)
    frozen.load_host_weights(oracle.random_weights(CFG.oracle_cfg(), seed=32, std=0.05), dev)
    pa = train.Policy(CFG, w, dev, matmul_planes=planes)
    pb = train.Policy(CFG, w, dev, matmul_planes=planes)
    G, B = 8, 2
    prompts = torch.from_numpy(np.random.default_rng(6).integers(0, CFG.vocab, (B * G, 8))
                               .astype(np.int32)).to(dev)
    tok = torch.from_numpy(np.random.default_rng(7).integers(0, CFG.vocab, (B * G, 6))
                           .astype(np.int32)).to(dev)
    beh = torch.full(tok.shape, -7.0, device=dev)
    rewards = torch.from_numpy(np.random.default_rng(8).random((B, G)).astype(np.float32)).to(dev)
    a = pa.prepare(frozen, prompts, tok, beh, rewards, kl_coefficient=0.04)
    b = pb.prepare(None, prompts, tok, beh, rewards, kl_coefficient=0.04,
                   reference_lp=a["lp_ref"].clone())
    for k in ("lp_cur", "stats", "dlp", "flags"):
        assert torch.equal(a[k], b[k]), k
    assert float(a["stats"][:, 3].abs().sum()) > 0  # the KL term took part
    for k in train.LAYER_KEYS:
        for layer in range(CFG.layers):
            assert torch.equal(pa.tensor(k, layer, gradient=True),
                               pb.tensor(k, layer, gradient=True)), (k, layer)
    for k in ("lm_head", "final_norm"):
        assert torch.equal(pa.tensor(k, gradient=True), pb.tensor(k, gradient=True)), k
    # the embedding gradient is a scatter of atomic f32 adds (sm_embed_backward):
    # repeated ids add in run-dependent order, so it is equal up to f32 rounding
    torch.testing.assert_close(pa.tensor("embed", gradient=True),
                               pb.tensor("embed", gradient=True), rtol=1e-5, atol=1e-8)
    with pytest.raises(_lib.SummaError, match="reference log-probs"):
        _lib.call("sm_policy_prepare_with_ref", pb._h, None, prompts.data_ptr(),
                  tok.data_ptr(), beh.data_ptr(), rewards.data_ptr(), None, B, G, 8, 6, 0.2,
                  1e-6, 0.04, a["lp_cur"].data_ptr(), a["stats"].data_ptr(),
                  a["dlp"].data_ptr(), a["flags"].data_ptr(),
                  torch.cuda.current_stream().cuda_stream)


def test_quantized_policy_recompute_equals_rollout_model(dev):
    """A quantized config trains f32 masters with fake-quantized forward
    weights: its recompute equals the installed Q4 model's log-probs (2e-3,
    the 16-bit KV cache of the model being the only difference), and an
    update moves the installed model."""
    qc = ModelConfig(layers=2, d_model=256, heads=4, kv_heads=2, head_dim=64, ffn=512,
                     vocab=1024, max_seq=32, quantized=True)
    w = oracle.random_weights(qc.oracle_cfg(), seed=16, std=0.05)
    pol = train.Policy(qc, w, dev)
    model = Model(qc)
    pol.install(model)
    prompts, _, rewards = _batch(qc, 6, dev)
    tok, beh = model.generate(prompts, 6, temperature=1.0, seed=3)
    out = pol.prepare(None, prompts, tok, beh, rewards, kl_coefficient=0.0)
    err = float((out["lp_cur"] - beh).abs().max())
    print(f"quantized policy recompute vs Q4 rollout log-probs: {err:.2e}", flush=True)
    assert err <= 2e-3
    before = model.logprobs(prompts, tok)
    pol.optimizer_step(1.0)
    pol.install(model)
    assert float((model.logprobs(prompts, tok) - before).abs().max()) > 1e-4


def test_quantized_moe_policy_recompute_equals_rollout_model(dev):
    """The same for an MoE config (4 experts, top-2, Q4G128 experts, f32
    router): the policy's recompute against the installed Q4 model's rollout
    log-probs (the router decisions of the two agree except at near-ties of
    the 16-bit-activation logits, so the bound is checked on 95 % of the
    positions and every position stays within 0.5), and an update moves the
    installed model."""
    qc = ModelConfig(layers=2, d_model=256, heads=4, kv_heads=2, head_dim=64, ffn=512,
                     vocab=1024, max_seq=32, quantized=True, experts=4, expert_ffn=128)
    w = oracle.random_weights(qc.oracle_cfg(), seed=17, std=0.05)
    pol = train.Policy(qc, w, dev)
    model = Model(qc)
    pol.install(model)
    prompts, _, rewards = _batch(qc, 8, dev)
    tok, beh = model.generate(prompts, 6, temperature=1.0, seed=3)
    out = pol.prepare(None, prompts, tok, beh, rewards, kl_coefficient=0.0)
    diff = (out["lp_cur"] - beh).abs().flatten().cpu()
    q95 = float(diff.quantile(0.95))
    print(f"quantized MoE policy recompute vs Q4 rollout: max {float(diff.max()):.2e}, "
          f"95th percentile {q95:.2e}", flush=True)
    assert q95 <= 2e-3 and float(diff.max()) <= 0.5
    before = model.logprobs(prompts, tok)
    pol.optimizer_step(1.0)
    pol.install(model)
    assert float((model.logprobs(prompts, tok) - before).abs().max()) > 1e-4


def test_policy_rejects_bad_config(dev):
    bad = ModelConfig(layers=1, d_model=256, heads=4, kv_heads=4, head_dim=64, ffn=512,
                      vocab=100, max_seq=16, quantized=True, experts=1, expert_ffn=256)
    with pytest.raises(_lib.SummaError, match="2..=64 experts"):
        train.Policy(bad, {}, dev)
    bad.experts, bad.expert_ffn = 4, 200  # quantized experts need 128-wide groups
    with pytest.raises(_lib.SummaError, match="% 128 == 0"):
        train.Policy(bad, {}, dev)
    dense = ModelConfig(layers=1, d_model=256, heads=4, kv_heads=4, head_dim=64, ffn=512,
                        vocab=100, max_seq=16, quantized=False)
    pol = train.Policy(dense, {}, dev)
    buf = torch.empty(16, device=dev)
    with pytest.raises(_lib.SummaError, match="not part of this policy"):
        _lib.call("sm_policy_get_tensor", pol._h, 9, 0, buf.data_ptr(), 0,
                  torch.cuda.current_stream().cuda_stream)
