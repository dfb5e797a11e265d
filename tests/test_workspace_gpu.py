"""Caller-bound RL workspace (sm_rl_workspace_bytes / sm_model_bind_workspace):
with a bound workspace the hot calls carve their buffers from it (no device
allocation), give the same bits as the model's own grow-only buffers, accept
smaller shapes and reject larger ones with a clear error."""
import numpy as np
import pytest
import torch

import oracle
from summa_amd import _lib
from summa_amd.model import Model, ModelConfig, rl_prepare

pytestmark = pytest.mark.gpu

GEOMS = {
    "q4": ModelConfig(layers=2, d_model=768, heads=12, kv_heads=4, head_dim=64, ffn=3072,
                      vocab=4096, max_seq=160, quantized=True),
    "moe": ModelConfig(layers=2, d_model=512, heads=4, kv_heads=2, head_dim=128, ffn=256,
                       vocab=4096, max_seq=160, quantized=True, experts=8, expert_ffn=256),
    "fp32": ModelConfig(layers=2, d_model=256, heads=4, kv_heads=4, head_dim=64, ffn=1024,
                        vocab=4096, max_seq=160, quantized=False),
}


def _pair(mc, seed, dev):
    w = oracle.random_weights(mc.oracle_cfg(), seed=seed, std=0.02)
    models = []
    for _ in range(2):
        m = Model(mc)
        m.load_host_weights(w, dev)
        models.append(m)
    return models


def _step(policy, ref, prompts, N, rewards, mtpf):
    tok, lp_beh = policy.generate(prompts, N, temperature=1.0, seed=5)
    out = rl_prepare(policy, ref, prompts, tok, lp_beh, rewards,
                     max_tokens_per_forward=mtpf)
    torch.cuda.synchronize()
    return tok, lp_beh, out


@pytest.mark.parametrize("geom", sorted(GEOMS))
def test_bound_workspace_equals_own_buffers(dev, geom):
    print(f"case workspace {geom}", flush=True)
    mc = GEOMS[geom]
    groups, G, P, N, mtpf = 4, 8, 40, 12, 600
    S = groups * G
    g = torch.Generator().manual_seed(1)
    prompts = torch.randint(0, mc.vocab, (S, P), generator=g, dtype=torch.int32).to(dev)
    rewards = torch.rand(groups, G, generator=g).to(dev)
    a_pol, a_ref = _pair(mc, 3, dev)
    b_pol, b_ref = _pair(mc, 3, dev)
    for m in (b_pol, b_ref):
        ws = m.bind_workspace(S, P, N, mtpf)
        assert ws.numel() >= m.workspace_bytes(S, P, N, mtpf)
    ta, la, oa = _step(a_pol, a_ref, prompts, N, rewards, mtpf)
    tb, lb, ob = _step(b_pol, b_ref, prompts, N, rewards, mtpf)
    assert torch.equal(ta, tb) and torch.equal(la, lb)
    for k in ("lp_cur", "lp_ref", "stats", "dlp", "flags"):
        assert torch.equal(oa[k], ob[k]), k
    # smaller shapes fit the bound workspace
    t2, l2 = b_pol.generate(prompts[:S // 2, :P - 5], N - 3, temperature=1.0, seed=5)
    t3, l3 = a_pol.generate(prompts[:S // 2, :P - 5], N - 3, temperature=1.0, seed=5)
    assert torch.equal(t2, t3) and torch.equal(l2, l3)
    # larger ones are refused before any launch
    big = torch.randint(0, mc.vocab, (2 * S, P), generator=g, dtype=torch.int32).to(dev)
    with pytest.raises(_lib.SummaError, match="bound workspace holds"):
        b_pol.generate(big, N, temperature=1.0, seed=5)
    # unbinding returns the model to its own buffers
    b_pol.unbind_workspace()
    t4, l4 = b_pol.generate(big, N, temperature=1.0, seed=5)
    t5, l5 = a_pol.generate(big, N, temperature=1.0, seed=5)
    assert torch.equal(t4, t5) and torch.equal(l4, l5)


def test_bound_workspace_prompt_groups(dev):
    """Shared prompts (sm_model_set_prompt_groups) with a bound workspace and a
    budget whose continuation chunks score more rows than the budget (cc = 600
    // 11 = 54 rollouts of N = 12 scored rows: 648 > 600): the bound model's
    rollout and recompute equal the own-buffer model's bit for bit."""
    mc = GEOMS["q4"]
    groups, G, P, N, mtpf = 8, 8, 40, 12, 600
    S = groups * G
    g = torch.Generator().manual_seed(7)
    prompts = torch.randint(0, mc.vocab, (groups, P), generator=g,
                            dtype=torch.int32).repeat_interleave(G, 0).to(dev)
    rewards = torch.rand(groups, G, generator=g).to(dev)
    a_pol, a_ref = _pair(mc, 5, dev)
    b_pol, b_ref = _pair(mc, 5, dev)
    for m in (a_pol, a_ref, b_pol, b_ref):
        m.set_prompt_groups(G)
    for m in (b_pol, b_ref):
        m.bind_workspace(S, P, N, mtpf)
    ta, la, oa = _step(a_pol, a_ref, prompts, N, rewards, mtpf)
    tb, lb, ob = _step(b_pol, b_ref, prompts, N, rewards, mtpf)
    assert torch.equal(ta, tb) and torch.equal(la, lb)
    for k in ("lp_cur", "lp_ref", "stats", "dlp", "flags"):
        assert torch.equal(oa[k], ob[k]), k


def test_bound_calls_allocate_nothing(dev):
    """A bound model's first rollout and recompute leave the device's free
    memory unchanged; the same calls on an unbound model take hundreds of MB
    (the control that shows the measurement sees the library's buffers)."""
    mc = GEOMS["q4"]
    S, P, N = 256, 150, 8
    g = torch.Generator().manual_seed(2)
    prompts = torch.randint(0, mc.vocab, (S, P), generator=g, dtype=torch.int32).to(dev)
    tok = torch.randint(0, mc.vocab, (S, N), generator=g, dtype=torch.int32).to(dev)
    bound, own = _pair(mc, 4, dev)
    bound.bind_workspace(S, P, N)
    for m in (bound, own):
        # torch's own output tensors come from its caching allocator: warm it
        m_out = [torch.empty(S, N, dtype=torch.int32, device=dev) for _ in range(4)]
        del m_out
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        m.generate(prompts, N, temperature=1.0, seed=1)
        m.logprobs(prompts, tok)
        torch.cuda.synchronize()
        used = free0 - torch.cuda.mem_get_info()[0]
        print(f"{'bound' if m is bound else 'own'}: device memory taken {used / 2**20:.1f} MiB",
              flush=True)
        if m is bound:
            assert used <= 8 << 20
        else:
            assert used >= 200 << 20


def test_workspace_query_rejects_bad_shapes(dev):
    m = Model(GEOMS["fp32"])
    assert _lib.lib().sm_rl_workspace_bytes(m.handle, 0, 4, 4, 0) == -1
    with pytest.raises(_lib.SummaError, match="256-byte aligned"):
        buf = torch.empty(1 << 20, dtype=torch.uint8, device=dev)
        _lib.call("sm_model_bind_workspace", m.handle, buf.data_ptr() + 16, 1 << 19, 1, 4, 4, 0)
    need = m.workspace_bytes(2, 8, 4)
    buf = torch.empty(need, dtype=torch.uint8, device=dev)
    with pytest.raises(_lib.SummaError, match="needed"):
        _lib.call("sm_model_bind_workspace", m.handle, buf.data_ptr(), need - 1, 2, 8, 4, 0)
    assert np.isfinite(need)
