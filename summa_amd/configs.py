"""The five BASELINE workloads as data (model geometry + GRPO step shape).

Config numbering follows BASELINE.json ``configs[0..4]``. The model geometry
is the MAL ModelDef subset the decoder implements (summa-mal/src/lib.rs:140-150,
280-292); the step shape is one GRPO update of summa-train's post-training
loop (prompts x group rollouts, prompt length, new tokens, reward law;
posttrain.rs:4339-4440). Config 3 is the fused cross-entropy stress test and
has no model.
"""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass(frozen=True)
class RlWorkload:
    index: int
    model: dict            # ModelConfig keyword arguments (max_seq is derived)
    prompts: int
    group: int
    prompt_len: int
    new_tokens: int
    temperature: float
    rewards: str           # "bernoulli0.5" | "bernoulli0.3" | "uniform"
    quantized: bool
    extra: dict = field(default_factory=dict)

    @property
    def rollouts(self) -> int:
        return self.prompts * self.group

    @property
    def max_seq(self) -> int:
        return self.prompt_len + self.new_tokens

    def model_config(self):
        from .model import ModelConfig
        return ModelConfig(**self.model, max_seq=self.max_seq, quantized=self.quantized)

    def reward_label(self) -> str:
        return {"bernoulli0.5": "Bernoulli(0.5)", "bernoulli0.3": "Bernoulli(0.3)",
                "uniform": "U[0,1]"}[self.rewards]

    def sample_rewards(self, generator):
        """[prompts, group] f32 rewards on the host from a torch.Generator."""
        import torch
        shape = (self.prompts, self.group)
        if self.rewards == "uniform":
            return torch.rand(shape, generator=generator)
        p = 0.5 if self.rewards == "bernoulli0.5" else 0.3
        return torch.bernoulli(torch.full(shape, p), generator=generator)


CFG0_MODEL = dict(layers=2, d_model=256, heads=4, kv_heads=4, head_dim=64, ffn=1024, vocab=4096)
CFG1_MODEL = dict(layers=12, d_model=768, heads=12, kv_heads=12, head_dim=64, ffn=3072,
                  vocab=32768)
CFG2_MODEL = dict(layers=24, d_model=2048, heads=16, kv_heads=4, head_dim=128, ffn=5632,
                  vocab=65536)
# config[4]: the attention geometry is not given by the config; H16 = KVH16,
# head_dim 128 (d_model / heads). All layers are MoE, so the dense FFN width
# is unused.
CFG4_MODEL = dict(layers=16, d_model=2048, heads=16, kv_heads=16, head_dim=128, ffn=1408,
                  vocab=65536, experts=32, expert_ffn=1408)

RL_WORKLOADS = {
    0: RlWorkload(0, CFG0_MODEL, 4, 8, 32, 64, 0.0, "bernoulli0.5", quantized=False),
    1: RlWorkload(1, CFG1_MODEL, 16, 8, 128, 256, 1.0, "bernoulli0.3", quantized=True),
    2: RlWorkload(2, CFG2_MODEL, 32, 8, 512, 512, 1.0, "uniform", quantized=True),
    4: RlWorkload(4, CFG4_MODEL, 16, 8, 256, 256, 1.0, "bernoulli0.3", quantized=True),
}

# GRPO loss settings shared by every config (config[0]: PPO clip 0.2, KL 0.04;
# the advantage epsilon is posttrain.rs:69-83's default).
CLIP_EPSILON = 0.2
KL_COEFFICIENT = 0.04
ADVANTAGE_EPSILON = 1e-6

# config[3]: bf16 logits [65536, 131072] ~ N(0, 3) plus a +8 spike at a random
# int32 target per row.
CE_STRESS = dict(rows=65536, vocab=131072, std=3.0, spike=8.0)
