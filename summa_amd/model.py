"""Host-side mirror of the reference's model / RL runtime entry points.

``Model`` wraps an ``sm_model`` (weights resident in HBM) and exposes the
GrpoDeviceBatchRuntime operations (summa-train/src/posttrain.rs:1288-1305):
``generate`` (generate_device_batch), ``logprobs`` (the recompute inside
prepare_device_batch) and ``rl_prepare`` (recompute + GRPO loss).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import call

# tensor kinds (include/summa_amd.h SM_W_*)
KIND = {"embed": 0, "attn_norm": 1, "qkv": 2, "o": 3, "ffn_norm": 4, "in": 5, "down": 6,
        "final_norm": 7, "lm_head": 8, "router": 9, "exp_in": 10, "exp_down": 11}
PER_LAYER = ("attn_norm", "ffn_norm", "qkv", "o", "in", "down", "router", "exp_in", "exp_down")


class ModelConfigC(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("layers", "d_model", "heads", "kv_heads", "head_dim",
                                         "ffn", "vocab", "max_seq")] + \
        [("norm_eps", C.c_float), ("rope_theta", C.c_float), ("quantized", C.c_int32),
         ("experts", C.c_int32), ("expert_ffn", C.c_int32)]


@dataclass
class ModelConfig:
    """Decoder geometry (MAL ModelDef subset, summa-mal/src/lib.rs:140-150, 280-292)."""
    layers: int
    d_model: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    max_seq: int
    quantized: bool
    norm_eps: float = 1e-5
    rope_theta: float = 1e4
    experts: int = 0
    expert_ffn: int = 0

    def c(self) -> ModelConfigC:
        return ModelConfigC(self.layers, self.d_model, self.heads, self.kv_heads, self.head_dim,
                            self.ffn, self.vocab, self.max_seq, self.norm_eps, self.rope_theta,
                            int(self.quantized), self.experts, self.expert_ffn)

    def oracle_cfg(self) -> dict:
        cfg = {"layers": self.layers, "d": self.d_model, "H": self.heads, "KVH": self.kv_heads,
               "hd": self.head_dim, "F": self.ffn, "V": self.vocab, "eps": self.norm_eps,
               "theta": self.rope_theta}
        if self.experts:
            cfg.update(E=self.experts, Fe=self.expert_ffn)
        return cfg


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


class Model:
    def __init__(self, cfg: ModelConfig):
        self.cfg = cfg
        self._h = C.c_void_p()
        lib = _lib.lib()
        lib.sm_model_create.argtypes = [C.POINTER(ModelConfigC), C.POINTER(C.c_void_p)]
        cc = cfg.c()
        _lib.check(lib.sm_model_create(C.byref(cc), C.byref(self._h)))

    @property
    def handle(self) -> int:
        return self._h.value

    def close(self) -> None:
        if self._h.value:
            _lib.lib().sm_model_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def weight_bytes(self) -> int:
        return int(_lib.lib().sm_model_weight_bytes(self._h))

    def set_tensor(self, name: str, src: torch.Tensor, layer: int = -1) -> None:
        """Load a dense float32 device tensor (linears in [out, in] layout)."""
        src = src.contiguous().float()
        call("sm_model_set_tensor", self._h, KIND[name], layer, src.data_ptr(), _stream())

    def load_packed(self, name: str, packed, layer: int = -1, layout: int = 0) -> None:
        """Install an HQUANT ``PackedTensor`` (``sm_model_load_packed``):
        layout 0 = rows [out, in], 1 = Burn's [in, out] Linear layout."""
        from .hquant import DevicePacked
        dev = torch.device("cuda", torch.cuda.current_device())
        d = DevicePacked(packed, dev)
        call("sm_model_load_packed", self._h, KIND[name], layer, C.addressof(d.c), int(layout),
             _stream())
        torch.cuda.current_stream().synchronize()

    def load_host_weights(self, weights: dict, device) -> None:
        """weights as produced by ``oracle.random_weights`` style dicts (numpy)."""
        for name, arr in weights.items():
            t = torch.from_numpy(arr).to(device)
            if name in PER_LAYER:
                for layer in range(self.cfg.layers):
                    self.set_tensor(name, t[layer], layer)
            else:
                self.set_tensor(name, t)
        torch.cuda.synchronize()

    def trace_routes(self, capacity: int, logits: bool = True):
        """Start an MoE router trace of ``capacity`` token entries
        (``sm_model_trace_routes``): returns the device buffers it fills, ids
        [capacity, 2] int32 and router logits [capacity, experts] f32 (or None).
        ``stop_trace`` ends it."""
        dev = torch.device("cuda", torch.cuda.current_device())
        idx = torch.full((capacity, 2), -1, dtype=torch.int32, device=dev)
        lg = (torch.zeros((capacity, self.cfg.experts), dtype=torch.float32, device=dev)
              if logits else None)
        call("sm_model_trace_routes", self._h, idx.data_ptr(),
             None if lg is None else lg.data_ptr(), int(capacity))
        self._trace = (idx, lg)
        return idx, lg

    def route_trace_count(self):
        """(recorded, dropped) token entries of the current trace."""
        rec, drop = C.c_int64(), C.c_int64()
        call("sm_model_route_trace_count", self._h, C.byref(rec), C.byref(drop))
        return rec.value, drop.value

    def stop_trace(self) -> None:
        call("sm_model_trace_routes", self._h, None, None, 0)
        self._trace = None

    def set_prompt_groups(self, group_size: int) -> None:
        """sm_model_set_prompt_groups: rollouts g*G .. g*G+G-1 of later RL
        calls share one prompt, computed once per group (1 = off). Set before
        binding a workspace."""
        call("sm_model_set_prompt_groups", self._h, int(group_size))
        self.prompt_group = int(group_size)

    def workspace_bytes(self, S: int, P: int, N: int, max_tokens_per_forward: int = 0) -> int:
        """sm_rl_workspace_bytes: device bytes the RL calls need for these shapes."""
        n = int(_lib.lib().sm_rl_workspace_bytes(self._h, S, P, N, int(max_tokens_per_forward)))
        if n < 0:
            raise ValueError("sm_rl_workspace_bytes: bad shape")
        return n

    def bind_workspace(self, S: int, P: int, N: int, max_tokens_per_forward: int = 0):
        """Allocate a workspace for RL calls of up to these shapes and bind it
        (sm_model_bind_workspace): later generate / logprobs / rl_prepare calls
        on this model allocate nothing. Returns the workspace tensor."""
        n = self.workspace_bytes(S, P, N, max_tokens_per_forward)
        dev = torch.device("cuda", torch.cuda.current_device())
        ws = torch.empty(n + 256, dtype=torch.uint8, device=dev)
        base = (ws.data_ptr() + 255) // 256 * 256
        call("sm_model_bind_workspace", self._h, base, n, S, P, N, int(max_tokens_per_forward))
        self._ws = ws
        return ws

    def unbind_workspace(self) -> None:
        call("sm_model_bind_workspace", self._h, None, 0, 0, 0, 0, 0)
        self._ws = None

    def init_random(self, seed: int = 0, std: float = 0.02) -> None:
        call("sm_model_init_random", self._h, int(seed), float(std), _stream())

    def generate(self, prompts: torch.Tensor, max_new_tokens: int, temperature: float = 0.0,
                 seed: int = 0):
        """Batched rollouts: prompts [S, P] int32 -> (tokens [S, N], behavior_lp [S, N])."""
        S, P = prompts.shape
        N = int(max_new_tokens)
        tok = torch.empty(S, N, dtype=torch.int32, device=prompts.device)
        lp = torch.empty(S, N, dtype=torch.float32, device=prompts.device)
        call("sm_rl_generate", self._h, prompts.data_ptr(), S, P, N, float(temperature), int(seed),
             tok.data_ptr(), lp.data_ptr(), _stream())
        return tok, lp

    def generate_ex(self, prompts: torch.Tensor, config, seed: int | None = None):
        """Batched rollouts with a ``sampling.SamplingConfig`` (top-k, repetition
        penalty, EOS, nucleus): (tokens [S, N], behavior_lp [S, N], lengths [S]).
        ``seed`` defaults to ``config.seed`` (0 when neither is given)."""
        import ctypes as C
        S, P = prompts.shape
        N = int(config.max_new_tokens)
        tok = torch.empty(S, N, dtype=torch.int32, device=prompts.device)
        lp = torch.empty(S, N, dtype=torch.float32, device=prompts.device)
        lens = torch.empty(S, dtype=torch.int32, device=prompts.device)
        sc = config.c()
        seed = config.seed if seed is None else seed
        call("sm_rl_generate_ex", self._h, prompts.data_ptr(), S, P, N, C.addressof(sc),
             int(seed or 0), tok.data_ptr(), lp.data_ptr(), lens.data_ptr(), _stream())
        return tok, lp, lens

    def logprobs(self, prompts: torch.Tensor, tokens: torch.Tensor, max_tokens_per_forward=0):
        S, P = prompts.shape
        N = tokens.shape[1]
        lp = torch.empty(S, N, dtype=torch.float32, device=prompts.device)
        call("sm_rl_logprobs", self._h, prompts.data_ptr(), tokens.data_ptr(), S, P, N,
             int(max_tokens_per_forward), lp.data_ptr(), _stream())
        return lp


def completion_mask(lengths: torch.Tensor, N: int) -> torch.Tensor:
    """sm_completion_mask: f32 [S, N], 1 for n < lengths[s] (EOS included)."""
    S = lengths.shape[0]
    mask = torch.empty(S, N, dtype=torch.float32, device=lengths.device)
    call("sm_completion_mask", lengths.data_ptr(), S, N, mask.data_ptr(), _stream())
    return mask


def rl_prepare(policy: Model, reference: Model | None, prompts, tokens, behavior_lp, rewards,
               mask=None, clip_epsilon=0.2, advantage_epsilon=1e-6, kl_coefficient=0.04,
               max_tokens_per_forward=0, lengths=None):
    """prepare_device_batch numerics: returns dict of device tensors (lp_cur, lp_ref,
    stats [groups, 5], dlp [S, N], flags [groups]) and the GrpoDeviceBatchResult sums.
    Rollouts from ``generate_ex`` that stopped at EOS pass their ``lengths``
    (the completion mask is built from them) or an explicit ``mask``."""
    groups, G = rewards.shape
    S, P = prompts.shape
    N = tokens.shape[1]
    dev = prompts.device
    if lengths is not None:
        if mask is not None:
            raise ValueError("rl_prepare: pass either mask or lengths")
        mask = completion_mask(lengths, N)
    lp_cur = torch.empty(S, N, dtype=torch.float32, device=dev)
    lp_ref = torch.empty(S, N, dtype=torch.float32, device=dev) if reference is not None else None
    stats = torch.empty(groups, 5, dtype=torch.float32, device=dev)
    dlp = torch.empty(S, N, dtype=torch.float32, device=dev)
    flags = torch.empty(groups, dtype=torch.int32, device=dev)
    call("sm_rl_prepare", policy.handle, reference.handle if reference is not None else None,
         prompts.data_ptr(), tokens.data_ptr(), behavior_lp.data_ptr(), rewards.data_ptr(),
         None if mask is None else mask.data_ptr(), groups, G, P, N, float(clip_epsilon),
         float(advantage_epsilon), float(kl_coefficient), int(max_tokens_per_forward),
         lp_cur.data_ptr(), None if lp_ref is None else lp_ref.data_ptr(), stats.data_ptr(),
         dlp.data_ptr(), flags.data_ptr(), _stream())
    return {"lp_cur": lp_cur, "lp_ref": lp_ref, "stats": stats, "dlp": dlp, "flags": flags}


def batch_result(out: dict) -> dict:
    """GrpoDeviceBatchResult sums over groups (posttrain.rs:1234-1244); one host read."""
    f = out["flags"].cpu()
    bad = [int(v) for v in f.tolist() if v]
    if bad:
        from .ops import GrpoValidationError
        raise GrpoValidationError(_lib.lib().sm_grpo_flags_message(bad[0]).decode())
    s = out["stats"].double().sum(0).cpu().tolist()
    return {"examples": out["stats"].shape[0], "rollouts": out["dlp"].shape[0],
            "loss_sum": s[0], "mean_reward_sum": s[1], "reward_stddev_sum": s[2],
            "mean_kl_sum": s[3], "clipped_fraction_sum": s[4]}
