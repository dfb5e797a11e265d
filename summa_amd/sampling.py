"""Sampling options and the device sampler (host side of ``sampling.hip``).

``SamplingConfig`` mirrors ``SamplingConfig`` of summa-llm/src/generate.rs:12-36
(field names, defaults, ``None`` for "off"), ``RolloutSampling`` mirrors
summa-train/src/posttrain.rs:353-387 (defaults and ``validate`` messages). Both
lower to the C struct ``sm_sampling``; the checks run in the library, which
reports the reference's messages.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import call

MAX_POST_TRAINING_SEQUENCE_TOKENS = 1_048_576  # posttrain.rs:54


class SamplingC(C.Structure):
    """``sm_sampling`` of include/summa_amd.h."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int32),
                ("repetition_penalty", C.c_float), ("eos_token", C.c_int32),
                ("top_p", C.c_float), ("apply_top_p", C.c_int32)]


@dataclass
class SamplingConfig:
    """generate.rs:12-36. ``temperature <= 0`` is greedy; ``top_k``/``eos_token``
    ``None`` are off; ``repetition_penalty`` 1.0 is off. ``top_p`` and
    ``apply_top_p`` extend it with the rollout nucleus option (``apply_top_p``
    False keeps the reference's behaviour: validated, not applied)."""
    max_new_tokens: int = 100
    temperature: float = 0.9
    top_k: int | None = None
    repetition_penalty: float = 1.0
    eos_token: int | None = None
    seed: int | None = None
    top_p: float = 1.0
    apply_top_p: bool = False

    def c(self) -> SamplingC:
        return SamplingC(float(self.temperature), -1 if self.top_k is None else int(self.top_k),
                         float(self.repetition_penalty),
                         -1 if self.eos_token is None else int(self.eos_token),
                         float(self.top_p), int(bool(self.apply_top_p)))


@dataclass
class RolloutSampling:
    """posttrain.rs:353-387: the GRPO rollout options."""
    max_new_tokens: int = 512
    temperature: float = 0.7
    top_p: float = 0.95

    def validate(self) -> None:
        if not 1 <= self.max_new_tokens <= MAX_POST_TRAINING_SEQUENCE_TOKENS:
            raise ValueError(
                f"max_new_tokens must be in 1..={MAX_POST_TRAINING_SEQUENCE_TOKENS}")
        t = float(self.temperature)
        if not (t == t and abs(t) != float("inf") and t > 0.0):
            raise ValueError("rollout temperature must be finite and positive")
        p = float(self.top_p)
        if not (p == p and abs(p) != float("inf") and 0.0 < p <= 1.0):
            raise ValueError("rollout top_p must be finite and in (0, 1]")

    def sampling_config(self, seed: int | None = None) -> SamplingConfig:
        """The per-rollout options: temperature sampling, top_p validated only."""
        self.validate()
        return SamplingConfig(max_new_tokens=self.max_new_tokens, temperature=self.temperature,
                              seed=seed, top_p=self.top_p)


def seen_words(vocab: int) -> int:
    return (vocab + 31) // 32


def seen_tokens(ids: torch.Tensor, vocab: int, seen: torch.Tensor | None = None,
                clear: bool = True) -> torch.Tensor:
    """The prior-token set of apply_repetition_penalty as a device bitmap
    [rows, ceil(vocab / 32)] int32 (bit v of word v // 32)."""
    ids = ids.contiguous()
    if ids.dtype != torch.int32 or ids.dim() != 2 or not ids.is_cuda:
        raise ValueError("ids must be a CUDA int32 [rows, n] tensor")
    rows, n = ids.shape
    if seen is None:
        seen = torch.empty(rows, seen_words(vocab), dtype=torch.int32, device=ids.device)
    call("sm_seen_tokens", ids.data_ptr(), rows, n, n, vocab, seen.data_ptr(), seen.shape[1],
         int(clear), torch.cuda.current_stream(ids.device).cuda_stream)
    return seen


def sample(logits: torch.Tensor, cfg: SamplingConfig, seed: int, step: int, *,
           seen: torch.Tensor | None = None, done: torch.Tensor | None = None,
           lengths: torch.Tensor | None = None):
    """``sm_sample_ex`` over f32 logits [rows, vocab]: (tokens int32, log-probs f32)."""
    if logits.dtype != torch.float32 or logits.dim() != 2 or not logits.is_cuda:
        raise ValueError("logits must be a CUDA f32 [rows, vocab] tensor")
    if logits.stride(1) != 1:
        raise ValueError("logits rows must be contiguous")
    rows, vocab = logits.shape
    tok = torch.empty(rows, dtype=torch.int32, device=logits.device)
    lp = torch.empty(rows, dtype=torch.float32, device=logits.device)
    sc = cfg.c()
    call("sm_sample_ex", logits.data_ptr(), rows, logits.stride(0), vocab, C.addressof(sc),
         int(seed), int(step), None if seen is None else seen.data_ptr(),
         0 if seen is None else seen.shape[1], None if done is None else done.data_ptr(),
         None if lengths is None else lengths.data_ptr(), tok.data_ptr(), 1, lp.data_ptr(), 1,
         None, torch.cuda.current_stream(logits.device).cuda_stream)
    return tok, lp
