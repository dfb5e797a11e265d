"""Host-side mirror of the reference's kernel entry points, over the C ABI.

Tensors are torch device tensors (torch is only the allocator and stream
provider here); every computation runs in ``libsumma_amd.so``. Names and
argument meaning follow the reference interfaces cited in each docstring.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from ._lib import SM_BF16, SM_F16, SM_F32, call

_DTYPES = {torch.float32: SM_F32, torch.bfloat16: SM_BF16, torch.float16: SM_F16}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dt(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError as e:
        raise TypeError(f"unsupported dtype {t.dtype}") from e


def _p(t):
    return None if t is None else t.data_ptr()


def _dev(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


# ------------------------------------------------------------------- CE ---

def ce_rows(logits: torch.Tensor, targets: torch.Tensor, logical_vocab: int | None = None, *,
            grad_in_place: bool = False, grad_scale: float = 1.0,
            row_scale: torch.Tensor | None = None, want_lse: bool = False,
            want_loss: bool = True):
    """Row-wise fused log-softmax / CE / token log-prob.

    Mirrors ``ce_row_statistics`` + ``ce_row_gradient``
    (summa-llm/src/model/linear_cross_entropy/gpu.rs:29-158) and the
    ``log_softmax(..).gather(targets)`` of tensor_sleep.rs:2609-2614.
    Returns ``(token_logprob [rows] f32, loss [1] f32 or None, lse or None)``;
    with ``grad_in_place`` the logits buffer is overwritten by
    ``(softmax - onehot) * grad_scale * row_scale``.
    """
    _dev(logits, "logits")
    _dev(targets, "targets")
    if targets.dtype != torch.int32:
        raise TypeError("targets must be int32")
    rows, stored = logits.shape
    lv = stored if logical_vocab is None else int(logical_vocab)
    lp = torch.empty(rows, dtype=torch.float32, device=logits.device)
    loss = torch.empty(1, dtype=torch.float32, device=logits.device) if want_loss else None
    lse = torch.empty(rows, dtype=torch.float32, device=logits.device) if want_lse else None
    if row_scale is not None:
        _dev(row_scale, "row_scale")
    call("sm_ce_rows", logits.data_ptr(), _dt(logits), targets.data_ptr(), rows, stored, lv,
         lp.data_ptr(), _p(lse), logits.data_ptr() if grad_in_place else None, float(grad_scale),
         _p(row_scale), _p(loss), _stream())
    return lp, loss, lse


def _lce_args(hidden, weight, bias, targets, logical_vocab, chunk_size):
    for t, name in ((hidden, "hidden"), (weight, "weight"), (targets, "targets")):
        _dev(t, name)
    if hidden.dtype != torch.float32 or weight.dtype != torch.float32:
        raise TypeError("hidden and weight must be float32")
    if targets.dtype != torch.int32:
        raise TypeError("targets must be int32")
    tokens, d = hidden.shape
    stored, dw = weight.shape
    if dw != d or targets.shape != (tokens,):
        raise ValueError("linear cross-entropy: hidden [T, d], weight [V, d], targets [T]")
    if bias is not None:
        _dev(bias, "bias")
        if bias.dtype != torch.float32 or bias.shape != (stored,):
            raise ValueError("bias must be float32 [V]")
    lv = stored if logical_vocab is None else int(logical_vocab)
    nbytes = int(_lib.lib().sm_linear_cross_entropy_workspace_bytes(
        tokens, d, stored, int(chunk_size), int(bias is not None)))
    ws = torch.empty(max(nbytes, 0) + 256, dtype=torch.uint8, device=hidden.device)
    base = (ws.data_ptr() + 255) // 256 * 256
    return tokens, d, stored, lv, ws, base, nbytes


def linear_cross_entropy(hidden: torch.Tensor, weight: torch.Tensor, bias, targets: torch.Tensor,
                         logical_vocab: int | None = None, chunk_size: int = 1024,
                         want_logprob: bool = False):
    """Fused linear head + cross-entropy (``sm_linear_cross_entropy``): the
    mean over tokens of -log_softmax(hidden W^T + b)[target] over the logical
    vocabulary, computed in chunks of ``chunk_size`` rows
    (linear_cross_entropy_inner, summa-llm/src/model/linear_cross_entropy/mod.rs:33-43,
    reference.rs:42-92). Returns ``loss [1]`` (and the per-token log-probs with
    ``want_logprob``)."""
    tokens, d, stored, lv, ws, base, nbytes = _lce_args(hidden, weight, bias, targets,
                                                        logical_vocab, chunk_size)
    loss = torch.empty(1, dtype=torch.float32, device=hidden.device)
    lp = torch.empty(tokens, dtype=torch.float32, device=hidden.device) if want_logprob else None
    call("sm_linear_cross_entropy", hidden.data_ptr(), weight.data_ptr(), _p(bias),
         targets.data_ptr(), tokens, d, stored, lv, int(chunk_size), int(bias is not None),
         loss.data_ptr(), _p(lp), base, nbytes, _stream())
    return (loss, lp) if want_logprob else loss


def linear_cross_entropy_backward(hidden: torch.Tensor, weight: torch.Tensor, bias,
                                  targets: torch.Tensor, grad_output: torch.Tensor,
                                  logical_vocab: int | None = None, chunk_size: int = 1024):
    """The three gradients (hidden [T, d], weight [V, d], bias [V] or None) of
    ``linear_cross_entropy`` for the upstream gradient ``grad_output`` [1]
    (``sm_linear_cross_entropy_backward``; linear_cross_entropy_backward,
    mod.rs:45-57, reference.rs:94-159, gpu.rs:313-426)."""
    tokens, d, stored, lv, ws, base, nbytes = _lce_args(hidden, weight, bias, targets,
                                                        logical_vocab, chunk_size)
    _dev(grad_output, "grad_output")
    go = grad_output.reshape(1).to(torch.float32).contiguous()
    gh = torch.empty_like(hidden)
    gw = torch.empty_like(weight)
    gb = torch.empty_like(bias) if bias is not None else None
    call("sm_linear_cross_entropy_backward", hidden.data_ptr(), weight.data_ptr(), _p(bias),
         targets.data_ptr(), go.data_ptr(), tokens, d, stored, lv, int(chunk_size),
         int(bias is not None), gh.data_ptr(), gw.data_ptr(), _p(gb), base, nbytes, _stream())
    return gh, gw, gb


# ----------------------------------------------------------------- GRPO ---

class GrpoValidationError(ValueError):
    """Raised with the reference's message when a device validation flag is set."""


def grpo_loss_batched(rewards: torch.Tensor, current: torch.Tensor, behavior: torch.Tensor,
                      reference: torch.Tensor | None, active_mask: torch.Tensor | None,
                      clip_epsilon: float = 0.2, advantage_epsilon: float = 1e-6,
                      kl_coefficient: float = 0.04, *, validate: bool = True):
    """GRPO loss for ``B`` prompt groups at once.

    ``rewards`` [B, G]; ``current``/``behavior``/``reference``/``active_mask``
    [B, G, T] float32. Returns a dict of device tensors: ``stats`` [B, 5]
    (loss, mean_reward, reward_stddev, mean_kl, clipped_fraction),
    ``advantages`` [B, G], ``dlp`` [B, G, T], ``flags`` [B].
    Follows grpo_loss_tensor (summa-train/src/posttrain.rs:874-1028). With
    ``validate`` it performs the reference's single validation readback
    (posttrain.rs:1007-1025) and raises GrpoValidationError.
    """
    for name, t in (("rewards", rewards), ("current", current), ("behavior", behavior)):
        _dev(t, name)
        if t.dtype != torch.float32:
            raise TypeError(f"{name} must be float32")
    B, G, T = current.shape
    if tuple(rewards.shape) != (B, G):
        raise ValueError(f"GRPO rewards must have shape [{B}, {G}]")
    for name, t in (("behavior", behavior), ("active_mask", active_mask), ("reference", reference)):
        if t is not None:
            _dev(t, name)
            if tuple(t.shape) != (B, G, T):
                raise ValueError(f"GRPO {name} tensor must have shape [{G}, {T}]")
    dev = current.device
    stats = torch.empty(B, 5, dtype=torch.float32, device=dev)
    adv = torch.empty(B, G, dtype=torch.float32, device=dev)
    dlp = torch.empty(B, G, T, dtype=torch.float32, device=dev)
    flags = torch.empty(B, dtype=torch.int32, device=dev)
    call("sm_grpo_loss", rewards.data_ptr(), current.data_ptr(), behavior.data_ptr(),
         _p(reference), _p(active_mask), B, G, T, float(clip_epsilon), float(advantage_epsilon),
         float(kl_coefficient), stats.data_ptr(), adv.data_ptr(), dlp.data_ptr(),
         flags.data_ptr(), _stream())
    if validate:
        bad = flags.cpu()
        for f in bad.tolist():
            if f:
                raise GrpoValidationError(_lib.lib().sm_grpo_flags_message(f).decode())
    return {"stats": stats, "advantages": adv, "dlp": dlp, "flags": flags}


def grpo_loss_tensor(rewards, current, behavior, reference, active_mask, clip_epsilon,
                     advantage_epsilon, kl_coefficient):
    """Single-group form of grpo_loss_tensor (posttrain.rs:874): [G] rewards,
    [G, T] log-probs and mask; returns the scalar loss as a [1] device tensor."""
    out = grpo_loss_batched(
        rewards.unsqueeze(0), current.unsqueeze(0), behavior.unsqueeze(0),
        None if reference is None else reference.unsqueeze(0),
        None if active_mask is None else active_mask.unsqueeze(0),
        clip_epsilon, advantage_epsilon, kl_coefficient)
    return out["stats"][0, 0:1]


# ------------------------------------------------------------ synthetic ---

def fill_normal(t: torch.Tensor, mean: float, std: float, seed: int) -> torch.Tensor:
    _dev(t, "out")
    call("sm_fill_normal", t.data_ptr(), _dt(t), t.numel(), float(mean), float(std), int(seed),
         _stream())
    return t


def fill_ce_stress(logits: torch.Tensor, targets: torch.Tensor, std: float = 3.0,
                   spike: float = 8.0, seed: int = 0):
    _dev(logits, "logits")
    rows, vocab = logits.shape
    call("sm_fill_ce_stress", logits.data_ptr(), _dt(logits), targets.data_ptr(), rows, vocab,
         float(std), float(spike), int(seed), _stream())
    return logits, targets


# ----------------------------------------------------------------- Q4G128 ---

class Q4Weight:
    """A Q4G128 weight resident in HBM: W[N, K] (out x in).

    Device counterpart of ``PackedTensor`` (summa-train/src/quantization.rs:416-423)
    for this build's 4-bit format (HQUANT tag 4). ``codes``/``scales`` hold the
    row-major codec (the interchange format); ``tcodes``/``tscales`` the
    prepared tiled copy the matmul kernels read (sm_q4_pack)."""

    def __init__(self, codes: torch.Tensor, scales: torch.Tensor, n: int, k: int):
        self.codes, self.scales, self.n, self.k = codes, scales, n, k
        self.tcodes = self.tscales = None
        if k % 128 == 0:  # groups never straddle rows: the matmul layout exists
            rows = (n + 15) // 16 * 16
            self.tcodes = torch.empty(rows * k // 2, dtype=torch.uint8, device=codes.device)
            self.tscales = torch.empty(rows * k // 128, dtype=torch.int16, device=codes.device)
            call("sm_q4_pack", codes.data_ptr(), scales.data_ptr(), n, k, self.tcodes.data_ptr(),
                 self.tscales.data_ptr(), _stream())

    @property
    def nbytes(self) -> int:
        """Algorithmic bytes of the weight: N*K/2 codes + N*K/128 bf16 scales."""
        return self.n * self.k // 2 + 2 * (self.n * self.k // 128)

    def drop_rowmajor(self) -> None:
        """Free the row-major copy (the kernels only read the tiled one)."""
        self.codes = self.scales = None

    @classmethod
    def quantize(cls, w: torch.Tensor) -> "Q4Weight":
        """Quantize a dense device weight [N, K] (f32 or bf16)."""
        _dev(w, "weight")
        n, k = w.shape
        groups = (w.numel() + 127) // 128
        codes = torch.empty(groups * 64, dtype=torch.uint8, device=w.device)
        scales = torch.empty(groups, dtype=torch.int16, device=w.device)
        bad = torch.zeros(1, dtype=torch.int32, device=w.device)
        call("sm_q4_quantize", w.data_ptr(), _dt(w), w.numel(), codes.data_ptr(),
             scales.data_ptr(), bad.data_ptr(), _stream())
        if int(bad.item()):
            raise ValueError(f"{int(bad.item())} Q4 groups have a scale outside the f16 normal range")
        return cls(codes, scales, n, k)

    @classmethod
    def from_host(cls, codes, scales, n: int, k: int, device) -> "Q4Weight":
        """Upload host codes (uint8) and scales (bf16 bits as uint16)."""
        import numpy as np

        c = torch.from_numpy(np.ascontiguousarray(codes)).to(device)
        s = torch.from_numpy(np.ascontiguousarray(scales).view(np.int16)).to(device)
        return cls(c, s, n, k)


def q4_workspace(m: int, n: int, k: int, epilogue: int, device) -> torch.Tensor:
    """Device workspace sized by sm_q4_matmul_workspace_bytes."""
    nbytes = int(_lib.lib().sm_q4_matmul_workspace_bytes(m, n, k, int(epilogue)))
    return torch.zeros(max(nbytes, 16), dtype=torch.uint8, device=device)


def f16_pair(x: torch.Tensor) -> torch.Tensor:
    """fp32 [M, K] -> SM_F16X2 rows [M, 2K] f16: hi = f16(x), lo = f16(x - hi)."""
    hi = x.to(torch.float16)
    lo = (x - hi.float()).to(torch.float16)
    return torch.cat([hi, lo], dim=1).contiguous()


def unpair(y: torch.Tensor) -> torch.Tensor:
    """SM_F16X2 rows [M, 2K] -> fp32 [M, K] (hi + lo)."""
    k = y.shape[1] // 2
    return y[:, :k].float() + y[:, k:].float()


def _x_dtype(x: torch.Tensor, pair: bool) -> int:
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("x must be bfloat16 or float16")
    if pair and x.dtype != torch.float16:
        raise TypeError("f16 pairs are float16 rows of [hi | lo]")
    return _lib.SM_F16X2 if pair else _dt(x)


def _out_spec(epilogue: int, rows: int, n: int):
    if epilogue == _lib.SM_EPI_SWIGLU_BF16:
        return (rows, n // 2), torch.bfloat16
    if epilogue == _lib.SM_EPI_SWIGLU_F16:
        return (rows, n // 2), torch.float16
    if epilogue == _lib.SM_EPI_SWIGLU_F16X2:
        return (rows, 2 * (n // 2)), torch.float16
    if epilogue == _lib.SM_EPI_STORE_BF16:
        return (rows, n), torch.bfloat16
    return (rows, n), torch.float32


def q4_matmul(w: Q4Weight, x: torch.Tensor, out: torch.Tensor | None = None,
              epilogue: int = _lib.SM_EPI_STORE_F32, *, pair: bool = False,
              workspace: torch.Tensor | None = None) -> torch.Tensor:
    """y = x . W^T with Q4G128 weights; x bf16 or f16 [M, K], or with ``pair``
    f16 [M, 2K] SM_F16X2 rows (see f16_pair). ``workspace`` (a device byte
    tensor) lets batch calls split K (sm_q4_matmul_ws)."""
    _dev(x, "x")
    xdt = _x_dtype(x, pair)
    M, K = x.shape
    if pair:
        K //= 2
    if K != w.k:
        raise ValueError(f"packed linear input width mismatch ({K} != {w.k})")
    if w.tcodes is None:
        raise ValueError(f"Q4 matmul needs K % 128 == 0 (K={w.k})")
    shape, dt = _out_spec(epilogue, M, w.n)
    if out is None:
        if epilogue == _lib.SM_EPI_ADD_F32:
            raise ValueError("SM_EPI_ADD_F32 needs an output to accumulate into")
        out = torch.empty(shape, dtype=dt, device=x.device)
    _dev(out, "out")
    if workspace is None:
        call("sm_q4_matmul", w.tcodes.data_ptr(), w.tscales.data_ptr(), w.n, w.k, x.data_ptr(),
             xdt, M, x.stride(0), out.data_ptr(), out.stride(0), int(epilogue), _stream())
    else:
        _dev(workspace, "workspace")
        call("sm_q4_matmul_ws", w.tcodes.data_ptr(), w.tscales.data_ptr(), w.n, w.k,
             x.data_ptr(), xdt, M, x.stride(0), out.data_ptr(), out.stride(0), int(epilogue),
             workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream())
    return out


class GemvBatch:
    """Independent one-row Q4 GEMVs launched together (sm_q4_gemv_multi).

    ``jobs``: (Q4Weight, x [K] or [1, K] f16 — [2K] f16 pairs with ``pair`` —,
    y [N] f32/bf16, epilogue). The plan (job table and block -> job table) is
    built once on the host and kept in device memory; ``launch()`` then runs
    every job in one kernel, as often as needed, while the tensors stay
    alive."""

    def __init__(self, jobs, *, pair: bool = False):
        import numpy as np
        n = len(jobs)
        host = (_lib.GemvJob * n)()
        kmax = 0
        self._keep = []  # the tensors the table points at
        for i, (w, x, y, epi) in enumerate(jobs):
            _dev(x, "x")
            _dev(y, "y")
            if w.tcodes is None:
                raise ValueError(f"Q4 GEMV needs K % 128 == 0 (K={w.k})")
            if x.numel() != (2 if pair else 1) * w.k or y.numel() != w.n:
                raise ValueError(f"job {i}: x / y sizes do not match the weight [{w.n}, {w.k}]")
            host[i] = _lib.GemvJob(w.tcodes.data_ptr(), w.tscales.data_ptr(), x.data_ptr(),
                                   y.data_ptr(), w.n, w.k, int(epi), 0)
            kmax = max(kmax, w.k)
            self._keep += [w, x, y]
        L = _lib.lib()
        total = L.sm_q4_gemv_multi_plan(C.byref(host), n, None)
        if total < 0:
            raise _lib.SummaError(L.sm_last_error().decode())
        table = np.empty(total, dtype=np.int32)
        L.sm_q4_gemv_multi_plan(C.byref(host), n, table.ctypes.data_as(C.c_void_p))
        dev = jobs[0][1].device
        raw = bytes(memoryview(host))
        self.jobs_dev = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(dev)
        self.table_dev = torch.from_numpy(table).to(dev)
        self.njobs, self.nblocks, self.max_k = n, int(total), kmax
        self.x_dtype = _lib.SM_F16X2 if pair else _lib.SM_F16
        self.weight_bytes = sum(w.nbytes for w, _, _, _ in jobs)

    def launch(self) -> None:
        call("sm_q4_gemv_multi", self.jobs_dev.data_ptr(), self.njobs, self.table_dev.data_ptr(),
             self.nblocks, self.max_k, self.x_dtype, _stream())


# ------------------------------------------------------------------ MoE ---

class ExpertBank:
    """Stacked Q4G128 expert weights W_e[N, K], e < E, resident in HBM.

    Counterpart of ``ExpertBank`` (summa-llm/src/model/ffn.rs:146-217, stacked
    ``[E, d, 2F]`` / ``[E, F, d]``) in this build's [out, in] Q4 layout: each
    expert is quantized as its own tensor and stored in the prepared tiled
    layout, expert e at a fixed stride."""

    def __init__(self, experts: list[Q4Weight]):
        if not experts:
            raise ValueError("an expert bank needs at least one expert")
        n, k = experts[0].n, experts[0].k
        if any(e.n != n or e.k != k for e in experts):
            raise ValueError("experts must share one shape")
        if experts[0].tcodes is None:
            raise ValueError(f"grouped Q4 matmul needs K % 128 == 0 (K={k})")
        self.n, self.k, self.experts = n, k, len(experts)
        self.tcodes = torch.stack([e.tcodes for e in experts]).contiguous()
        self.tscales = torch.stack([e.tscales for e in experts]).contiguous()

    @classmethod
    def quantize(cls, w: torch.Tensor) -> "ExpertBank":
        """Quantize dense device experts [E, N, K]."""
        return cls([Q4Weight.quantize(w[e].contiguous()) for e in range(w.shape[0])])


class RoutePlan:
    """Device route plan of ``route_plan`` (summa-llm/src/model/moe_route.rs:22,
    kernels :61-142): routes r = t*top_k + j sorted stably by expert. Views:
    counts [E], offsets [E+1], order [R] (route id at each sorted position),
    inverse [R] (sorted position of each route), src_rows [R] (token of each
    sorted position)."""

    def __init__(self, words: torch.Tensor, tokens: int, top_k: int, experts: int,
                 error: torch.Tensor):
        self.words, self.tokens, self.top_k, self.experts, self.error = (
            words, tokens, top_k, experts, error)
        R, E = tokens * top_k, experts
        o = [0]
        for n in (E, E + 1, R, R, R):
            o.append(o[-1] + n)
        self.counts, self.offsets, self.order, self.inverse, self.src_rows = (
            words[o[i]:o[i + 1]] for i in range(5))


def moe_top2_indices(h: torch.Tensor, router: torch.Tensor, *, want_logits: bool = False,
                     pair: bool = False):
    """Router logits (fp32 h . W_r^T, ffn.rs:489-490), strict top-2 with the
    first index winning ties (moe_topk.rs:74-104) and the softmax over the
    selected pair (ffn.rs:514). h [T, d] f32/f16 (or f16 pairs [T, 2d] with
    ``pair``), router [E, d] f32.
    Returns (top_idx [T, 2] int32, top_w [T, 2] f32, logits [T, E] or None)."""
    _dev(h, "h")
    _dev(router, "router")
    T, d = h.shape
    if pair:
        d //= 2
    E = router.shape[0]
    if router.dtype != torch.float32 or router.shape[1] != d:
        raise ValueError("router must be f32 [experts, d]")
    idx = torch.empty((T, 2), dtype=torch.int32, device=h.device)
    wts = torch.empty((T, 2), dtype=torch.float32, device=h.device)
    logits = torch.empty((T, E), dtype=torch.float32, device=h.device) if want_logits else None
    call("sm_moe_router_top2", h.data_ptr(), _lib.SM_F16X2 if pair else _dt(h),
         router.data_ptr(), T, d, E, _p(logits),
         idx.data_ptr(), wts.data_ptr(), _stream())
    return idx, wts, logits


def moe_route_plan(top_idx: torch.Tensor, experts: int) -> RoutePlan:
    """Stable expert-major route plan of top_idx [T, k] (moe_route.rs:22)."""
    _dev(top_idx, "top_idx")
    if top_idx.dtype != torch.int32:
        raise TypeError("top_idx must be int32")
    T, k = top_idx.shape
    words = torch.empty(int(_lib.lib().sm_moe_plan_words(T, k, experts)), dtype=torch.int32,
                        device=top_idx.device)
    error = torch.zeros(1, dtype=torch.int32, device=top_idx.device)
    call("sm_moe_route_plan", top_idx.data_ptr(), T, k, experts, words.data_ptr(),
         error.data_ptr(), _stream())
    return RoutePlan(words, T, k, experts, error)


def moe_route_plan_logits(logits: torch.Tensor) -> tuple:
    """Top-2 routing from router logits [T, E] and its stable route plan in one
    launch (``sm_moe_route_plan_logits``; moe_topk.rs:36-104 + moe_route.rs:22).
    Returns (top_idx [T, 2] int32, top_w [T, 2] f32, RoutePlan)."""
    _dev(logits, "logits")
    if logits.dtype != torch.float32:
        raise TypeError("logits must be float32")
    T, E = logits.shape
    idx = torch.empty((T, 2), dtype=torch.int32, device=logits.device)
    wts = torch.empty((T, 2), dtype=torch.float32, device=logits.device)
    words = torch.empty(int(_lib.lib().sm_moe_plan_words(T, 2, E)), dtype=torch.int32,
                        device=logits.device)
    error = torch.zeros(1, dtype=torch.int32, device=logits.device)
    call("sm_moe_route_plan_logits", logits.data_ptr(), T, E, idx.data_ptr(), wts.data_ptr(),
         words.data_ptr(), error.data_ptr(), _stream())
    return idx, wts, RoutePlan(words, T, 2, E, error)


def grouped_q4_matmul(bank: ExpertBank, x: torch.Tensor, plan: RoutePlan, *, gather: bool,
                      epilogue: int = _lib.SM_EPI_STORE_F32, pair: bool = False) -> torch.Tensor:
    """Per-expert y[p] = x[row(p)] . W_e^T over the plan's sorted positions p
    (grouped_linear.rs:65 / forward_grouped_swiglu ffn.rs:321). With ``gather``
    row(p) = src_rows[p] (the token; route_gather folded in), else row(p) = p."""
    _dev(x, "x")
    xdt = _x_dtype(x, pair)
    width = x.shape[1] // 2 if pair else x.shape[1]
    if width != bank.k:
        raise ValueError(f"grouped linear input width mismatch ({width} != {bank.k})")
    R = plan.tokens * plan.top_k
    shape, dt = _out_spec(epilogue, R, bank.n)
    out = torch.empty(shape, dtype=dt, device=x.device)
    call("sm_q4_grouped_matmul", bank.tcodes.data_ptr(), bank.tscales.data_ptr(), bank.experts,
         bank.n, bank.k, x.data_ptr(), xdt, x.stride(0), int(gather), plan.words.data_ptr(),
         plan.tokens, plan.top_k, out.data_ptr(), out.stride(0), int(epilogue), _stream())
    return out


def moe_route_combine(routed: torch.Tensor, top_w: torch.Tensor, plan: RoutePlan,
                      x: torch.Tensor) -> torch.Tensor:
    """x[t] += sum_j top_w[t, j] * routed[inverse[t*k + j]] in f32
    (route_combine_forward, moe_dispatch.rs:290-312), in place on x."""
    for t, n in ((routed, "routed"), (top_w, "top_w"), (x, "x")):
        _dev(t, n)
        if t.dtype != torch.float32:
            raise TypeError(f"{n} must be float32")
    call("sm_moe_combine", routed.data_ptr(), top_w.data_ptr(), plan.words.data_ptr(),
         plan.tokens, plan.top_k, plan.experts, x.shape[1], x.data_ptr(), _stream())
    return x


# ------------------------------------------------------ MoE training kernels --

def _f32_or_bf16(t: torch.Tensor, name: str) -> int:
    _dev(t, name)
    if t.dtype == torch.float32:
        return _lib.SM_F32
    if t.dtype == torch.bfloat16:
        return _lib.SM_BF16
    raise TypeError(f"{name} must be float32 or bfloat16")


def moe_gather(x: torch.Tensor, plan: RoutePlan) -> torch.Tensor:
    """routed[p] = x[order[p] // k] (route_gather_forward, moe_dispatch.rs:244-264)."""
    dt = _f32_or_bf16(x, "x")
    x = x.contiguous()
    out = torch.empty(plan.tokens * plan.top_k, x.shape[1], dtype=x.dtype, device=x.device)
    call("sm_moe_gather", x.data_ptr(), dt, plan.words.data_ptr(), plan.tokens, plan.top_k,
         plan.experts, x.shape[1], out.data_ptr(), _stream())
    return out


def moe_gather_backward(grad_routed: torch.Tensor, plan: RoutePlan) -> torch.Tensor:
    """grad_x[t] = sum_j grad_routed[inverse[t*k + j]] (route_gather_backward, :266-286)."""
    dt = _f32_or_bf16(grad_routed, "grad_routed")
    g = grad_routed.contiguous()
    out = torch.empty(plan.tokens, g.shape[1], dtype=g.dtype, device=g.device)
    call("sm_moe_gather_backward", g.data_ptr(), dt, plan.words.data_ptr(), plan.tokens,
         plan.top_k, plan.experts, g.shape[1], out.data_ptr(), _stream())
    return out


def moe_combine_backward(grad_x: torch.Tensor, routed: torch.Tensor, top_w: torch.Tensor,
                         plan: RoutePlan):
    """(grad_routed, grad_w) of x += sum_j w[t,j] routed[inverse[t*k+j]]
    (route_combine_routed_backward / route_combine_weight_backward, :314-384)."""
    dt = _f32_or_bf16(grad_x, "grad_x")
    if routed.dtype != grad_x.dtype or top_w.dtype != torch.float32:
        raise TypeError("routed must match grad_x; top_w must be float32")
    g, r, w = grad_x.contiguous(), routed.contiguous(), top_w.contiguous()
    gr = torch.zeros_like(r)
    gw = torch.empty(plan.tokens, plan.top_k, dtype=torch.float32, device=g.device)
    call("sm_moe_combine_backward", g.data_ptr(), r.data_ptr(), dt, w.data_ptr(),
         plan.words.data_ptr(), plan.tokens, plan.top_k, plan.experts, g.shape[1], gr.data_ptr(),
         gw.data_ptr(), _stream())
    return gr, gw


def swiglu(gate_value: torch.Tensor) -> torch.Tensor:
    """silu(gate) * value over [gate | value] rows (swiglu_forward, fused_swiglu.rs:106-124)."""
    dt = _f32_or_bf16(gate_value, "gate_value")
    gv = gate_value.contiguous()
    F = gv.shape[1] // 2
    out = torch.empty(gv.shape[0], F, dtype=gv.dtype, device=gv.device)
    call("sm_swiglu", gv.data_ptr(), dt, gv.shape[0], F, out.data_ptr(), _stream())
    return out


def swiglu_backward(gate_value: torch.Tensor, grad: torch.Tensor) -> torch.Tensor:
    """d[gate | value] of swiglu (swiglu_backward, fused_swiglu.rs:126-150)."""
    dt = _f32_or_bf16(gate_value, "gate_value")
    gv, g = gate_value.contiguous(), grad.contiguous()
    out = torch.empty_like(gv)
    call("sm_swiglu_backward", gv.data_ptr(), g.data_ptr(), dt, gv.shape[0], gv.shape[1] // 2,
         out.data_ptr(), _stream())
    return out


# ------------------------------------- float-weight grouped experts, permute --

def _host_counts(counts, experts: int, routes: int):
    import numpy as np
    c = np.ascontiguousarray([int(x) for x in counts], dtype=np.int64)
    if c.shape != (experts,):
        raise ValueError("one route count is required per expert")
    if int(c.sum()) != routes:
        raise ValueError("route counts must cover the input")
    return c


def _f32_dev(t: torch.Tensor, name: str) -> torch.Tensor:
    _dev(t, name)
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32")
    return t.contiguous()


def grouped_linear(input: torch.Tensor, weight: torch.Tensor, counts) -> torch.Tensor:
    """GroupedLinearBackend::grouped_linear_inner (grouped_linear.rs:23-28,
    65-86): input [routes, d_in] with counts[e] consecutive rows per expert,
    weight [E, d_in, d_out] -> [routes, d_out] (sm_grouped_linear)."""
    x, w = _f32_dev(input, "input"), _f32_dev(weight, "weight")
    R, din = x.shape
    E, wdin, dout = w.shape
    if wdin != din:
        raise ValueError("grouped linear input width mismatch")
    c = _host_counts(counts, E, R)
    out = torch.empty(R, dout, dtype=torch.float32, device=x.device)
    call("sm_grouped_linear", x.data_ptr(), w.data_ptr(), c.ctypes.data, E, R, din, dout,
         out.data_ptr(), _stream())
    return out


def grouped_linear_backward(input: torch.Tensor, weight: torch.Tensor, grad: torch.Tensor,
                            counts) -> tuple:
    """grouped_linear_backward (grouped_linear.rs:30-37): (grad_input,
    grad_weight), zero weight gradient for an expert without rows."""
    x, w, g = _f32_dev(input, "input"), _f32_dev(weight, "weight"), _f32_dev(grad, "grad")
    R, din = x.shape
    E, _, dout = w.shape
    c = _host_counts(counts, E, R)
    gx, gw = torch.empty_like(x), torch.empty_like(w)
    call("sm_grouped_linear_backward", x.data_ptr(), w.data_ptr(), g.data_ptr(), c.ctypes.data,
         E, R, din, dout, gx.data_ptr(), gw.data_ptr(), _stream())
    return gx, gw


def grouped_swiglu_mlp(input: torch.Tensor, in_weight: torch.Tensor, down_weight: torch.Tensor,
                       counts, intermediate: int) -> tuple:
    """grouped_swiglu_mlp_inner (grouped_linear.rs:40-49, 779-799):
    (output [routes, d_out], projected [routes, 2I] as [gate | value],
    hidden [routes, I])."""
    x = _f32_dev(input, "input")
    wi, wd = _f32_dev(in_weight, "in_weight"), _f32_dev(down_weight, "down_weight")
    R, d = x.shape
    E, _, two_i = wi.shape
    if two_i != 2 * intermediate or wd.shape[1] != intermediate or wd.shape[0] != E:
        raise ValueError("grouped SwiGLU MLP weight shapes do not match the intermediate width")
    dout = wd.shape[2]
    c = _host_counts(counts, E, R)
    out = torch.empty(R, dout, dtype=torch.float32, device=x.device)
    proj = torch.empty(R, 2 * intermediate, dtype=torch.float32, device=x.device)
    hid = torch.empty(R, intermediate, dtype=torch.float32, device=x.device)
    call("sm_grouped_swiglu_mlp", x.data_ptr(), wi.data_ptr(), wd.data_ptr(), c.ctypes.data, E, R,
         d, intermediate, dout, out.data_ptr(), proj.data_ptr(), hid.data_ptr(), _stream())
    return out, proj, hid


def grouped_swiglu_mlp_backward(input, in_weight, down_weight, counts, projected, hidden, grad,
                                intermediate: int) -> tuple:
    """grouped_swiglu_mlp_backward (grouped_linear.rs:50-60, 801-826):
    (grad_input, grad_in_weight, grad_down_weight)."""
    x = _f32_dev(input, "input")
    wi, wd = _f32_dev(in_weight, "in_weight"), _f32_dev(down_weight, "down_weight")
    p, h, g = _f32_dev(projected, "projected"), _f32_dev(hidden, "hidden"), _f32_dev(grad, "grad")
    R, d = x.shape
    E = wi.shape[0]
    dout = wd.shape[2]
    c = _host_counts(counts, E, R)
    gx, gwi, gwd = torch.empty_like(x), torch.empty_like(wi), torch.empty_like(wd)
    scratch = torch.empty(max(R, 1) * 3 * intermediate, dtype=torch.float32, device=x.device)
    call("sm_grouped_swiglu_mlp_backward", x.data_ptr(), wi.data_ptr(), wd.data_ptr(),
         c.ctypes.data, E, R, d, intermediate, dout, p.data_ptr(), h.data_ptr(), g.data_ptr(),
         gx.data_ptr(), gwi.data_ptr(), gwd.data_ptr(), scratch.data_ptr(), _stream())
    return gx, gwi, gwd


def row_permute(input: torch.Tensor, order: torch.Tensor, inverse: torch.Tensor | None = None
                ) -> torch.Tensor:
    """RowPermutationBackend::row_permute_inner (row_permute.rs:33-41):
    out[i] = input[order[i]] over the rows (bits copied); ``inverse`` is the
    backward's order (accepted for the trait's signature, unused here)."""
    _dev(input, "input")
    _dev(order, "order")
    dt = {torch.float32: SM_F32, torch.bfloat16: SM_BF16, torch.float16: SM_F16}.get(input.dtype)
    if dt is None:
        raise TypeError("input must be float32, bfloat16 or float16")
    if input.dim() != 2 or order.dtype != torch.int32 or order.shape != (input.shape[0],):
        raise ValueError("row_permute takes [rows, cols] input and int32 order [rows]")
    x, o = input.contiguous(), order.contiguous()
    out = torch.empty_like(x)
    call("sm_row_permute", x.data_ptr(), dt, x.shape[0], x.shape[1], o.data_ptr(), out.data_ptr(),
         _stream())
    return out


# ------------------------------------------------------------- attention ---

def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = True,
              want_lse: bool = False):
    """AttentionBackend::attention_inner (fused_attention.rs:37-55) in the
    reference's layout: q [B, H, S, hd], k / v [B, KVH, S, hd] (KVH divides H)
    of one dtype (f32, bf16 or f16) -> out [B, H, S, hd] (and lse [B*H, S] f32)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _dev(t, n)
    B, H, S, hd = q.shape
    KVH = k.shape[1]
    if k.shape != (B, KVH, S, hd) or v.shape != k.shape or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("attention: k and v must be [B, KVH, S, hd] in q's dtype")
    out = torch.empty_like(q)
    lse = torch.empty(B * H, S, dtype=torch.float32, device=q.device) if want_lse else None
    call("sm_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), _dt(q), B, H, KVH, S, hd,
         int(causal), out.data_ptr(), _p(lse), _stream())
    return (out, lse) if want_lse else out


def attention_backward(q, k, v, out, grad_out, lse, causal: bool = True):
    """AttentionBackend::attention_backward (fused_attention.rs:57-68), f32:
    (dq [B, H, S, hd], dk [B, KVH, S, hd], dv [B, KVH, S, hd])."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (out, "out"), (grad_out, "grad_out"), (lse, "lse")):
        _dev(t, n)
    B, H, S, hd = q.shape
    KVH = k.shape[1]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    delta = torch.empty(B * H * S, dtype=torch.float32, device=q.device)
    call("sm_attention_backward", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
         grad_out.data_ptr(), lse.data_ptr(), B, H, KVH, S, hd, int(causal), dq.data_ptr(),
         dk.data_ptr(), dv.data_ptr(), delta.data_ptr(), _stream())
    return dq, dk, dv
