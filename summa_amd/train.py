"""GRPO policy update for fp32 models on the device (host composition).

The reference trains with Burn's autodiff: ``prepare_device_batch`` recomputes
the policy's token log-probs, ``grpo_loss_tensor`` gives the loss, its
backward reaches every parameter, and ``optimizer_step`` applies Muon to the
2-D matrices and AdamW to the rest (summa-train/src/posttrain.rs:874-1028,
1288-1305; trainer.rs:1974-1975; muon.rs:196-285). Here the recompute forward
keeps its activations, and the backward is spelled out layer by layer over the
library's kernels: the fused CE gradient (``sm_ce_rows``), ``sm_gemm_ex`` for
data and weight gradients, ``sm_rmsnorm_backward``, ``sm_rope_qk``,
``sm_attn_backward_f32``, ``sm_swiglu_backward``, ``sm_embed_backward``; the
optimizers are ``sm_adamw_step`` and Muon's momentum / Newton-Schulz over
``sm_gemm_ex``. Weights are f32 master copies in the model's [out, in] rows;
``to_model`` installs them into an inference ``Model``.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import ops
from ._lib import SM_F32, call
from .model import Model, ModelConfig

LAYER_KEYS = ("attn_norm", "qkv", "o", "ffn_norm", "in", "down")
# per-layer tensors of an MoE policy (stacked experts, the f32 router)
MOE_LAYER_KEYS = ("router", "exp_in", "exp_down")
MUON_MOMENTUM = 0.95                       # muon.rs:10
NS_COEFFICIENTS = (3.4445, -4.775, 2.0315)  # muon.rs:11
NS_STEPS = 5                               # muon.rs:12
MUON_EPSILON = 1e-7                        # muon.rs:13


def _st() -> int:
    return torch.cuda.current_stream().cuda_stream


def gemm(a, b, *, ta=False, tb=False, out=None, alpha=1.0, beta=0.0, entry="sm_gemm_ex"):
    """out = alpha op(a) op(b) + beta out (sm_gemm_ex, or ``entry`` =
    "sm_gemm_mfma" for the matrix-core kernel at any size), f32 2-D tensors."""
    M = a.shape[1] if ta else a.shape[0]
    K = a.shape[0] if ta else a.shape[1]
    N = b.shape[0] if tb else b.shape[1]
    if (b.shape[1] if tb else b.shape[0]) != K:
        raise ValueError(f"gemm: inner dimensions {K} and {b.shape} differ")
    if out is None:
        out = torch.empty(M, N, dtype=torch.float32, device=a.device)
        beta = 0.0
    call(entry, int(ta), int(tb), M, N, K, float(alpha), a.data_ptr(), a.stride(0),
         b.data_ptr(), b.stride(0), float(beta), out.data_ptr(), out.stride(0), _st())
    return out


def rope_table(cfg: ModelConfig, device) -> torch.Tensor:
    """(cos, sin) per (position, pair) as the model builds it (model.hip)."""
    half = cfg.head_dim // 2
    freq = np.power(float(cfg.rope_theta), -2.0 * np.arange(half) / cfg.head_dim)
    ang = np.arange(cfg.max_seq)[:, None] * freq[None, :]
    tab = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    return torch.from_numpy(tab).to(device)


class Fp32Policy:
    """f32 master weights + the recompute forward / backward of a decoder."""

    def __init__(self, cfg: ModelConfig, weights: dict, device):
        if cfg.quantized or cfg.experts:
            raise ValueError("Fp32Policy trains dense fp32 decoders")
        if cfg.head_dim not in (64, 128):
            raise ValueError("head_dim must be 64 or 128")
        self.cfg, self.dev = cfg, device
        self.p = {k: torch.as_tensor(np.ascontiguousarray(v, dtype=np.float32)).to(device)
                  for k, v in weights.items()}
        self.rope = rope_table(cfg, device)
        self._adam, self._muon_v, self._step = {}, {}, 0

    # ------------------------------------------------------------- forward --
    def _rmsnorm(self, x, g):
        y = torch.empty_like(x)
        call("sm_rmsnorm", x.data_ptr(), g.data_ptr(), x.shape[0], x.shape[1],
             float(self.cfg.norm_eps), y.data_ptr(), SM_F32, _st())
        return y

    def forward(self, prompts: torch.Tensor, tokens: torch.Tensor):
        """lp [S, N] of tokens[:, n] given prompt + tokens[:, :n] (the recompute
        of sm_rl_logprobs), keeping what the backward needs."""
        c = self.cfg
        S, P = prompts.shape
        N = tokens.shape[1]
        L = P + N - 1
        if L > c.max_seq:
            raise ValueError(f"sequence length {L} exceeds max_seq_len {c.max_seq}")
        ids = torch.cat([prompts, tokens[:, :N - 1]], 1).contiguous()
        M, d, H, KVH, hd = S * L, c.d_model, c.heads, c.kv_heads, c.head_dim
        x = torch.empty(M, d, device=self.dev)
        call("sm_embed", self.p["embed"].data_ptr(), SM_F32, ids.data_ptr(), M, d, c.vocab, 1.0,
             x.data_ptr(), _st())
        pos0 = torch.zeros(S, dtype=torch.int32, device=self.dev)
        saved = []
        for i in range(c.layers):
            W = {k: self.p[k][i] for k in LAYER_KEYS}
            x0 = x
            h = self._rmsnorm(x0, W["attn_norm"])
            qkv = gemm(h, W["qkv"], tb=True)
            call("sm_rope_qk", qkv.data_ptr(), self.rope.data_ptr(), pos0.data_ptr(), S, L, H, KVH,
                 hd, 0, _st())
            q = qkv[:, :H * hd].contiguous()
            k = qkv[:, H * hd:(H + KVH) * hd].reshape(S, L, KVH, hd).permute(0, 2, 1, 3).contiguous()
            v = qkv[:, (H + KVH) * hd:].reshape(S, L, KVH, hd).permute(0, 2, 1, 3).contiguous()
            o = torch.empty(M, H * hd, device=self.dev)
            lse = torch.empty(S * H, L, device=self.dev)
            call("sm_attn_prefill_lse", q.data_ptr(), k.data_ptr(), v.data_ptr(), pos0.data_ptr(),
                 o.data_ptr(), lse.data_ptr(), SM_F32, SM_F32, S, L, H, KVH, L, hd, _st())
            x1 = gemm(o, W["o"], tb=True, out=x0.clone(), beta=1.0)
            h2 = self._rmsnorm(x1, W["ffn_norm"])
            u = gemm(h2, W["in"], tb=True)
            a = ops.swiglu(u)
            x = gemm(a, W["down"], tb=True, out=x1.clone(), beta=1.0)
            saved.append(dict(x0=x0, h=h, qkv=qkv, q=q, k=k, v=v, o=o, lse=lse, x1=x1, h2=h2, u=u,
                              a=a))
        hf = self._rmsnorm(x, self.p["final_norm"])
        rows = (torch.arange(S, device=self.dev)[:, None] * L + (P - 1) +
                torch.arange(N, device=self.dev)[None, :]).reshape(-1)
        hr = hf[rows].contiguous()
        logits = gemm(hr, self.p["lm_head"], tb=True)
        tgt = tokens.reshape(-1).contiguous()
        lp, _, _ = ops.ce_rows(logits, tgt, want_loss=False)
        self._fw = dict(S=S, P=P, N=N, L=L, ids=ids, saved=saved, x=x, hf=hf, rows=rows, hr=hr,
                        logits=logits, tgt=tgt, pos0=pos0)
        return lp.view(S, N)

    # ------------------------------------------------------------ backward --
    def backward(self, dlp: torch.Tensor) -> dict:
        """Gradients of sum(dlp * lp) with respect to every weight."""
        fw, c = self._fw, self.cfg
        S, L, N = fw["S"], fw["L"], fw["N"]
        M, d, H, KVH, hd = S * L, c.d_model, c.heads, c.kv_heads, c.head_dim
        g = {k: torch.zeros_like(v) for k, v in self.p.items()}
        # d lp / d logits = onehot - softmax: the CE gradient scaled by -dlp per row
        dlog = fw["logits"]
        ops.ce_rows(dlog, fw["tgt"], grad_in_place=True, grad_scale=-1.0,
                    row_scale=dlp.reshape(-1).contiguous().float(), want_loss=False)
        gemm(dlog, fw["hr"], ta=True, out=g["lm_head"])
        dhr = gemm(dlog, self.p["lm_head"])
        dhf = torch.zeros(M, d, device=self.dev)
        dhf[fw["rows"]] = dhr
        dx = torch.empty(M, d, device=self.dev)
        rinv = torch.empty(M, device=self.dev)
        call("sm_rmsnorm_backward", fw["x"].data_ptr(), self.p["final_norm"].data_ptr(),
             dhf.data_ptr(), M, d, float(c.norm_eps), 0, dx.data_ptr(), g["final_norm"].data_ptr(),
             rinv.data_ptr(), _st())
        delta = torch.empty(S * H * L, device=self.dev)
        for i in reversed(range(c.layers)):
            s = fw["saved"][i]
            W = {k: self.p[k][i] for k in LAYER_KEYS}
            # FFN: x = x1 + swiglu(h2 W_in^T) W_down^T
            da = gemm(dx, W["down"])
            gemm(dx, s["a"], ta=True, out=g["down"][i])
            du = ops.swiglu_backward(s["u"], da)
            gemm(du, s["h2"], ta=True, out=g["in"][i])
            dh2 = gemm(du, W["in"])
            call("sm_rmsnorm_backward", s["x1"].data_ptr(), W["ffn_norm"].data_ptr(), dh2.data_ptr(),
                 M, d, float(c.norm_eps), 1, dx.data_ptr(), g["ffn_norm"][i].data_ptr(),
                 rinv.data_ptr(), _st())
            # attention: x1 = x0 + attn(rope(h W_qkv^T)) W_o^T
            do = gemm(dx, W["o"])
            gemm(dx, s["o"], ta=True, out=g["o"][i])
            dq = torch.empty(M, H * hd, device=self.dev)
            dk = torch.empty(S, KVH, L, hd, device=self.dev)
            dv = torch.empty(S, KVH, L, hd, device=self.dev)
            call("sm_attn_backward_f32", s["q"].data_ptr(), s["k"].data_ptr(), s["v"].data_ptr(),
                 s["o"].data_ptr(), do.data_ptr(), s["lse"].data_ptr(), S, L, H, KVH, hd,
                 dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr(), _st())
            dqkv = torch.cat([dq, dk.permute(0, 2, 1, 3).reshape(M, KVH * hd),
                              dv.permute(0, 2, 1, 3).reshape(M, KVH * hd)], 1).contiguous()
            call("sm_rope_qk", dqkv.data_ptr(), self.rope.data_ptr(), fw["pos0"].data_ptr(), S, L,
                 H, KVH, hd, 1, _st())
            gemm(dqkv, s["h"], ta=True, out=g["qkv"][i])
            dh = gemm(dqkv, W["qkv"])
            call("sm_rmsnorm_backward", s["x0"].data_ptr(), W["attn_norm"].data_ptr(), dh.data_ptr(),
                 M, d, float(c.norm_eps), 1, dx.data_ptr(), g["attn_norm"][i].data_ptr(),
                 rinv.data_ptr(), _st())
        call("sm_embed_backward", fw["ids"].data_ptr(), dx.data_ptr(), M, d, c.vocab,
             g["embed"].data_ptr(), _st())
        return g

    # ---------------------------------------------------------- optimizers --
    def muon_keys(self):
        """2-D matrices (per layer) go to Muon, the rest to AdamW (trainer.rs:1974)."""
        return ("qkv", "o", "in", "down")

    def adamw_step(self, grads: dict, keys, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, wd=0.1):
        """AdamW with the trainer's settings: beta1 0.9, beta2 0.95, eps 1e-8
        (summa-train/src/trainer.rs:1124-1129), lr 3e-4 and weight decay 0.1
        (the CLI defaults, summa-train/src/main.rs:171-174)."""
        self._step += 1
        for k in keys:
            p, gr = self.p[k], grads[k].contiguous()
            if k not in self._adam:
                self._adam[k] = (torch.zeros_like(p), torch.zeros_like(p))
            m, v = self._adam[k]
            call("sm_adamw_step", p.data_ptr(), gr.data_ptr(), m.data_ptr(), v.data_ptr(),
                 p.numel(), float(lr), float(betas[0]), float(betas[1]), float(eps), float(wd),
                 self._step, _st())

    def muon_step(self, grads: dict, keys, lr=0.02):
        """BatchedMuon::step (muon.rs:196-215) with Newton-Schulz in f32 (the
        reference's CPU path; its CUDA path runs the iteration in bf16)."""
        for k in keys:
            for i in range(self.p[k].shape[0]):
                p, gr = self.p[k][i], grads[k][i].contiguous()
                key = (k, i)
                first = key not in self._muon_v
                if first:
                    self._muon_v[key] = torch.zeros_like(p)
                upd = torch.empty_like(p)
                call("sm_muon_momentum", gr.data_ptr(), self._muon_v[key].data_ptr(),
                     upd.data_ptr(), p.numel(), MUON_MOMENTUM, int(first), _st())
                orth = newton_schulz(upd)
                # Burn Linear weights are [d_in, d_out]: scale by that shape
                rows, cols = p.shape[1], p.shape[0]
                adj = lr * max(1.0, rows / cols) ** 0.5
                call("sm_axpby", orth.data_ptr(), p.data_ptr(), p.numel(), -float(adj), 1.0, _st())

    def to_model(self, model: Model) -> None:
        for k, v in self.p.items():
            if k in LAYER_KEYS:
                for i in range(self.cfg.layers):
                    model.set_tensor(k, v[i], i)
            else:
                model.set_tensor(k, v)
        torch.cuda.synchronize()


def newton_schulz(g: torch.Tensor) -> torch.Tensor:
    """zeropower_via_newton_schulz (muon.rs:257-285) of one matrix, in the
    orientation the reference sees it (Burn [d_in, d_out] = this [out, in]^T):
    the short side first, Frobenius-normalised, five quintic steps."""
    x = g.t().contiguous()  # Burn orientation
    transpose = x.shape[0] > x.shape[1]
    if transpose:
        x = x.t().contiguous()
    norm = torch.empty(1, device=x.device)
    call("sm_frobenius_normalize", x.data_ptr(), x.numel(), MUON_EPSILON, norm.data_ptr(), _st())
    a, b, c = NS_COEFFICIENTS
    for _ in range(NS_STEPS):
        gram = gemm(x, x, tb=True)
        poly = gemm(gram, gram, alpha=c)
        call("sm_axpby", gram.data_ptr(), poly.data_ptr(), poly.numel(), float(b), 1.0, _st())
        x = gemm(poly, x, out=x.clone(), beta=a)
    if transpose:
        x = x.t().contiguous()
    return x.t().contiguous()  # back to [out, in]


# ------------------------------------------------------- native policy ---

class OptimizerConfigC(C.Structure):
    _fields_ = [(n, C.c_float) for n in ("lr", "beta1", "beta2", "eps", "weight_decay",
                                         "muon_lr", "grad_clip")]


_POLICY_KINDS = {"embed": 0, "attn_norm": 1, "qkv": 2, "o": 3, "ffn_norm": 4, "in": 5,
                 "down": 6, "final_norm": 7, "lm_head": 8, "router": 9, "exp_in": 10,
                 "exp_down": 11}


class Policy:
    """The library's trainable policy (``sm_policy``): prepare_device_batch's
    recompute, GRPO loss and staged backward in one call, optimizer_step in
    another (posttrain.rs:1288-1305), with the trainer's optimizer settings as
    defaults (AdamW 3e-4 / 0.9 / 0.95 / 1e-8 / wd 0.1, global-norm clip 1.0: the
    CLI defaults of summa-train/src/main.rs:171-176 and trainer.rs:1124-1129;
    ``muon_lr > 0`` adds Muon for the per-layer projections).
    ``matmul_planes``: bf16 planes per GEMM operand in ``prepare``
    (sm_policy_set_matmul_planes): 3 f32-grade, 2 16-bit operands, 1 bf16
    operands with f32 accumulation (the reference's CUDA-path matmul)."""

    def __init__(self, cfg: ModelConfig, weights: dict, device, lr=3e-4, betas=(0.9, 0.95),
                 eps=1e-8, weight_decay=0.1, muon_lr=0.0, grad_clip=1.0, matmul_planes=3):
        from . import _lib
        self.cfg, self.dev = cfg, device
        self._h = C.c_void_p()
        oc = OptimizerConfigC(lr, betas[0], betas[1], eps, weight_decay, muon_lr, grad_clip)
        cc = cfg.c()
        _lib.check(_lib.lib().sm_policy_create(C.byref(cc), C.byref(oc), C.byref(self._h)))
        if matmul_planes != 3:
            self.set_matmul_planes(matmul_planes)
        for name, arr in weights.items():
            if isinstance(arr, torch.Tensor):  # host or device tensors
                t = arr.to(device=device, dtype=torch.float32).contiguous()
            else:
                t = torch.as_tensor(np.ascontiguousarray(arr, dtype=np.float32)).to(device)
            if name in LAYER_KEYS or name in MOE_LAYER_KEYS:
                for i in range(cfg.layers):
                    call("sm_policy_set_tensor", self._h, _POLICY_KINDS[name], i,
                         t[i].contiguous().data_ptr(), _st())
            else:
                call("sm_policy_set_tensor", self._h, _POLICY_KINDS[name], -1, t.data_ptr(),
                     _st())
        torch.cuda.synchronize()

    def set_matmul_planes(self, planes: int) -> None:
        """bf16 planes per operand of the prepare's GEMMs (1, 2 or 3)."""
        call("sm_policy_set_matmul_planes", self._h, int(planes))

    def close(self):
        if self._h.value:
            from . import _lib
            _lib.lib().sm_policy_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor(self, name: str, layer: int = -1, gradient: bool = False) -> torch.Tensor:
        """A master weight (or its staged gradient), [out, in] rows."""
        c = self.cfg
        d, F, qn = c.d_model, c.ffn, (c.heads + 2 * c.kv_heads) * c.head_dim
        E, Fe = c.experts, c.expert_ffn
        shape = {"embed": (c.vocab, d), "lm_head": (c.vocab, d), "attn_norm": (d,),
                 "ffn_norm": (d,), "final_norm": (d,), "qkv": (qn, d),
                 "o": (d, c.heads * c.head_dim), "in": (2 * F, d), "down": (d, F),
                 "router": (E, d), "exp_in": (E, 2 * Fe, d), "exp_down": (E, d, Fe)}[name]
        out = torch.empty(shape, dtype=torch.float32, device=self.dev)
        call("sm_policy_get_tensor", self._h, _POLICY_KINDS[name], layer, out.data_ptr(),
             int(gradient), _st())
        return out

    def prepare(self, reference, prompts, tokens, behavior_lp, rewards, mask=None,
                clip_epsilon=0.2, advantage_epsilon=1e-6, kl_coefficient=0.04,
                reference_lp=None):
        """sm_policy_prepare: like ``model.rl_prepare`` for the trainable
        policy; the gradient of the loss is added to the staged gradients.
        With ``reference`` None and ``reference_lp`` given ([S, N] f32, the
        frozen model's log-probs over the same tokens, e.g. the step's
        ``rl_prepare`` output) it runs sm_policy_prepare_with_ref, which does
        not run the frozen model again."""
        groups, G = rewards.shape
        S, P = prompts.shape
        N = tokens.shape[1]
        dev = prompts.device
        lp_cur = torch.empty(S, N, dtype=torch.float32, device=dev)
        stats = torch.empty(groups, 5, dtype=torch.float32, device=dev)
        dlp = torch.empty(S, N, dtype=torch.float32, device=dev)
        flags = torch.empty(groups, dtype=torch.int32, device=dev)
        msk = None if mask is None else mask.data_ptr()
        if reference is None and reference_lp is not None:
            if reference_lp.shape != (S, N) or reference_lp.dtype != torch.float32:
                raise ValueError("reference_lp must be float32 [S, N]")
            ref = reference_lp.contiguous()
            call("sm_policy_prepare_with_ref", self._h, ref.data_ptr(), prompts.data_ptr(),
                 tokens.data_ptr(), behavior_lp.data_ptr(), rewards.data_ptr(), msk, groups, G,
                 P, N, float(clip_epsilon), float(advantage_epsilon), float(kl_coefficient),
                 lp_cur.data_ptr(), stats.data_ptr(), dlp.data_ptr(), flags.data_ptr(), _st())
            return {"lp_cur": lp_cur, "lp_ref": ref, "stats": stats, "dlp": dlp,
                    "flags": flags}
        lp_ref = (torch.empty(S, N, dtype=torch.float32, device=dev)
                  if reference is not None else None)
        call("sm_policy_prepare", self._h, reference.handle if reference is not None else None,
             prompts.data_ptr(), tokens.data_ptr(), behavior_lp.data_ptr(), rewards.data_ptr(),
             msk, groups, G, P, N, float(clip_epsilon),
             float(advantage_epsilon), float(kl_coefficient), lp_cur.data_ptr(),
             None if lp_ref is None else lp_ref.data_ptr(), stats.data_ptr(), dlp.data_ptr(),
             flags.data_ptr(), _st())
        return {"lp_cur": lp_cur, "lp_ref": lp_ref, "stats": stats, "dlp": dlp, "flags": flags}

    def optimizer_step(self, learning_rate_scale: float = 1.0) -> float:
        """sm_policy_optimizer_step; returns the pre-clip global gradient norm."""
        norm = C.c_float()
        call("sm_policy_optimizer_step", self._h, float(learning_rate_scale), C.byref(norm),
             _st())
        return norm.value

    def install(self, model: Model) -> None:
        call("sm_policy_install", self._h, model.handle, _st())
        torch.cuda.synchronize()
