"""CPU oracle bindings — TEST INFRASTRUCTURE ONLY.

Restates the reference's CPU path (see ``oracle.h`` for the file:line each
function follows). Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker. The product library ``summa_amd`` never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# SUMMA_ORACLE_LIB selects another build of the checker (the AddressSanitizer
# one, `make -C oracle asan`)
LIB_PATH = Path(os.environ.get("SUMMA_ORACLE_LIB", HERE / "liboracle.so"))

_lib = None

f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


def _declare(L: C.CDLL) -> None:
    vp, i64, d = C.c_void_p, C.c_int64, C.c_double
    L.or_ce_rows.argtypes = [vp, C.c_int, i32p, i64, i64, i64, vp, vp, vp, d, vp]
    L.or_ce_rows.restype = None
    L.or_grpo_loss.argtypes = [f64p, f64p, f64p, vp, vp, i64, i64, i64, d, d, d, f64p, f64p, f64p]
    L.or_grpo_loss.restype = C.c_int
    L.or_q4_quantize.argtypes = [f32p, i64, u8p, u16p]
    L.or_q4_decode.argtypes = [u8p, u16p, i64, f32p]
    L.or_q4_matvec.argtypes = [u8p, u16p, i64, i64, f32p, f32p]
    for name in ("or_q4_quantize", "or_q4_decode", "or_q4_matvec"):
        getattr(L, name).restype = None
    L.or_round_f16.argtypes = [C.c_float]
    L.or_round_f16.restype = C.c_float
    L.or_bf16_bits.argtypes = [vp, i64, vp]
    L.or_bf16_bits.restype = None
    L.or_set_threads.argtypes = [C.c_int]
    L.or_set_threads.restype = None
    L.or_max_threads.argtypes = []
    L.or_max_threads.restype = C.c_int
    _declare_model(L)


class OrModel(C.Structure):
    """Mirror of ``or_model`` in model.c (host weight pointers)."""
    _fields_ = [(n, C.c_int32) for n in ("layers", "d", "H", "KVH", "hd", "F", "V", "quantized",
                                         "acc64")] + \
        [("eps", C.c_float), ("theta", C.c_float)] + \
        [(n, C.c_void_p) for n in ("embed", "attn_norm", "ffn_norm", "final_norm",
                                   "qkv", "o", "in_", "down", "lm_head",
                                   "qkv_c", "o_c", "in_c", "down_c", "lm_c",
                                   "qkv_s", "o_s", "in_s", "down_s", "lm_s")] + \
        [("experts", C.c_int32), ("expert_ffn", C.c_int32)] + \
        [(n, C.c_void_p) for n in ("router", "exp_in", "exp_down", "exp_in_c", "exp_down_c",
                                   "exp_in_s", "exp_down_s", "router_gap", "route_hint")] + \
        [("hint_margin", C.c_float), ("hint_conflicts", C.c_void_p), ("kv_f32", C.c_int32)]


def _declare_model(L: C.CDLL) -> None:
    vp, i32, i64 = C.c_void_p, C.c_int, C.c_int64
    L.or_model_forward.argtypes = [C.POINTER(OrModel), vp, i32, i32, i32, vp, vp, i32, vp]
    L.or_model_logits.argtypes = [C.POINTER(OrModel), vp, i64, vp]
    L.or_sample.argtypes = [vp, i64, i64, C.c_float, C.c_uint64, i64, vp, i64, vp, i64]
    L.or_generate.argtypes = [C.POINTER(OrModel), vp, i32, i32, i32, C.c_float, C.c_uint64, vp, vp]
    L.or_logprobs.argtypes = [C.POINTER(OrModel), vp, vp, i32, i32, i32, vp]
    f32 = C.c_float
    L.or_apply_penalty.argtypes = [vp, i64, vp, i64, f32]
    L.or_apply_penalty.restype = i32
    L.or_sample_ex_row.argtypes = [vp, i64, f32, i32, f32, f32, i32, C.c_uint64, i64, i64, vp, i64,
                                   vp, vp]
    L.or_sample_ex_row.restype = i32
    L.or_generate_ex.argtypes = [C.POINTER(OrModel), vp, i32, i32, i32, f32, i32, f32, f32, i32,
                                 i32, C.c_uint64, vp, vp, vp]
    for n in ("or_model_forward", "or_model_logits", "or_sample", "or_generate", "or_logprobs",
              "or_generate_ex"):
        getattr(L, n).restype = None


def _ptr(a):
    return None if a is None else a.ctypes.data


# ---------------------------------------------------------------- helpers ---

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (NaN kept quiet):
    ``or_f32_to_bf16`` per element."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    r = np.empty(a.shape, np.uint16)
    lib().or_bf16_bits(a.ctypes.data, a.size, r.ctypes.data)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_to_f32(bf16_bits(x))


# --------------------------------------------------------------------- CE ---

def ce_rows(logits: np.ndarray, targets: np.ndarray, logical_vocab: int | None = None,
            grad: bool = False, grad_scale: float = 1.0, row_scale=None):
    """Row-wise log-softmax / CE in f64. ``logits`` float32 or uint16 (bf16 bits)."""
    rows, stored = logits.shape
    lv = stored if logical_vocab is None else logical_vocab
    dtype = 1 if logits.dtype == np.uint16 else 0
    lg = np.ascontiguousarray(logits)
    tg = np.ascontiguousarray(targets, dtype=np.int32)
    lp = np.empty(rows, np.float64)
    lse = np.empty(rows, np.float64)
    g = np.empty((rows, stored), np.float32) if grad else None
    rs = None if row_scale is None else np.ascontiguousarray(row_scale, dtype=np.float64)
    lib().or_ce_rows(lg.ctypes.data, dtype, tg, rows, stored, lv, lp.ctypes.data,
                     lse.ctypes.data, _ptr(g), grad_scale, _ptr(rs))
    return lp, lse, g


# ------------------------------------------------------------------- GRPO ---

class GrpoError(ValueError):
    pass


def grpo_loss(rewards, lp_cur, lp_beh, lp_ref=None, mask=None, clip=0.2, adv_eps=1e-6, beta=0.04):
    """Batched GRPO loss. Arrays: rewards [B, G]; log-probs / mask [B, G, T].

    Returns (stats [B, 5], advantages [B, G], dlp [B, G, T], error_flags)."""
    r = np.ascontiguousarray(rewards, dtype=np.float64)
    B, G = r.shape
    cur = np.ascontiguousarray(lp_cur, dtype=np.float64)
    T = cur.shape[-1]
    beh = np.ascontiguousarray(lp_beh, dtype=np.float64)
    ref = None if lp_ref is None else np.ascontiguousarray(lp_ref, dtype=np.float64)
    mk = None if mask is None else np.ascontiguousarray(mask, dtype=np.float64)
    stats = np.empty((B, 5), np.float64)
    adv = np.empty((B, G), np.float64)
    dlp = np.empty((B, G, T), np.float64)
    err = lib().or_grpo_loss(r, cur, beh, _ptr(ref), _ptr(mk), B, G, T, clip, adv_eps, beta,
                             stats, adv, dlp)
    return stats, adv, dlp, err


# ----------------------------------------------------------------- Q4G128 ---

def q4_quantize(w: np.ndarray):
    """Returns (codes uint8 [ceil(n/128)*64], scales uint16 [ceil(n/128)])."""
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    n = w.size
    groups = (n + 127) // 128
    codes = np.empty(groups * 64, np.uint8)
    scales = np.empty(groups, np.uint16)
    lib().or_q4_quantize(w, n, codes, scales)
    return codes, scales


def q4_decode(codes, scales, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().or_q4_decode(np.ascontiguousarray(codes), np.ascontiguousarray(scales), n, out)
    return out


def q4_matvec(codes, scales, rows: int, cols: int, x) -> np.ndarray:
    y = np.empty(rows, np.float32)
    lib().or_q4_matvec(np.ascontiguousarray(codes), np.ascontiguousarray(scales), rows, cols,
                       np.ascontiguousarray(x, dtype=np.float32), y)
    return y


# ------------------------------------------------------------------ model ---

class HostModel:
    """Host copy of a decoder's weights for the oracle.

    ``weights`` maps names to float32 arrays: embed [V, d], attn_norm / ffn_norm
    [layers, d], final_norm [d], and linears qkv / o / in / down [layers, N, K],
    lm_head [V, d] in [out, in] layout; MoE models (cfg "E", "Fe") carry router
    [layers, E, d], exp_in [layers, E, 2Fe, d], exp_down [layers, E, d, Fe]
    instead of in / down, each expert quantized as its own tensor. When ``quantized`` the linears are
    packed with the Q4G128 oracle codec and the embedding is rounded to bf16.
    ``acc64`` (default: on for quantized models) accumulates matmuls in f64.
    ``kv_f32`` keeps a quantized model's q, k and v in f32 (the trainable
    policy's forward) instead of rounding them to f16 (the inference cache).
    """

    def __init__(self, cfg: dict, weights: dict, quantized: bool, acc64: bool | None = None,
                 kv_f32: bool = False):
        self.cfg, self.quantized = cfg, quantized
        self._keep = []
        w = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in weights.items()}
        if quantized:
            w["embed"] = round_bf16(w["embed"])
        self.w = w
        m = OrModel()
        for k in ("layers", "d", "H", "KVH", "hd", "F", "V"):
            setattr(m, k, int(cfg[k]))
        m.quantized = int(quantized)
        m.acc64 = int(quantized if acc64 is None else acc64)
        m.kv_f32 = int(kv_f32)
        m.eps, m.theta = float(cfg.get("eps", 1e-5)), float(cfg.get("theta", 1e4))
        for k in ("embed", "attn_norm", "ffn_norm", "final_norm"):
            setattr(m, k, self._ptr(w[k]))
        self.packed = {}
        m.experts = int(cfg.get("E", 0))
        m.expert_ffn = int(cfg.get("Fe", 0))
        if m.experts:
            if quantized and (2 * m.expert_ffn * m.d) % 128:
                raise ValueError("quantized experts need 2 * Fe * d % 128 == 0")
            m.router = self._ptr(w["router"])
            for k in ("exp_in", "exp_down"):
                if quantized:
                    arr = w[k].reshape(-1, *w[k].shape[2:])  # [layers*E, N, K]
                    cs, ss = zip(*[q4_quantize(a) for a in arr])
                    codes, scales = np.concatenate(cs), np.concatenate(ss)
                    self.packed[k] = (codes, scales)
                    setattr(m, k + "_c", self._ptr(codes))
                    setattr(m, k + "_s", self._ptr(scales))
                else:
                    setattr(m, k, self._ptr(w[k]))
        names = {"qkv": "qkv", "o": "o", "in": "in_", "down": "down", "lm_head": "lm_head"}
        short = {"qkv": "qkv", "o": "o", "in": "in", "down": "down", "lm_head": "lm"}
        for k, field in names.items():
            if k not in w:  # MoE models have no dense FFN
                continue
            if quantized:
                arr = w[k] if k != "lm_head" else w[k][None]
                cs, ss = zip(*[q4_quantize(a) for a in arr])
                codes, scales = np.concatenate(cs), np.concatenate(ss)
                self.packed[k] = (codes, scales)
                setattr(m, short[k] + "_c", self._ptr(codes))
                setattr(m, short[k] + "_s", self._ptr(scales))
            else:
                setattr(m, field, self._ptr(w[k]))
        self.m = m

    def _ptr(self, a):
        a = np.ascontiguousarray(a)
        self._keep.append(a)
        return a.ctypes.data

    def generate(self, prompts, N, temperature=0.0, seed=0):
        prompts = np.ascontiguousarray(prompts, dtype=np.int32)
        S, P = prompts.shape
        tok = np.empty((S, N), np.int32)
        lp = np.empty((S, N), np.float64)
        lib().or_generate(C.byref(self.m), prompts.ctypes.data, S, P, N, temperature, seed,
                          tok.ctypes.data, lp.ctypes.data)
        return tok, lp

    def generate_ex(self, prompts, N, *, temperature=0.0, top_k=-1, repetition_penalty=1.0,
                    top_p=1.0, apply_top_p=False, eos_token=-1, seed=0):
        """``or_generate_ex``: rollouts with the full sampling options;
        returns (tokens [S, N], log-probs [S, N] f64, lengths [S])."""
        prompts = np.ascontiguousarray(prompts, dtype=np.int32)
        S, P = prompts.shape
        tok = np.empty((S, N), np.int32)
        lp = np.empty((S, N), np.float64)
        lens = np.empty(S, np.int32)
        lib().or_generate_ex(C.byref(self.m), prompts.ctypes.data, S, P, N, temperature, top_k,
                             repetition_penalty, top_p, int(apply_top_p), eos_token, seed,
                             tok.ctypes.data, lp.ctypes.data, lens.ctypes.data)
        return tok, lp, lens

    def logprobs(self, prompts, tokens):
        prompts = np.ascontiguousarray(prompts, dtype=np.int32)
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        S, P = prompts.shape
        N = tokens.shape[1]
        lp = np.empty((S, N), np.float64)
        lib().or_logprobs(C.byref(self.m), prompts.ctypes.data, tokens.ctypes.data, S, P, N,
                          lp.ctypes.data)
        return lp

    def continuation(self, prompts, tokens, route_hint=None, hint_margin=0.0):
        """Teacher-forced recompute of ``or_logprobs`` that also returns the
        logits: (lp [S, N] f64, logits [S, N, V] f32), row n being the
        prediction of tokens[:, n] from prompt ‖ tokens[:, :n].

        MoE models: ``route_hint`` [layers, S, P + N - 1, 2] expert ids of
        another computation of the same forward; a token whose top-2 margin
        (2nd minus 3rd router logit) is below ``hint_margin`` takes the hinted
        pair. Returns (lp, logits, conflicts): conflicts counts hinted pairs
        that differ from the oracle's own where its margin is not below it."""
        prompts = np.ascontiguousarray(prompts, dtype=np.int32)
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        S, P = prompts.shape
        N = tokens.shape[1]
        L = P + N - 1
        c = self.cfg
        ids = np.ascontiguousarray(np.concatenate([prompts, tokens[:, :N - 1]], 1))
        kc = np.zeros(c["layers"] * S * c["KVH"] * L * c["hd"], np.float32)
        vc = np.zeros_like(kc)
        x = np.empty((S, L, c["d"]), np.float32)
        conflicts = np.zeros(1, np.int32)
        if route_hint is not None:
            hint = np.ascontiguousarray(route_hint, dtype=np.int32)
            assert hint.shape == (c["layers"], S, L, 2)
            self.m.route_hint = hint.ctypes.data
            self.m.hint_margin = float(hint_margin)
            self.m.hint_conflicts = conflicts.ctypes.data
        try:
            lib().or_model_forward(C.byref(self.m), ids.ctypes.data, S, L, 0, kc.ctypes.data,
                                   vc.ctypes.data, L, x.ctypes.data)
        finally:
            self.m.route_hint = None
            self.m.hint_conflicts = None
        del kc, vc
        rows = np.ascontiguousarray(x[:, P - 1:, :]).reshape(S * N, c["d"])
        logits = np.empty((S * N, c["V"]), np.float32)
        lib().or_model_logits(C.byref(self.m), rows.ctypes.data, S * N, logits.ctypes.data)
        lp, _, _ = ce_rows(logits, tokens.reshape(-1))
        if route_hint is None:
            return lp.reshape(S, N), logits.reshape(S, N, c["V"])
        return lp.reshape(S, N), logits.reshape(S, N, c["V"]), int(conflicts[0])

    def decode_steps(self, prompt, steps, temperature=1.0, seed=0, on_step=None):
        """One rollout as ``or_generate`` runs it (generate.rs:68-124): a
        prefill over ``prompt`` [P], then ``steps`` cached single-token steps.
        ``on_step(i)`` is called before decode step i (timing hooks); returns
        the sampled tokens [steps + 1]."""
        c = self.cfg
        P = len(prompt)
        cap = P + steps
        kc = np.zeros(c["layers"] * c["KVH"] * cap * c["hd"], np.float32)
        vc = np.zeros_like(kc)
        ids = np.ascontiguousarray(prompt, dtype=np.int32)
        x = np.empty((P, c["d"]), np.float32)
        lib().or_model_forward(C.byref(self.m), ids.ctypes.data, 1, P, 0, kc.ctypes.data,
                               vc.ctypes.data, cap, x.ctypes.data)
        last = np.ascontiguousarray(x[P - 1:])
        logits = np.empty((1, c["V"]), np.float32)
        toks = np.empty(steps + 1, np.int32)
        lp = np.empty(1, np.float64)
        for t in range(steps + 1):
            if t > 0:
                if on_step is not None:
                    on_step(t - 1)
                one = np.array([toks[t - 1]], np.int32)
                lib().or_model_forward(C.byref(self.m), one.ctypes.data, 1, 1, P + t - 1,
                                       kc.ctypes.data, vc.ctypes.data, cap, last.ctypes.data)
            lib().or_model_logits(C.byref(self.m), last.ctypes.data, 1, logits.ctypes.data)
            lib().or_sample(logits.ctypes.data, 1, c["V"], temperature, seed, t,
                            toks[t:].ctypes.data, 1, lp.ctypes.data, 1)
        return toks

    def forward_at(self, ids, pos0, kc, vc, cap):
        """One sequence's forward of ids [R] at positions pos0 .. pos0 + R - 1
        over caller caches kc / vc (float32, [layers, KVH, cap, hd] each; the
        positions before pos0 are read as they are): ``or_model_forward`` with
        S = 1. Returns the hidden rows [R, d]."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        R = ids.shape[0]
        c = self.cfg
        assert kc.dtype == np.float32 and kc.size == c["layers"] * c["KVH"] * cap * c["hd"]
        assert vc.dtype == np.float32 and vc.size == kc.size and pos0 + R <= cap
        x = np.empty((R, c["d"]), np.float32)
        lib().or_model_forward(C.byref(self.m), ids.ctypes.data, 1, R, int(pos0), kc.ctypes.data,
                               vc.ctypes.data, int(cap), x.ctypes.data)
        return x

    def logits(self, x):
        """Final norm + LM head of hidden rows x [R, d]: logits [R, V] f32."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty((x.shape[0], self.cfg["V"]), np.float32)
        lib().or_model_logits(C.byref(self.m), x.ctypes.data, x.shape[0], out.ctypes.data)
        return out

    def forward_logits(self, ids):
        """Full causal forward over ids [S, L]; returns logits [S, L, V] (float32)."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        S, L = ids.shape
        c = self.cfg
        kc = np.zeros(c["layers"] * S * c["KVH"] * L * c["hd"], np.float32)
        vc = np.zeros_like(kc)
        x = np.empty((S * L, c["d"]), np.float32)
        lib().or_model_forward(C.byref(self.m), ids.ctypes.data, S, L, 0, kc.ctypes.data,
                               vc.ctypes.data, L, x.ctypes.data)
        logits = np.empty((S * L, c["V"]), np.float32)
        lib().or_model_logits(C.byref(self.m), x.ctypes.data, S * L, logits.ctypes.data)
        return logits.reshape(S, L, c["V"])


    def router_gaps(self, ids):
        """MoE router margins of a full forward over ids [S, L]: [layers, S, L]
        array of (2nd-largest - 3rd-largest) router logit per token; a small
        margin means the top-2 expert set is a near-tie."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        S, L = ids.shape
        c = self.cfg
        gaps = np.full((c["layers"], S * L), np.inf, np.float32)
        kc = np.zeros(c["layers"] * S * c["KVH"] * L * c["hd"], np.float32)
        vc = np.zeros_like(kc)
        x = np.empty((S * L, c["d"]), np.float32)
        self.m.router_gap = gaps.ctypes.data
        try:
            lib().or_model_forward(C.byref(self.m), ids.ctypes.data, S, L, 0, kc.ctypes.data,
                                   vc.ctypes.data, L, x.ctypes.data)
        finally:
            self.m.router_gap = None
        return gaps.reshape(c["layers"], S, L)


def set_threads(n: int) -> int:
    """OpenMP threads for the oracle (n <= 0: every core); returns the count."""
    lib().or_set_threads(int(n))
    return int(lib().or_max_threads())


def sample(logits, temperature, seed, step):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows, V = logits.shape
    tok = np.empty(rows, np.int32)
    lp = np.empty(rows, np.float64)
    lib().or_sample(logits.ctypes.data, rows, V, temperature, seed, step, tok.ctypes.data, 1,
                    lp.ctypes.data, 1)
    return tok, lp


def apply_penalty(values, prior, penalty):
    """``or_apply_penalty`` on a copy of ``values`` (apply_repetition_penalty)."""
    v = np.array(values, dtype=np.float32)
    pr = np.ascontiguousarray(prior, dtype=np.int32)
    if lib().or_apply_penalty(v.ctypes.data, v.size, pr.ctypes.data, pr.size, penalty) != 0:
        raise ValueError("token id outside the model vocabulary")
    return v


def sample_ex(logits, *, temperature, seed, step, top_k=-1, repetition_penalty=1.0, top_p=1.0,
              apply_top_p=False, prior=None, row0=0):
    """``or_sample_ex_row`` per row. prior: list (per row) of prior token ids;
    row r draws from the counter stream of row ``row0 + r``."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows, V = logits.shape
    tok = np.empty(rows, np.int32)
    lp = np.empty(rows, np.float64)
    for r in range(rows):
        pr = np.ascontiguousarray(prior[r] if prior is not None else [], dtype=np.int32)
        t = np.empty(1, np.int32)
        l = np.empty(1, np.float64)
        rc = lib().or_sample_ex_row(logits[r].ctypes.data, V, temperature, top_k,
                                    repetition_penalty, top_p, int(apply_top_p), seed, row0 + r,
                                    step,
                                    pr.ctypes.data, pr.size, t.ctypes.data, l.ctypes.data)
        if rc != 0:
            raise ValueError("token id outside the model vocabulary")
        tok[r], lp[r] = t[0], l[0]
    return tok, lp


def fnv1a64(data: bytes) -> int:
    L = lib()
    L.or_fnv1a64.restype = C.c_uint64
    L.or_fnv1a64.argtypes = [C.c_char_p, C.c_int64]
    return int(L.or_fnv1a64(data, len(data)))


def hq_quantize(values, fmt: int):
    """``quantize_tensor`` for HQUANT formats 1-3: (scales u16 FP16 bits, codes u8)."""
    v = np.ascontiguousarray(values, dtype=np.float32).ravel()
    L = lib()
    L.or_hq_bytes_per_group.restype = C.c_int64
    L.or_hq_bytes_per_group.argtypes = [C.c_int]
    L.or_hq_quantize.restype = C.c_int
    L.or_hq_quantize.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_void_p, C.c_void_p]
    groups = (v.size + 127) // 128
    scales = np.zeros(groups, np.uint16)
    codes = np.zeros(groups * L.or_hq_bytes_per_group(fmt), np.uint8)
    if L.or_hq_quantize(v.ctypes.data, v.size, fmt, scales.ctypes.data, codes.ctypes.data) != 0:
        raise ValueError("quantization group scale is outside finite FP16 range")
    return scales, codes


def hq_decode(fmt: int, n: int, scales, codes):
    """``PackedTensor::decode`` (formats 1-3; 4 = the Q4G128 codec): f32 [n]."""
    L = lib()
    L.or_hq_decode.restype = None
    L.or_hq_decode.argtypes = [C.c_int, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p]
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(n, np.float32)
    L.or_hq_decode(fmt, n, s.ctypes.data, c.ctypes.data, out.ctypes.data)
    return out


def f32_to_f16_bits(x) -> np.ndarray:
    L = lib()
    L.or_f32_to_f16_bits.restype = C.c_uint16
    L.or_f32_to_f16_bits.argtypes = [C.c_float]
    return np.array([L.or_f32_to_f16_bits(float(v)) for v in np.ravel(x)], np.uint16)


def random_weights(cfg: dict, seed: int = 0, std: float = 0.02) -> dict:
    """N(0, std) linears and embedding, unit norms (the configs' synthetic init).
    MoE configs (cfg["E"] > 0) get a router ~ N(0, 1/sqrt(d)) (router logits
    ~ N(0, 1)) and stacked experts instead of the dense FFN."""
    rng = np.random.default_rng(seed)
    Lr, d, H, KVH, hd, F, V = (cfg[k] for k in ("layers", "d", "H", "KVH", "hd", "F", "V"))
    qn = H * hd + 2 * KVH * hd
    n = lambda *s: rng.normal(0, std, s).astype(np.float32)  # noqa: E731
    w = {"embed": n(V, d), "attn_norm": np.ones((Lr, d), np.float32),
         "ffn_norm": np.ones((Lr, d), np.float32), "final_norm": np.ones(d, np.float32),
         "qkv": n(Lr, qn, d), "o": n(Lr, d, H * hd), "lm_head": n(V, d)}
    E = cfg.get("E", 0)
    if E:
        Fe = cfg["Fe"]
        w["router"] = rng.normal(0, 1 / np.sqrt(d), (Lr, E, d)).astype(np.float32)
        w["exp_in"] = n(Lr, E, 2 * Fe, d)
        w["exp_down"] = n(Lr, E, d, Fe)
    else:
        w["in"] = n(Lr, 2 * F, d)
        w["down"] = n(Lr, d, F)
    return w
