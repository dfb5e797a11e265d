"""Checkpoints: safetensors files and quantized archives into a ``Model``.

``load_safetensors`` mirrors summa-llm/src/model/weights.rs:18-69 (strict:
missing, unexpected and shape-mismatched tensors are errors, and nothing is
applied unless the whole file matches), ``load_archive`` the
``QuantizedModelBackend`` install of a validated ``QuantizedArchive``
(summa-train/src/quantization.rs:1183-1189). Tensor names follow Burn's record
paths of the reference modules (``Transformer`` transformer.rs:367-381,
``TransformerBlock`` block.rs:25-31, ``MultiHeadAttention`` attention.rs:43-48,
``FeedForward`` / ``SparseMoe`` / ``ExpertBank`` ffn.rs:35-54, 146-160, 449-452,
``Norm::Rms`` norm.rs:16-19 with enum variants skipped as weights.rs:48 asks);
Burn stores a ``Linear`` weight as ``[d_in, d_out]``, so linears are
transposed into this model's ``[out, in]`` rows on load.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import torch

from .hquant import FORMATS, HQuantError, QuantizedArchive
from .model import KIND, Model, ModelConfig

SAFETENSORS_DTYPES = {"F32": np.float32, "F16": np.float16, "BF16": np.uint16, "F64": np.float64}


class CheckpointError(ValueError):
    pass


def burn_names(cfg: ModelConfig) -> dict:
    """Record path -> (kind, layer, expected Burn shape, transpose rule).
    Rules: "none"; "t" (2-D transpose); "te" (transpose each expert)."""
    d, hd = cfg.d_model, cfg.head_dim
    qn = (cfg.heads + 2 * cfg.kv_heads) * hd
    names = {"embedding.weight": ("embed", -1, (cfg.vocab, d), "none"),
             "final_norm.gamma": ("final_norm", -1, (d,), "none"),
             "lm_head.weight": ("lm_head", -1, (d, cfg.vocab), "t")}
    for i in range(cfg.layers):
        p = f"layers.{i}."
        names[p + "attention.qkv_proj.weight"] = ("qkv", i, (d, qn), "t")
        names[p + "attention.o_proj.weight"] = ("o", i, (cfg.heads * hd, d), "t")
        names[p + "attn_norm.gamma"] = ("attn_norm", i, (d,), "none")
        names[p + "ffn_norm.gamma"] = ("ffn_norm", i, (d,), "none")
        if cfg.experts:
            e, fe = cfg.experts, cfg.expert_ffn
            names[p + "feed_forward.moe.router.weight"] = ("router", i, (d, e), "t")
            names[p + "feed_forward.moe.experts.in_weight"] = ("exp_in", i, (e, d, 2 * fe), "te")
            names[p + "feed_forward.moe.experts.down_weight"] = ("exp_down", i, (e, fe, d), "te")
        else:
            names[p + "feed_forward.in_proj.weight"] = ("in", i, (d, 2 * cfg.ffn), "t")
            names[p + "feed_forward.down_proj.weight"] = ("down", i, (cfg.ffn, d), "t")
    return names


def _to_model_layout(a: np.ndarray, rule: str) -> np.ndarray:
    if rule == "t":
        return np.ascontiguousarray(a.T)
    if rule == "te":
        return np.ascontiguousarray(np.transpose(a, (0, 2, 1)))
    return np.ascontiguousarray(a)


# ------------------------------------------------------------- safetensors --

def read_safetensors(path) -> dict:
    """name -> float32 array (F32 / F16 / BF16 / F64 payloads)."""
    data = Path(path).read_bytes()
    if len(data) < 8:
        raise CheckpointError("safetensors file is truncated")
    (hlen,) = struct.unpack("<Q", data[:8])
    if 8 + hlen > len(data):
        raise CheckpointError("safetensors header exceeds the file")
    header = json.loads(data[8:8 + hlen])
    body = memoryview(data)[8 + hlen:]
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        dt = info["dtype"]
        if dt not in SAFETENSORS_DTYPES:
            raise CheckpointError(f"tensor `{name}` has unsupported dtype {dt}")
        b, e = info["data_offsets"]
        if not 0 <= b <= e <= len(body):
            raise CheckpointError(f"tensor `{name}` data offsets are out of range")
        a = np.frombuffer(body[b:e], dtype=SAFETENSORS_DTYPES[dt])
        if dt == "BF16":
            a = (a.astype(np.uint32) << 16).view(np.float32)
        shape = tuple(info["shape"])
        if a.size != int(np.prod(shape, dtype=np.int64)):
            raise CheckpointError(f"tensor `{name}` byte count does not match its shape")
        out[name] = a.astype(np.float32).reshape(shape)
    return out


def write_safetensors(path, tensors: dict, dtype: str = "F32") -> None:
    """Canonical file: header keys in lexical order (weights.rs:84-90)."""
    header, blobs, off = {}, [], 0
    for name in sorted(tensors):
        a = np.ascontiguousarray(tensors[name], dtype=np.float32)
        if dtype == "BF16":
            u = a.view(np.uint32)
            b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).tobytes()
        elif dtype == "F16":
            b = a.astype(np.float16).tobytes()
        else:
            b = a.tobytes()
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header, sort_keys=True, separators=(",", ":")).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    Path(path).write_bytes(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def load_safetensors(model: Model, path) -> dict:
    """Strict load (weights.rs:18-60). A checkpoint without ``lm_head.weight``
    ties the output matrix to the embedding (transformer.rs:372-373).
    Returns {"applied": [...], "tied": bool}."""
    tensors = read_safetensors(path)
    names = burn_names(model.cfg)
    tied = "lm_head.weight" not in tensors
    if tied:
        names.pop("lm_head.weight")
    missing = sorted(set(names) - set(tensors))
    unused = sorted(set(tensors) - set(names))
    errors = [f"{n}: shape {tuple(tensors[n].shape)}, expected {names[n][2]}"
              for n in sorted(set(names) & set(tensors)) if tuple(tensors[n].shape) != names[n][2]]
    if missing or unused or errors:
        raise CheckpointError(f"checkpoint {path} does not match the model topology:\n"
                              f"missing: {missing}\nunused: {unused}\nerrors: {errors}")
    dev = torch.device("cuda", torch.cuda.current_device())
    for name, (kind, layer, _, rule) in names.items():
        t = torch.from_numpy(_to_model_layout(tensors[name], rule)).to(dev)
        model.set_tensor(kind, t, layer)
    if tied:
        model.set_tensor("lm_head", torch.from_numpy(tensors["embedding.weight"]).to(dev))
    torch.cuda.synchronize()
    return {"applied": sorted(names), "tied": tied}


# ---------------------------------------------------------------- archives --

def load_archive(model: Model, root) -> dict:
    """Install a validated archive: quantized matrices through
    ``sm_model_load_packed`` (reference formats in Burn's [in, out] layout;
    q4_g128 archives in the model's [out, in] rows, installed bit for bit
    into a quantized model), floating tensors like ``load_safetensors``."""
    arc = QuantizedArchive.open(root)
    names = burn_names(model.cfg)
    q4 = FORMATS[arc.manifest["recipe"]["format"]] == FORMATS["q4_g128"]
    present = set(arc.matrices) | set(arc.floating)
    tied = "lm_head.weight" not in present
    if tied:
        names.pop("lm_head.weight")
    missing = sorted(set(names) - present)
    unused = sorted(present - set(names))
    if missing or unused:
        raise CheckpointError(f"archive {root} does not match the model topology:\n"
                              f"missing: {missing}\nunused: {unused}")
    dev = torch.device("cuda", torch.cuda.current_device())
    for name, (kind, layer, burn_shape, rule) in names.items():
        if name in arc.matrices:
            t = arc.matrices[name]
            want = burn_shape
            if q4:  # model layout
                want = burn_shape[::-1] if rule == "t" else \
                    (burn_shape[0], burn_shape[2], burn_shape[1]) if rule == "te" else burn_shape
            if t.shape != tuple(want):
                raise CheckpointError(f"{name}: shape {t.shape}, expected {tuple(want)}")
            if rule == "te" and not q4:
                # per-expert transpose: decode, then install as a dense tensor
                a = t.decode(dev).cpu().numpy()
                model.set_tensor(kind, torch.from_numpy(_to_model_layout(a, rule)).to(dev), layer)
            else:
                model.load_packed(kind, t, layer, layout=0 if (q4 or rule == "none") else 1)
        else:
            f = arc.floating[name]
            if f.shape != burn_shape:
                raise CheckpointError(f"{name}: shape {f.shape}, expected {burn_shape}")
            a = np.require(_to_model_layout(f.to_f32(), rule), requirements="W")
            model.set_tensor(kind, torch.from_numpy(a).to(dev), layer)
    if tied:
        if "embedding.weight" in arc.matrices:
            emb = arc.matrices["embedding.weight"].decode(dev)
        else:
            emb = torch.from_numpy(np.require(arc.floating["embedding.weight"].to_f32(),
                                              requirements="W")).to(dev)
        model.set_tensor("lm_head", emb)
    torch.cuda.synchronize()
    return {"format": arc.manifest["recipe"]["format"], "tied": tied,
            "matrices": len(arc.matrices), "floating": len(arc.floating)}


def export_q4_archive(weights: dict, cfg: ModelConfig, root, base_checkpoint_hash: str) -> dict:
    """Q4G128 export of host f32 weights given by Burn record path in Burn
    layout: linears are quantized on the device in the model's [out, in]
    rows (format q4_g128), norms and the embedding stay F32 floating tensors."""
    from .hquant import q4_packed, write_archive
    names = burn_names(cfg)
    dev = torch.device("cuda", torch.cuda.current_device())
    mats, flts = {}, {}
    for name, a in weights.items():
        if name not in names:
            raise CheckpointError(f"unexpected tensor `{name}`")
        kind, _, _, rule = names[name]
        a = np.asarray(a, dtype=np.float32)
        if rule in ("t", "te") and kind != "router":
            mats[name] = q4_packed(torch.from_numpy(_to_model_layout(a, rule)).to(dev))
        else:
            flts[name] = ("F32", a.shape, np.ascontiguousarray(a).tobytes())
    try:
        return write_archive(root, mats, flts, "q4_g128", base_checkpoint_hash)
    except HQuantError as e:
        raise CheckpointError(str(e)) from None
