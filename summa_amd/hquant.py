"""HQUANT packed tensors and quantized weight archives (host side).

Mirrors the reference codec and archive of summa-train/src/quantization.rs:
``PackedTensor`` (:414-689; container bytes :502-597) and ``QuantizedArchive``
(:1163-1346: ``manifest.json`` + one member file per tensor, every member
verified by size and SHA-256 before any tensor is exposed). Parsing,
validation and serialisation of a container run in the native library
(``sm_hquant_parse`` / ``sm_hquant_write``), decoding on the device
(``sm_hquant_decode``); installing a tensor into a model goes through
``sm_model_load_packed`` (the ``QuantizedModelBackend`` seam, :1183-1189).

Formats 1-3 are the reference's; format 4 (``q4_g128``) is this build's 4-bit
codec, whose archives store linear weights in the model's ``[out, in]`` row
layout (reference archives store Burn's ``[in, out]`` Linear layout).
"""
from __future__ import annotations

import ctypes as C
import hashlib
import json
import os
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

from . import _lib

FORMATS = {"binary_g128": 1, "ternary_g128": 2, "ternary_entropy_g128": 3, "q4_g128": 4}
FORMAT_NAMES = {v: k for k, v in FORMATS.items()}
BYTES_PER_GROUP = {1: 16, 2: 32, 3: 26, 4: 64}
GROUP = 128
ARCHIVE_VERSION = 2                    # QUANTIZATION_ARCHIVE_VERSION, :37
MAX_MANIFEST_BYTES = 16 * 1024 * 1024  # :39
MAX_MEMBERS = 65_536                   # :40
MAX_RANK = 32
DTYPE_BITS = {"F4": 4, "F6_E2M3": 6, "F6_E3M2": 6, "BOOL": 8, "U8": 8, "I8": 8, "F8_E5M2": 8,
              "F8_E4M3": 8, "F8_E8M0": 8, "I16": 16, "U16": 16, "F16": 16, "BF16": 16,
              "I32": 32, "U32": 32, "F32": 32, "C64": 64, "F64": 64, "I64": 64,
              "U64": 64}  # tensor_storage_bytes, :1997-2013


class HQuantError(ValueError):
    pass


class HQuantC(C.Structure):
    """``sm_hquant`` of include/summa_amd.h."""
    _fields_ = [("format", C.c_int32), ("group_size", C.c_int32), ("rank", C.c_int32),
                ("shape", C.c_int64 * 32), ("elements", C.c_int64), ("scales", C.c_void_p),
                ("nscales", C.c_int64), ("codes", C.c_void_p), ("ncodes", C.c_int64)]


def _check(status: int) -> None:
    if status != 0:
        raise HQuantError(_lib.lib().sm_last_error().decode(errors="replace"))


def sha256_identity(data: bytes) -> str:
    """``sha256_identity`` (artifact_io.rs:42): ``sha256:`` + 64 lowercase hex."""
    return "sha256:" + hashlib.sha256(data).hexdigest()


@dataclass
class PackedTensor:
    """``PackedTensor`` (:414-423): shape, g128 scales (FP16 bits; bf16 bits
    for q4_g128) and packed codes."""
    format: int
    shape: tuple
    scales: np.ndarray
    codes: np.ndarray
    group_size: int = GROUP

    @property
    def elements(self) -> int:
        return int(np.prod(self.shape, dtype=object))

    def _c(self, scales_ptr: int, codes_ptr: int) -> HQuantC:
        t = HQuantC()
        t.format, t.group_size, t.rank = self.format, self.group_size, len(self.shape)
        if not 1 <= t.rank <= MAX_RANK:
            raise HQuantError(f"packed tensor rank must be in 1..={MAX_RANK}")
        for i, d in enumerate(self.shape):
            t.shape[i] = int(d)
        t.elements = self.elements
        t.scales, t.nscales = scales_ptr, int(self.scales.size)
        t.codes, t.ncodes = codes_ptr, int(self.codes.size)
        return t

    def bits_per_weight(self) -> float:
        """Codec payload rate (:435-443): 8 * (2 * scales + codes) / elements."""
        self.to_bytes()  # validates
        return 8.0 * (2 * self.scales.size + self.codes.size) / self.elements

    def to_bytes(self) -> bytes:
        s = np.ascontiguousarray(self.scales, dtype=np.uint16)
        c = np.ascontiguousarray(self.codes, dtype=np.uint8)
        t = self._c(s.ctypes.data, c.ctypes.data)
        L = _lib.lib()
        n = L.sm_hquant_bytes(C.byref(t))
        if n < 0:
            raise HQuantError("packed tensor rank must be in 1..=32")
        out = np.empty(n, np.uint8)
        written = C.c_int64(0)
        _check(L.sm_hquant_write(C.byref(t), out.ctypes.data, n, C.byref(written)))
        return out[:written.value].tobytes()

    @classmethod
    def from_bytes(cls, data: bytes) -> "PackedTensor":
        buf = np.frombuffer(data, dtype=np.uint8).copy()  # aligned, owned
        t = HQuantC()
        _check(_lib.lib().sm_hquant_parse(buf.ctypes.data, buf.size, C.byref(t)))
        so = t.scales - buf.ctypes.data
        co = t.codes - buf.ctypes.data
        return cls(int(t.format), tuple(int(t.shape[i]) for i in range(t.rank)),
                   buf[so:so + 2 * t.nscales].view(np.uint16).copy(),
                   buf[co:co + t.ncodes].copy(), int(t.group_size))

    def save(self, path) -> None:
        Path(path).write_bytes(self.to_bytes())

    @classmethod
    def load(cls, path) -> "PackedTensor":
        return cls.from_bytes(Path(path).read_bytes())

    def to_device(self, device) -> "DevicePacked":
        return DevicePacked(self, device)

    def decode(self, device, transpose: bool = False) -> torch.Tensor:
        """Device decode (PackedTensor::decode, :445-497): f32, shaped like the
        tensor, or a rank-2 tensor transposed."""
        d = self.to_device(device)
        shape = (self.shape[1], self.shape[0]) if transpose else self.shape
        out = torch.empty(shape, dtype=torch.float32, device=device)
        _check(_lib.lib().sm_hquant_decode(C.byref(d.c), out.data_ptr(), int(transpose),
                                           torch.cuda.current_stream(device).cuda_stream))
        return out


class DevicePacked:
    """A packed tensor's scales / codes in device memory with the C view."""

    def __init__(self, t: PackedTensor, device):
        self.scales = torch.from_numpy(np.ascontiguousarray(t.scales).view(np.int16)).to(device)
        self.codes = torch.from_numpy(np.ascontiguousarray(t.codes)).to(device)
        self.c = t._c(self.scales.data_ptr(), self.codes.data_ptr())


def q4_packed(w: torch.Tensor) -> PackedTensor:
    """Q4G128 packed tensor of a device weight (the device quantizer,
    sm_q4_quantize): the q4_g128 export of a model linear [out, in]."""
    from .ops import Q4Weight
    q = Q4Weight.quantize(w)
    return PackedTensor(4, tuple(w.shape), q.scales.cpu().numpy().view(np.uint16),
                        q.codes.cpu().numpy())


# ------------------------------------------------------------------ archive --

def _storage_bytes(dtype: str, elements: int) -> int:
    if dtype not in DTYPE_BITS:
        raise HQuantError(f"unsupported floating tensor dtype `{dtype}` in quantized archive")
    return (elements * DTYPE_BITS[dtype] + 7) // 8


def _packed_bytes(shape, fmt: int) -> int:
    """packed_tensor_storage_bytes (:1962-1995): header + payload + checksum."""
    elements = int(np.prod(shape, dtype=object))
    if elements <= 0:
        raise HQuantError("packed tensor is empty")
    groups = -(-elements // GROUP)
    return 8 + 2 + 1 + 2 + 1 + 8 * len(shape) + 16 + groups * (2 + BYTES_PER_GROUP[fmt]) + 8


def _member(root: Path, file: str) -> Path:
    """checked_archive_member: a relative path inside the archive root."""
    p = Path(file)
    if p.is_absolute() or not file or any(part in ("..", ".", "") for part in p.parts):
        raise HQuantError(f"archive member path `{file}` is not a plain relative path")
    full = root / p
    if full.is_symlink() or not full.is_file():
        raise HQuantError(f"archive member `{file}` must be a regular file")
    return full


def _read_verified(path: Path, size: int, sha: str) -> bytes:
    data = path.read_bytes()
    if len(data) != size:
        raise HQuantError(f"archive member {path.name} has {len(data)} bytes, manifest says {size}")
    if sha256_identity(data) != sha:
        raise HQuantError(f"archive member {path.name} SHA-256 mismatch")
    return data


@dataclass
class FloatingTensor:
    name: str
    dtype: str
    shape: tuple
    data: bytes

    def to_f32(self) -> np.ndarray:
        if self.dtype == "F32":
            a = np.frombuffer(self.data, np.float32)
        elif self.dtype == "BF16":
            a = (np.frombuffer(self.data, np.uint16).astype(np.uint32) << 16).view(np.float32)
        elif self.dtype == "F16":
            a = np.frombuffer(self.data, np.float16).astype(np.float32)
        else:
            raise HQuantError(f"floating tensor `{self.name}` dtype {self.dtype} is not loadable")
        return a.reshape(self.shape)


@dataclass
class QuantizedArchive:
    """A validated archive (QuantizedArchive::open, :1192-1346)."""
    root: Path
    manifest: dict
    matrices: dict = field(default_factory=dict)    # name -> PackedTensor
    floating: dict = field(default_factory=dict)    # name -> FloatingTensor

    @classmethod
    def open(cls, root) -> "QuantizedArchive":
        root = Path(root)
        if not root.is_dir() or root.is_symlink():
            raise HQuantError("quantized archive root must be a real directory")
        mpath = root / "manifest.json"
        if mpath.is_symlink() or not mpath.is_file():
            raise HQuantError("quantization manifest must be a regular file")
        if mpath.stat().st_size > MAX_MANIFEST_BYTES:
            raise HQuantError("quantization manifest exceeds its size limit")
        try:
            m = json.loads(mpath.read_bytes())
        except ValueError as e:
            raise HQuantError(f"invalid quantization manifest: {e}") from None
        if m.get("version") != ARCHIVE_VERSION:
            raise HQuantError(f"unsupported quantization manifest version {m.get('version')}")
        if not str(m.get("base_checkpoint_hash", "")).strip():
            raise HQuantError("base checkpoint hash is empty")
        recipe = m.get("recipe", {})
        if recipe.get("group_size", GROUP) != GROUP:
            raise HQuantError("Bonsai-compatible codecs require group_size 128")
        if recipe.get("format") not in FORMATS:
            raise HQuantError(f"unknown quantization format {recipe.get('format')!r}")
        mats, flts = m.get("matrices", []), m.get("floating_tensors", [])
        if not mats:
            raise HQuantError("quantization archive contains no quantized matrices")
        if len(mats) + len(flts) > MAX_MEMBERS:
            raise HQuantError(f"quantization archive exceeds its {MAX_MEMBERS}-member limit")
        arc = cls(root, m)
        names, files = set(), set()
        for rec in mats + flts:
            if rec["name"] in names or rec["file"] in files:
                raise HQuantError(f"duplicate archive member `{rec['name']}`")
            names.add(rec["name"])
            files.add(rec["file"])
        for rec in mats:
            shape = tuple(rec["shape"])
            if not 2 <= len(shape) <= MAX_RANK:
                raise HQuantError(f"quantized matrix `{rec['name']}` rank must be in 2..={MAX_RANK}")
            if rec["elements"] != int(np.prod(shape, dtype=object)):
                raise HQuantError(f"quantized matrix `{rec['name']}` element count mismatch")
            fmt = FORMATS.get(rec["format"])
            if rec["packed_bytes"] != _packed_bytes(shape, fmt):
                raise HQuantError(f"quantized matrix `{rec['name']}` packed byte count does not "
                                  "match its shape and format")
            data = _read_verified(_member(root, rec["file"]), rec["packed_bytes"], rec["sha256"])
            try:
                t = PackedTensor.from_bytes(data)
            except HQuantError as e:
                raise HQuantError(f"invalid quantized matrix `{rec['name']}`: {e}") from None
            if not (fmt == FORMATS[recipe["format"]] and t.format == fmt and t.shape == shape):
                raise HQuantError(f"quantized matrix `{rec['name']}` does not match its manifest")
            arc.matrices[rec["name"]] = t
        for rec in flts:
            shape = tuple(rec["shape"])
            elements = int(np.prod(shape, dtype=object))
            if rec["elements"] != elements:
                raise HQuantError(f"floating tensor `{rec['name']}` element count mismatch")
            if rec["bytes"] != _storage_bytes(rec["dtype"], elements):
                raise HQuantError(f"floating tensor `{rec['name']}` byte count does not match "
                                  "dtype and shape")
            data = _read_verified(_member(root, rec["file"]), rec["bytes"], rec["sha256"])
            arc.floating[rec["name"]] = FloatingTensor(rec["name"], rec["dtype"], shape, data)
        # inventory: nothing but the manifest and its members
        found = {str(p.relative_to(root)) for p in root.rglob("*") if p.is_file()}
        extra = found - files - {"manifest.json"}
        if extra:
            raise HQuantError(f"quantized archive contains unexpected files: {sorted(extra)}")
        return arc


def write_archive(root, matrices: dict, floating: dict, fmt: str, base_checkpoint_hash: str,
                  errors: dict | None = None) -> dict:
    """Write an archive: ``matrices`` name -> PackedTensor (all of format
    ``fmt``), ``floating`` name -> (dtype, shape, bytes). Returns the manifest."""
    root = Path(root)
    root.mkdir(parents=True, exist_ok=False)
    man = {"version": ARCHIVE_VERSION, "base_checkpoint_hash": base_checkpoint_hash,
           "recipe": {"format": fmt, "group_size": GROUP, "fake_quant_start_step": 0,
                      "ternary_warmup_steps": 0, "distillation_weight": 0.0,
                      "quantize_embeddings": False, "quantize_lm_head": True},
           "matrices": [], "floating_tensors": []}
    for i, (name, t) in enumerate(sorted(matrices.items())):
        data = t.to_bytes()
        file = f"matrices/{i:05d}.hquant"
        (root / "matrices").mkdir(exist_ok=True)
        (root / file).write_bytes(data)
        mse, mae = (errors or {}).get(name, (0.0, 0.0))
        man["matrices"].append({"name": name, "shape": list(t.shape), "elements": t.elements,
                                "format": fmt, "file": file, "packed_bytes": len(data),
                                "sha256": sha256_identity(data), "mean_squared_error": mse,
                                "maximum_absolute_error": mae})
    for i, (name, (dtype, shape, data)) in enumerate(sorted(floating.items())):
        file = f"floating/{i:05d}.bin"
        (root / "floating").mkdir(exist_ok=True)
        (root / file).write_bytes(data)
        man["floating_tensors"].append({"name": name, "dtype": dtype, "shape": list(shape),
                                        "elements": int(np.prod(shape, dtype=object)),
                                        "file": file, "bytes": len(data),
                                        "sha256": sha256_identity(data)})
    tmp = root / "manifest.json.tmp"
    tmp.write_text(json.dumps(man, sort_keys=True))
    os.replace(tmp, root / "manifest.json")
    return man
