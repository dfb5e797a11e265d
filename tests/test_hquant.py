"""HQUANT codec (summa-train/src/quantization.rs): the oracle restatement
pinned by the reference's codec tests and closed forms, and the native
container parse / serialise (C ABI, host memory, no GPU), archives and
safetensors files on the CPU."""
import hashlib
import json
import math

import numpy as np
import pytest

import oracle
from summa_amd import hquant
from summa_amd.hquant import HQuantError, PackedTensor, QuantizedArchive


def weights():
    # quantization.rs:2287-2291
    i = np.arange(256, dtype=np.float32)
    return (np.sin(i * np.float32(0.37)) * 2.0 + (np.arange(256) % 7) * 0.01).astype(np.float32)


def packed(values, shape, fmt):
    s, c = oracle.hq_quantize(values, fmt)
    return PackedTensor(fmt, tuple(shape), s, c)


def test_fnv1a64_published_vectors():
    assert oracle.fnv1a64(b"") == 0xcbf29ce484222325
    assert oracle.fnv1a64(b"a") == 0xaf63dc4c8601ec8c
    assert oracle.fnv1a64(b"foobar") == 0x85944171f73967e8
    from summa_amd import _lib
    import ctypes
    L = _lib.lib()
    assert L.sm_fnv1a64(b"foobar", 6) == 0x85944171f73967e8


def test_binary_storage_rate_golden():
    # binary_g128_has_prism_public_storage_rate_and_roundtrips (:2501-2515)
    t = packed(weights(), (2, 128), 1)
    assert t.codes.size == 32 and t.scales.size == 2
    assert abs(t.bits_per_weight() - 1.125) < 1e-9
    d = oracle.hq_decode(1, 256, t.scales, t.codes)
    assert d.size == 256 and np.all(np.isfinite(d))


def test_binary_scale_is_mean_abs_and_sign_codes():
    v = weights()
    t = packed(v, (256,), 1)
    for g in range(2):
        grp = v[g * 128:(g + 1) * 128]
        want = np.float16(np.abs(grp.astype(np.float64)).mean()).view(np.uint16)
        assert t.scales[g] == want
    d = oracle.hq_decode(1, 256, t.scales, t.codes)
    s = np.repeat(t.scales.view(np.float16).astype(np.float32), 128)
    np.testing.assert_array_equal(d, np.where(v >= 0, s, -s))


def test_ternary_codecs_decode_identically_golden():
    # ternary_codecs_decode_identically_and_entropy_pack_is_smaller (:2549-2569)
    dense = packed(weights(), (2, 128), 2)
    ent = packed(weights(), (2, 128), 3)
    np.testing.assert_array_equal(oracle.hq_decode(2, 256, dense.scales, dense.codes),
                                  oracle.hq_decode(3, 256, ent.scales, ent.codes))
    assert ent.codes.size < dense.codes.size
    assert dense.bits_per_weight() == 2.125 and ent.bits_per_weight() == 1.75


@pytest.mark.parametrize("seed", range(6))
def test_ternary_is_the_squared_error_minimiser(seed):
    """optimal_ternary (:934-978) against brute force over every nonzero count."""
    rng = np.random.default_rng(seed)
    g = rng.normal(0, 1, 128).astype(np.float32)
    g[rng.integers(0, 128, 10)] = 0.0
    t = packed(g, (128,), 2)
    d = oracle.hq_decode(2, 128, t.scales, t.codes)
    mags = np.sort(np.abs(g.astype(np.float64)))[::-1]
    errs = [np.sum(mags ** 2) - np.sum(mags[:k]) ** 2 / k for k in range(1, 129)]
    k = int(np.argmin(errs)) + 1
    assert np.count_nonzero(d) == k
    s = np.float16(mags[:k].mean()).astype(np.float32)
    nz = d[d != 0]
    assert np.all(np.abs(nz) == s)
    np.testing.assert_array_equal(np.sign(nz), np.sign(g[d != 0]))


@pytest.mark.parametrize("fmt", [1, 2, 3])
def test_final_partial_group_golden(fmt):
    # final_partial_group_is_padded_only_in_storage (:2571-2589)
    v = np.arange(137, dtype=np.float32) - 70.0
    t = packed(v, (137,), fmt)
    assert t.scales.size == 2
    assert oracle.hq_decode(fmt, 137, t.scales, t.codes).size == 137
    back = PackedTensor.from_bytes(t.to_bytes())
    assert back.format == fmt and back.shape == (137,)
    np.testing.assert_array_equal(back.scales, t.scales)
    np.testing.assert_array_equal(back.codes, t.codes)


@pytest.mark.parametrize("fmt", [1, 2, 3])
def test_packed_linear_equals_decode_times_x(fmt):
    # direct_packed_linear_matches_decode_reference (:2591-2618): row . x over
    # the decoded codes, against value-at-a-time accumulation in f32
    t = packed(weights(), (2, 128), fmt)
    x = np.cos(np.arange(128, dtype=np.float32) * np.float32(0.2))
    d = oracle.hq_decode(fmt, 256, t.scales, t.codes).reshape(2, 128)
    for r in range(2):
        acc = np.float32(0)
        for c in range(128):
            acc = np.float32(acc + d[r, c] * x[c])
        assert abs(acc - float(d[r].astype(np.float64) @ x)) < 1e-5


def test_container_layout_and_checksum():
    t = packed(weights(), (2, 128), 1)
    b = t.to_bytes()
    assert b[:8] == b"HQUANT1\0" and b[8:10] == (1).to_bytes(2, "little") and b[10] == 1
    assert int.from_bytes(b[11:13], "little") == 128 and b[13] == 2
    assert int.from_bytes(b[-8:], "little") == oracle.fnv1a64(b[:-8])
    assert len(b) == 8 + 2 + 1 + 2 + 1 + 16 + 16 + 4 + 32 + 8


def _reseal(b: bytes) -> bytes:
    return b[:-8] + oracle.fnv1a64(b[:-8]).to_bytes(8, "little")


@pytest.mark.parametrize("mutate,msg", [
    (lambda b: b[:-9] + bytes([b[-9] ^ 1]) + b[-8:], "quantized tensor checksum mismatch"),
    (lambda b: _reseal(b"HQUANT2\0" + b[8:]), "invalid quantized tensor magic"),
    (lambda b: _reseal(b[:8] + (2).to_bytes(2, "little") + b[10:]), "unsupported quantized tensor version 2"),
    (lambda b: _reseal(b[:10] + bytes([9]) + b[11:]), "unknown ultra-quant format tag 9"),
    (lambda b: b[:12], "quantized tensor is truncated"),
    (lambda b: _reseal(b[:-9] + b[-8:]), "quantized tensor declared payload size mismatch"),
])
def test_container_rejections(mutate, msg):
    b = packed(weights(), (2, 128), 2).to_bytes()
    with pytest.raises(HQuantError, match=msg):
        PackedTensor.from_bytes(mutate(b))


def test_reserved_and_padding_codes_rejected():
    t = packed(weights(), (2, 128), 2)
    bad = t.codes.copy()
    bad[0] |= 3  # reserved ternary code 3
    with pytest.raises(HQuantError, match="reserved ternary code 3"):
        PackedTensor(2, (2, 128), t.scales, bad).to_bytes()
    e = packed(np.arange(137, dtype=np.float32), (137,), 3)
    bad = e.codes.copy()
    bad[-1] = 242  # nonzero trits past element 137
    with pytest.raises(HQuantError, match="non-canonical final-group padding"):
        PackedTensor(3, (137,), e.scales, bad).to_bytes()
    bad = e.codes.copy()
    bad[25] = 200  # spare trits of a full base-3 group
    with pytest.raises(HQuantError, match="non-canonical base-3 group padding"):
        PackedTensor(3, (137,), e.scales, bad).to_bytes()
    s = t.scales.copy()
    s[0] = 0x8000  # negative zero is non-canonical
    with pytest.raises(HQuantError, match="invalid or non-canonical scale"):
        PackedTensor(2, (2, 128), s, t.codes).to_bytes()


def _archive(tmp_path, fmt=2):
    mats = {"layers.0.attention.o_proj.weight": packed(weights(), (2, 128), fmt)}
    g = np.arange(4, dtype=np.float32)
    flts = {"final_norm.gamma": ("F32", (4,), g.tobytes())}
    root = tmp_path / "arc"
    hquant.write_archive(root, mats, flts, hquant.FORMAT_NAMES[fmt],
                         "sha256:" + hashlib.sha256(b"src").hexdigest())
    return root


def test_archive_roundtrip_and_member_verification(tmp_path):
    root = _archive(tmp_path)
    arc = QuantizedArchive.open(root)
    t = arc.matrices["layers.0.attention.o_proj.weight"]
    assert t.shape == (2, 128) and t.format == 2
    np.testing.assert_array_equal(arc.floating["final_norm.gamma"].to_f32(), np.arange(4))
    f = next((root / "matrices").iterdir())
    data = bytearray(f.read_bytes())
    data[40] ^= 1
    f.write_bytes(bytes(data))
    with pytest.raises(HQuantError, match="SHA-256 mismatch"):
        QuantizedArchive.open(root)


def test_archive_rejects_extra_files_and_bad_manifests(tmp_path):
    root = _archive(tmp_path)
    (root / "stray.bin").write_bytes(b"x")
    with pytest.raises(HQuantError, match="unexpected files"):
        QuantizedArchive.open(root)
    (root / "stray.bin").unlink()
    m = json.loads((root / "manifest.json").read_text())
    m["version"] = 1
    (root / "manifest.json").write_text(json.dumps(m))
    with pytest.raises(HQuantError, match="unsupported quantization manifest version 1"):
        QuantizedArchive.open(root)
    m["version"] = 2
    m["matrices"][0]["packed_bytes"] += 1
    (root / "manifest.json").write_text(json.dumps(m))
    with pytest.raises(HQuantError, match="packed byte count does not match"):
        QuantizedArchive.open(root)


@pytest.mark.parametrize("dtype", ["F32", "BF16", "F16"])
def test_safetensors_roundtrip(tmp_path, dtype):
    from summa_amd.checkpoint import read_safetensors, write_safetensors
    rng = np.random.default_rng(1)
    t = {"b": rng.normal(0, 1, (3, 5)).astype(np.float32), "a": np.arange(7, dtype=np.float32)}
    p = tmp_path / "w.safetensors"
    write_safetensors(p, t, dtype)
    raw = p.read_bytes()
    hlen = int.from_bytes(raw[:8], "little")
    assert list(json.loads(raw[8:8 + hlen])) == ["a", "b"] and hlen % 8 == 0
    back = read_safetensors(p)
    for k, v in t.items():
        want = {"F32": v, "BF16": oracle.round_bf16(v), "F16": v.astype(np.float16).astype(np.float32)}[dtype]
        np.testing.assert_array_equal(back[k], want)
