"""Checkpoints into a device model: HQUANT device decode against the oracle,
safetensors (Burn record paths and [in, out] Linear layout) and quantized
archives through sm_model_load_packed, end to end through the decoder."""
import hashlib

import numpy as np
import pytest
import torch

import oracle
from summa_amd import checkpoint, hquant
from summa_amd.hquant import PackedTensor
from summa_amd.model import Model, ModelConfig

pytestmark = pytest.mark.gpu

CFG = ModelConfig(layers=2, d_model=256, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=1000,
                  max_seq=64, quantized=False)
SRC = "sha256:" + hashlib.sha256(b"synthetic source").hexdigest()


def burn_weights(w, cfg, tied=False):
    """oracle.random_weights (model layout) -> Burn record paths / layout."""
    out = {"embedding.weight": w["embed"], "final_norm.gamma": w["final_norm"]}
    if not tied:
        out["lm_head.weight"] = w["lm_head"].T
    for i in range(cfg.layers):
        p = f"layers.{i}."
        out[p + "attention.qkv_proj.weight"] = w["qkv"][i].T
        out[p + "attention.o_proj.weight"] = w["o"][i].T
        out[p + "attn_norm.gamma"] = w["attn_norm"][i]
        out[p + "ffn_norm.gamma"] = w["ffn_norm"][i]
        out[p + "feed_forward.in_proj.weight"] = w["in"][i].T
        out[p + "feed_forward.down_proj.weight"] = w["down"][i].T
    return {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in out.items()}


def _lp(m, dev, seed=0):
    rng = np.random.default_rng(seed)
    prompts = torch.from_numpy(rng.integers(0, CFG.vocab, (4, 12)).astype(np.int32)).to(dev)
    toks = torch.from_numpy(rng.integers(0, CFG.vocab, (4, 6)).astype(np.int32)).to(dev)
    return prompts, toks, m.logprobs(prompts, toks).cpu().numpy()


@pytest.mark.parametrize("fmt", [1, 2, 3, 4])
@pytest.mark.parametrize("n", [256, 137, 1000])
def test_device_decode_matches_oracle(dev, fmt, n):
    rng = np.random.default_rng(fmt * n)
    v = rng.normal(0, 1, n).astype(np.float32)
    if fmt == 4:
        from summa_amd import ops
        q = ops.Q4Weight.quantize(torch.from_numpy(np.pad(v, (0, -n % 128))).to(dev).view(1, -1))
        t = PackedTensor(4, (n,), q.scales.cpu().numpy().view(np.uint16),
                         q.codes.cpu().numpy()[:((n + 127) // 128) * 64])
        # elements past n in the last group were quantized from zeros: codes 0
    else:
        s, c = oracle.hq_quantize(v, fmt)
        t = PackedTensor(fmt, (n,), s, c)
    PackedTensor.from_bytes(t.to_bytes())  # canonical
    got = t.decode(dev).cpu().numpy()
    np.testing.assert_array_equal(got, oracle.hq_decode(fmt, n, t.scales, t.codes))
    if n % 8 == 0:
        t2 = PackedTensor(t.format, (8, n // 8), t.scales, t.codes)
        gt = t2.decode(dev, transpose=True).cpu().numpy()
        np.testing.assert_array_equal(gt, got.reshape(8, n // 8).T)


def test_safetensors_load_matches_host_weights(dev, tmp_path):
    cfg = CFG.oracle_cfg()
    w = oracle.random_weights(cfg, seed=3, std=0.05)
    ref = Model(CFG)
    ref.load_host_weights(w, dev)
    p = tmp_path / "model.safetensors"
    checkpoint.write_safetensors(p, burn_weights(w, CFG))
    m = Model(CFG)
    info = checkpoint.load_safetensors(m, p)
    assert not info["tied"]
    _, _, a = _lp(ref, dev)
    _, _, b = _lp(m, dev)
    np.testing.assert_array_equal(a, b)


def test_safetensors_tied_output_and_strictness(dev, tmp_path):
    cfg = CFG.oracle_cfg()
    w = oracle.random_weights(cfg, seed=4, std=0.05)
    w_tied = dict(w, lm_head=w["embed"].copy())
    ref = Model(CFG)
    ref.load_host_weights(w_tied, dev)
    p = tmp_path / "tied.safetensors"
    checkpoint.write_safetensors(p, burn_weights(w, CFG, tied=True))
    m = Model(CFG)
    assert checkpoint.load_safetensors(m, p)["tied"]
    np.testing.assert_array_equal(_lp(ref, dev)[2], _lp(m, dev)[2])
    bw = burn_weights(w, CFG)
    for mutate, msg in [(lambda d: d.pop("layers.1.ffn_norm.gamma"), "missing: \\['layers.1.ffn_norm.gamma'\\]"),
                        (lambda d: d.__setitem__("extra.bias", np.zeros(3, np.float32)), "unused: \\['extra.bias'\\]"),
                        (lambda d: d.__setitem__("final_norm.gamma", np.zeros(5, np.float32)), "final_norm.gamma: shape")]:
        d = dict(bw)
        mutate(d)
        q = tmp_path / "bad.safetensors"
        checkpoint.write_safetensors(q, d)
        with pytest.raises(checkpoint.CheckpointError, match=msg):
            checkpoint.load_safetensors(Model(CFG), q)


@pytest.mark.parametrize("fmt", ["binary_g128", "ternary_g128", "ternary_entropy_g128"])
def test_reference_format_archive_into_fp32_model(dev, tmp_path, fmt):
    """Matrices packed by the reference codec (oracle restatement) in Burn's
    [in, out] layout: the model computes with exactly the decoded weights."""
    cfg = CFG.oracle_cfg()
    w = oracle.random_weights(cfg, seed=5, std=0.05)
    bw = burn_weights(w, CFG)
    f = hquant.FORMATS[fmt]
    mats, flts, decoded = {}, {}, {}
    for name, a in bw.items():
        if a.ndim == 2 and name != "embedding.weight":
            s, c = oracle.hq_quantize(a, f)
            mats[name] = PackedTensor(f, a.shape, s, c)
            decoded[name] = oracle.hq_decode(f, a.size, s, c).reshape(a.shape)
        else:
            flts[name] = ("F32", a.shape, a.tobytes())
            decoded[name] = a
    root = tmp_path / "arc"
    hquant.write_archive(root, mats, flts, fmt, SRC)
    m = Model(CFG)
    info = checkpoint.load_archive(m, root)
    assert info["matrices"] == len(mats)
    # the same weights decoded on the host, installed densely
    p = tmp_path / "decoded.safetensors"
    checkpoint.write_safetensors(p, decoded)
    ref = Model(CFG)
    checkpoint.load_safetensors(ref, p)
    np.testing.assert_array_equal(_lp(ref, dev)[2], _lp(m, dev)[2])


def test_q4_archive_export_roundtrip_is_bit_exact(dev, tmp_path):
    """Q4G128 export of a model's weights, re-imported into a quantized model:
    the same codes and scales as quantizing on load, so the same log-probs."""
    qc = ModelConfig(**{**CFG.__dict__, "quantized": True})
    cfg = qc.oracle_cfg()
    w = oracle.random_weights(cfg, seed=6, std=0.05)
    ref = Model(qc)
    ref.load_host_weights(w, dev)
    root = tmp_path / "q4"
    man = checkpoint.export_q4_archive(burn_weights(w, qc), qc, root, SRC)
    assert man["recipe"]["format"] == "q4_g128"
    m = Model(qc)
    checkpoint.load_archive(m, root)
    np.testing.assert_array_equal(_lp(ref, dev)[2], _lp(m, dev)[2])
    arc = hquant.QuantizedArchive.open(root)
    t = arc.matrices["layers.0.attention.qkv_proj.weight"]
    assert t.format == 4 and t.shape == ((CFG.heads + 2 * CFG.kv_heads) * CFG.head_dim, CFG.d_model)
