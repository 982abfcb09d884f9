"""vx_load_safetensors: a local safetensors file of mixed dtypes loaded
into the engine with the reference's conversions, then a decode step
against the oracle given the same converted weights."""
import json
import struct

import numpy as np
import pytest

import oracle as O
import voxtral_amd as V
from vxtest import fill_oracle_kv, gpu_engine, max_rel_err, oracle_engine

pytestmark = pytest.mark.gpu


def write_safetensors(path, tensors):
    """tensors: name -> (dtype string, numpy array of the raw element type)"""
    header, blobs, off = {"__metadata__": {"format": "pt"}}, [], 0
    for name, (dt, arr) in tensors.items():
        raw = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def to_bf16_bits(x):
    """f32 -> BF16 bits, round to nearest even"""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def test_load_mixed_dtypes_then_decode(tmp_path):
    g = gpu_engine(n_layers=1, max_seq=64)
    o = oracle_engine(n_layers=1, max_seq=64)
    try:
        rng = np.random.default_rng(5)
        wq = (rng.standard_normal((4096, 3072)) * 0.02).astype(np.float32)
        wo = (rng.standard_normal((3072, 4096)) * 0.02).astype(np.float32)
        an = (1 + rng.standard_normal(3072) * 0.1).astype(np.float32)
        fn16 = (1 + rng.standard_normal(3072) * 0.1).astype(np.float16)
        path = tmp_path / "model.safetensors"
        write_safetensors(path, {
            "layers.0.attention.wq.weight": ("BF16", to_bf16_bits(wq)),
            "layers.0.attention.wo.weight": ("BF16", to_bf16_bits(wo)),
            "layers.0.attention_norm.weight": ("F32", an),
            "layers.0.ffn_norm.weight": ("F16", fn16.view(np.uint16)),
            "audio_tokenizer.decoder.weight": ("BF16", np.zeros((4, 4), np.uint16)),
            "something.else": ("F32", np.zeros(3, np.float32)),
        })
        loaded, skipped = g.load_safetensors(path)
        assert (loaded, skipped) == (4, 2)
        expect = {
            "layers.0.attention.wq.weight": V.bf16_to_f16(to_bf16_bits(wq)).ravel(),
            "layers.0.attention.wo.weight": V.bf16_to_f16(to_bf16_bits(wo)).ravel(),
            "layers.0.attention_norm.weight": V.f32_to_f16_trunc(an),
            "layers.0.ffn_norm.weight": fn16.view(np.uint16),
        }
        for name, bits in expect.items():
            assert np.array_equal(g.read_tensor(name, bits.size), bits), name
            o.set_weight(name, bits)
        # the engine computes with exactly these weights
        x = O.gen_f32(9, "input.hidden", 3072)
        g.fill_kv_synthetic(0, 20)
        fill_oracle_kv(o, 0, 20)
        g.position = 20
        o.position = 20
        _, gn = g.backbone_step(precomputed=x)
        o.backbone_step(precomputed=x)
        assert max_rel_err(gn, o.buffer("normed")) < 1e-3
    finally:
        g.destroy()
        o.close()


def test_loader_errors(tmp_path):
    g = gpu_engine(n_layers=1, max_seq=16)
    try:
        with pytest.raises(V.VoxtralError, match="cannot open"):
            g.load_safetensors(tmp_path / "missing.safetensors")
        bad = tmp_path / "bad.safetensors"
        bad.write_bytes(struct.pack("<Q", 5) + b"{oops")
        with pytest.raises(V.VoxtralError, match="header"):
            g.load_safetensors(bad)
        # a deeply nested value (rejected, not recursed into) and an offset
        # outside int64
        for hdr in (b'{"__metadata__":' + b"[" * 200000 + b"]" * 200000 + b"}",
                    b'{"norm.weight":{"dtype":"F16","shape":[3072],"data_offsets":[0,99999999999999999999]}}'):
            bad.write_bytes(struct.pack("<Q", len(hdr)) + hdr)
            with pytest.raises(V.VoxtralError, match="header"):
                g.load_safetensors(bad)
        p = tmp_path / "dtype.safetensors"
        write_safetensors(p, {"layers.0.ffn_norm.weight": ("I32", np.zeros(3072, np.int32))})
        with pytest.raises(V.VoxtralError, match="Unsupported dtype for layers.0.ffn_norm.weight: I32"):
            g.load_safetensors(p)
        p = tmp_path / "shape.safetensors"
        write_safetensors(p, {"layers.0.ffn_norm.weight": ("F16", np.zeros(3000, np.uint16))})
        with pytest.raises(V.VoxtralError, match="expected"):
            g.load_safetensors(p)
        p = tmp_path / "short.safetensors"
        write_safetensors(p, {"layers.0.ffn_norm.weight": ("F16", np.zeros(3072, np.uint16))})
        raw = p.read_bytes()
        p.write_bytes(raw[:-100])
        with pytest.raises(V.VoxtralError):
            g.load_safetensors(p)
        assert g.is_ready  # nothing was half-loaded by the failures
    finally:
        g.destroy()
