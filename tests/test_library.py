"""CPU-side checks of the C ABI library: it loads, exports exactly what
include/voxtral_engine.h declares, and fails loudly without a device."""
import ctypes
import os
import re

import pytest

import voxtral_amd as V

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "voxtral_engine.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(vx_[a-z0-9_]+)\s*\(", text)
    return sorted(set(n for n in names if not n.endswith("_cb")))


def test_library_exports_every_declared_symbol():
    lib = V.load_library()
    declared = header_functions()
    assert len(declared) >= 25
    for name in declared:
        assert hasattr(lib, name), f"{name} declared but not exported"
    # and the Python binding covers every declared entry point
    assert sorted(V.exported_symbols()) == declared


def test_config_default_matches_reference_types():
    c = V.default_config()
    assert (c.dim, c.n_layers, c.head_dim, c.hidden_dim, c.n_heads, c.n_kv_heads) == (3072, 26, 128, 9216, 32, 8)
    assert c.vocab_size == 131072 and abs(c.rope_theta - 1e6) < 1 and abs(c.norm_eps - 1e-5) < 1e-12
    assert (c.fm_layers, c.nfe, c.n_acoustic_out, c.semantic_vocab) == (3, 8, 36, 8320)
    assert abs(c.cfg_alpha - 1.2) < 1e-6 and c.acoustic_levels == 21


def _has_gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device error path")
def test_create_without_device_fails_loudly():
    with pytest.raises(V.VoxtralError) as ei:
        V.VoxtralEngine().init()
    assert ei.value.code == V.VX_E_DEVICE
    assert "device" in str(ei.value).lower()


def test_create_rejects_unsupported_shapes():
    cfg = V.default_config(dim=1024)
    with pytest.raises(V.VoxtralError) as ei:
        V.VoxtralEngine(cfg).init()
    assert ei.value.code == V.VX_E_INVALID
    assert "unsupported shape" in str(ei.value)


def test_null_handle_calls_are_rejected():
    lib = V.load_library()
    assert lib.vx_reset(None) == V.VX_E_INVALID
    assert lib.vx_is_ready(None) == 0
    assert lib.vx_position(None) == -1
    lib.vx_destroy(None)
    assert isinstance(lib.vx_last_error(None), bytes)
    f = ctypes.c_float()
    assert lib.vx_time_backbone_steps(None, 1, 0, ctypes.byref(f)) == V.VX_E_INVALID
