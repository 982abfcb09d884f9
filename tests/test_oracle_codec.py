"""The oracle's codec decoder (oracle/vx_oracle_codec.c) pinned against
torch's own float64 operators and known answers: conv and transposed conv
with weight norm, RMSNorm, per-head QK norm, windowed ALiBi attention, VQ
codebook normalisation, FSQ dequantisation, and the whole decoder (every
debugCodecDecode intermediate) against tests/codec_f64.py."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import codec_f64 as R
import oracle as O
from vxtest import max_rel_err


def f16bits(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def test_fsq_dequant_known_answers():
    codes = np.array([2, 12, 22, 7, 17, 0], np.uint32)
    out = np.empty(6, np.float32)
    O.lib().vxo_fsq_dequant(codes, out, 6, 21, 2)
    assert list(out[:5]) == [-1.0, 0.0, 1.0, -0.5, 0.5]
    # code 0: u32 wrap-around of code - 2, as the shader's u32 arithmetic does
    assert out[5] == np.float32(np.float32(2 ** 32 - 2) * 2 / 20 - 1)


def test_vq_normalize_and_lookup():
    rng = np.random.default_rng(1)
    n, d = 37, 16
    s = f16bits(rng.standard_normal((n, d)))
    u = f16bits(np.abs(rng.standard_normal(n)) * 3)
    u[3] = f16bits([0.0])[0]           # max(usage, eps) clamps to eps
    u[4] = f16bits([1e-7])[0]          # f16 subnormal below eps
    cb = np.empty(n * d, np.uint16)
    O.lib().vxo_normalize_codebook(s.ravel(), u, cb, n, d, np.float32(1e-5))
    uf = np.maximum(u.view(np.float16).astype(np.float32), np.float32(1e-5))
    with np.errstate(over="ignore"):  # clamped usage: f16 overflow to inf, as in the kernel
        expect = (s.view(np.float16).astype(np.float32) / uf[:, None]).astype(np.float16).view(np.uint16)
    assert np.array_equal(cb.reshape(n, d), expect)
    codes = np.array([0, 36, 5, 37, 1000], np.uint32)
    out = np.empty(5 * d, np.float32)
    O.lib().vxo_vq_lookup(codes, cb, out, 5, d, n)
    out = out.reshape(5, d)
    cbf = cb.view(np.float16).astype(np.float32).reshape(n, d)
    assert np.array_equal(out[:3], cbf[[0, 36, 5]])
    assert not out[3:].any()  # rows past the table read as zero


@pytest.mark.parametrize("c_in,c_out,k,T", [(6, 5, 3, 7), (292, 16, 3, 4), (32, 12, 7, 9)])
def test_causal_conv1d_vs_torch(c_in, c_out, k, T):
    rng = np.random.default_rng(c_in + k)
    x = rng.standard_normal((T, c_in)).astype(np.float32)
    v = f16bits(rng.standard_normal((c_out, c_in, k)) * 0.1)
    g = f16bits(1 + rng.standard_normal(c_out) * 0.2)
    out = np.empty(T * c_out, np.float32)
    O.lib().vxo_causal_conv1d(x, v.ravel(), g, out, c_in, c_out, k, T, 1)
    ref = R.causal_conv(torch.from_numpy(x.astype(np.float64)), R.w64(v, v.shape), R.w64(g, (c_out,)), k)
    assert max_rel_err(out.reshape(T, c_out), ref.numpy()) < 1e-5


@pytest.mark.parametrize("c_in,c_out,T", [(8, 6, 5), (64, 16, 3)])
def test_conv_transpose_vs_torch(c_in, c_out, T):
    rng = np.random.default_rng(c_in)
    x = rng.standard_normal((T, c_in)).astype(np.float32)
    v = f16bits(rng.standard_normal((c_in, c_out, 4)) * 0.1)
    g = f16bits(1 + rng.standard_normal(c_in) * 0.2)
    scale = np.empty(c_in, np.float32)
    O.lib().vxo_conv_transpose_scale(v.ravel(), g, scale, c_in, c_out, 4)
    norm = np.sqrt((v.view(np.float16).astype(np.float64) ** 2).sum(axis=(1, 2)))
    assert max_rel_err(scale, g.view(np.float16).astype(np.float64) / norm) < 1e-6
    out = np.empty(2 * T * c_out, np.float32)
    O.lib().vxo_conv_transpose1d(x, v.ravel(), scale, out, c_in, c_out, 4, 2 * T, 2)
    ref = R.conv_up(torch.from_numpy(x.astype(np.float64)), R.w64(v, v.shape), R.w64(g, (c_in,)))
    assert max_rel_err(out.reshape(2 * T, c_out), ref.numpy()) < 1e-5


def test_rmsnorm_and_qk_norm_vs_torch():
    rng = np.random.default_rng(4)
    T, H, hd = 5, 8, 16
    x = rng.standard_normal((T, H * hd)).astype(np.float32)
    w = f16bits(1 + rng.standard_normal(H * hd) * 0.1)
    out = np.empty_like(x)
    O.lib().vxo_batched_rmsnorm(x, w, out, H * hd, T, np.float32(0.01))
    ref = F.rms_norm(torch.from_numpy(x.astype(np.float64)), (H * hd,), R.w64(w, (H * hd,)), 0.01)
    assert max_rel_err(out, ref.numpy()) < 1e-6
    q = x.copy()
    O.lib().vxo_qk_norm(q, w, H, hd, T, np.float32(1e-6))
    ref = R.qk_norm(torch.from_numpy(x.astype(np.float64)), R.w64(w, (H * hd,)), H, 1e-6)
    assert max_rel_err(q, ref.numpy()) < 1e-6


@pytest.mark.parametrize("W", [1, 2, 5, 16])
def test_windowed_alibi_attention_vs_dense(W):
    rng = np.random.default_rng(W)
    T, H, hd = 11, 8, 16
    q, k, v = (rng.standard_normal((T, H * hd)).astype(np.float32) for _ in range(3))
    out = np.empty_like(q)
    O.lib().vxo_codec_attention(q, k, v, out, H, hd, T, W)
    t64 = lambda a: torch.from_numpy(a.astype(np.float64))
    ref = R.attention(t64(q), t64(k), t64(v), H, W)
    assert max_rel_err(out, ref.numpy()) < 1e-5
    if W == 1:  # only the key itself: the output is V
        assert max_rel_err(out, v) < 1e-6


def test_batched_matvec_matches_single():
    rng = np.random.default_rng(9)
    M, K, T = 24, 512, 11
    A = f16bits(rng.standard_normal((M, K)) * 0.1)
    x = rng.standard_normal((T, K)).astype(np.float32)
    out = np.empty((T, M), np.float32)
    O.lib().vxo_batched_matvec_f16(A, x, out, M, K, T)
    for t in range(T):
        assert np.array_equal(out[t], O.matvec_f16(A, x[t]))


@pytest.fixture(scope="module")
def codec():
    c = O.OracleCodec()
    c.init_synthetic(0, 0.02)
    yield c
    c.close()


def test_weight_table(codec):
    names = codec.names()
    assert len(names) == len(set(names)) == 2 + 4 * 2 * 13 + 3 * 2 + 2 + 2
    assert "audio_tokenizer.decoder_blocks.7.layers.1.ffn_scale" in names
    assert "audio_tokenizer.decoder_blocks.6.conv.parametrizations.weight.original1" in names
    assert "audio_tokenizer.decoder_blocks.8.conv.parametrizations.weight.original1" not in names


@pytest.mark.parametrize("T", [1, 3])
def test_decoder_vs_f64_model(codec, T):
    rng = np.random.default_rng(T)
    sem = rng.integers(2, 8194, T).astype(np.uint32)
    sem[0] = 8193  # past the 8192-row codebook: a zero row
    ac = rng.integers(2, 23, (T, 36)).astype(np.uint32)
    weights = {n: codec.weight(n) for n in codec.names()}
    ref = R.decode(weights, sem, ac)
    # f32 against f64 through 8 layers and 4 convs: the error grows to about
    # 2e-6 of each tensor's largest value (1e-4 at the 1e-2 floor of
    # max_rel_err); an indexing or term mistake shows at 1e-2 or more
    for name in O.CODEC_STOPS:
        got = codec.decode(sem, ac, name)
        r = ref[name].ravel()
        err = max_rel_err(got, r)
        assert err < 1e-3 and np.abs(got - r).max() < 1e-5 * np.abs(r).max(), (name, err)
    assert not codec.decode(sem, ac, "concat")[:256].any()
    assert codec.decode(sem, ac).size == 1920 * T
