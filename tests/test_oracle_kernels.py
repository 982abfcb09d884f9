"""Pins each oracle kernel against float64 mathematics: numpy closed forms and
torch CPU library routines (rms_norm, silu, scaled_dot_product_attention)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
import oracle_np as R

RS = np.random.RandomState(1234)


def f16_bits(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("M,K", [(7, 36), (64, 3072), (33, 4096), (16, 9216), (5, 2)])
def test_matvec_f16(M, K):
    A = f16_bits(RS.randn(M, K) * 0.02)
    x = RS.randn(K).astype(np.float32)
    y = O.matvec_f16(A, x)
    ref = R.f16(A) @ x.astype(np.float64)
    scale = np.abs(R.f16(A)) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(y - ref) <= 4e-7 * scale + 1e-30)
    # a transposed operand or a dropped pair half fails
    assert not np.allclose(y, R.f16(A)[:, ::2] @ x[::2], rtol=1e-3)


def test_rmsnorm_vs_torch():
    x = RS.randn(3072).astype(np.float32) * 3
    w = f16_bits(1 + 0.02 * RS.randn(3072))
    y = O.rmsnorm(x, w, 1e-5)
    ref = F.rms_norm(torch.tensor(x, dtype=torch.float64), (3072,),
                     torch.tensor(R.f16(w)), eps=1e-5).numpy()
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("pos", [0, 1, 128, 4095])
def test_rope_closed_form(pos):
    q = RS.randn(32 * 128).astype(np.float32)
    y = O.rope(q, 128, pos, 1e6)
    ref = R.rope_interleaved(q, 128, pos, 1e6)
    # f32 angle = pos*freq carries relative error ~2^-24 * pos
    np.testing.assert_allclose(y, ref, rtol=0, atol=2e-6 * max(1, pos) ** 0.5 * 8)
    if pos == 0:
        assert np.array_equal(y, q)
    # rotation preserves each pair's norm
    n0 = q.reshape(-1, 2) ** 2
    n1 = y.reshape(-1, 2) ** 2
    np.testing.assert_allclose(n1.sum(1), n0.sum(1), rtol=1e-5)


@pytest.mark.parametrize("seq", [1, 129, 513, 1000])
def test_attention_decode_vs_sdpa(seq):
    nh, nkv, hd = 32, 8, 128
    q = RS.randn(nh * hd).astype(np.float32)
    K = RS.randn(seq, nkv * hd).astype(np.float32)
    V = RS.randn(seq, nkv * hd).astype(np.float32)
    out, scores = O.attention_decode(q, K, V, nh, nkv, hd, seq)
    qt = torch.tensor(q, dtype=torch.float64).view(1, nh, 1, hd)
    kt = torch.tensor(K, dtype=torch.float64).view(seq, nkv, hd).permute(1, 0, 2).repeat_interleave(nh // nkv, 0)[None]
    vt = torch.tensor(V, dtype=torch.float64).view(seq, nkv, hd).permute(1, 0, 2).repeat_interleave(nh // nkv, 0)[None]
    ref = F.scaled_dot_product_attention(qt, kt, vt).view(-1).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=2e-5)
    np.testing.assert_allclose(scores.reshape(nh, seq).sum(1), 1.0, rtol=1e-5)
    assert np.allclose(out, R.gqa_decode(q.astype(np.float64), K.astype(np.float64), V.astype(np.float64), nh, nkv, hd), atol=2e-5)


def test_attention_identical_keys_is_mean_of_v():
    nh, nkv, hd, seq = 8, 2, 64, 50
    q = RS.randn(nh * hd).astype(np.float32)
    K = np.tile(RS.randn(1, nkv * hd).astype(np.float32), (seq, 1))
    V = RS.randn(seq, nkv * hd).astype(np.float32)
    out, _ = O.attention_decode(q, K, V, nh, nkv, hd, seq)
    mean = V.astype(np.float64).mean(0).reshape(nkv, hd)
    ref = np.repeat(mean, nh // nkv, 0).ravel()
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_swiglu_vs_torch():
    g = (RS.randn(9216) * 4).astype(np.float32)
    u = RS.randn(9216).astype(np.float32)
    y = O.swiglu(g, u)
    ref = (F.silu(torch.tensor(g, dtype=torch.float64)) * torch.tensor(u, dtype=torch.float64)).numpy()
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("t", [0.0, 1 / 7, 3 / 7, 6 / 7])
def test_time_embedding_closed_form(t):
    y = O.time_embedding(3072, np.float32(t))
    np.testing.assert_allclose(y, R.time_embedding(3072, np.float32(t)), atol=3e-7)
    if t == 0.0:
        assert np.all(y[:1536] == 1.0) and np.all(y[1536:] == 0.0)


def test_cfg_and_euler():
    vc = RS.randn(36).astype(np.float32)
    vu = RS.randn(36).astype(np.float32)
    np.testing.assert_allclose(O.cfg_combine(vc, vu, 1.2), 1.2 * vc.astype(np.float64) - 0.2 * vu, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(O.cfg_combine(vc, vc, 1.2), vc, rtol=1e-6)
    x = RS.randn(36).astype(np.float32)
    assert np.array_equal(O.euler_step(x, np.zeros(36, np.float32), np.float32(1 / 7)), x)
    np.testing.assert_allclose(O.euler_step(x, vc, np.float32(1 / 7)), x + vc / 7.0, rtol=1e-6, atol=1e-7)


def test_fsq_known_answers():
    # exact ties: (x+1)*0.5*20 = 2.5, 12.5, 7.5, 17.5 for x = -0.75, 0.25, -0.25, 0.75;
    # half-to-even gives 2, 12, 8, 18 (half-away-from-zero would give 3, 13)
    x = np.array([-1.0, 0.0, 1.0, -5.0, 5.0, -0.75, 0.25, -0.25, 0.75], np.float32)
    assert list(O.fsq_quantize(x)) == [2, 12, 22, 2, 22, 4, 14, 10, 20]
    xs = np.linspace(-1.2, 1.2, 2001).astype(np.float32)
    ref = np.clip(np.rint((np.clip(xs, -1, 1) + 1) * np.float32(0.5) * 20), 0, 20).astype(np.uint32) + 2
    assert np.array_equal(O.fsq_quantize(xs), ref)


def test_argmax_tree_tie_rule():
    x = RS.randn(131072).astype(np.float32)
    assert O.argmax(x) == int(np.argmax(x))  # tie-free data: the maximum
    # Exact ties follow the shader's 256-lane tree (src/shaders.ts:1154-1211).
    # Hand trace for maxima at 5 (lane 5), 700 (lane 188), 131000 (lane 184):
    # s=128 moves 184->56 and 188->60; s=32 moves 56->24, 60->28; s=16 ->8, 12;
    # s=8 -> 0, 4; s=4: lane 0 (131000) ties lane 4 (700) and keeps 131000,
    # lane 1 takes lane 5; s=1: lane 0 ties lane 1 and keeps 131000.
    x[[5, 700, 131000]] = 100.0
    assert O.argmax(x) == 131000
    # ties inside one lane's strided run keep the first index
    y = np.zeros(8320, np.float32)
    y[[3, 3 + 256, 3 + 512]] = 1.0
    assert O.argmax(y) == 3
    # all-equal input: lane 0, index 0
    assert O.argmax(np.zeros(8320, np.float32)) == 0


def test_multi_codebook_embed_rows():
    dim = 64
    table = f16_bits(RS.randn(9088, dim))
    sem = 4321
    ac = RS.randint(2, 23, 36).astype(np.uint32)
    out = O.multi_codebook_embed(table, sem, ac, dim)
    rows = [sem] + [8194 + k * 23 + int(ac[k]) for k in range(36)]
    ref = R.f16(table)[rows].sum(0)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)


def test_bi_attention_vs_sdpa():
    nh, nkv, hd = 32, 8, 128
    q = RS.randn(3, nh * hd).astype(np.float32)
    k = RS.randn(3, nkv * hd).astype(np.float32)
    v = RS.randn(3, nkv * hd).astype(np.float32)
    out, scores = O.bi_attention(q, k, v, nh, nkv, hd)
    qt = torch.tensor(q, dtype=torch.float64).view(3, nh, hd).permute(1, 0, 2)[None]
    kt = torch.tensor(k, dtype=torch.float64).view(3, nkv, hd).permute(1, 0, 2).repeat_interleave(4, 0)[None]
    vt = torch.tensor(v, dtype=torch.float64).view(3, nkv, hd).permute(1, 0, 2).repeat_interleave(4, 0)[None]
    ref = F.scaled_dot_product_attention(qt, kt, vt)[0].permute(1, 0, 2).reshape(-1).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(scores.reshape(-1, 3).sum(1), 1.0, rtol=1e-6)
