"""Pins the oracle's number plumbing: f16 conversion, splitmix64, and the
counter-based normal generator shared with the GPU initialiser."""
import ctypes

import numpy as np

import oracle as O


def test_splitmix64_published_vectors():
    # First outputs of splitmix64 from state 0 (Vigna's reference generator).
    s = ctypes.c_uint64(0)
    got = [O.lib().vxo_splitmix64_next(ctypes.byref(s)) for _ in range(3)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([O.lib().vxo_f16_to_f32(int(b)) for b in bits], np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    # and every finite half round-trips through f32 -> f16
    back = np.array([O.lib().vxo_f32_to_f16(float(v)) for v in ref[finite]], np.uint16)
    assert np.array_equal(back, bits[finite])


def test_f32_to_f16_rne_matches_numpy():
    rs = np.random.RandomState(0)
    x = (rs.randn(50000) * 10.0 ** rs.uniform(-9, 5.5, 50000)).astype(np.float32)
    edges = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2 ** -24, 2 ** -25,
                      2 ** -25 * 1.0000001, 3 * 2 ** -25, 2 ** -14, 2 ** -14 * (1 - 2 ** -11),
                      1 + 2 ** -11, 1 + 3 * 2 ** -11, 1 + 2 ** -11 + 2 ** -20], np.float32)
    x = np.concatenate([x, edges, -edges])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = np.array([O.lib().vxo_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, ref)


def _mix64(z):
    z = np.uint64(z)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def test_normal_generator_definition():
    seed, name = 7, "layers.0.attention.wq.weight"
    stream = O.name_stream(name)
    # FNV-1a 64 of the name
    h = 0xcbf29ce484222325
    for ch in name.encode():
        h = ((h ^ ch) * 0x100000001b3) & (2 ** 64 - 1)
    assert stream == h
    s0 = int(_mix64(seed)) ^ stream
    for idx in (0, 1, 12345, 10 ** 9):
        tot = 0
        for j in range(4):
            with np.errstate(over="ignore"):
                st = np.uint64((s0 + (4 * idx + j + 1) * 0x9E3779B97F4A7C15) % 2 ** 64)
            hh = int(_mix64(st))
            tot += (hh & 0xFFFFF) + ((hh >> 20) & 0xFFFFF) + ((hh >> 40) & 0xFFFFF)
        expect = np.float32(tot - 6 * 0xFFFFF) * np.float32(2.0 ** -20)
        assert O.lib().vxo_normal(seed, stream, idx) == expect


def test_normal_generator_moments_and_streams():
    z = O.gen_f32(0, "a", 1 << 20)
    assert abs(z.mean()) < 3e-3 and abs(z.std() - 1.0) < 3e-3
    assert np.abs(z).max() <= 6.0
    z2 = O.gen_f32(0, "b", 1 << 16)
    z3 = O.gen_f32(1, "a", 1 << 16)
    assert abs(np.corrcoef(z[: 1 << 16], z2)[0, 1]) < 0.02
    assert abs(np.corrcoef(z[: 1 << 16], z3)[0, 1]) < 0.02
    w = O.gen_f16(0, "a", 1 << 16, 0.0, 0.02)
    assert np.array_equal(w, (z[: 1 << 16] * np.float32(0.02)).astype(np.float16).view(np.uint16))
    g = O.gen_f16(0, "a", 1 << 16, 1.0, 0.02)
    assert np.array_equal(g, (np.float32(1.0) + z[: 1 << 16] * np.float32(0.02)).astype(np.float16).view(np.uint16))
