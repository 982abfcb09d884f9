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


# --- Box-Muller generator of the FM noise (vxo_gauss) -----------------------
_LOGC = [float.fromhex(h) for h in (
    "0x1.5555555555555p-2", "0x1.999999999999ap-3", "0x1.2492492492492p-3", "0x1.c71c71c71c71cp-4",
    "0x1.745d1745d1746p-4", "0x1.3b13b13b13b14p-4", "0x1.1111111111111p-4", "0x1.e1e1e1e1e1e1ep-5")]
_COSC = [float.fromhex(h) for h in (
    "-0x1.0000000000000p-1", "0x1.5555555555555p-5", "-0x1.6c16c16c16c17p-10", "0x1.a01a01a01a01ap-16",
    "-0x1.27e4fb7789f5cp-22", "0x1.1eed8eff8d898p-29", "-0x1.93974a8c07c9dp-37", "0x1.ae7f3e733b81fp-45",
    "-0x1.6827863b97d97p-53", "0x1.e542ba4020225p-62")]
_SINC = [float.fromhex(h) for h in (
    "-0x1.5555555555555p-3", "0x1.1111111111111p-7", "-0x1.a01a01a01a01ap-13", "0x1.71de3a556c734p-19",
    "-0x1.ae64567f544e4p-26", "0x1.6124613a86d09p-33", "-0x1.ae7f3e733b81fp-41", "0x1.952c77030ad4ap-49",
    "-0x1.2f49b46814157p-57", "0x1.71b8ef6dcf572p-66")]


def _fma(a, b, c):
    from fractions import Fraction
    return float(Fraction(a) * Fraction(b) + Fraction(c))  # exact product and sum, one rounding


def _uniform_pair(seed, stream, idx):
    s0 = int(_mix64(seed)) ^ stream
    h = []
    for j in (1, 2):
        with np.errstate(over="ignore"):
            st = np.uint64((s0 + (2 * idx + j) * 0x9E3779B97F4A7C15) % 2 ** 64)
        h.append(int(_mix64(st)))
    return (h[0] >> 11) + 1, h[1] >> 11  # u1 = N 2^-53 in (0, 1], u2 = U 2^-53 in [0, 1)


def _gauss_restated(seed, stream, idx):
    """The generator's operations in Python doubles (each fma exact, then
    rounded once), i.e. what a correct implementation must return bit for bit."""
    import math
    N, U = _uniform_pair(seed, stream, idx)
    m, e = math.frexp(float(N))
    m, e = m * 2.0, e - 1  # N = m 2^e, m in [1, 2)
    if m > float.fromhex("0x1.6a09e667f3bcdp+0"):
        m, e = m * 0.5, e + 1
    s = (m - 1.0) / (m + 1.0)
    s2 = s * s
    p = _LOGC[7]
    for k in range(6, -1, -1):
        p = _fma(s2, p, _LOGC[k])
    lu = _fma(float(e - 53), float.fromhex("0x1.62e42fefa39efp-1"), 2.0 * _fma(s * s2, p, s))
    r = math.sqrt(-2.0 * lu)
    q = U >> 51
    x = (float(U & ((1 << 51) - 1)) * 2.0 ** -51) * float.fromhex("0x1.921fb54442d18p+0")
    x2 = x * x
    c, sn = _COSC[9], _SINC[9]
    for k in range(8, -1, -1):
        c = _fma(x2, c, _COSC[k])
        sn = _fma(x2, sn, _SINC[k])
    c = _fma(x2, c, 1.0)
    sn = _fma(x * x2, sn, x)
    return np.float32(r * (c, -sn, -c, sn)[q])


def test_gauss_generator_is_its_restatement_bit_for_bit():
    stream = O.name_stream("fm.noise")
    for seed in (0, 1, 12345):
        for idx in list(range(40)) + [10 ** 6, 2 ** 40 + 7]:
            got = np.float32(O.lib().vxo_gauss(seed, stream, idx))
            assert got.view(np.uint32) == _gauss_restated(seed, stream, idx).view(np.uint32), (seed, idx)


def test_gauss_generator_is_box_muller():
    """src/engine.ts:1264-1273: sqrt(-2 ln u1) cos(2 pi u2), here with the
    library log / cos in float64 (the series agree to f32 rounding)."""
    stream = O.name_stream("fm.noise")
    n = 2000
    got = O.gen_gauss_f32(7, "fm.noise", n).astype(np.float64)
    pairs = np.array([_uniform_pair(7, stream, i) for i in range(n)], np.float64)
    u1, u2 = pairs[:, 0] * 2.0 ** -53, pairs[:, 1] * 2.0 ** -53
    ref = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    assert np.max(np.abs(got - ref) / (1.0 + np.abs(ref))) < 2e-7


def test_gauss_generator_moments_and_tails():
    z = O.gen_gauss_f32(0, "a", 1 << 20).astype(np.float64)
    assert abs(z.mean()) < 3e-3 and abs(z.std() - 1.0) < 3e-3
    kurt = np.mean((z - z.mean()) ** 4) / z.var() ** 2
    assert abs(kurt - 3.0) < 0.03  # the Irwin-Hall(12) sum has 2.9
    # Gaussian tails: P(|z| > 4) = 6.3e-5, about 66 of 2^20; Irwin-Hall(12) stops at 6
    n4 = int(np.sum(np.abs(z) > 4.0))
    assert 40 < n4 < 100
    assert np.abs(z).max() > 4.5
