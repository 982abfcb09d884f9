"""The reference's dtype conversions of the safetensors loader
(src/weights.ts), run by the library on the host."""
import numpy as np
import pytest

import voxtral_amd as V


def bf16_value(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def f16_value(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def test_bf16_normal_range_is_exact():
    """Every BF16 value inside the f16 normal range converts exactly (BF16
    has 7 mantissa bits, f16 10)."""
    b = np.arange(65536, dtype=np.uint16)
    f = V.bf16_to_f16(b)
    v = bf16_value(b)
    normal = np.isfinite(v) & (np.abs(v) >= 2.0 ** -14) & (np.abs(v) <= 65504)
    assert normal.sum() == 2 * 30 * 128  # signs x f16 normal exponents x BF16 mantissas
    assert np.array_equal(f16_value(f[normal]), v[normal])
    # sign symmetry over the whole table
    assert np.array_equal(f[b >= 0x8000] & 0x7FFF, f[b < 0x8000])
    assert np.all(f[b >= 0x8000] & 0x8000)


def test_bf16_special_values():
    f = V.bf16_to_f16(np.array([0x0000, 0x8000, 0x0001, 0x7F80, 0xFF80, 0x7FC0, 0x7F81,
                                0x4780, 0xC780, 0x477F], np.uint16))
    # zero, BF16 subnormal -> zero, inf, NaN (f16 NaN 0x7E00), overflow -> inf,
    # the largest value below 65536 (65280) exactly
    assert list(f) == [0x0000, 0x8000, 0x0000, 0x7C00, 0xFC00, 0x7E00, 0x7E00, 0x7C00, 0xFC00, 0x7BF8]
    assert f16_value([0x7BF8])[0] == 65280.0


def test_bf16_subnormal_branch_follows_the_reference():
    """Below 2^-14 the reference shifts the mantissa (src/weights.ts:117-126)
    rather than rounding: 2^-15 becomes 0x0020 (2^-19), where a correctly
    rounded conversion gives 0x0200; values below 2^-24 become zero."""
    f = V.bf16_to_f16(np.array([0x3800, 0x3780, 0x3400, 0x3380, 0x3300, 0xB800], np.uint16))
    # 2^-15, 2^-16, 2^-23, 2^-24, 2^-25, -2^-15
    assert list(f) == [0x0020, 0x0010, 0x0000, 0x0000, 0x0000, 0x8020]
    correct = np.float32(2.0 ** -15).astype(np.float16).view(np.uint16)
    assert correct == 0x0200


def test_f32_to_f16_truncates():
    x = np.array([1.0, 1 + 2 ** -10, 1 + 3 * 2 ** -12, -2.5, 1e-6, 6.2e-5, 70000.0, np.inf,
                  -np.inf, np.nan, 65519.0, 0.0], np.float32)
    f = V.f32_to_f16_trunc(x)
    # 1 + 3*2^-12 truncates to 1.0 (round-to-nearest would give 0x3C01); no
    # subnormals: 1e-6 -> 0; 6.2e-5 is normal (0x0410); overflow, inf and NaN -> inf
    assert list(f) == [0x3C00, 0x3C01, 0x3C00, 0xC100, 0x0000, 0x0410, 0x7C00, 0x7C00, 0xFC00,
                       0x7C00, 0x7BFF, 0x0000]
    assert np.float32(1 + 3 * 2 ** -12).astype(np.float16).view(np.uint16) == 0x3C01
