"""The oracle's fp16 conversion and q8_0 quantizer, pinned by numpy float16,
numpy rint / float64 half-away rounding and closed-form known answers."""
import numpy as np
import pytest

from _refs import q8_block_ref, dequant_ref

RNE, ROUNDF = 0, 1


def _special_f32():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e10, -1e10, np.inf, -np.inf,
            6.103515625e-05, 6.0975552e-05, 5.960464477539063e-08, 2.9802322387695312e-08,
            2.98023259e-08, 1e-30, -1e-30, 1.401298464324817e-45, 0.5, 1.0009765625, 1.00048828125,
            1.00146484375, 2049.0, 2051.0, 3.0517578125e-05, 1.52587890625e-05]
    return np.array(vals, dtype=np.float32)


@pytest.mark.filterwarnings("ignore:overflow")
def test_f16_matches_numpy_specials(oracle):
    x = _special_f32()
    got = oracle.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, ref)


@pytest.mark.filterwarnings("ignore:overflow")
def test_f16_matches_numpy_sweep(oracle):
    rng = np.random.default_rng(1)
    # every exponent band, including the subnormal and overflow edges of binary16
    bits = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    got = oracle.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, ref)
    # dense sweep around the binary16 range, where rounding matters
    y = (rng.standard_normal(200_000) * np.exp2(rng.integers(-30, 17, 200_000))).astype(np.float32)
    np.testing.assert_array_equal(oracle.f32_to_f16_bits(y), y.astype(np.float16).view(np.uint16))


def test_f16_nan_stays_nan(oracle):
    h = oracle.f32_to_f16_bits(np.array([np.nan], dtype=np.float32))[0]
    assert (h & 0x7C00) == 0x7C00 and (h & 0x3FF) != 0


def test_f16_to_f32_exact(oracle):
    h = np.arange(0, 65536, 97, dtype=np.uint16)
    h = h[(h & 0x7C00) != 0x7C00]
    got = oracle.f16_bits_to_f32(h)
    np.testing.assert_array_equal(got, h.view(np.float16).astype(np.float32))


@pytest.mark.parametrize("variant", [RNE, ROUNDF])
def test_q8_zero_block(oracle, variant):
    d, qs = oracle.quantize_block(np.zeros(32, np.float32), variant)
    assert d == 0 and not qs.any()


@pytest.mark.parametrize("variant", [RNE, ROUNDF])
def test_q8_integer_block_is_identity(oracle, variant):
    x = np.arange(-16, 16, dtype=np.float32) * 4
    x[0] = -127.0
    x[5] = 127.0
    d, qs = oracle.quantize_block(x, variant)
    assert d == 0x3C00                          # fp16 1.0
    np.testing.assert_array_equal(qs, x.astype(np.int8))


@pytest.mark.parametrize("variant", [RNE, ROUNDF])
@pytest.mark.parametrize("a", [1.0, 3.5, 1e-3, 250.0])
def test_q8_single_spike(oracle, variant, a):
    x = np.zeros(32, np.float32)
    x[7] = -a
    d, qs = oracle.quantize_block(x, variant)
    assert qs[7] == -127 and np.count_nonzero(qs) == 1
    assert d == int(np.float16(np.float32(a) / np.float32(127)).view(np.uint16))


@pytest.mark.parametrize("variant", [RNE, ROUNDF])
def test_q8_power_of_two_scaling(oracle, variant):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(32).astype(np.float32)
    d0, q0 = oracle.quantize_block(x, variant)
    for k in (-6, -1, 3, 9):
        d1, q1 = oracle.quantize_block(np.ldexp(x, k).astype(np.float32), variant)
        np.testing.assert_array_equal(q0, q1)
        assert np.float16(np.uint16(d1).view(np.float16)) == np.ldexp(np.uint16(d0).view(np.float16), k)


def test_q8_tie_rule_distinguishes_variants(oracle):
    # amax = 127 -> id = 1 for both variants; x = k + 0.5 is an exact tie.
    x = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5] + [0.0] * 24, np.float32)
    _, q_rne = oracle.quantize_block(x, RNE)
    _, q_rf = oracle.quantize_block(x, ROUNDF)
    np.testing.assert_array_equal(q_rne[:8], [127, 0, 2, 2, 0, -2, -2, 4])
    np.testing.assert_array_equal(q_rf[:8], [127, 1, 2, 3, -1, -2, -3, 4])


@pytest.mark.parametrize("variant", [RNE, ROUNDF])
def test_q8_matches_numpy_restatement(oracle, variant):
    rng = np.random.default_rng(3)
    for trial in range(3000):
        scale = np.float32(np.exp(rng.uniform(np.log(1e-4), np.log(1e4))))
        x = (rng.standard_normal(32) * scale).astype(np.float32)
        d, qs = oracle.quantize_block(x, variant)
        dr, qr = q8_block_ref(x, variant)
        assert d == dr, (trial, d, dr)
        np.testing.assert_array_equal(qs, qr, err_msg=f"trial {trial}")


@pytest.mark.parametrize("variant", [RNE, ROUNDF])
def test_q8_invariants(oracle, variant):
    rng = np.random.default_rng(4)
    for _ in range(500):
        x = (rng.standard_normal(32) * rng.uniform(0.01, 100)).astype(np.float32)
        d, qs = oracle.quantize_block(x, variant)
        assert np.abs(qs.astype(int)).max() == 127
        deq = dequant_ref(d, qs)
        d32 = np.uint16(d).view(np.float16).astype(np.float32)
        # |x - d16*q| <= d16/2 plus the scale's own fp16 rounding (|q| <= 127)
        amax = np.abs(x).max()
        bound = d32 / 2 + 127 * abs(d32 - amax / 127) + 1e-6 * amax
        assert np.abs(x - deq).max() <= bound


def test_q8_row_ggml_layout(oracle):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(256).astype(np.float32)
    b = oracle.quantize_row_ggml(x, RNE)
    assert b.size == 8 * 34
    for k in range(8):
        d, qs = oracle.quantize_block(x[32 * k:32 * k + 32], RNE)
        assert int(b[34 * k:34 * k + 2].view(np.uint16)[0]) == d
        np.testing.assert_array_equal(b[34 * k + 2:34 * k + 34].view(np.int8), qs)


@pytest.mark.parametrize("variant", [RNE, ROUNDF])
def test_q8_nonfinite_documented_values(oracle, variant):
    x = np.ones(32, np.float32)
    x[3] = np.nan
    d, qs = oracle.quantize_block(x, variant)
    assert qs[3] == 0 and qs[0] == 127 and d == int(np.float16(np.float32(1) / 127).view(np.uint16))
    x[3] = np.inf
    d, qs = oracle.quantize_block(x, variant)
    assert d == 0x7C00 and not qs.any()
