"""Round-to-nearest-even fp32 -> FP16 of the oracle (the append conversion)
against numpy's IEEE float16 cast, and the synthetic generator's invariants."""
import numpy as np


def _rne(oracle_lib, bits):
    L = oracle_lib.lib()
    return np.array([L.sao_float_to_half_rne(float(np.uint32(u).view(np.float32))) for u in bits], np.uint16)


def test_rne_matches_numpy_random_bits(oracle_lib):
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 2**32, size=300_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    bits = bits[~np.isnan(f)]
    got = _rne(oracle_lib, bits)
    with np.errstate(over="ignore"):
        expect = bits.view(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, expect)


def test_rne_matches_numpy_near_boundaries(oracle_lib):
    """Every fp32 within a few ulps of each FP16 rounding midpoint, across the
    normal, subnormal, overflow and underflow ranges."""
    halves = np.arange(0, 0x7c00, dtype=np.uint32).astype(np.uint16)
    lo = halves.view(np.float16).astype(np.float32)
    hi = (halves + 1).view(np.float16).astype(np.float32)
    mid = ((lo.astype(np.float64) + hi.astype(np.float64)) / 2).astype(np.float32)
    bits = mid.view(np.uint32).astype(np.int64)
    cand = np.concatenate([bits + k for k in (-2, -1, 0, 1, 2)])
    cand = cand[cand >= 0].astype(np.uint32)
    cand = cand[~np.isnan(cand.view(np.float32))]
    cand = np.concatenate([cand, cand | 0x80000000])
    got = _rne(oracle_lib, cand)
    with np.errstate(over="ignore"):
        expect = cand.view(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, expect)


def test_rne_specials(oracle_lib):
    L = oracle_lib.lib()
    assert L.sao_float_to_half_rne(float("inf")) == 0x7C00
    assert L.sao_float_to_half_rne(float("-inf")) == 0xFC00
    assert L.sao_float_to_half_rne(65520.0) == 0x7C00
    assert L.sao_float_to_half_rne(65519.99) == 0x7BFF
    assert L.sao_float_to_half_rne(-0.0) == 0x8000
    h = L.sao_float_to_half_rne(float("nan"))
    assert (h & 0x7C00) == 0x7C00 and (h & 0x3FF) != 0


def test_synthetic_normal_moments_and_determinism(oracle_lib):
    O = oracle_lib
    x = O.synth_float(1234, 0, 200_000)
    assert abs(float(x.mean())) < 0.01
    assert abs(float(x.std()) - 1.0) < 0.01
    assert np.array_equal(x, O.synth_float(1234, 0, 200_000))
    # a window of the stream equals the same window generated on its own
    assert np.array_equal(x[5000:6000], O.synth_float(1234, 5000, 1000))
    h = O.synth_half(1234, 0, 1000)
    assert np.array_equal(h, x[:1000].astype(np.float16).view(np.uint16))
