"""The restated glibc expf (sao_expf_glibc) and the InfLLM builder variant
that uses it (the arithmetic of the GPU builder).

The reference's builder (cpp/src/selection.cpp:12-94) calls std::exp on
floats, i.e. glibc's expf.  The oracle restates glibc 2.35's method (a
32-entry 2^(i/32) table, a degree-3 polynomial in double and the fused
multiply-adds of its x86-64 FMA build) so that the GPU builder can run the
same operations.  Pinned here: the table against its high-precision
derivation (oracle/gen_expf_table.py), the function against libm's expf over
a strided sweep of every float in [-110, 90] plus dense windows around the
two arguments where a reduction without the fused multiply-add (a plausible
mistake) differs, and the builder variant against the reference's own
builder (oracle/_ref, built from its sources) on random windows and seeds,
its golden outputs and the published C2.1 offset hash."""
import ctypes
import ctypes.util
import os
import struct
import sys

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)

from cases import REPRESENTATIVES, representative_inputs  # noqa: E402

GOLD = np.load(os.path.join(HERE, "reference_outputs.npz"), allow_pickle=False)


def bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def test_table_equals_its_derivation(oracle_lib):
    sys.path.insert(0, os.path.dirname(oracle_lib.__file__))
    from gen_expf_table import expf_table
    assert oracle_lib.expf_glibc_table() == expf_table()


def test_equals_libm_expf_on_a_sweep_of_every_float(oracle_lib):
    """Every 16th float bit pattern of [-110, -0] and [+0, 90]: no difference
    from libm's expf (an exhaustive run over all 2,240,806,914 floats of the
    range found none either)."""
    assert oracle_lib.expf_glibc_mismatches(0x80000000, bits(-110.0), 16) == 0
    assert oracle_lib.expf_glibc_mismatches(0x00000000, bits(90.0), 16) == 0


@pytest.mark.parametrize("center", [float.fromhex("0x1.04845ep+5"), float.fromhex("-0x1.f8cbb2p+5")])
def test_equals_libm_where_an_unfused_reduction_differs(oracle_lib, center):
    """The two floats of the range where r = z - k without the fused
    multiply-add rounds differently from libm, with 2^20 neighbours each."""
    u = bits(center)
    assert oracle_lib.expf_glibc_mismatches(u - (1 << 19), u + (1 << 19), 1) == 0


def test_special_values(oracle_lib):
    f = oracle_lib.lib().sao_expf_glibc
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    for x in (0.0, -0.0, 1.0, -1.0, -87.33654, -88.72284, -103.27893, -103.97208, -104.0, -200.0, 88.7, 89.0,
              200.0, float("inf"), float("-inf")):
        assert bits(f(x)) == bits(libm.expf(x)), x
    assert f(0.0) == 1.0 and f(-200.0) == 0.0 and f(200.0) == float("inf")
    assert np.isnan(f(float("nan")))


@pytest.mark.parametrize("name", sorted(REPRESENTATIVES))
def test_restated_builder_equals_reference_on_golden(oracle_lib, name):
    """The reference's tokens and representative bits on every golden case."""
    c = REPRESENTATIVES[name]
    pq, kv = representative_inputs(c)
    vals, offs, received = oracle_lib.local_causal_representatives_restated(pq, kv, c["tokens"], c["hq"], c["hkv"],
                                                                            128, 32, c["window"], c["topk"])
    assert np.array_equal(offs.astype(np.int64), GOLD[f"representatives/{name}/offsets"])
    assert np.array_equal(vals.view(np.uint32), GOLD[f"representatives/{name}/values"])
    # every query spreads a mass of one over its window
    assert abs(float(received.astype(np.float64).sum()) - c["hq"] * c["tokens"]) < 1e-3 * c["hq"] * c["tokens"]


@pytest.mark.parametrize("seed,tokens,hq,hkv,window,topk,scale",
                         [(1, 256, 4, 2, 32, 4, 1.0), (2, 128, 8, 2, 7, 3, 1.0), (3, 192, 4, 1, 64, 8, 3.0),
                          (4, 96, 2, 2, 2, 32, 1.0), (5, 256, 4, 4, 200, 5, 8.0), (6, 64, 8, 8, 33, 1, 0.25)])
def test_restated_builder_equals_reference_builder(ref_lib, seed, tokens, hq, hkv, window, topk, scale):
    """Random windows and seeds: offsets and representative bits equal the
    reference's own builder (std::exp = libm's expf), run from oracle/_ref."""
    rng = np.random.default_rng(seed)
    pq = (rng.standard_normal(hq * tokens * 128) * scale).astype(np.float32)
    kv = (rng.standard_normal(tokens * 2 * hkv * 128) * scale).astype(np.float16).view(np.uint16)
    vals, offs, _ = ref_lib.local_causal_representatives_restated(pq, kv, tokens, hq, hkv, 128, 32, window, topk)
    rvals, roffs = ref_lib.local_causal_representatives(pq, kv, tokens, hq, hkv, 128, 32, window, topk, use_ref=True)
    assert np.array_equal(offs.astype(np.int64).ravel(), np.asarray(roffs).astype(np.int64).ravel())
    assert np.array_equal(vals.view(np.uint32).ravel(), np.asarray(rvals, np.float32).view(np.uint32).ravel())


@pytest.mark.parametrize("d,block,window,topk,hq,hkv,tokens", [
    (128, 32, 1100, 8, 2, 1, 1280), (128, 32, 5000, 4, 2, 2, 512), (64, 16, 48, 5, 8, 4, 160),
    (36, 8, 20, 3, 4, 2, 96), (256, 64, 100, 10, 4, 1, 256), (128, 100, 64, 7, 2, 1, 300), (8, 1, 3, 1, 2, 2, 40)])
def test_restated_builder_equals_reference_general_shapes(ref_lib, d, block, window, topk, hq, hkv, tokens):
    """The shapes the general GPU kernels take (any head_dim, block size and
    window, selection.cpp:12-23): offsets and representative bits equal the
    reference's own builder, run from oracle/_ref."""
    rng = np.random.default_rng(d * 131 + block * 7 + window)
    pq = rng.standard_normal(hq * tokens * d).astype(np.float32)
    kv = rng.standard_normal(tokens * 2 * hkv * d).astype(np.float16).view(np.uint16)
    vals, offs, received = ref_lib.local_causal_representatives_restated(pq, kv, tokens, hq, hkv, d, block, window,
                                                                         topk)
    rvals, roffs = ref_lib.local_causal_representatives(pq, kv, tokens, hq, hkv, d, block, window, topk, use_ref=True)
    assert np.array_equal(offs.astype(np.int64).ravel(), np.asarray(roffs).astype(np.int64).ravel())
    assert np.array_equal(vals.view(np.uint32).ravel(), np.asarray(rvals, np.float32).view(np.uint32).ravel())
    # every query spreads a mass of one over its window
    assert abs(float(received.astype(np.float64).sum()) - hq * tokens) < 1e-3 * hq * tokens


def test_restated_builder_c21_offset_hash(oracle_lib):
    """The published C2.1 golden: offset FNV hash 7873450381430813043
    (docs/cpp-versions/C2.1-infllm-selection-uring.md:40-42)."""
    kv, pq = oracle_lib.fixture_c2(512, 16, 8, 128)
    _, offs, _ = oracle_lib.local_causal_representatives_restated(pq, kv, 512, 16, 8, 128, 32, 32, 4)
    h = 1469598103934665603
    for o in offs.ravel():
        h ^= int(o)
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    assert h == 7873450381430813043


def test_window_one_received_mass_is_one(oracle_lib):
    """Closed form (reference tests/test_selection.py:6-12): with a window of
    one every key receives exactly mass 1.0."""
    rng = np.random.default_rng(3)
    pq = rng.standard_normal(4 * 64 * 128).astype(np.float32)
    kv = rng.standard_normal(64 * 2 * 2 * 128).astype(np.float16).view(np.uint16)
    _, _, received = oracle_lib.local_causal_representatives_restated(pq, kv, 64, 4, 2, 128, 32, 1, 4)
    assert (received == 1.0).all()
