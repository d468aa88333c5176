"""The deterministic exponential (sao_exp_det) and the InfLLM builder variant
that uses it (the arithmetic of the GPU builder).

The reference's builder (cpp/src/selection.cpp:12-94) calls std::exp on
floats, i.e. glibc's expf, which is not reproducible on the GPU.  Both the
GPU builder and sao_build_local_causal_representatives_det use sao_exp_det;
these tests pin that function to the mathematics (correctly rounded exp from
float64) and the det builder to the reference (golden fixtures written by the
reference's own builder, the published C2.1 offset hash)."""
import ctypes
import ctypes.util
import os
import sys

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)

from cases import REPRESENTATIVES, representative_inputs  # noqa: E402

GOLD = np.load(os.path.join(HERE, "reference_outputs.npz"), allow_pickle=False)


def correctly_rounded_exp(x):
    return np.exp(np.asarray(x, np.float64)).astype(np.float32)


def test_exp_det_is_correctly_rounded(oracle_lib):
    """On 200k arguments over the softmax range [-104, 0] (and a few
    positives) the result equals exp computed in float64 then rounded."""
    rng = np.random.default_rng(7)
    x = np.concatenate([-rng.exponential(3.0, 100_000), rng.uniform(-104, 0, 99_000), rng.uniform(0, 80, 1000),
                        [0.0, -0.0, -1e-30, -87.33654, -88.72284, -103.27893, -103.97208, -110.0, 88.7]]).astype(
                            np.float32)
    got = oracle_lib.exp_det(x)
    expect = correctly_rounded_exp(x)
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))


def test_exp_det_special_values(oracle_lib):
    f = oracle_lib.lib().sao_exp_det
    assert f(0.0) == 1.0
    assert f(-200.0) == 0.0
    assert f(200.0) == float("inf")
    assert np.isnan(f(float("nan")))
    assert f(1.0) == np.float32(np.e)


def test_exp_det_vs_glibc_expf_agree_nearly_always(oracle_lib):
    """glibc's expf is within 0.502 ulp, so it differs from the correctly
    rounded result on a small fraction of inputs only (measured here)."""
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    rng = np.random.default_rng(8)
    x = (-rng.exponential(3.0, 20_000)).astype(np.float32)
    got = oracle_lib.exp_det(x)
    glibc = np.array([libm.expf(float(v)) for v in x], np.float32)
    differ = int((got.view(np.uint32) != glibc.view(np.uint32)).sum())
    ulps = np.abs(got.view(np.int32).astype(np.int64) - glibc.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1
    assert differ <= 0.01 * x.size


@pytest.mark.parametrize("name", sorted(REPRESENTATIVES))
def test_det_builder_equals_reference_on_golden(oracle_lib, name):
    """The det builder picks the reference's tokens and writes the reference's
    representative bits on every golden case."""
    c = REPRESENTATIVES[name]
    pq, kv = representative_inputs(c)
    vals, offs, received = oracle_lib.local_causal_representatives_det(pq, kv, c["tokens"], c["hq"], c["hkv"], 128,
                                                                       32, c["window"], c["topk"])
    assert np.array_equal(offs.astype(np.int64), GOLD[f"representatives/{name}/offsets"])
    assert np.array_equal(vals.view(np.uint32), GOLD[f"representatives/{name}/values"])
    # every query spreads a mass of one over its window
    assert abs(float(received.astype(np.float64).sum()) - c["hq"] * c["tokens"]) < 1e-3 * c["hq"] * c["tokens"]


def test_det_builder_c21_offset_hash(oracle_lib):
    """The published C2.1 golden: offset FNV hash 7873450381430813043
    (docs/cpp-versions/C2.1-infllm-selection-uring.md:40-42)."""
    kv, pq = oracle_lib.fixture_c2(512, 16, 8, 128)
    _, offs, _ = oracle_lib.local_causal_representatives_det(pq, kv, 512, 16, 8, 128, 32, 32, 4)
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
    _, _, received = oracle_lib.local_causal_representatives_det(pq, kv, 64, 4, 2, 128, 32, 1, 4)
    assert (received == 1.0).all()
