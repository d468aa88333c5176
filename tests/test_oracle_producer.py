"""The oracle's query producer / output consumer (rms_norm, the [out][in]
projections, per-head RMS + RoPE; reference cpp/src/qwen_layer_main.cpp
:125-183) pinned by independent computations and by invariants that a
dropped term, a swapped pair or a sign error would break."""
import numpy as np

import oracle as O


def test_rms_norm_matches_float64_and_closed_form():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 1024)).astype(np.float32) * 3
    w = rng.standard_normal(1024).astype(np.float32)
    got = O.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)
    # constant row c: out = w * c / sqrt(c^2 + eps)
    c = np.full((1, 1024), -0.75, np.float32)
    np.testing.assert_allclose(O.rms_norm(c, w, 1e-6)[0], w * (-0.75 / np.sqrt(0.5625 + 1e-6)), rtol=1e-6)


def test_linear_matches_matmul_and_residual():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((7, 256)).astype(np.float32)
    w = rng.standard_normal((96, 256)).astype(np.float32)
    r = rng.standard_normal((7, 96)).astype(np.float32)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(O.linear(x, w), ref, rtol=1e-6, atol=1e-5)
    np.testing.assert_allclose(O.linear(x, w, r), ref + r, rtol=1e-6, atol=1e-5)
    # a transposed weight would give a different (wrong-shaped) product
    assert O.linear(x, w).shape == (7, 96)


def test_rope_frequencies_closed_form():
    f = O.rope_inv_freq(1e6, 128)
    assert f[0] == 1.0
    assert abs(float(f[32]) - 1e-3) < 1e-3 * 2 ** -23  # theta^(-1/2)
    assert np.all(np.diff(f.astype(np.float64)) < 0)


def test_rope_is_a_rotation_of_each_half_pair():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 4, 128)).astype(np.float32)
    pos = np.array([0, 7, 4093], np.int32)
    y = O.qk_norm_rope(x, None, pos)
    assert np.array_equal(y[0], x[0])  # position 0 is the identity
    # |(x_d, x_{d+64})| is preserved; the complex form z = x_d + i x_{d+64}
    # turns by position * f_d
    zx = x[..., :64].astype(np.float64) + 1j * x[..., 64:].astype(np.float64)
    zy = y[..., :64].astype(np.float64) + 1j * y[..., 64:].astype(np.float64)
    np.testing.assert_allclose(np.abs(zy), np.abs(zx), rtol=1e-6)
    f = O.rope_inv_freq(1e6, 128).astype(np.float32)
    for r in range(3):
        ang = (np.float32(pos[r]) * f).astype(np.float64)
        np.testing.assert_allclose(zy[r], zx[r] * np.exp(1j * ang), rtol=1e-6, atol=1e-6)


def test_rope_scores_depend_on_relative_position_only():
    """q.k after RoPE depends on the position difference: shifting both
    positions by s leaves every score unchanged (small positions, where the
    fp32 angle is exact to ~1e-6)."""
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, 1, 128)).astype(np.float32)
    k = rng.standard_normal((1, 1, 128)).astype(np.float32)
    base = None
    for s in (0, 3, 11, 40):
        rq = O.qk_norm_rope(q, None, np.array([9 + s], np.int32))
        rk = O.qk_norm_rope(k, None, np.array([2 + s], np.int32))
        score = float(np.dot(rq.ravel().astype(np.float64), rk.ravel().astype(np.float64)))
        if base is None:
            base = score
        assert abs(score - base) < 1e-4 * max(1.0, abs(base)), (s, score, base)


def test_head_rms_norm():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 3, 128)).astype(np.float32) * 5
    w = np.ones(128, np.float32)
    y = O.qk_norm_rope(x, w, None)
    rms = np.sqrt((y.astype(np.float64) ** 2).mean(axis=2))
    np.testing.assert_allclose(rms, 1.0, rtol=1e-5)
    w2 = rng.standard_normal(128).astype(np.float32)
    np.testing.assert_allclose(O.qk_norm_rope(x, w2, None), y * w2, rtol=1e-6, atol=1e-6)
