"""Golden-fixture cases: seeds and shapes, and the input generators shared by
tests/golden/make_golden.py (which records the reference's outputs) and the
tests that check the oracle and the GPU path against them."""
from __future__ import annotations

import hashlib

import numpy as np

D = 128

ATTENTION = {
    "rand_33_g2": {"seed": 11, "tokens": 33, "hq": 16, "hkv": 8, "d": D},
    "rand_97_g4": {"seed": 12, "tokens": 97, "hq": 32, "hkv": 8, "d": D},
    "rand_256_g2": {"seed": 13, "tokens": 256, "hq": 16, "hkv": 8, "d": D},
    "outliers_64_g2": {"seed": 14, "tokens": 64, "hq": 16, "hkv": 8, "d": D, "outliers": 0.02},
    "one_token_g1": {"seed": 15, "tokens": 1, "hq": 8, "hkv": 8, "d": D},
}

SELECTION = {
    # reference C2 call shape: 16 heads, 16 blocks, budget 4 = init 1 + local 1 + 2
    "c2_shape": {"seed": 21, "heads": 16, "blocks": 16, "budget": 4, "init": 1, "local": 1},
    # one KV group of the Qwen3-0.6B shape: 2 heads, 512 blocks, 4 + 8 + 52
    "group2_512": {"seed": 22, "heads": 2, "blocks": 512, "budget": 64, "init": 4, "local": 8},
    # quantised values: many equal scores
    "ties": {"seed": 23, "heads": 2, "blocks": 300, "budget": 40, "init": 1, "local": 2, "quantised": True},
    # all-zero representatives: every score 0, lowest ids win
    "zeros": {"seed": 24, "heads": 4, "blocks": 50, "budget": 10, "init": 2, "local": 2, "zero_reps": True},
}

REPRESENTATIVES = {
    # the C2.1 builder settings (window 32, top 4) at 128 tokens
    "w32_top4_128": {"seed": 31, "tokens": 128, "hq": 16, "hkv": 8, "window": 32, "topk": 4},
    # window 1, top 32: the mean key of every block
    "w1_top32_96": {"seed": 32, "tokens": 96, "hq": 16, "hkv": 8, "window": 1, "topk": 32},
    # four query heads per KV head, window 8, top 8
    "w8_top8_g4_96": {"seed": 33, "tokens": 96, "hq": 8, "hkv": 2, "window": 8, "topk": 8},
}

CODEC = {
    "float_to_half_4096": {"seed": 41, "count": 4096},
}


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def _half(rng, n, scale=1.0):
    return (rng.standard_normal(n) * scale).astype(np.float16).view(np.uint16)


def attention_inputs(c):
    """kv: FP16 bits [tokens][2][hkv][d] (token-major K/V interleaved); q: [hq][d]."""
    rng = np.random.default_rng(c["seed"])
    kv = _half(rng, c["tokens"] * 2 * c["hkv"] * c["d"])
    q = rng.standard_normal(c["hq"] * c["d"]).astype(np.float32)
    if c.get("outliers"):
        mask = rng.random(kv.size) < c["outliers"]
        sign = np.where(rng.random(kv.size) < 0.5, -1.0, 1.0)
        big = (sign * 60000.0).astype(np.float16).view(np.uint16)
        kv = np.where(mask, big, kv).astype(np.uint16)
    return kv, q


def selection_inputs(c):
    """q: [heads][D]; reps: [heads][blocks][D] (the reference's layout)."""
    rng = np.random.default_rng(c["seed"])
    q = rng.standard_normal(c["heads"] * D).astype(np.float32)
    reps = rng.standard_normal(c["heads"] * c["blocks"] * D).astype(np.float32)
    if c.get("quantised"):
        q = (rng.integers(-1, 2, size=q.size) * 0.25).astype(np.float32)
        reps = (rng.integers(-1, 2, size=reps.size) * 0.5).astype(np.float32)
    if c.get("zero_reps"):
        reps[:] = 0.0
    return q, reps


def representative_inputs(c):
    """prompt queries [hq][tokens][D] fp32; kv FP16 bits [tokens][2][hkv][D]."""
    rng = np.random.default_rng(c["seed"])
    pq = rng.standard_normal(c["hq"] * c["tokens"] * D).astype(np.float32)
    kv = _half(rng, c["tokens"] * 2 * c["hkv"] * D)
    return pq, kv


def codec_inputs(c):
    """fp32 values over the FP16 range and beyond, plus rounding edges."""
    rng = np.random.default_rng(c["seed"])
    mags = np.exp2(rng.uniform(-26, 17, size=c["count"] - 16))
    x = (mags * np.where(rng.random(mags.size) < 0.5, -1, 1)).astype(np.float32)
    edges = np.array([0.0, -0.0, 1.0, 1.99999, 65504.0, 65519.0, 65520.0, 6.1035156e-05, 5.9604645e-08,
                      2.9802322e-08, 3.0e-08, -65520.0, 0.5, 0.33333334, 1024.5, 2049.0], np.float32)
    return np.concatenate([x, edges]).astype(np.float32)
