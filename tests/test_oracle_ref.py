"""The oracle restatement against the reference's own CPU functions, compiled
from the reference sources into oracle/_ref/libsa_ref.so (bit-exact,
many seeds), plus closed-form checks that hold without the reference build.
"""
import numpy as np
import pytest


def rand_half(rng, n, scale=1.0):
    """Random FP16 bit patterns of N(0, scale^2) values (finite)."""
    return (rng.standard_normal(n) * scale).astype(np.float16).view(np.uint16)


def test_half_to_float_all_patterns_vs_ref(ref_lib):
    O = ref_lib
    L, R = O.lib(), O.ref()
    for h in range(0, 65536):
        a = np.float32(L.sao_half_to_float(h)).view(np.uint32)
        b = np.float32(R.saref_half_to_float(h)).view(np.uint32)
        assert a == b, hex(h)


def test_half_to_float_matches_ieee_decode(oracle_lib):
    """Closed form: the exact decode equals numpy's float16 -> float32 for every
    non-NaN pattern (NaNs keep their payload bits)."""
    L = oracle_lib.lib()
    hs = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expect = hs.view(np.float16).astype(np.float32)
    got = np.array([L.sao_half_to_float(int(h)) for h in hs], np.float32)
    nan = np.isnan(expect)
    assert np.array_equal(got[~nan].view(np.uint32), expect[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


def test_float_to_half_vs_ref(ref_lib):
    O = ref_lib
    L, R = O.lib(), O.ref()
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0, 0x80000000, 0x3fffffff, 0x3ffff000, 0x3ffff001, 0x477fe000, 0x477ff000,
                         0x47800000, 0x7f800000, 0xff800000, 0x7fc00000, 0x33000000, 0x33000001,
                         0x387fc000, 0x38800000, 0x00000001], np.uint32)
    for u in np.concatenate([bits, specials]):
        f = float(np.uint32(u).view(np.float32))
        assert L.sao_float_to_half(f) == R.saref_float_to_half(f), hex(int(u))


def test_float_to_half_quirk(oracle_lib):
    """The fixture encoder's carry is OR-ed into the exponent: 1.99999f -> 1.0."""
    L = oracle_lib.lib()
    assert L.sao_float_to_half(1.99999) == 0x3C00
    assert L.sao_float_to_half(1.0) == 0x3C00
    assert L.sao_float_to_half(0.5) == 0x3800


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("tokens,hq,hkv", [(1, 4, 2), (33, 16, 8), (128, 16, 8), (97, 32, 8), (64, 8, 8)])
def test_attention_reference_bit_exact(ref_lib, seed, tokens, hq, hkv):
    O = ref_lib
    rng = np.random.default_rng(seed * 1000 + tokens)
    d = 128
    kv = rand_half(rng, tokens * 2 * hkv * d)
    q = rng.standard_normal(hq * d).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    a = O.attention_reference(kv, q, tokens, hq, hkv, d, scale)
    b = O.attention_reference(kv, q, tokens, hq, hkv, d, scale, use_ref=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_attention_single_token_closed_form(oracle_lib):
    """One token: softmax weight is exactly 1, so out = V exactly."""
    O = oracle_lib
    rng = np.random.default_rng(7)
    kv = rand_half(rng, 2 * 8 * 128)
    q = rng.standard_normal(16 * 128).astype(np.float32)
    out = O.attention_reference(kv, q, 1, 16, 8, 128, 0.1)
    v = kv.reshape(2, 8, 128)[1].view(np.float16).astype(np.float32)
    assert np.array_equal(out, np.repeat(v, 2, axis=0))


@pytest.mark.parametrize("seed", range(3))
@pytest.mark.parametrize("window,topk", [(1, 1), (1, 32), (32, 4), (7, 3), (64, 16)])
def test_local_causal_representatives_bit_exact(ref_lib, seed, window, topk):
    O = ref_lib
    rng = np.random.default_rng(seed)
    tokens, hq, hkv, d = 128, 8, 4, 128
    kv = rand_half(rng, tokens * 2 * hkv * d, 0.5)
    pq = rng.standard_normal(hq * tokens * d).astype(np.float32)
    a, ao = O.local_causal_representatives(pq, kv, tokens, hq, hkv, d, 32, window, topk)
    b, bo = O.local_causal_representatives(pq, kv, tokens, hq, hkv, d, 32, window, topk, use_ref=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(ao, bo)


def test_mean_key_equals_window1_topk32(ref_lib):
    """Mean-key representative == the reference builder with window 1 and
    top-k = block tokens (every received mass is exactly 1)."""
    O = ref_lib
    rng = np.random.default_rng(3)
    tokens, hq, hkv, d = 256, 16, 8, 128
    kv = rand_half(rng, tokens * 2 * hkv * d)
    pq = rng.standard_normal(hq * tokens * d).astype(np.float32)
    ref_vals, _ = O.local_causal_representatives(pq, kv, tokens, hq, hkv, d, 32, 1, 32, use_ref=True)
    mean = O.mean_key_representatives(kv, tokens, hkv, d, 32)
    expanded = np.repeat(mean, hq // hkv, axis=0)
    assert np.array_equal(ref_vals.view(np.uint32), expanded.view(np.uint32))


def _quantized_reps(rng, heads, blocks, d, levels):
    """Representatives with few distinct values so that scores tie often."""
    return (rng.integers(-levels, levels + 1, size=heads * blocks * d) * 0.25).astype(np.float32)


@pytest.mark.parametrize("seed", range(12))
def test_select_shared_blocks_bit_exact(ref_lib, seed):
    O = ref_lib
    rng = np.random.default_rng(seed)
    heads = int(rng.choice([1, 2, 4, 16]))
    blocks = int(rng.integers(1, 300))
    d = 128
    budget = int(rng.integers(1, blocks + 1))
    init = int(rng.integers(0, budget + 1))
    local = int(rng.integers(0, budget - init + 1))
    if seed % 3 == 0:
        reps = _quantized_reps(rng, heads, blocks, d, 1)
        q = (rng.integers(-1, 2, size=heads * d) * 0.5).astype(np.float32)
    else:
        reps = rng.standard_normal(heads * blocks * d).astype(np.float32)
        q = rng.standard_normal(heads * d).astype(np.float32)
    a, sa_ = O.select_shared_blocks(q, reps, heads, blocks, d, budget, init, local)
    b, sb = O.select_shared_blocks(q, reps, heads, blocks, d, budget, init, local, use_ref=True)
    assert a.tolist() == b.tolist()
    assert np.array_equal(sa_.view(np.uint32), sb.view(np.uint32))


def test_select_zero_scores_tie_on_id(ref_lib):
    """-0.0 and +0.0 are equal for the reference comparator: ties go to the
    lower block id."""
    O = ref_lib
    heads, blocks, d = 1, 8, 128
    reps = np.zeros(heads * blocks * d, np.float32)
    reps[3 * d] = -0.0
    reps[5 * d] = 1e-30
    q = np.zeros(d, np.float32)
    q[0] = -1.0  # block 5 scores -1e-30 (< 0), block 3 scores +0.0 * -1 = -0.0
    a, _ = O.select_shared_blocks(q, reps, heads, blocks, d, 3, 0, 0)
    b, _ = O.select_shared_blocks(q, reps, heads, blocks, d, 3, 0, 0, use_ref=True)
    assert a.tolist() == b.tolist() == [0, 1, 2]


def test_select_rejects_invalid_like_reference(oracle_lib):
    O = oracle_lib
    q = np.zeros(128, np.float32)
    reps = np.zeros(4 * 128, np.float32)
    with pytest.raises(ValueError):
        O.select_shared_blocks(q, reps, 1, 4, 128, 5, 0, 0)  # budget > blocks
    with pytest.raises(ValueError):
        O.select_shared_blocks(q, reps, 1, 4, 128, 2, 2, 1)  # init + local > budget
