"""CPU: the InfLLM builder's received-mass order for inputs the reference's
comparator leaves unordered.  The reference ranks keys with
std::stable_sort(a > b) (selection.cpp:71-76); a NaN mass (from a non-finite
query) is unordered under a > b, so the reference's order is undefined
there.  The oracle and both GPU builders rank NaN after every number, NaNs in
token order, numbers exactly as a > b with ties in token order.  Pinned here
by brute force on the oracle's own received masses."""
import numpy as np
import pytest

import oracle as O


def nan_last_order(masses):
    """Stable descending order, NaN after every number (token order among
    NaNs): sort keys (is_nan, -mass, token)."""
    idx = list(range(len(masses)))
    return sorted(idx, key=lambda j: (bool(np.isnan(masses[j])), 0.0 if np.isnan(masses[j]) else -float(masses[j]), j))


@pytest.mark.parametrize("nan_at", [[37], [3, 40, 41], []])
def test_builder_ranks_nan_masses_last(oracle_lib, nan_at):
    rng = np.random.default_rng(31 + len(nan_at))
    tokens, hq, hkv, window, topk = 96, 4, 2, 8, 12
    pq = rng.standard_normal((hq, tokens, 128)).astype(np.float32)
    for t in nan_at:
        pq[1, t, 5] = np.nan  # query head 1: the masses of the keys in its window become NaN
    kv = rng.standard_normal(tokens * 2 * hkv * 128).astype(np.float16).view(np.uint16)
    vals, offs, rec = O.local_causal_representatives_restated(pq, kv, tokens, hq, hkv, 128, 32, window, topk)
    assert np.isnan(rec).any() == bool(nan_at)
    for h in range(hq):
        for b in range(tokens // 32):
            masses = rec[h, b * 32:(b + 1) * 32]
            assert offs[h, b].tolist() == nan_last_order(masses)[:topk], (h, b)
    # libm's expf gives the same order
    _, loffs = O.local_causal_representatives(pq, kv, tokens, hq, hkv, 128, 32, window, topk)
    assert np.array_equal(loffs, offs)
