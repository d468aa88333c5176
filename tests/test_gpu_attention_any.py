"""GPU: attention over a contiguous K/V buffer for head dimensions other
than 128 (csrc/attention_any.hip, routed by sa_hip_attention_contiguous), the
reference's attention_reference (attention_reference.cpp:55-96) for any
head_dim, within 2e-3 of the oracle's restatement of it.  Also through the
C++ backend: make_hip_backend()'s attention variants at head_dim 64
(tests/cpp/backend_check, C1 case)."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import assert_close_2e3, to_dev

pytestmark = pytest.mark.gpu


def case(seed, tokens, hq, hkv, d, kv_scale=1.0):
    rng = np.random.default_rng(seed)
    kv = (rng.standard_normal((tokens, 2, hkv, d)) * kv_scale).astype(np.float16)
    q = rng.standard_normal((hq, d)).astype(np.float32)
    return kv.view(np.uint16), q


@pytest.mark.parametrize("d", [8, 64, 80, 96, 192, 256, 512])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8), (64, 8)])
def test_attention_any_head_dim(hip, d, hq, hkv):
    tokens = 700 + d
    kv, q = case(d * 31 + hq, tokens, hq, hkv, d)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    print(f"case: attention_any d={d} hq={hq} hkv={hkv} tokens={tokens}", flush=True)
    out = hip.attention_contiguous(to_dev(kv.view(np.int16)).view(torch.uint16), to_dev(q), tokens, hq, hkv, scale,
                                   head_dim=d)
    torch.cuda.synchronize()
    expect = O.attention_reference(kv, q, tokens, hq, hkv, d, scale)
    assert_close_2e3(out.cpu().numpy(), expect)


@pytest.mark.parametrize("tokens", [1, 2, 63, 64, 65, 257, 4096, 40000])
def test_attention_any_token_counts(hip, tokens):
    """Tails of a 64-token tile, one token, and the split + merge path
    (thousands of tokens over 8 KV heads)."""
    d, hq, hkv = 64, 16, 8
    kv, q = case(tokens, tokens, hq, hkv, d)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    print(f"case: attention_any tokens={tokens}", flush=True)
    out = hip.attention_contiguous(to_dev(kv.view(np.int16)).view(torch.uint16), to_dev(q), tokens, hq, hkv, scale,
                                   head_dim=d)
    torch.cuda.synchronize()
    assert_close_2e3(out.cpu().numpy(), O.attention_reference(kv, q, tokens, hq, hkv, d, scale))


def test_attention_any_large_logits(hip):
    """Logits far from zero (keys scaled by 40): the running max keeps the
    exponentials finite."""
    d, hq, hkv, tokens = 96, 32, 8, 3000
    kv, q = case(5, tokens, hq, hkv, d, kv_scale=40.0)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    out = hip.attention_contiguous(to_dev(kv.view(np.int16)).view(torch.uint16), to_dev(q), tokens, hq, hkv, scale,
                                   head_dim=d)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    assert_close_2e3(got, O.attention_reference(kv, q, tokens, hq, hkv, d, scale))
