"""GPU parity: InfLLM local-causal block representatives of a prefill
(sa_hip_local_causal_representatives), the reference's
build_local_causal_representatives (cpp/src/selection.cpp:12-94).

The GPU builder's exponential restates glibc's expf, the reference's
std::exp.  Bars: bit-exact chosen offsets and representative bits against the
oracle's builder with libm's expf (the reference's own arithmetic,
sao_build_local_causal_representatives) and, with the received-mass bits,
against the oracle's builder with the restated expf
(sao_build_local_causal_representatives_restated); bit-exact offsets and
representatives against the reference's own outputs on the committed golden
cases and the published C2.1 offset hash; the C2.1 chain (GPU builder, then
GPU selection) returns the published ids [0, 8, 13, 15]."""
import os
import sys

import numpy as np
import pytest
import torch

import oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)

from cases import REPRESENTATIVES, representative_inputs  # noqa: E402

pytestmark = pytest.mark.gpu

GOLD = np.load(os.path.join(HERE, "reference_outputs.npz"), allow_pickle=False)


def gpu_build(hip, pq, kv, tokens, hq, hkv, window, topk, want_reps=False, d=128, block=32):
    dq = torch.from_numpy(np.ascontiguousarray(pq)).cuda()
    dkv = torch.from_numpy(np.ascontiguousarray(kv).view(np.int16)).cuda().view(torch.uint16)
    received = torch.empty((hq, tokens), dtype=torch.float32, device="cuda")
    blocks = tokens // block
    rep_stride = (blocks + 3) // 4 * 4
    reps = torch.zeros((hq, d, rep_stride), dtype=torch.float32, device="cuda") if want_reps else None
    vals, offs = hip.local_causal_representatives(dq, dkv, tokens, hq, hkv, window, topk, reps=reps,
                                                  rep_stride=rep_stride if want_reps else 0, received=received,
                                                  head_dim=d, block_tokens=block)
    torch.cuda.synchronize()
    out = (vals.cpu().numpy(), offs.cpu().numpy().astype(np.int64), received.cpu().numpy())
    return out + ((reps.cpu().numpy()[:, :, :blocks],) if want_reps else ())


def check_vs_oracle(hip, pq, kv, tokens, hq, hkv, window, topk, d=128, block=32, want_reps=False):
    got = gpu_build(hip, pq, kv, tokens, hq, hkv, window, topk, want_reps=want_reps, d=d, block=block)
    vals, offs, rec = got[:3]
    evals, eoffs, erec = O.local_causal_representatives_restated(pq, kv, tokens, hq, hkv, d, block, window, topk)
    assert np.array_equal(rec.view(np.uint32), erec.view(np.uint32)), "received mass differs"
    assert np.array_equal(offs, eoffs.astype(np.int64)), "chosen offsets differ"
    assert np.array_equal(vals.view(np.uint32), evals.view(np.uint32)), "representative bits differ"
    if want_reps:  # the d-major copy holds the same bits
        assert np.array_equal(got[3].transpose(0, 2, 1).view(np.uint32), vals.view(np.uint32))
    # the reference's arithmetic: libm's expf
    lvals, loffs = O.local_causal_representatives(pq, kv, tokens, hq, hkv, d, block, window, topk)
    assert np.array_equal(offs, loffs.astype(np.int64)), "chosen offsets differ from the libm builder"
    assert np.array_equal(vals.view(np.uint32), lvals.view(np.uint32)), "representative bits differ from libm"


@pytest.mark.parametrize("name", sorted(REPRESENTATIVES))
def test_gpu_builder_vs_reference_golden(hip, name):
    c = REPRESENTATIVES[name]
    print(f"case: representatives/{name}", flush=True)
    pq, kv = representative_inputs(c)
    vals, offs, _ = gpu_build(hip, pq, kv, c["tokens"], c["hq"], c["hkv"], c["window"], c["topk"])
    assert np.array_equal(offs, GOLD[f"representatives/{name}/offsets"])
    assert np.array_equal(vals.view(np.uint32), GOLD[f"representatives/{name}/values"])


@pytest.mark.parametrize("window,topk,hq,hkv,tokens", [
    (1, 1, 4, 4, 64), (2, 3, 8, 4, 96), (5, 4, 8, 2, 160), (32, 4, 16, 8, 512), (64, 8, 8, 8, 256),
    (100, 16, 4, 1, 320), (256, 32, 8, 2, 544), (33, 32, 2, 2, 64),
    # whole-row staging in the block kernel (windows 4..64, powers of two),
    # including prompts shorter than a block's 32 + W - 1 query rows
    (4, 2, 8, 4, 128), (8, 3, 4, 2, 96), (16, 5, 8, 8, 224), (64, 4, 4, 2, 64), (32, 32, 2, 1, 32)])
def test_gpu_builder_vs_oracle(hip, window, topk, hq, hkv, tokens):
    print(f"case: window={window} topk={topk} hq={hq} hkv={hkv} tokens={tokens}", flush=True)
    rng = np.random.default_rng(window * 7 + tokens)
    pq = rng.standard_normal(hq * tokens * 128).astype(np.float32)
    kv = rng.standard_normal(tokens * 2 * hkv * 128).astype(np.float16).view(np.uint16)
    check_vs_oracle(hip, pq, kv, tokens, hq, hkv, window, topk)


@pytest.mark.parametrize("d,block,window,topk,hq,hkv,tokens", [
    (128, 32, 257, 4, 4, 2, 640),     # the first window past the tiled kernels
    (128, 32, 1100, 8, 2, 1, 1280),   # windows over one 1024-entry denominator chunk
    (128, 32, 5000, 4, 2, 2, 512),    # a window longer than the prompt
    (64, 16, 48, 5, 8, 4, 160),       # head_dim 64, 16-token blocks
    (36, 8, 20, 3, 4, 2, 96),         # head_dim not a multiple of 8 (2-byte key reads)
    (256, 64, 100, 10, 4, 1, 256),    # head_dim 256, 64-token blocks
    (128, 100, 64, 7, 2, 1, 300),     # blocks of 100 tokens (more than a wave's lanes)
    (8, 1, 3, 1, 2, 2, 40),           # one-token blocks
    (128, 32, 300, 32, 2, 2, 96)])    # topk = block_tokens
def test_gpu_builder_general_shapes(hip, d, block, window, topk, hq, hkv, tokens):
    """The reference's builder takes any head_dim, block size and window
    (selection.cpp:12-23); shapes outside the tiled kernels' (head_dim 128,
    32-token blocks, window <= 256) run the general kernels: received-mass
    bits, offsets and representative bits equal the oracle's."""
    print(f"case: d={d} block={block} window={window} topk={topk} hq={hq} hkv={hkv} tokens={tokens}", flush=True)
    rng = np.random.default_rng(d * 131 + block * 7 + window)
    pq = rng.standard_normal(hq * tokens * d).astype(np.float32)
    kv = rng.standard_normal(tokens * 2 * hkv * d).astype(np.float16).view(np.uint16)
    check_vs_oracle(hip, pq, kv, tokens, hq, hkv, window, topk, d=d, block=block, want_reps=True)


def test_gpu_builder_general_shapes_ties_and_nan(hip):
    """The general kernels' rank on repeated tokens (equal mass keeps token
    order) and NaN masses (ranked last), at head_dim 64 with 48-token blocks
    and a 300-token window."""
    rng = np.random.default_rng(5)
    d, block, tokens, hq, hkv, window, topk = 64, 48, 384, 4, 2, 300, 9
    pq = rng.standard_normal((hq, tokens, d)).astype(np.float32)
    pq[2, 200, 3] = np.nan
    kv = rng.standard_normal((tokens, 2, hkv, d)).astype(np.float16)
    kv[96:120] = kv[96]
    vals, offs, rec = gpu_build(hip, pq, kv.view(np.uint16).ravel(), tokens, hq, hkv, window, topk, d=d,
                                block=block)
    evals, eoffs, erec = O.local_causal_representatives_restated(pq, kv.view(np.uint16).ravel(), tokens, hq, hkv,
                                                                 d, block, window, topk)
    assert np.isnan(erec).any()
    assert np.array_equal(np.isnan(rec), np.isnan(erec))
    finite = ~np.isnan(erec)
    assert np.array_equal(rec[finite].view(np.uint32), erec[finite].view(np.uint32))
    assert np.array_equal(offs, eoffs.astype(np.int64))
    assert np.array_equal(vals.view(np.uint32), evals.view(np.uint32))


@pytest.mark.parametrize("window", [32, 64])
def test_gpu_builder_unaligned_workspace(hip, window):
    """A workspace 4 bytes off a 16-byte boundary: the block kernel stages
    the probabilities per token column instead of as whole rows (its 16-byte
    copies need an aligned workspace); results bit-exact as with an aligned
    one."""
    rng = np.random.default_rng(700 + window)
    tokens, hq, hkv, topk = 320, 8, 4, 4
    pq = rng.standard_normal(hq * tokens * 128).astype(np.float32)
    kv = rng.standard_normal(tokens * 2 * hkv * 128).astype(np.float16).view(np.uint16)
    nbytes = hip.lib().sa_hip_local_causal_workspace_bytes(tokens, hq, window)
    base = torch.empty(nbytes // 4 + 4, dtype=torch.float32, device="cuda")
    ws = base[1:1 + nbytes // 4]
    assert ws.data_ptr() % 16 == 4
    dq = torch.from_numpy(pq).cuda()
    dkv = torch.from_numpy(kv.view(np.int16)).cuda().view(torch.uint16)
    received = torch.empty((hq, tokens), dtype=torch.float32, device="cuda")
    vals, offs = hip.local_causal_representatives(dq, dkv, tokens, hq, hkv, window, topk, received=received,
                                                  workspace=ws)
    torch.cuda.synchronize()
    evals, eoffs, erec = O.local_causal_representatives_restated(pq, kv, tokens, hq, hkv, 128, 32, window, topk)
    assert np.array_equal(received.cpu().numpy().view(np.uint32), erec.view(np.uint32))
    assert np.array_equal(offs.cpu().numpy().astype(np.int64), eoffs.astype(np.int64))
    assert np.array_equal(vals.cpu().numpy().view(np.uint32), evals.view(np.uint32))


def test_gpu_builder_outliers_and_ties(hip):
    """+-60000 keys (saturated softmax rows) and repeated tokens (equal mass:
    the stable rank keeps token order)."""
    rng = np.random.default_rng(99)
    tokens, hq, hkv = 128, 8, 4
    pq = rng.standard_normal(hq * tokens * 128).astype(np.float32)
    kv = rng.standard_normal((tokens, 2, hkv, 128)).astype(np.float16)
    kv[rng.random(tokens) < 0.05] = np.float16(60000)
    kv[40:56] = kv[40]  # a run of identical tokens
    check_vs_oracle(hip, pq, kv.view(np.uint16).ravel(), tokens, hq, hkv, 32, 4)


def test_gpu_builder_wide_logit_range(hip):
    """Queries and keys scaled x6: window logits spread over hundreds, so the
    exponentials cover the whole float range down to subnormals and zero."""
    rng = np.random.default_rng(123)
    tokens, hq, hkv = 384, 8, 2
    pq = (rng.standard_normal(hq * tokens * 128) * 6).astype(np.float32)
    kv = (rng.standard_normal(tokens * 2 * hkv * 128) * 6).astype(np.float16).view(np.uint16)
    check_vs_oracle(hip, pq, kv, tokens, hq, hkv, 48, 6)


def test_gpu_c21_chain(hip):
    """C2.1 end to end on the GPU: representatives of the reference's 512-token
    fixture (window 32, top 4), their offset hash, then the shared selection
    over them (budget 4 = init 1 + local 1 + 2) -> [0, 8, 13, 15]."""
    kv, pq = O.fixture_c2(512, 16, 8, 128)
    vals, offs, _, reps = gpu_build(hip, pq, kv, 512, 16, 8, 32, 4, want_reps=True)
    h = 1469598103934665603
    for o in offs.ravel():
        h ^= int(o)
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    assert h == 7873450381430813043
    assert np.array_equal(reps.transpose(0, 2, 1).view(np.uint32), vals.view(np.uint32))
    kvp = hip.PagedKV(1, 16, 8, table_stride=16, num_pages=16, rep_heads=16, rep_stride=16)
    kvp.reps[0].copy_(torch.from_numpy(np.ascontiguousarray(reps)))
    kvp.sealed.fill_(16)
    kvp.seq_len.fill_(512)
    query = pq.reshape(16, 512, 128)[:, 511, :].copy()
    sel, cnt = hip.score_select(kvp, torch.from_numpy(query.reshape(1, 16, 128)).cuda(), 1, 4, 1, 1)
    torch.cuda.synchronize()
    assert sel[0, 0, : int(cnt.item())].cpu().numpy().tolist() == [0, 8, 13, 15]


def test_gpu_builder_nan_queries_rank_last(hip):
    """Non-finite prompt queries give NaN received masses to the keys in
    their windows; the GPU builder ranks them after every number in token
    order, as the oracle does (the reference's a > b leaves NaN unordered):
    offsets and representative bits equal the oracle's, NaN masses where
    the oracle has them and equal bits elsewhere."""
    rng = np.random.default_rng(321)
    tokens, hq, hkv, window, topk = 160, 8, 4, 8, 12
    pq = rng.standard_normal((hq, tokens, 128)).astype(np.float32)
    pq[1, 37, 5] = np.nan
    pq[6, [3, 40, 41, 130], 0] = np.inf
    kv = rng.standard_normal(tokens * 2 * hkv * 128).astype(np.float16).view(np.uint16)
    vals, offs, rec = gpu_build(hip, pq, kv, tokens, hq, hkv, window, topk)
    evals, eoffs, erec = O.local_causal_representatives_restated(pq, kv, tokens, hq, hkv, 128, 32, window, topk)
    assert np.isnan(erec).any()
    assert np.array_equal(np.isnan(rec), np.isnan(erec))
    finite = ~np.isnan(erec)
    assert np.array_equal(rec[finite].view(np.uint32), erec[finite].view(np.uint32))
    assert np.array_equal(offs, eoffs.astype(np.int64))
    assert np.array_equal(vals.view(np.uint32), evals.view(np.uint32))
