"""GPU parity: the InfLLM online seal (sa_hip_decode_step_online,
sa_hip_append_seal_online), the reference's P1.3c.4
(cpp/src/online_seal_main.cpp:41-44).

When a decode step seals a block, the representative of each query head is
build_local_causal_representatives (cpp/src/selection.cpp:12-94) over that
block alone: its 32 keys and the 32 decode queries issued with them.  Bars:
page bytes, representatives (bits), counters and the query ring equal the
oracle's after every step (the oracle's builder with libm's expf, which the
CPU suite pins to the reference's own builder); selected ids bit-exact; the
attention within 2e-3.  The P1.3c.4 closed form: 28 layers, each sealing its
32-token tail (window 32, top 4) as block 16 behind a 16-block prompt; the
stored block equals the tail; the selection over the new block alone
(select_shared_blocks(last query, new representative, 16 heads, 1 block,
budget 1)) picks it on all 28 layers."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import assert_close_2e3, device_kv, pool_numpy, status_tensor, to_dev
from paged_case import D, PAGE, make_case, oracle_online_append_seal, oracle_select_attend

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128)))


def check_state(kv, case, seal, ring):
    assert np.array_equal(kv.seq_len.cpu().numpy(), case.seq_len)
    assert np.array_equal(kv.sealed.cpu().numpy(), case.sealed)
    assert np.array_equal(kv.generation.cpu().numpy(), case.generation)
    assert np.array_equal(pool_numpy(kv), case.pool)
    assert np.array_equal(kv.reps.cpu().numpy().view(np.uint32), case.reps.view(np.uint32))
    assert np.array_equal(seal.ring.cpu().numpy().view(np.uint32), ring.view(np.uint32))


def start_ring(hip, kv, case, rng, ring_tokens, window, topk):
    """The caller's prefill queries of the unsealed tail positions, in the ring."""
    seal = hip.OnlineSeal(kv, ring_tokens=ring_tokens, window=window, topk=topk)
    ring = np.zeros((case.batch, case.hq, ring_tokens, D), np.float32)
    for b in range(case.batch):
        for p in range(int(case.sealed[b]) * PAGE, int(case.seq_len[b])):
            ring[b, :, p % ring_tokens, :] = rng.standard_normal((case.hq, D)).astype(np.float32)
    seal.ring.copy_(torch.from_numpy(ring))
    return seal, ring


@pytest.mark.parametrize("hq,local_tokens,ring_tokens,window,topk",
                         [(16, 0, 32, 32, 4), (32, 0, 32, 32, 4), (16, 32, 64, 8, 2), (32, 32, 96, 32, 32),
                          (8, 0, 40, 5, 1)])
def test_decode_step_online_bit_exact(hip, hq, local_tokens, ring_tokens, window, topk):
    """40 fused decode steps across seal boundaries: state and ring bit-exact
    every few steps, ids bit-exact and outputs within 2e-3 every step."""
    print(f"case: hq={hq} local={local_tokens} ring={ring_tokens} window={window} topk={topk}", flush=True)
    lengths = [32 * 40 + 30 + local_tokens, 32 * 12 + local_tokens, 32 * 9 + 13 + local_tokens]
    case = make_case(900 + hq + local_tokens, 3, hq, 8, lengths, table_stride=60, local_tokens=local_tokens,
                     rep_heads=hq, planted=3)
    kv = device_kv(case)
    rng = np.random.default_rng(hq + topk)
    seal, ring = start_ring(hip, kv, case, rng, ring_tokens, window, topk)
    budget, init, local = 16, 2, 3
    assert hip.select_attend_fused(kv, 8, sel_stride=budget)
    ws, _ = hip.decode_step_workspace(kv)
    st = status_tensor()
    seals = 0
    for step in range(40):
        k = (rng.standard_normal((3, 8, D)) * 2).astype(np.float32)
        v = (rng.standard_normal((3, 8, D)) * 2).astype(np.float32)
        case.query[:] = rng.standard_normal(case.query.shape).astype(np.float32)
        sel, cnt, out = hip.decode_step_online(kv, to_dev(k), to_dev(v), local_tokens, to_dev(case.query), seal, 8,
                                               budget, init, local, SCALE, ws, status=st)
        before = case.sealed.copy()
        oracle_online_append_seal(case, ring, k, v, case.query, local_tokens, window, topk)
        seals += int((case.sealed - before).sum())
        esel, ecnt, expect = oracle_select_attend(case, budget, init, local, budget, SCALE)
        torch.cuda.synchronize()
        assert int(st.item()) == 0, step
        got_sel, got_cnt = sel.cpu().numpy(), cnt.cpu().numpy()
        assert np.array_equal(got_cnt, ecnt), step
        for b in range(3):
            for g in range(8):
                assert got_sel[b, g, : ecnt[b, g]].tolist() == esel[b, g, : ecnt[b, g]].tolist(), (step, b, g)
        assert_close_2e3(out.cpu().numpy(), expect)
        if step % 7 == 0 or step == 39:
            check_state(kv, case, seal, ring)
    assert seals >= 4
    assert int(ws[:kv.batch].abs().sum().item()) == 0


@pytest.mark.parametrize("hq,splits", [(64, 1), (16, 2), (32, 2)])
def test_online_seal_separate_launches(hip, hq, splits):
    """8 query heads per KV head (no fused kernel) and split requests run
    sa_hip_append_seal_online + selection + attention: the same results."""
    print(f"case: hq={hq} splits={splits}", flush=True)
    case = make_case(950 + hq, 2, hq, 8, [32 * 20 + 29, 32 * 7 + 31], table_stride=30, rep_heads=hq)
    kv = device_kv(case)
    rng = np.random.default_rng(5)
    seal, ring = start_ring(hip, kv, case, rng, 32, 32, 4)
    assert not hip.select_attend_fused(kv, 8, splits, sel_stride=12)
    ws, _ = hip.decode_step_workspace(kv, splits)
    st = status_tensor()
    for step in range(5):
        k = rng.standard_normal((2, 8, D)).astype(np.float32)
        v = rng.standard_normal((2, 8, D)).astype(np.float32)
        case.query[:] = rng.standard_normal(case.query.shape).astype(np.float32)
        sel, cnt, out = hip.decode_step_online(kv, to_dev(k), to_dev(v), 0, to_dev(case.query), seal, 8, 12, 2, 2,
                                               SCALE, ws, splits=splits, status=st)
        oracle_online_append_seal(case, ring, k, v, case.query, 0, 32, 4)
        esel, ecnt, expect = oracle_select_attend(case, 12, 2, 2, 12, SCALE)
        torch.cuda.synchronize()
        assert int(st.item()) == 0
        assert np.array_equal(cnt.cpu().numpy(), ecnt)
        got = sel.cpu().numpy()
        for b in range(2):
            for g in range(8):
                assert got[b, g, : ecnt[b, g]].tolist() == esel[b, g, : ecnt[b, g]].tolist()
        assert_close_2e3(out.cpu().numpy(), expect)
    check_state(kv, case, seal, ring)
    assert case.sealed.tolist() == [21, 8]


def test_p13c4_online_seal_28_layers(hip):
    """P1.3c.4 (online_seal_main.cpp:23-47, docs P1.3c.4): 28 layers (here 28
    sequences of one launch), 16 query / 8 KV heads; each holds a 512-token
    prompt (16 sealed blocks) and a 31-token tail whose queries are in the
    ring; one decode step appends the 32nd tail token and seals the tail as
    block 16 with window 32, top 4.  The new representatives equal the
    reference's builder over the tail, the sealed page equals the tail bytes,
    and the selection over the new block alone picks it on every layer."""
    layers, hq, hkv = 28, 16, 8
    case = make_case(1304, layers, hq, hkv, [32 * 16 + 31] * layers, table_stride=20, rep_heads=hq)
    kv = device_kv(case)
    rng = np.random.default_rng(13)
    seal, ring = start_ring(hip, kv, case, rng, 32, 32, 4)
    k = rng.standard_normal((layers, hkv, D)).astype(np.float32)
    v = rng.standard_normal((layers, hkv, D)).astype(np.float32)
    ws, _ = hip.decode_step_workspace(kv)
    st = status_tensor()
    hip.decode_step_online(kv, to_dev(k), to_dev(v), 0, to_dev(case.query), seal, 8, 4, 1, 1, SCALE, ws, status=st)
    oracle_online_append_seal(case, ring, k, v, case.query, 0, 32, 4, use_ref=O.ref_available())
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    check_state(kv, case, seal, ring)
    sealed_layers = int((kv.sealed.cpu().numpy() == 17).sum())
    assert sealed_layers == 28
    # the stored block 16 is the tail: 31 prefilled tokens + the appended one
    pool = pool_numpy(kv)
    for b in range(layers):
        assert np.array_equal(pool[case.table[b, 16]], case.pool[case.table[b, 16]])
    # select_shared_blocks(last query, the new representative, 16 heads, 1 block, budget 1, init 0, local 0)
    view = hip.PagedKV(layers, hq, hkv, kv.table_stride, num_pages=kv.num_pages, rep_heads=hq,
                       rep_stride=kv.rep_stride, pool=kv.pool)
    view.reps = kv.reps[:, :, :, 16:]
    view.sealed.fill_(1)
    view.seq_len.fill_(32)
    sel, cnt = hip.score_select(view, to_dev(case.query), 1, 1, 0, 0)
    torch.cuda.synchronize()
    selected = 0
    for b in range(layers):
        rep_new = np.ascontiguousarray(case.reps[b, :, :, 16])[:, None, :]
        ids, _ = O.select_shared_blocks(case.query[b], rep_new, hq, 1, D, 1, 0, 0)
        assert ids.tolist() == [0]
        selected += int(cnt[b, 0].item() == 1 and sel[b, 0, 0].item() == 0)
    assert selected == 28
    assert case.reps[:, :, :, 16].size == 28 * 16 * 128  # representative values of P1.3c.4


@pytest.mark.parametrize("hq,fused", [(16, True), (64, False)])
def test_online_seal_nan_queries_in_ring(hip, hq, fused):
    """Non-finite prefill queries in the ring: the sealed blocks' received
    masses go NaN for the keys in their windows and rank after every number
    (token order among them), on the GPU as in the oracle, so the page
    bytes, representatives, counters and ring equal the oracle's bit for
    bit; decode queries stay finite."""
    print(f"case: NaN ring queries hq={hq} fused={fused}", flush=True)
    case = make_case(960 + hq, 2, hq, 8, [32 * 5 + 20, 32 * 3 + 30], table_stride=12, rep_heads=hq)
    kv = device_kv(case)
    rng = np.random.default_rng(17)
    seal, ring = start_ring(hip, kv, case, rng, 32, 8, 6)
    ring[0, 3, (32 * 5 + 5) % 32, 7] = np.nan
    ring[1, 0, (32 * 3 + 9) % 32, :] = np.inf
    ring[1, hq - 1, (32 * 3 + 29) % 32, 100] = np.nan
    seal.ring.copy_(torch.from_numpy(ring))
    assert hip.select_attend_fused(kv, 8, sel_stride=8) == fused
    ws, _ = hip.decode_step_workspace(kv)
    st = status_tensor()
    for step in range(13):
        k = rng.standard_normal((2, 8, D)).astype(np.float32)
        v = rng.standard_normal((2, 8, D)).astype(np.float32)
        case.query[:] = rng.standard_normal(case.query.shape).astype(np.float32)
        hip.decode_step_online(kv, to_dev(k), to_dev(v), 0, to_dev(case.query), seal, 8, 8, 2, 2, SCALE, ws,
                               status=st)
        oracle_online_append_seal(case, ring, k, v, case.query, 0, 8, 6)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    assert case.sealed.tolist() == [6, 4]
    check_state(kv, case, seal, ring)
