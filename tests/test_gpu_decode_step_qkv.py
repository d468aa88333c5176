"""GPU parity: the decode step fed by its q/k/v producer
(sa_hip_decode_step_qkv) against the two calls it replaces
(sa_hip_qkv_project_rms, then sa_hip_decode_step; reference
cpp/src/qwen_chain_main.cpp:365-395), on two copies of the same paged state
over steps that seal blocks.

Bar: bit for bit.  Where the step's one launch applies with 1 or 2 query heads
per KV head, its workgroups run the producer's epilogue (the same device
function as the producer's reduce launch) and attend from the same query
values, so q, k, v, the pool, representatives, counters, ids and the
attention output are equal bit for bit; elsewhere the entry runs the two calls
themselves.  The two calls are held to the oracle in test_gpu_producer.py and
the decode step tests; one step of the producer-fed path is also checked
against the oracle's attention here."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import device_kv, status_tensor, to_dev
from paged_case import PAGE, make_case

pytestmark = pytest.mark.gpu


def make_weights(rng, hidden, hq, hkv):
    s = 1.0 / np.sqrt(hidden)
    return dict(
        wq=to_dev((rng.standard_normal((hq * 128, hidden)) * s).astype(np.float32)),
        wk=to_dev((rng.standard_normal((hkv * 128, hidden)) * s).astype(np.float32)),
        wv=to_dev((rng.standard_normal((hkv * 128, hidden)) * s).astype(np.float32)),
        qn=to_dev((1 + 0.1 * rng.standard_normal(128)).astype(np.float32)),
        kn=to_dev((1 + 0.1 * rng.standard_normal(128)).astype(np.float32)),
        inorm=to_dev((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)))


def state(kv):
    return [t.clone() for t in (kv.pool, kv.reps, kv.seq_len, kv.sealed, kv.generation)]


@pytest.mark.parametrize("hq,hkv,rep_heads,splits,rms,batch", [
    (16, 8, None, 1, True, 4),     # two launches: 2 query heads per KV head, representatives per KV head
    (16, 8, 16, 1, True, 4),       # two launches: 2 query heads, representatives per query head
    (8, 8, None, 1, False, 4),     # two launches: 1 query head per KV head, no input RMSNorm
    (32, 8, None, 1, True, 4),     # 4 query heads per KV head: the two calls
    (16, 8, None, 2, True, 4),     # split attention: the two calls
    (16, 8, None, 1, True, 70),    # two launches over two 64-row tiles of the projection
])
def test_decode_step_qkv_equals_two_calls(hip, hq, hkv, rep_heads, splits, rms, batch):
    print(f"case: decode_step_qkv hq={hq} hkv={hkv} rep_heads={rep_heads} splits={splits} rms={rms} batch={batch}",
          flush=True)
    rng = np.random.default_rng(hq * 10 + hkv + (rep_heads or 0) + splits + batch)
    hidden = 1024
    lengths = ([32 * 40 + 25, 32 * 17 + 5, 32 * 25 + 30, 32 * 9] * 18)[:batch]
    case = make_case(300 + hq + splits, batch, hq, hkv, lengths, rep_heads=rep_heads, planted=2)
    kva, kvb = device_kv(case), device_kv(case)
    W = make_weights(rng, hidden, hq, hkv)
    inorm = W["inorm"] if rms else None
    budget, init, local = 16, 1, 2
    scale = float(np.float32(1.0) / np.sqrt(np.float32(128)))
    assert hip.select_attend_fused(kva, hkv, splits) == (splits == 1)
    wsa, _ = hip.decode_step_workspace(kva, splits)
    wsb, _ = hip.decode_step_workspace(kvb, splits)
    qws = torch.empty(hip.lib().sa_hip_qkv_workspace_bytes(batch, hidden, hq, hkv) // 4, dtype=torch.float32,
                      device="cuda")
    qa, qb = (torch.empty((batch, hq, 128), dtype=torch.float32, device="cuda") for _ in range(2))
    ka, kb, va, vb = (torch.empty((batch, hkv, 128), dtype=torch.float32, device="cuda") for _ in range(4))
    sta, stb = status_tensor(), status_tensor()
    for step in range(12):
        x = to_dev(rng.standard_normal((batch, hidden)).astype(np.float32))
        hip.qkv_project(x, W["wq"], W["wk"], W["wv"], W["qn"], W["kn"], kva.seq_len, hq, hkv, q=qa, k=ka, v=va,
                        workspace=qws, input_norm=inorm)
        sa_, ca, oa = hip.decode_step(kva, ka, va, 0, qa, hkv, budget, init, local, scale, wsa, splits=splits,
                                      status=sta)
        if step == 0:
            # the producer-fed step against the oracle on its own q/k/v
            pre = [kvb.pool.view(torch.int16).cpu().numpy().view(np.uint16).copy()] + \
                  [t.cpu().numpy().copy() for t in (kvb.reps, kvb.seq_len, kvb.sealed, kvb.generation)]
        sb, cb, ob = hip.decode_step_qkv(kvb, x, W["wq"], W["wk"], W["wv"], W["qn"], W["kn"], kvb.seq_len, qb, kb, vb,
                                         qws, 0, hkv, budget, init, local, scale, wsb, input_norm=inorm,
                                         splits=splits, status=stb)
        torch.cuda.synchronize()
        assert int(sta.item()) == 0 and int(stb.item()) == 0, step
        for a, b, what in ((qa, qb, "q"), (ka, kb, "k"), (va, vb, "v"), (sa_, sb, "ids"), (ca, cb, "counts"),
                           (oa, ob, "out")):
            assert torch.equal(a.view(torch.int32) if a.dtype == torch.float32 else a,
                               b.view(torch.int32) if b.dtype == torch.float32 else b), (step, what)
        if step == 0:
            pool, reps, seq_len, sealed, gen = pre
            gq, gk, gv = qb.cpu().numpy(), kb.cpu().numpy(), vb.cpu().numpy()
            O.paged_append(pool, PAGE, case.table, seq_len, k=gk.reshape(batch, -1), v=gv.reshape(batch, -1),
                           batch=batch, hkv=hkv, d=128)
            O.paged_seal(pool, PAGE, case.table, seq_len, sealed, gen, reps, case.rep_heads, case.rep_stride, batch,
                         hq, hkv, 128, 0)
            esel, ecnt = O.paged_score_select(gq, reps, sealed, batch, hq, hkv, 128, case.rep_heads,
                                              case.rep_stride, hkv, budget, init, local)
            eout = O.paged_sparse_attention(pool, PAGE, case.table, seq_len, sealed, esel, ecnt, hkv, gq, batch, hq,
                                            hkv, 128, scale)
            assert np.array_equal(cb.cpu().numpy(), ecnt) and np.array_equal(sb.cpu().numpy(), esel)
            err = np.abs(ob.cpu().numpy().astype(np.float64) - eout)
            assert ((err <= 2e-3) | (err <= 2e-3 * np.abs(eout))).all(), float(err.max())
    for a, b in zip(state(kva), state(kvb)):
        assert torch.equal(a, b)
    assert torch.equal(wsb[:batch], torch.zeros_like(wsb[:batch]))  # arrival counters left at zero
    sealed_now = kvb.sealed.cpu().numpy()
    assert (sealed_now > case.sealed).any()  # the steps sealed blocks


def test_decode_step_qkv_graph_replays(hip):
    """The two-launch form captured in a HIP graph: every replay equals the
    eager two calls on a copy of the state."""
    rng = np.random.default_rng(5)
    batch, hq, hkv, hidden = 4, 16, 8, 1024
    case = make_case(77, batch, hq, hkv, [32 * 20 + 30, 32 * 11 + 2, 32 * 7 + 31, 32 * 30])
    kva, kvb = device_kv(case), device_kv(case)
    W = make_weights(rng, hidden, hq, hkv)
    budget, init, local = 16, 1, 2
    scale = float(np.float32(1.0) / np.sqrt(np.float32(128)))
    wsa, _ = hip.decode_step_workspace(kva, 1)
    wsb, _ = hip.decode_step_workspace(kvb, 1)
    qws = torch.empty(hip.lib().sa_hip_qkv_workspace_bytes(batch, hidden, hq, hkv) // 4, dtype=torch.float32,
                      device="cuda")
    qa, qb = (torch.empty((batch, hq, 128), dtype=torch.float32, device="cuda") for _ in range(2))
    ka, kb, va, vb = (torch.empty((batch, hkv, 128), dtype=torch.float32, device="cuda") for _ in range(4))
    sel = torch.full((batch, hkv, budget), -1, dtype=torch.int32, device="cuda")
    cnt = torch.zeros((batch, hkv), dtype=torch.int32, device="cuda")
    out = torch.empty((batch, hq, 128), dtype=torch.float32, device="cuda")
    x = torch.empty((batch, hidden), dtype=torch.float32, device="cuda")
    st = status_tensor()

    def fused():
        hip.decode_step_qkv(kvb, x, W["wq"], W["wk"], W["wv"], W["qn"], W["kn"], kvb.seq_len, qb, kb, vb, qws, 0, hkv,
                            budget, init, local, scale, wsb, input_norm=W["inorm"], selected=sel, counts=cnt, out=out,
                            status=st)

    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        # capture only: a captured launch does not run, so kvb is unchanged
        with torch.cuda.graph(g, stream=s):
            fused()
    torch.cuda.synchronize()
    for step in range(6):
        x.copy_(to_dev(rng.standard_normal((batch, hidden)).astype(np.float32)))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        hip.qkv_project(x, W["wq"], W["wk"], W["wv"], W["qn"], W["kn"], kva.seq_len, hq, hkv, q=qa, k=ka, v=va,
                        input_norm=W["inorm"])
        sa_, ca, oa = hip.decode_step(kva, ka, va, 0, qa, hkv, budget, init, local, scale, wsa)
        torch.cuda.synchronize()
        assert int(st.item()) == 0
        assert torch.equal(qa, qb) and torch.equal(ka, kb) and torch.equal(va, vb), step
        assert torch.equal(sa_, sel) and torch.equal(ca, cnt), step
        assert torch.equal(oa.view(torch.int32), out.view(torch.int32)), step
    for a, b in zip(state(kva), state(kvb)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("seed", range(8))
def test_decode_step_qkv_sweep(hip, seed):
    """Seeded configurations of the producer-fed step against the two calls,
    bit for bit: batch 1-6, 1 or 2 query heads per KV head, budgets 3-20
    blocks with init 0-2 and local 0-3, local_tokens 0, 5 or 32, with and
    without the input RMSNorm, 6 steps each."""
    rng = np.random.default_rng(900 + seed)
    hkv = int(rng.choice([2, 4, 8]))
    hq = hkv * int(rng.choice([1, 2]))
    batch = int(rng.integers(1, 7))
    local_tokens = int(rng.choice([0, 5, 32]))
    lengths = [int(rng.integers(40, 32 * 50)) for _ in range(batch)]
    budget = int(rng.integers(3, 21))
    init = int(rng.integers(0, 3))
    loc = int(rng.integers(0, 4))
    rms = bool(rng.integers(0, 2))
    print(f"case: decode_step_qkv sweep seed={seed} hq={hq} hkv={hkv} batch={batch} local_tokens={local_tokens} "
          f"budget={budget} init={init} local={loc} rms={rms}", flush=True)
    case = make_case(950 + seed, batch, hq, hkv, lengths, local_tokens=local_tokens)
    kva, kvb = device_kv(case), device_kv(case)
    hidden = 1024
    W = make_weights(rng, hidden, hq, hkv)
    inorm = W["inorm"] if rms else None
    scale = float(np.float32(1.0) / np.sqrt(np.float32(128)))
    wsa, _ = hip.decode_step_workspace(kva, 1)
    wsb, _ = hip.decode_step_workspace(kvb, 1)
    qws = torch.empty(hip.lib().sa_hip_qkv_workspace_bytes(batch, hidden, hq, hkv) // 4, dtype=torch.float32,
                      device="cuda")
    qa, qb = (torch.empty((batch, hq, 128), dtype=torch.float32, device="cuda") for _ in range(2))
    ka, kb, va, vb = (torch.empty((batch, hkv, 128), dtype=torch.float32, device="cuda") for _ in range(4))
    sta, stb = status_tensor(), status_tensor()
    for step in range(6):
        x = to_dev(rng.standard_normal((batch, hidden)).astype(np.float32))
        hip.qkv_project(x, W["wq"], W["wk"], W["wv"], W["qn"], W["kn"], kva.seq_len, hq, hkv, q=qa, k=ka, v=va,
                        workspace=qws, input_norm=inorm)
        sa_, ca, oa = hip.decode_step(kva, ka, va, local_tokens, qa, hkv, budget, init, loc, scale, wsa, status=sta)
        sb, cb, ob = hip.decode_step_qkv(kvb, x, W["wq"], W["wk"], W["wv"], W["qn"], W["kn"], kvb.seq_len, qb, kb, vb,
                                         qws, local_tokens, hkv, budget, init, loc, scale, wsb, input_norm=inorm,
                                         status=stb)
        torch.cuda.synchronize()
        assert int(sta.item()) == int(stb.item()), step
        for a, b, what in ((qa, qb, "q"), (ka, kb, "k"), (va, vb, "v"), (sa_, sb, "ids"), (ca, cb, "counts"),
                           (oa, ob, "out")):
            assert torch.equal(a.view(torch.int32) if a.dtype == torch.float32 else a,
                               b.view(torch.int32) if b.dtype == torch.float32 else b), (step, what)
    for a, b in zip(state(kva), state(kvb)):
        assert torch.equal(a, b)
