"""GPU parity sweep of the decode step (sa_hip_decode_step: append + seal +
score + select + attend) over seeded random configurations, against the
oracle step by step: query heads per KV head 1/2/4, 1-8 KV heads, 1-5
sequences with lengths at and around block boundaries (and empty ones),
local tails of 0-64 tokens, representatives per KV head or per query head,
padded and unpadded rep_stride, init/local/budget splits including budgets
that take every block, and per-sequence budgets.  Each configuration runs 5
steps; every step's ids and counts must equal the oracle's
(select_shared_blocks, cpp/src/selection.cpp:96-147), its attention be within
2e-3 (attention_reference.cpp:55-96), and the pool bytes, representatives and
counters after the last step be bit-exact (kv_lifecycle_main.cpp:92-113)."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import assert_close_2e3, device_kv, pool_numpy, status_tensor, to_dev
from paged_case import D, PAGE, make_case

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128)))
STEPS = 5


def config(seed):
    rng = np.random.default_rng(seed)
    group = int(rng.choice([1, 2, 4]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    batch = int(rng.integers(1, 6))
    lengths = []
    for _ in range(batch):
        kind = rng.integers(0, 4)
        if kind == 0:
            lengths.append(int(rng.integers(0, 64)))
        else:
            m = int(rng.integers(1, 200))
            lengths.append(max(0, 32 * m + int(rng.choice([-2, -1, 0, 1, 2, 17]))))
    local_tokens = int(rng.choice([0, 32, 64]))
    rep_heads = None if rng.random() < 0.6 else hkv * group
    init = int(rng.integers(0, 5))
    local = int(rng.integers(0, 9))
    budget = int(rng.integers(init + local + 1, init + local + 60))
    sel_stride = budget + int(rng.choice([0, 0, 7]))
    budgets = None
    if rng.random() < 0.3:
        budgets = rng.integers(init + local, sel_stride + 1, size=batch).astype(np.int32)
        budgets = np.maximum(budgets, 1)
    need = max(lengths) // PAGE + 2 + (STEPS + PAGE - 1) // PAGE
    table_stride = need + int(rng.integers(0, 4))
    rep_stride = None if rng.random() < 0.5 else (table_stride + 31) // 32 * 32
    return dict(group=group, hkv=hkv, batch=batch, lengths=lengths, local_tokens=local_tokens, rep_heads=rep_heads,
                init=init, local=local, budget=budget, sel_stride=sel_stride, budgets=budgets,
                table_stride=table_stride, rep_stride=rep_stride)


def oracle_step(case, k, v, c, groups=None):
    """groups: selection groups (default: one per KV head; 1: the shared selection)."""
    groups = groups or case.hkv
    O.paged_append(case.pool, PAGE, case.table, case.seq_len, k=k, v=v, batch=case.batch, hkv=case.hkv, d=D)
    O.paged_seal(case.pool, PAGE, case.table, case.seq_len, case.sealed, case.generation, case.reps,
                 case.rep_heads, case.rep_stride, case.batch, case.hq, case.hkv, D, c["local_tokens"])
    sel_stride = c["sel_stride"]
    esel = np.full((case.batch, groups, sel_stride), -1, np.int32)
    ecnt = np.zeros((case.batch, groups), np.int32)
    for b in range(case.batch):
        bud = c["budget"] if c["budgets"] is None else int(c["budgets"][b])
        s_, n_ = O.paged_score_select(case.query[b:b + 1], case.reps[b:b + 1], case.sealed[b:b + 1], 1, case.hq,
                                      case.hkv, D, case.rep_heads, case.rep_stride, groups, bud, c["init"],
                                      c["local"], sel_stride=sel_stride)
        esel[b], ecnt[b] = s_[0], n_[0]
    expect = O.paged_sparse_attention(case.pool, PAGE, case.table, case.seq_len, case.sealed, esel, ecnt, groups,
                                      case.query, case.batch, case.hq, case.hkv, D, SCALE)
    return esel, ecnt, expect


@pytest.mark.parametrize("seed", range(64))
def test_decode_step_sweep(hip, seed):
    run_sweep(hip, seed, 9100, 9200, None)


@pytest.mark.parametrize("seed", range(32))
def test_decode_step_shared_sweep(hip, seed):
    """The same sweep with the shared selection (select_groups 1): one launch
    where the lists are short enough (select_attend_shared_supported), the
    separate launches otherwise; both against the oracle's shared selection."""
    run_sweep(hip, seed, 9300, 9400, 1)


def run_sweep(hip, seed, config_base, case_base, groups):
    c = config(config_base + seed)
    print(f"case: sweep seed={seed} groups={groups} {c}", flush=True)
    hq = c["hkv"] * c["group"]
    case = make_case(case_base + seed, c["batch"], hq, c["hkv"], c["lengths"], table_stride=c["table_stride"],
                     rep_heads=c["rep_heads"], local_tokens=c["local_tokens"], rep_stride=c["rep_stride"],
                     planted=2)
    groups = groups or c["hkv"]
    kv = device_kv(case)
    ws, _ = hip.decode_step_workspace(kv)
    st = status_tensor()
    budgets = None if c["budgets"] is None else to_dev(c["budgets"])
    rng = np.random.default_rng(seed)
    for step in range(STEPS):
        k = (rng.standard_normal((c["batch"], c["hkv"], D)) * 2).astype(np.float32)
        v = (rng.standard_normal((c["batch"], c["hkv"], D)) * 2).astype(np.float32)
        case.query[:] = rng.standard_normal(case.query.shape).astype(np.float32)
        sel, cnt, out = hip.decode_step(kv, to_dev(k), to_dev(v), c["local_tokens"], to_dev(case.query), groups,
                                        c["budget"], c["init"], c["local"], SCALE, ws, status=st,
                                        sel_stride=c["sel_stride"], budgets=budgets)
        esel, ecnt, expect = oracle_step(case, k, v, c, groups)
        torch.cuda.synchronize()
        assert int(st.item()) == 0, step
        got_sel, got_cnt = sel.cpu().numpy(), cnt.cpu().numpy()
        assert np.array_equal(got_cnt, ecnt), step
        for b in range(c["batch"]):
            for g in range(groups):
                n = int(ecnt[b, g])
                assert got_sel[b, g, :n].tolist() == esel[b, g, :n].tolist(), (step, b, g)
        got = out.cpu().numpy()
        assert np.isfinite(got).all(), step
        assert_close_2e3(got, expect)
    assert np.array_equal(kv.seq_len.cpu().numpy(), case.seq_len)
    assert np.array_equal(kv.sealed.cpu().numpy(), case.sealed)
    assert np.array_equal(kv.generation.cpu().numpy(), case.generation)
    assert np.array_equal(pool_numpy(kv), case.pool)
    assert np.array_equal(kv.reps.cpu().numpy().view(np.uint32), case.reps.view(np.uint32))
    assert int(ws[:kv.batch].abs().sum().item()) == 0, "arrival counters must be left at zero"
