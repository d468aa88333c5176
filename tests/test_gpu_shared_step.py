"""GPU parity: the shared selection as one launch (decode_step and
select_attend with select_groups 1: one block set per sequence over every
query head, the reference's shared mode, select_shared_blocks over all heads,
cpp/src/selection.cpp:96-147, as selection_main.cpp:178-181 and
pipeline_main.cpp:480-499 call it).

Every workgroup of a sequence scores the whole shared set itself and seals
every KV head's representative of a filled block (the new token's key from
the step's input).  Ids and counts must be bit-exact with the oracle every
step, attention within 2e-3 of the oracle (attention_reference semantics,
attention_reference.cpp:55-96), and the pool, representatives and counters
bit-exact after the checked steps, also when a step seals the block that
holds its own new token (local tail 0).  The split launches on a copy of the
state give the same ids and state bit for bit."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import assert_close_2e3, device_kv, pool_numpy, status_tensor, to_dev
from paged_case import D, PAGE, make_case

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128)))


def oracle_shared(case, budget, init, local, sel_stride, budgets=None):
    """Shared selection (one list per sequence) + attention, per sequence."""
    esel = np.full((case.batch, 1, sel_stride), -1, np.int32)
    ecnt = np.zeros((case.batch, 1), np.int32)
    for b in range(case.batch):
        bud = budget if budgets is None else int(budgets[b])
        s_, c_ = O.paged_score_select(case.query[b:b + 1], case.reps[b:b + 1], case.sealed[b:b + 1], 1, case.hq,
                                      case.hkv, D, case.rep_heads, case.rep_stride, 1, bud, init, local,
                                      sel_stride=sel_stride)
        esel[b], ecnt[b] = s_[0], c_[0]
    expect = O.paged_sparse_attention(case.pool, PAGE, case.table, case.seq_len, case.sealed, esel, ecnt, 1,
                                      case.query, case.batch, case.hq, case.hkv, D, SCALE)
    return esel, ecnt, expect


def oracle_shared_decode(case, local_tokens, budget, init, local, sel_stride, k=None, v=None, k16=None, v16=None,
                         budgets=None):
    if k16 is not None:
        O.paged_append(case.pool, PAGE, case.table, case.seq_len, k16=k16, v16=v16, batch=case.batch, hkv=case.hkv,
                       d=D)
    else:
        O.paged_append(case.pool, PAGE, case.table, case.seq_len, k=k, v=v, batch=case.batch, hkv=case.hkv, d=D)
    O.paged_seal(case.pool, PAGE, case.table, case.seq_len, case.sealed, case.generation, case.reps,
                 case.rep_heads, case.rep_stride, case.batch, case.hq, case.hkv, D, local_tokens)
    return oracle_shared(case, budget, init, local, sel_stride, budgets)


def check_state(kv, case):
    assert np.array_equal(kv.seq_len.cpu().numpy(), case.seq_len)
    assert np.array_equal(kv.sealed.cpu().numpy(), case.sealed)
    assert np.array_equal(kv.generation.cpu().numpy(), case.generation)
    assert np.array_equal(pool_numpy(kv), case.pool)
    assert np.array_equal(kv.reps.cpu().numpy().view(np.uint32), case.reps.view(np.uint32))


def check_ids(sel, cnt, esel, ecnt, tag):
    assert np.array_equal(cnt, ecnt), tag
    for b in range(esel.shape[0]):
        c = int(ecnt[b, 0])
        assert sel[b, 0, :c].tolist() == esel[b, 0, :c].tolist(), (tag, b)


@pytest.mark.parametrize("hq,local_tokens,f16", [(16, 0, False), (16, 16, False), (8, 0, False), (16, 0, True),
                                                  (32, 0, False), (32, 16, True)])
def test_shared_decode_steps_bit_exact(hip, hq, local_tokens, f16):
    """36 one-launch steps of three sequences (tails of 30, 0 and 25 tokens:
    every sequence crosses a seal), queries and tokens fresh each step."""
    print(f"case: shared decode steps hq={hq} local_tokens={local_tokens} f16={f16}", flush=True)
    case = make_case(900 + hq + local_tokens + int(f16), 3, hq, 8, [32 * 60 + 30, 32 * 9, 32 * 30 + 25],
                     table_stride=64, local_tokens=local_tokens, planted=4)
    kv = device_kv(case)
    assert hip.select_attend_fused(kv, 1)
    ws, _ = hip.decode_step_workspace(kv)
    st = status_tensor()
    rng = np.random.default_rng(17 + hq)
    budget, init, local = 16, 1, 2
    for step in range(36):
        case.query[:] = rng.standard_normal(case.query.shape).astype(np.float32)
        if f16:
            k16 = (rng.standard_normal((3, 8, D)) * 2).astype(np.float16).view(np.uint16)
            v16 = (rng.standard_normal((3, 8, D)) * 2).astype(np.float16).view(np.uint16)
            kd = to_dev(k16.view(np.int16)).view(torch.uint16)
            vd = to_dev(v16.view(np.int16)).view(torch.uint16)
            esel, ecnt, expect = oracle_shared_decode(case, local_tokens, budget, init, local, budget, k16=k16,
                                                      v16=v16)
        else:
            k = (rng.standard_normal((3, 8, D)) * 2).astype(np.float32)
            v = (rng.standard_normal((3, 8, D)) * 2).astype(np.float32)
            kd, vd = to_dev(k), to_dev(v)
            esel, ecnt, expect = oracle_shared_decode(case, local_tokens, budget, init, local, budget, k=k, v=v)
        sel, cnt, out = hip.decode_step(kv, kd, vd, local_tokens, to_dev(case.query), 1, budget, init, local, SCALE,
                                        ws, status=st)
        torch.cuda.synchronize()
        assert int(st.item()) == 0, step
        check_ids(sel.cpu().numpy(), cnt.cpu().numpy(), esel, ecnt, step)
        assert_close_2e3(out.cpu().numpy(), expect)
        if step % 11 == 0 or step == 35:
            check_state(kv, case)
    assert int(ws[:kv.batch].abs().sum().item()) == 0, "arrival counters must be left at zero"


def test_c1_shape_shared_decode_steps_equal_split_launches(hip):
    """The reference's C1/C2 shape (1 sequence, 16 query / 8 KV heads, 2048
    tokens, budget 16 = init 1 + local 2 + 13): 40 one-launch steps against
    the same steps as separate launches (splits 2) on a copy of the state:
    ids, counts, pool, representatives and counters equal bit for bit, the
    outputs to fp32 rounding (the pages are visited in another order), and
    both within 2e-3 of the oracle."""
    case = make_case(910, 1, 16, 8, [2047], table_stride=68, planted=4)
    kv_a, kv_b = device_kv(case), device_kv(case)
    assert hip.select_attend_fused(kv_a, 1) and not hip.select_attend_fused(kv_a, 1, splits=2)
    ws_a, _ = hip.decode_step_workspace(kv_a)
    ws_b, _ = hip.decode_step_workspace(kv_b, 2)
    st = status_tensor()
    rng = np.random.default_rng(23)
    budget, init, local = 16, 1, 2
    for step in range(40):
        case.query[:] = rng.standard_normal(case.query.shape).astype(np.float32)
        k = (rng.standard_normal((1, 8, D)) * 2).astype(np.float32)
        v = (rng.standard_normal((1, 8, D)) * 2).astype(np.float32)
        q = to_dev(case.query)
        sel_a, cnt_a, out_a = hip.decode_step(kv_a, to_dev(k), to_dev(v), 0, q, 1, budget, init, local, SCALE, ws_a,
                                              status=st)
        sel_b, cnt_b, out_b = hip.decode_step(kv_b, to_dev(k), to_dev(v), 0, q, 1, budget, init, local, SCALE, ws_b,
                                              splits=2, status=st)
        esel, ecnt, expect = oracle_shared_decode(case, 0, budget, init, local, budget, k=k, v=v)
        torch.cuda.synchronize()
        assert int(st.item()) == 0, step
        check_ids(sel_a.cpu().numpy(), cnt_a.cpu().numpy(), esel, ecnt, step)
        assert np.array_equal(sel_a.cpu().numpy(), sel_b.cpu().numpy()), step
        assert np.array_equal(cnt_a.cpu().numpy(), cnt_b.cpu().numpy()), step
        a, b = out_a.cpu().numpy(), out_b.cpu().numpy()
        err = np.abs(a.astype(np.float64) - b)
        assert (err <= 1e-5 + 1e-5 * np.abs(b)).all(), (step, float(err.max()))
        assert_close_2e3(a, expect)
    check_state(kv_a, case)
    check_state(kv_b, case)
    assert int(case.sealed[0]) == 65


@pytest.mark.parametrize("hq", [16, 8, 32])
def test_shared_select_attend_budgets_and_ties(hip, hq):
    """select_attend (no append) with select_groups 1 in one launch: mixed
    lengths (empty, a single block, under and over the budget, 120 blocks),
    per-sequence budgets, and duplicated representatives (equal scores,
    lowest id first)."""
    print(f"case: shared select_attend hq={hq}", flush=True)
    lengths = [0, 32, 32 * 5 + 7, 32 * 120 + 3, 32 * 40]
    case = make_case(920 + hq, 5, hq, 8, lengths, table_stride=122, planted=3)
    for b in (3, 4):
        case.reps[b, :, :, 20:30] = case.reps[b, :, :, 10:11]  # ties with block 10
    kv = device_kv(case)
    assert hip.select_attend_fused(kv, 1)
    budgets = np.array([8, 8, 4, 40, 12], np.int32)
    st = status_tensor()
    sel, cnt, out = hip.select_attend(kv, to_dev(case.query), 1, 40, 2, 2, SCALE, status=st, sel_stride=40,
                                      budgets=to_dev(budgets))
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    esel, ecnt, expect = oracle_shared(case, 40, 2, 2, 40, budgets)
    check_ids(sel.cpu().numpy(), cnt.cpu().numpy(), esel, ecnt, "select_attend")
    assert_close_2e3(out.cpu().numpy(), expect)


def test_shared_one_launch_predicate(hip):
    """The one-launch shared form takes 1, 2 or 4 query heads per KV head,
    per-KV-head representatives, rows of at most 128 blocks and a bounded
    repeat of the representative reads; other shapes run the split launches."""
    def fused(batch, hq, table_stride, rep_heads=None):
        case = make_case(930, batch, hq, 8, [32 * 4] * batch, table_stride=table_stride, rep_heads=rep_heads)
        return hip.select_attend_fused(device_kv(case), 1)
    assert fused(1, 16, 64)
    assert fused(2, 8, 120)
    assert fused(1, 32, 64)
    assert not fused(1, 64, 64)            # 8 query heads per KV head
    assert not fused(1, 16, 130)           # rows past 128 blocks
    assert not fused(1, 16, 64, rep_heads=16)  # a representative per query head
    assert fused(16, 16, 64)
    assert not fused(20, 16, 64)           # the repeated reads past the byte budget


def test_shared_decode_steps_long_lists_split_selection(hip):
    """Shared lists past the one-launch form (rows of 520 blocks): the decode
    step runs as separate launches, its selection spread over the device with
    the scores in the step's workspace.  12 steps across a seal: ids bit-exact,
    attention within 2e-3, state bit-exact."""
    case = make_case(940, 2, 16, 8, [32 * 500 + 25, 32 * 300 + 5], table_stride=520, planted=4)
    kv = device_kv(case)
    assert not hip.select_attend_fused(kv, 1)
    ws, _ = hip.decode_step_workspace(kv)
    st = status_tensor()
    rng = np.random.default_rng(29)
    budget, init, local = 64, 4, 8
    for step in range(12):
        case.query[:] = rng.standard_normal(case.query.shape).astype(np.float32)
        k = (rng.standard_normal((2, 8, D)) * 2).astype(np.float32)
        v = (rng.standard_normal((2, 8, D)) * 2).astype(np.float32)
        sel, cnt, out = hip.decode_step(kv, to_dev(k), to_dev(v), 0, to_dev(case.query), 1, budget, init, local,
                                        SCALE, ws, status=st)
        esel, ecnt, expect = oracle_shared_decode(case, 0, budget, init, local, budget, k=k, v=v)
        torch.cuda.synchronize()
        assert int(st.item()) == 0, step
        check_ids(sel.cpu().numpy(), cnt.cpu().numpy(), esel, ecnt, step)
        assert_close_2e3(out.cpu().numpy(), expect)
    check_state(kv, case)
    assert int(case.sealed[0]) == 501


def test_shared_flags_bad_budget_and_capacity(hip):
    """The one-launch shared form flags a per-sequence budget below init +
    local (that sequence selects nothing, the others select) and a sequence
    with more sealed blocks than rep_stride (capacity: nothing selected, its
    tail attended), like the separate selection."""
    case = make_case(950, 2, 16, 8, [32 * 40 + 3, 32 * 30])
    kv = device_kv(case)
    assert hip.select_attend_fused(kv, 1)
    q = to_dev(case.query)
    st = status_tensor()
    budgets = to_dev(np.array([20, 10], np.int32))  # 10 < init + local
    sel, cnt, out = hip.select_attend(kv, q, 1, 20, 4, 8, SCALE, status=st, sel_stride=20, budgets=budgets)
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_BAD_BUDGET
    assert cnt.cpu().numpy()[:, 0].tolist() == [20, 0]
    kv.sealed.copy_(to_dev(np.array([case.rep_stride + 1, 30], np.int32)))
    kv.seq_len.copy_(to_dev(np.array([32 * (case.rep_stride + 1) + 3, 32 * 30], np.int32)))
    st.zero_()
    sel, cnt, out = hip.select_attend(kv, q, 1, 20, 4, 8, SCALE, status=st, sel_stride=20)
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_CAPACITY
    assert cnt.cpu().numpy()[:, 0].tolist() == [0, 20]
    assert np.isfinite(out.cpu().numpy()).all()
