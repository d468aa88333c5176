"""GPU parity: scoring + budgeted top-k selection, bit-exact against the
oracle (which is bit-exact against the reference's select_shared_blocks,
cpp/src/selection.cpp:96-147): same ids, same fp32 score bits."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import device_kv, status_tensor, to_dev
from paged_case import D, make_case

pytestmark = pytest.mark.gpu


MODES = ("single", "split", "chunked")


def gpu_select(hip, case, select_groups, budget, init, local, sel_stride=None, split=False, mode=None):
    """mode: "single" (one workgroup per list), "split" (scores in a first
    launch) or "chunked" (lists in chunks of blocks, one launch; run twice
    on one workspace, which the first call must leave reusable)."""
    mode = mode or ("split" if split else "single")
    kv = device_kv(case)
    sel_stride = sel_stride or budget
    scores = torch.zeros((case.batch, select_groups, case.rep_stride), dtype=torch.float32, device="cuda")
    st = status_tensor()
    if mode == "split":
        sel, cnt, _ = hip.score_select_split(kv, to_dev(case.query), select_groups, budget, init, local,
                                             scores=scores, status=st, sel_stride=sel_stride)
    elif mode == "chunked":
        ws, _ = hip.score_select_chunked_workspace(kv, select_groups, budget, init, local, sel_stride)
        for _ in range(2):
            sel, cnt = hip.score_select_chunked(kv, to_dev(case.query), select_groups, budget, init, local, ws,
                                                status=st, sel_stride=sel_stride)
        scores = None
    else:
        sel, cnt = hip.score_select(kv, to_dev(case.query), select_groups, budget, init, local, scores=scores,
                                    status=st, sel_stride=sel_stride)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    return sel.cpu().numpy(), cnt.cpu().numpy(), None if scores is None else scores.cpu().numpy()


def check(hip, case, select_groups, budget, init, local, modes=MODES):
    """Every form (one workgroup per list, the split scoring, the chunked
    lists) against the oracle: same ids, and same score bits where the form
    returns scores."""
    esel, ecnt, esc = O.paged_score_select(case.query, case.reps, case.sealed, case.batch, case.hq, case.hkv, D,
                                           case.rep_heads, case.rep_stride, select_groups, budget, init, local,
                                           want_scores=True)
    for mode in modes:
        sel, cnt, sc = gpu_select(hip, case, select_groups, budget, init, local, mode=mode)
        assert np.array_equal(cnt, ecnt), mode
        for b in range(case.batch):
            n = int(case.sealed[b])
            for g in range(select_groups):
                assert sel[b, g, : cnt[b, g]].tolist() == esel[b, g, : ecnt[b, g]].tolist(), (mode, b, g)
                if sc is not None:
                    assert np.array_equal(sc[b, g, :n].view(np.uint32), esc[b, g, :n].view(np.uint32)), (mode, b, g)


@pytest.mark.parametrize("group,hkv", [(2, 8), (4, 8), (1, 8), (8, 2)])
def test_group_selection_bit_exact(hip, group, hkv):
    case = make_case(100 + group, 4, group * hkv, hkv, [32 * 512, 32 * 300 + 17, 32 * 64, 32 * 13], planted=8)
    check(hip, case, hkv, 64, 4, 8)


def test_unpadded_rep_stride_scalar_path(hip):
    """rep_stride not a multiple of 4: the one-block-per-lane scoring path;
    the chunked form (16-byte loads only) refuses the layout."""
    case = make_case(109, 3, 16, 8, [32 * 129, 32 * 77 + 3, 32 * 7], table_stride=131, rep_stride=131)
    assert case.rep_stride % 4 != 0
    check(hip, case, 8, 32, 2, 4, modes=("single", "split"))
    check(hip, case, 1, 32, 2, 4, modes=("single", "split"))
    kv = device_kv(case)
    ws, _ = hip.score_select_chunked_workspace(kv, 8, 32, 2, 4)
    with pytest.raises(RuntimeError):
        hip.score_select_chunked(kv, to_dev(case.query), 8, 32, 2, 4, ws)


def test_chunked_mixed_lengths_and_budgets(hip):
    """Lists of 1 to 3 chunks of 1024 blocks (up to 2400 blocks) in one batch with
    per-sequence budgets, one of which takes every block (no scoring) and one
    of which is out of range (flagged, nothing selected): ids and counts
    equal the oracle's per sequence, over three calls on one workspace."""
    lengths = [32 * 2400 + 5, 32 * 511, 32 * 513, 32 * 1024, 32 * 40 + 7, 32 * 1700]
    case = make_case(150, len(lengths), 16, 8, lengths, planted=8)
    kv = device_kv(case)
    budgets = np.array([64, 64, 513, 16, 16, 300], np.int32)  # 513 >= 513 blocks: every block
    bd = to_dev(budgets)
    q = to_dev(case.query)
    ws, _ = hip.score_select_chunked_workspace(kv, 8, 600, 4, 8)
    expect = [O.paged_score_select(case.query[b:b + 1], case.reps[b:b + 1], case.sealed[b:b + 1], 1, 16, 8, D, 8,
                                   case.rep_stride, 8, int(budgets[b]), 4, 8) for b in range(case.batch)]
    assert (expect[2][1] == 513).all()  # the budget takes every block
    for it in range(3):
        print(f"case: chunked mixed lengths, call {it}", flush=True)
        st = status_tensor()
        sel, cnt = hip.score_select_chunked(kv, q, 8, 600, 4, 8, ws, status=st, sel_stride=600, budgets=bd)
        torch.cuda.synchronize()
        assert int(st.item()) == 0
        c, s_ = cnt.cpu().numpy(), sel.cpu().numpy()
        for b in range(case.batch):
            esel, ecnt = expect[b]
            assert np.array_equal(c[b], ecnt[0]), (it, b)
            for g in range(8):
                assert s_[b, g, : c[b, g]].tolist() == esel[0, g, : ecnt[0, g]].tolist(), (it, b, g)
    # a budget below init + local is flagged and selects nothing for that sequence
    bad = budgets.copy()
    bad[3] = 5
    st = status_tensor()
    _, cnt = hip.score_select_chunked(kv, q, 8, 600, 4, 8, ws, status=st, sel_stride=600, budgets=to_dev(bad))
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_BAD_BUDGET
    assert (cnt.cpu().numpy()[3] == 0).all()


def test_shared_selection_per_query_head_reps(hip):
    case = make_case(110, 2, 16, 8, [32 * 200, 32 * 77 + 3], rep_heads=16)
    check(hip, case, 1, 16, 1, 2)


def test_shared_selection_kv_reps(hip):
    case = make_case(111, 2, 32, 8, [32 * 300, 32 * 1000])
    check(hip, case, 1, 64, 4, 8)


@pytest.mark.parametrize("budget,init,local", [(1, 0, 0), (1, 1, 0), (1, 0, 1), (7, 3, 4), (13, 0, 0), (64, 4, 8)])
def test_budget_shapes(hip, budget, init, local):
    case = make_case(120 + budget, 3, 16, 8, [32 * 40, 32 * 9, 32 * 5 + 1])
    check(hip, case, 8, budget, init, local)


def test_init_local_overlap_and_clamp(hip):
    """init + local overlapping on short sequences; budget >= blocks selects all."""
    case = make_case(130, 4, 16, 8, [32 * 6, 32 * 3, 32 * 1, 32 * 100])
    check(hip, case, 8, 5, 2, 3)


def test_many_ties(hip):
    """Quantized representatives make many equal scores: ties must go to the
    lower block id exactly as the reference's stable sort does."""
    case = make_case(131, 2, 16, 8, [32 * 400, 32 * 257])
    rng = np.random.default_rng(5)
    case.reps[:] = (rng.integers(-1, 2, size=case.reps.shape) * 0.5).astype(np.float32)
    case.query[:] = (rng.integers(-1, 2, size=case.query.shape) * 0.25).astype(np.float32)
    check(hip, case, 8, 40, 1, 2)
    check(hip, case, 1, 40, 1, 2)


def test_zero_scores(hip):
    case = make_case(132, 1, 16, 8, [32 * 50])
    case.reps[:] = 0.0
    check(hip, case, 8, 10, 2, 2)


def test_long_context_4096_blocks(hip):
    """Long-context shape: 4096 blocks per sequence, budget 128."""
    case = make_case(133, 2, 32, 8, [32 * 4096, 32 * 3000 + 5], planted=16)
    check(hip, case, 8, 128, 4, 8)


def test_c21_golden_on_gpu(hip):
    """C2.1: the GPU selection over the reference's InfLLM representatives
    (per query head, shared selection, budget 4 = init 1 + local 1 + 2)
    returns the published ids [0, 8, 13, 15]."""
    kv16, pq = O.fixture_c2(512, 16, 8, 128)
    reps, _ = O.local_causal_representatives(pq, kv16, 512, 16, 8, 128, 32, 32, 4)  # [16][16][128]
    case = make_case(134, 1, 16, 8, [512], rep_heads=16, table_stride=16)
    case.reps[0, :, :, :16] = reps.transpose(0, 2, 1)
    case.query[0] = pq.reshape(16, 512, 128)[:, 511, :]
    sel, cnt, _ = gpu_select(hip, case, 1, 4, 1, 1)
    assert sel[0, 0, : cnt[0, 0]].tolist() == [0, 8, 13, 15]


def test_split_capacity_flag(hip):
    """The split form flags a sequence with more sealed blocks than
    rep_stride and selects nothing for it, like score_select, while the
    other sequence is selected as the oracle does."""
    case = make_case(135, 2, 16, 8, [32 * 40 + 3, 32 * 30])
    kv = device_kv(case)
    kv.sealed.copy_(to_dev(np.array([case.rep_stride + 1, 30], np.int32)))
    kv.seq_len.copy_(to_dev(np.array([32 * (case.rep_stride + 1) + 3, 32 * 30], np.int32)))
    st = status_tensor()
    sel, cnt, _ = hip.score_select_split(kv, to_dev(case.query), 8, 20, 4, 8, status=st, sel_stride=20)
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_CAPACITY
    c = cnt.cpu().numpy()
    assert (c[0] == 0).all()
    esel, ecnt = O.paged_score_select(case.query[1:], case.reps[1:], case.sealed[1:], 1, 16, 8, D, 8,
                                      case.rep_stride, 8, 20, 4, 8)
    assert np.array_equal(c[1], ecnt[0])
    s = sel.cpu().numpy()
    for g in range(8):
        assert s[1, g, : c[1, g]].tolist() == esel[0, g, : ecnt[0, g]].tolist()


@pytest.mark.parametrize("split", [False, True, "chunked"])
def test_selection_at_the_8192_block_limit(hip, split):
    """8192 sealed blocks (256K tokens) is the selection's limit: selected
    bit-exact with the oracle; 8193 blocks are flagged (capacity) and select
    nothing, in both forms."""
    rng = np.random.default_rng(140)
    n, hq, hkv, budget = 8192, 16, 8, 128
    rep_stride = n + 4
    kv = hip.PagedKV(1, hq, hkv, rep_stride, num_pages=4, rep_stride=rep_stride)
    reps = rng.standard_normal((1, hkv, D, rep_stride)).astype(np.float32)
    kv.reps.copy_(torch.from_numpy(reps))
    kv.sealed.fill_(n)
    kv.seq_len.fill_(n * 32)
    q = rng.standard_normal((1, hq, D)).astype(np.float32)
    st = status_tensor()
    scores = torch.zeros((1, hkv, rep_stride), dtype=torch.float32, device="cuda")
    print(f"case: {n} blocks split={split}", flush=True)
    if split == "chunked":
        ws, _ = hip.score_select_chunked_workspace(kv, hkv, budget, 4, 8)
        fn = lambda *a, scores=None, **k: hip.score_select_chunked(*a, ws, **k)  # noqa: E731
    else:
        fn = hip.score_select_split if split else hip.score_select
    res = fn(kv, to_dev(q), hkv, budget, 4, 8, scores=scores, status=st)
    sel, cnt = res[0], res[1]
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    esel, ecnt, esc = O.paged_score_select(q, reps, np.array([n], np.int32), 1, hq, hkv, D, hkv, rep_stride, hkv,
                                           budget, 4, 8, want_scores=True)
    assert np.array_equal(cnt.cpu().numpy(), ecnt)
    assert np.array_equal(sel.cpu().numpy(), esel)
    if split != "chunked":
        assert np.array_equal(scores.cpu().numpy()[..., :n].view(np.uint32), esc[..., :n].view(np.uint32))
    kv.sealed.fill_(n + 1)
    kv.seq_len.fill_((n + 1) * 32)
    st.zero_()
    res = fn(kv, to_dev(q), hkv, budget, 4, 8, scores=scores, status=st)
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_CAPACITY
    assert (res[1].cpu().numpy() == 0).all()


@pytest.mark.parametrize("lengths", [[32 * 4096, 32 * 4095 + 7], [32 * 64, 32 * 65 + 1, 32 * 1],
                                     [32 * 128, 32 * 129 + 5, 32 * 256, 32 * 127]])
def test_shared_selection_long_context_rows(hip, lengths):
    """The reference's shared mode at the long-context shape (32 query heads
    over 8 representative rows, 4096 blocks, budget 128 = 4 + 8 + 116) and
    at lengths around one 64- and one 128-block chunk: the split scoring
    spreads the rows over waves; ids (every form) and score bits equal the
    oracle's."""
    case = make_case(135, len(lengths), 32, 8, lengths, planted=16)
    check(hip, case, 1, 128, 4, 8)


def test_shared_selection_chunked_at_the_8192_block_limit(hip):
    """The shared mode (32 query heads, one list per sequence) in the
    chunked form at 8192 blocks (the last chunk selects from keys in LDS,
    past the register form's 4096), and a flagged 8193: ids equal the
    oracle's, twice on one workspace."""
    rng = np.random.default_rng(141)
    n, hq, hkv, budget = 8192, 32, 8, 128
    rep_stride = n + 4
    kv = hip.PagedKV(1, hq, hkv, rep_stride, num_pages=4, rep_stride=rep_stride)
    reps = rng.standard_normal((1, hkv, D, rep_stride)).astype(np.float32)
    kv.reps.copy_(torch.from_numpy(reps))
    kv.sealed.fill_(n)
    kv.seq_len.fill_(n * 32)
    q = rng.standard_normal((1, hq, D)).astype(np.float32)
    st = status_tensor()
    ws, _ = hip.score_select_chunked_workspace(kv, 1, budget, 4, 8)
    esel, ecnt = O.paged_score_select(q, reps, np.array([n], np.int32), 1, hq, hkv, D, hkv, rep_stride, 1,
                                      budget, 4, 8)
    for call in range(2):
        print(f"case: shared rows {n} blocks, call {call}", flush=True)
        sel, cnt = hip.score_select_chunked(kv, to_dev(q), 1, budget, 4, 8, ws, status=st)
        torch.cuda.synchronize()
        assert int(st.item()) == 0
        assert np.array_equal(cnt.cpu().numpy(), ecnt)
        assert np.array_equal(sel.cpu().numpy(), esel)
    kv.sealed.fill_(n + 1)
    kv.seq_len.fill_((n + 1) * 32)
    _, cnt = hip.score_select_chunked(kv, to_dev(q), 1, budget, 4, 8, ws, status=st)
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_CAPACITY
    assert (cnt.cpu().numpy() == 0).all()


@pytest.mark.parametrize("group", [4, 8])
def test_group_selection_per_query_head_reps_rows(hip, group):
    """Per-KV-group selection over per-query-head representatives (the
    online seal's layout): each group reads `group` rows, which the split
    scoring spreads over waves."""
    case = make_case(136 + group, 3, group * 4, 4, [32 * 700 + 3, 32 * 129, 32 * 2], rep_heads=group * 4)
    check(hip, case, 4, 32, 2, 4)
