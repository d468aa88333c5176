"""GPU parity on the stress shape (reduced batch so the oracle finishes in
seconds): mixed context lengths rounded to 32, pages drawn at random from
one shared fragmented pool, per-sequence budgets in {16, 64, all blocks},
1% of tokens at +-60000; selection bit-exact per sequence, attention within
2e-3, and full-budget sequences equal dense attention."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import assert_close_2e3, device_kv, status_tensor, to_dev
from paged_case import D, PAGE, make_case

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128)))
INIT, LOCAL = 4, 8


@pytest.mark.parametrize("seed", [0, 1])
def test_stress_mixed_lengths_budgets_outliers(hip, seed):
    rng = np.random.default_rng(500 + seed)
    batch = 12
    lengths = (rng.integers(1024, 12288, size=batch) // 32 * 32).astype(np.int64)
    case = make_case(600 + seed, batch, 16, 8, lengths.tolist(), outliers=0.01, spare_pages=64)
    n_blocks = case.sealed.astype(np.int64)
    choice = rng.integers(0, 3, size=batch)
    budgets = np.where(choice == 0, 16, np.where(choice == 1, 64, n_blocks)).astype(np.int32)
    budgets[0] = n_blocks[0]  # at least one full-context sequence
    sel_stride = int(n_blocks.max())
    print(f"case: seed={seed} lengths={lengths.tolist()} budgets={budgets.tolist()}", flush=True)

    kv = device_kv(case)
    st = status_tensor()
    q = to_dev(case.query)
    sel, cnt = hip.score_select(kv, q, 8, 64, INIT, LOCAL, status=st, sel_stride=sel_stride,
                                budgets=to_dev(budgets))
    sel2, cnt2, _ = hip.score_select_split(kv, q, 8, 64, INIT, LOCAL, status=st, sel_stride=sel_stride,
                                           budgets=to_dev(budgets))
    out = hip.sparse_decode_attention(kv, q, sel, cnt, SCALE, status=st)
    # the schedule for uneven lists: 16-page chunks, enough for the longest
    chunk = 16
    out_c = hip.sparse_decode_attention_chunked(kv, q, sel, cnt, SCALE, chunk, (sel_stride + 1) // chunk + 1,
                                                status=st)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    got_sel, got_cnt, got = sel.cpu().numpy(), cnt.cpu().numpy(), out.cpu().numpy()
    assert np.array_equal(cnt2.cpu().numpy(), got_cnt) and np.array_equal(sel2.cpu().numpy(), got_sel)
    got_c = out_c.cpu().numpy()

    esel = np.full((batch, 8, sel_stride), -1, np.int32)
    ecnt = np.zeros((batch, 8), np.int32)
    for b in range(batch):
        s_, c_ = O.paged_score_select(case.query[b:b + 1], case.reps[b:b + 1], case.sealed[b:b + 1], 1, 16, 8, D, 8,
                                      case.rep_stride, 8, int(budgets[b]), INIT, LOCAL, sel_stride=sel_stride)
        esel[b], ecnt[b] = s_[0], c_[0]
        for g in range(8):
            assert got_sel[b, g, : got_cnt[b, g]].tolist() == esel[b, g, : ecnt[b, g]].tolist(), (b, g)
    assert np.array_equal(got_cnt, ecnt)
    expect = O.paged_sparse_attention(case.pool, PAGE, case.table, case.seq_len, case.sealed, esel, ecnt, 8,
                                      case.query, batch, 16, 8, D, SCALE)
    assert np.isfinite(got).all() and np.isfinite(got_c).all()
    assert_close_2e3(got, expect)
    assert_close_2e3(got_c, expect)
    for b in np.nonzero(budgets == n_blocks)[0]:
        n = int(case.seq_len[b])
        pages = [case.pool[case.table[b, i]].reshape(PAGE, -1) for i in range(n // PAGE)]
        dense = O.attention_reference(np.concatenate(pages).ravel(), case.query[b], n, 16, 8, D, SCALE)
        assert_close_2e3(got[b], dense)
        assert_close_2e3(got_c[b], dense)


def test_bad_per_sequence_budget_is_flagged(hip):
    case = make_case(650, 2, 16, 8, [32 * 40, 32 * 30])
    kv = device_kv(case)
    st = status_tensor()
    budgets = np.array([20, 10], np.int32)  # 10 < init + local
    sel, cnt = hip.score_select(kv, to_dev(case.query), 8, 20, INIT, LOCAL, status=st, sel_stride=20,
                                budgets=to_dev(budgets))
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_BAD_BUDGET
    c = cnt.cpu().numpy()
    assert (c[1] == 0).all() and (c[0] == 20).all()
    st2 = status_tensor()
    _, cnt2, _ = hip.score_select_split(kv, to_dev(case.query), 8, 20, INIT, LOCAL, status=st2, sel_stride=20,
                                        budgets=to_dev(budgets))
    torch.cuda.synchronize()
    assert int(st2.item()) & hip.STATUS_BAD_BUDGET
    assert np.array_equal(cnt2.cpu().numpy(), c)


def test_stress_full_size_one_layer(hip, capsys):
    """The stress workload at its full size (batch 128, contexts 1K-64K, one
    layer, ~17 GiB of pages): append + seal, per-sequence budgets and chunked
    attention; the longest and shortest sequence and one of each budget
    class bit-exact in selection and within 2e-3 of the oracle, full-budget
    ones within 2e-3 of dense attention."""
    import argparse
    import json

    import bench_stress
    args = argparse.Namespace(layers=1, steps=1, warmup=1, seed=77, chunk=128, splits=0, check_seqs=1,
                              no_cpu_baseline=True)
    print("case: stress full size, 1 layer, chunk 128", flush=True)
    bench_stress.run(args)
    line = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    par = line["parity"]
    print(par, flush=True)
    assert par["selection_bit_exact"] and par["attention_within_2e-3"]
    assert par["full_budget_sequences"] >= 1 and par["full_budget_equals_dense_within_2e-3"]
