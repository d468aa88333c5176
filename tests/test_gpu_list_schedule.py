"""GPU: the longest-list-first schedules of the chunked selection and the
chunked attention (csrc/schedule.hpp).  Beyond 4096 (sequence, KV head)
lists neither schedule runs and the launches keep the grid order: the
selection must still equal the single-launch selection and the oracle
(select_shared_blocks, cpp/src/selection.cpp:96-147) bit for bit, and the
attention stay within 2e-3 of the oracle (attention_reference.cpp:55-96).
The scheduled attention replayed from a HIP graph (the schedule rewritten on
every replay) equals its eager launch bit for bit."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import assert_close_2e3, device_kv, status_tensor, to_dev
from paged_case import D, PAGE, make_case

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128)))


def test_many_lists_keep_grid_order(hip):
    batch, hq, hkv = 520, 8, 8  # 4160 lists: more than the schedules take
    rng = np.random.default_rng(811)
    lengths = rng.integers(33, 170, size=batch)
    case = make_case(812, batch, hq, hkv, lengths.tolist(), spare_pages=8)
    kind = rng.integers(0, 3, size=batch)
    budgets = np.where(kind == 0, 2, np.where(kind == 1, 3, np.maximum(case.sealed, 2))).astype(np.int32)
    init, local, budget = 1, 1, 3
    sel_stride = int(case.sealed.max())
    print(f"case: {batch * hkv} lists, sealed {int(case.sealed.min())}..{sel_stride}", flush=True)
    kv = device_kv(case)
    st = status_tensor()
    q = to_dev(case.query)
    b_dev = to_dev(budgets)
    ws, _ = hip.score_select_chunked_workspace(kv, hkv, budget, init, local, sel_stride=sel_stride)
    sel_c, cnt_c = hip.score_select_chunked(kv, q, hkv, budget, init, local, ws, status=st, sel_stride=sel_stride,
                                            budgets=b_dev)
    sel_s, cnt_s = hip.score_select(kv, q, hkv, budget, init, local, status=st, sel_stride=sel_stride,
                                    budgets=b_dev)
    out = hip.sparse_decode_attention_chunked(kv, q, sel_c, cnt_c, SCALE, 2, sel_stride // 2 + 2, status=st)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    got_sel, got_cnt = sel_c.cpu().numpy(), cnt_c.cpu().numpy()
    assert np.array_equal(got_cnt, cnt_s.cpu().numpy())
    assert np.array_equal(got_sel, sel_s.cpu().numpy())
    esel = np.full((batch, hkv, sel_stride), -1, np.int32)
    ecnt = np.zeros((batch, hkv), np.int32)
    for b in range(batch):
        s_, c_ = O.paged_score_select(case.query[b:b + 1], case.reps[b:b + 1], case.sealed[b:b + 1], 1, hq, hkv, D,
                                      case.rep_heads, case.rep_stride, hkv, int(budgets[b]), init, local,
                                      sel_stride=sel_stride)
        esel[b], ecnt[b] = s_[0], c_[0]
        for g in range(hkv):
            assert got_sel[b, g, :got_cnt[b, g]].tolist() == esel[b, g, :ecnt[b, g]].tolist(), (b, g)
    assert np.array_equal(got_cnt, ecnt)
    expect = O.paged_sparse_attention(case.pool, PAGE, case.table, case.seq_len, case.sealed, esel, ecnt, hkv,
                                      case.query, batch, hq, hkv, D, SCALE)
    assert_close_2e3(out.cpu().numpy(), expect)


def test_scheduled_chunked_attention_graph_replays(hip):
    lengths = [32 * 150 + 7, 20, 32 * 40 + 1, 32 * 99, 31, 32 * 7 + 3]
    case = make_case(813, len(lengths), 16, 8, lengths, planted=2)
    sel, cnt = O.paged_score_select(case.query, case.reps, case.sealed, case.batch, 16, 8, D, case.rep_heads,
                                    case.rep_stride, 8, 120, 1, 2)
    kv = device_kv(case)
    q, sel_d, cnt_d = to_dev(case.query), to_dev(sel), to_dev(cnt)
    chunk, max_chunks = 8, 20
    ws = torch.zeros(hip.lib().sa_hip_attention_chunked_workspace_bytes(kv.batch, 16, 8, 128, max_chunks) // 4,
                     dtype=torch.float32, device="cuda")
    out = torch.empty((kv.batch, 16, 128), dtype=torch.float32, device="cuda")
    st = status_tensor()
    hip.sparse_decode_attention_chunked(kv, q, sel_d, cnt_d, SCALE, chunk, max_chunks, out=out, workspace=ws,
                                        status=st)
    torch.cuda.synchronize()
    eager = out.cpu().numpy().copy()
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            hip.sparse_decode_attention_chunked(kv, q, sel_d, cnt_d, SCALE, chunk, max_chunks, out=out, workspace=ws,
                                                status=st, stream=stream)
    for rep in range(3):
        out.zero_()
        ws.fill_(7.0)  # the schedule and the records must be rewritten by each replay
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert int(st.item()) == 0, rep
        assert np.array_equal(out.cpu().numpy().view(np.uint32), eager.view(np.uint32)), rep
