"""The oracle's batched paged functions reduce to the reference functions:
identity tables, shared/group selection, budget clamp, full budget == dense,
append/seal bytes and representatives."""
import numpy as np
import pytest

import oracle as O
from paged_case import D, PAGE, make_case


def contiguous_tokens(case, b):
    """Tokens [0, seq_len) of sequence b in the reference token format."""
    pages = [case.pool[case.table[b, i]] for i in range((case.seq_len[b] + PAGE - 1) // PAGE)]
    flat = np.concatenate([p.reshape(PAGE, -1) for p in pages])[: case.seq_len[b]]
    return flat.ravel()


def test_paged_select_shared_equals_select_shared_blocks():
    case = make_case(1, 2, 16, 8, [32 * 40, 32 * 25 + 7], rep_heads=16)
    sel, cnt, sc = O.paged_score_select(case.query, case.reps, case.sealed, 2, 16, 8, D, 16, case.rep_stride,
                                        1, 10, 1, 2, want_scores=True)
    for b in range(2):
        n = int(case.sealed[b])
        reps_hbd = np.ascontiguousarray(case.reps[b, :, :, :n].transpose(0, 2, 1))  # [H][blocks][D]
        ids, scores = O.select_shared_blocks(case.query[b], reps_hbd, 16, n, D, 10, 1, 2)
        assert sel[b, 0, : cnt[b, 0]].tolist() == ids.tolist()
        assert np.array_equal(sc[b, 0, :n].view(np.uint32), scores.view(np.uint32))


def test_paged_select_group_equals_per_group_call():
    case = make_case(2, 3, 16, 8, [32 * 30, 32 * 31, 32 * 64 + 31], planted=4)
    sel, cnt = O.paged_score_select(case.query, case.reps, case.sealed, 3, 16, 8, D, 8, case.rep_stride,
                                    8, 12, 2, 3)
    for b in range(3):
        n = int(case.sealed[b])
        for g in range(8):
            reps_g = np.repeat(case.reps[b, g:g + 1, :, :n].transpose(0, 2, 1), 2, axis=0)
            ids, _ = O.select_shared_blocks(case.query[b, 2 * g:2 * g + 2], np.ascontiguousarray(reps_g), 2, n,
                                            D, 12, 2, 3)
            assert sel[b, g, : cnt[b, g]].tolist() == ids.tolist()


def test_paged_select_clamps_when_budget_covers_all():
    case = make_case(3, 2, 8, 8, [32 * 5, 32 * 3 + 3])
    sel, cnt = O.paged_score_select(case.query, case.reps, case.sealed, 2, 8, 8, D, 8, case.rep_stride, 8, 16, 1, 1)
    assert cnt[0].tolist() == [5] * 8 and cnt[1].tolist() == [3] * 8
    assert sel[0, 0, :5].tolist() == [0, 1, 2, 3, 4]


def test_full_budget_sparse_equals_dense():
    """Selecting every sealed block makes the sparse path the dense one."""
    case = make_case(4, 2, 16, 8, [32 * 9 + 5, 32 * 4])
    sel, cnt = O.paged_score_select(case.query, case.reps, case.sealed, 2, 16, 8, D, 8, case.rep_stride,
                                    8, 64, 1, 1, sel_stride=64)
    out = O.paged_sparse_attention(case.pool, PAGE, case.table, case.seq_len, case.sealed, sel, cnt, 8,
                                   case.query, 2, 16, 8, D, 0.0883883)
    for b in range(2):
        dense = O.attention_reference(contiguous_tokens(case, b), case.query[b], int(case.seq_len[b]), 16, 8, D,
                                      0.0883883)
        assert np.array_equal(out[b].view(np.uint32), dense.view(np.uint32))


def test_append_then_seal_bytes_and_reps():
    rng = np.random.default_rng(5)
    case = make_case(6, 2, 16, 8, [32 * 3 - 1, 32 * 2 + 10], table_stride=8)
    k = rng.standard_normal((2, 8, D)).astype(np.float32)
    v = rng.standard_normal((2, 8, D)).astype(np.float32)
    before = case.seq_len.copy()
    O.paged_append(case.pool, PAGE, case.table, case.seq_len, k=k, v=v, batch=2, hkv=8, d=D)
    assert (case.seq_len == before + 1).all()
    for b in range(2):
        t = int(before[b])
        tok = case.pool[case.table[b, t // PAGE], t % PAGE]
        assert np.array_equal(tok[0], k[b].astype(np.float16).view(np.uint16))
        assert np.array_equal(tok[1], v[b].astype(np.float16).view(np.uint16))
    O.paged_seal(case.pool, PAGE, case.table, case.seq_len, case.sealed, case.generation, case.reps, 8,
                 case.rep_stride, 2, 16, 8, D, 0)
    assert case.sealed.tolist() == [3, 2] and case.generation.tolist() == [3, 2]
    # the representative of the block completed by the append is its mean key
    blk = case.pool[case.table[0, 2]].reshape(PAGE, -1)
    mean = O.mean_key_representatives(blk.ravel(), PAGE, 8, D, PAGE)  # [8][1][D]
    assert np.array_equal(case.reps[0, :, :, 2].view(np.uint32), mean[:, 0, :].view(np.uint32))


def test_seal_keeps_local_window():
    case = make_case(7, 1, 16, 8, [32 * 5 + 3], local_tokens=32)
    # tail must stay within [local, local + 32)
    tail = int(case.seq_len[0]) - int(case.sealed[0]) * PAGE
    assert 32 <= tail < 64
    assert int(case.sealed[0]) == 4


def test_pack_blocks_is_a_page_copy():
    case = make_case(8, 1, 16, 8, [32 * 6])
    pages = case.table[0, [0, 3, 5]].astype(np.int32)
    out = np.zeros(3 * case.page_elems, np.uint16)
    O.lib().sao_pack_blocks(case.pool.ctypes.data, case.page_elems, pages.ctypes.data, 3, out.ctypes.data)
    assert np.array_equal(out.reshape(3, -1), case.pool.reshape(case.num_pages, -1)[pages])
