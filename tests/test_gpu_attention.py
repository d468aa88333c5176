"""GPU parity: sparse GQA decode attention (libsa_hip.so) against the oracle.

Bar: within 2e-3 absolute or relative of the oracle's fp32 two-pass
attention (attention_reference, reference cpp/src/attention_reference.cpp
:55-96) on the same tokens.  Selection ids come from the oracle here so the
attention kernel is checked on its own."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import assert_close_2e3, device_kv, status_tensor, to_dev
from paged_case import D, PAGE, make_case

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128)))


def run_case(hip, case, select_groups, budget, init, local, splits=None, chunk=None):
    sel, cnt = O.paged_score_select(case.query, case.reps, case.sealed, case.batch, case.hq, case.hkv, D,
                                    case.rep_heads, case.rep_stride, select_groups, budget, init, local)
    expect = O.paged_sparse_attention(case.pool, PAGE, case.table, case.seq_len, case.sealed, sel, cnt,
                                      select_groups, case.query, case.batch, case.hq, case.hkv, D, SCALE)
    kv = device_kv(case)
    st = status_tensor()
    if chunk:
        out = hip.sparse_decode_attention_chunked(kv, to_dev(case.query), to_dev(sel), to_dev(cnt), SCALE,
                                                  chunk[0], chunk[1], status=st)
    else:
        out = hip.sparse_decode_attention(kv, to_dev(case.query), to_dev(sel), to_dev(cnt), SCALE, splits=splits,
                                          status=st)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    return out.cpu().numpy(), expect


@pytest.mark.parametrize("group,hkv", [(2, 8), (4, 8), (1, 4), (8, 2)])
def test_paged_group_shapes(hip, group, hkv):
    print(f"case: group={group} hkv={hkv}", flush=True)
    case = make_case(10 + group, 3, group * hkv, hkv, [32 * 40 + 5, 32 * 17, 32 * 64 + 31], planted=3)
    got, expect = run_case(hip, case, hkv, 12, 1, 2)
    assert_close_2e3(got, expect)


@pytest.mark.parametrize("hq", [16, 32, 64])
@pytest.mark.parametrize("splits", [1, 2, 3, 8, 33])
def test_split_counts(hip, splits, hq):
    """Query heads per KV head 2 (register pages), 4 and 8 (LDS-staged
    pages, q.K on the matrix cores) under every split count."""
    print(f"case: splits={splits} hq={hq}", flush=True)
    case = make_case(20, 2, hq, 8, [32 * 70 + 9, 32 * 33 + 1])
    got, expect = run_case(hip, case, 8, 20, 2, 4, splits=splits)
    assert_close_2e3(got, expect)


@pytest.mark.parametrize("hq", [16, 32, 64])
@pytest.mark.parametrize("chunk,max_chunks", [(1, 200), (4, 3), (5, 9), (16, 8), (64, 2)])
def test_chunked_pages(hip, chunk, max_chunks, hq):
    """Lists of 41, 4, 34 and 1 pages cut into chunks: one page per chunk,
    a last chunk taking the remainder beyond max_chunks * chunk, chunks
    past the end of short lists, and a chunk longer than every list."""
    print(f"case: chunk={chunk} max_chunks={max_chunks} hq={hq}", flush=True)
    case = make_case(24, 4, hq, 8, [32 * 70 + 9, 32 * 3 + 5, 32 * 33 + 1, 31], planted=2)
    got, expect = run_case(hip, case, 8, 40, 1, 2, chunk=(chunk, max_chunks))
    assert_close_2e3(got, expect)


@pytest.mark.parametrize("hq,chunk,max_chunks", [(16, 4, 12), (32, 8, 7), (64, 3, 40), (16, 1, 200)])
def test_chunked_longest_first_equals_grid_order(hip, hq, chunk, max_chunks):
    """The longest-first schedule (a workspace of
    sa_hip_attention_chunked_workspace_bytes) attends the same chunks and
    merges them in the same order as the grid order (a workspace of
    sa_hip_attention_workspace_bytes): equal bit for bit, over lists of very
    different lengths, empty lists and lists longer than max_chunks chunks."""
    print(f"case: chunk schedule hq={hq} chunk={chunk} max_chunks={max_chunks}", flush=True)
    lengths = [32 * 200 + 9, 20, 32 * 3 + 5, 32 * 77 + 1, 31, 32 * 150, 32 * 12 + 17]
    case = make_case(26 + hq, len(lengths), hq, 8, lengths, planted=2)
    sel, cnt = O.paged_score_select(case.query, case.reps, case.sealed, case.batch, hq, 8, D, case.rep_heads,
                                    case.rep_stride, 8, 180, 1, 2)
    expect = O.paged_sparse_attention(case.pool, PAGE, case.table, case.seq_len, case.sealed, sel, cnt, 8,
                                      case.query, case.batch, hq, 8, D, SCALE)
    kv = device_kv(case)
    L = hip.lib()
    small = L.sa_hip_attention_workspace_bytes(kv.batch, hq, 8, 128, max_chunks)
    big = L.sa_hip_attention_chunked_workspace_bytes(kv.batch, hq, 8, 128, max_chunks)
    assert big > small
    outs = []
    for nbytes in (small, big, big):
        ws = torch.zeros(nbytes // 4, dtype=torch.float32, device="cuda")
        st = status_tensor()
        out = hip.sparse_decode_attention_chunked(kv, to_dev(case.query), to_dev(sel), to_dev(cnt), SCALE, chunk,
                                                  max_chunks, workspace=ws, status=st)
        torch.cuda.synchronize()
        assert int(st.item()) == 0
        outs.append(out.cpu().numpy())
    assert_close_2e3(outs[0], expect)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.array_equal(outs[1].view(np.uint32), outs[2].view(np.uint32))  # the schedule rebuilt each call


def test_chunked_equals_split_within_rounding(hip):
    """The chunked and the split schedules sum the same terms in another
    order: equal within fp32 rounding."""
    case = make_case(25, 3, 32, 8, [32 * 90 + 7, 32 * 12, 32 * 40 + 31])
    a, expect = run_case(hip, case, 8, 48, 2, 3, splits=3)
    b, _ = run_case(hip, case, 8, 48, 2, 3, chunk=(8, 7))
    assert_close_2e3(b, expect)
    np.testing.assert_allclose(b, a, rtol=1e-5, atol=1e-6)


def test_workspace_reuse_across_launches(hip):
    """Repeated launches on one workspace, with different inputs, all match
    the oracle."""
    case = make_case(21, 3, 16, 8, [32 * 30 + 3, 32 * 45, 32 * 9 + 30])
    sel, cnt = O.paged_score_select(case.query, case.reps, case.sealed, 3, 16, 8, D, 8, case.rep_stride, 8, 10,
                                    1, 2)
    kv = device_kv(case)
    splits = 4
    ws, nbytes = hip.attention_workspace(kv, splits)
    rng = np.random.default_rng(0)
    for rep in range(5):
        q = rng.standard_normal(case.query.shape).astype(np.float32)
        expect = O.paged_sparse_attention(case.pool, PAGE, case.table, case.seq_len, case.sealed, sel, cnt, 8, q,
                                          3, 16, 8, D, SCALE)
        out = hip.sparse_decode_attention(kv, to_dev(q), to_dev(sel), to_dev(cnt), SCALE, splits=splits,
                                          workspace=ws)
        torch.cuda.synchronize()
        assert_close_2e3(out.cpu().numpy(), expect)


@pytest.mark.parametrize("tail", [0, 1, 15, 31])
def test_tail_lengths(hip, tail):
    print(f"case: tail={tail}", flush=True)
    case = make_case(30 + tail, 2, 16, 8, [32 * 12 + tail, 32 * 3 + tail])
    got, expect = run_case(hip, case, 8, 6, 1, 1)
    assert_close_2e3(got, expect)


def test_local_window_tail_up_to_63(hip):
    """Seal with local_tokens=32 keeps 32..63 tail tokens (two tail pages)."""
    case = make_case(40, 3, 16, 8, [32 * 9 + 31, 32 * 9 + 2, 32 * 2], local_tokens=32)
    got, expect = run_case(hip, case, 8, 4, 1, 1)
    assert_close_2e3(got, expect)


def test_shared_selection_mode(hip):
    case = make_case(41, 2, 16, 8, [32 * 30, 32 * 18 + 3], rep_heads=16)
    got, expect = run_case(hip, case, 1, 5, 1, 1)
    assert_close_2e3(got, expect)


def test_tail_only_and_empty(hip):
    """A sequence with no sealed block attends its tail only; an empty
    sequence yields zeros."""
    case = make_case(42, 2, 16, 8, [20, 0])
    got, expect = run_case(hip, case, 8, 4, 0, 0)
    assert_close_2e3(got, expect)
    assert np.all(got[1] == 0)


def test_full_budget_equals_dense(hip):
    case = make_case(43, 2, 16, 8, [32 * 20 + 7, 32 * 11])
    got, expect = run_case(hip, case, 8, 64, 1, 1)
    for b in range(2):
        n = int(case.seq_len[b])
        pages = [case.pool[case.table[b, i]].reshape(PAGE, -1) for i in range((n + PAGE - 1) // PAGE)]
        dense = O.attention_reference(np.concatenate(pages)[:n].ravel(), case.query[b], n, 16, 8, D, SCALE)
        assert_close_2e3(got[b], dense)


def test_stress_outliers(hip):
    """1% of tokens at +-60000 exercise the stable softmax."""
    case = make_case(44, 2, 16, 8, [32 * 50 + 3, 32 * 40 + 31], outliers=0.01)
    got, expect = run_case(hip, case, 8, 16, 1, 2)
    assert np.isfinite(got).all()
    assert_close_2e3(got, expect)


def test_key_channel_outliers(hip):
    """Qwen3-8B-like post-RoPE key outliers: 4 of 128 channels x8."""
    case = make_case(45, 2, 32, 8, [32 * 64 + 5, 32 * 70], channel_scale=(4, 8.0))
    got, expect = run_case(hip, case, 8, 16, 2, 3)
    assert_close_2e3(got, expect)


def test_contiguous_c1_fixture(hip):
    """C1 fixture (reference attention_main.cpp:131-156): 128 tokens, 16/8/128."""
    kv, q = O.fixture_c1(128, 16, 8, 128)
    scale = 0.08838834764831845
    expect = O.attention_reference(kv, q, 128, 16, 8, 128, scale)
    out = hip.attention_contiguous(to_dev(kv.view(np.int16)).view(torch.uint16), to_dev(q), 128, 16, 8, scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_close_2e3(got, expect)
    # the reference's own C1 acceptance bar (attention_main.cpp:265-270)
    assert np.abs(got - expect).max() <= 2e-5
    cos = float((got.ravel().astype(np.float64) @ expect.ravel()) /
                np.sqrt((got.ravel().astype(np.float64) ** 2).sum() * (expect.ravel().astype(np.float64) ** 2).sum()))
    assert cos >= 0.999999


@pytest.mark.parametrize("tokens", [1, 31, 33, 257, 1000, 4096])
def test_contiguous_lengths(hip, tokens):
    rng = np.random.default_rng(tokens)
    kv = rng.standard_normal(tokens * 2 * 8 * 128).astype(np.float16).view(np.uint16)
    q = rng.standard_normal(16 * 128).astype(np.float32)
    expect = O.attention_reference(kv, q, tokens, 16, 8, 128, SCALE)
    out = hip.attention_contiguous(to_dev(kv.view(np.int16)).view(torch.uint16), to_dev(q), tokens, 16, 8, SCALE)
    torch.cuda.synchronize()
    assert_close_2e3(out.cpu().numpy(), expect)


@pytest.mark.parametrize("hq,hkv", [(32, 8), (64, 8), (16, 2)])
@pytest.mark.parametrize("tokens", [1, 33, 1000, 4096])
def test_contiguous_group_sizes(hip, tokens, hq, hkv):
    """Contiguous buffers at 4 and 8 query heads per KV head: full pages
    staged through LDS, a partial last page spread over the waves."""
    print(f"case: tokens={tokens} hq={hq} hkv={hkv}", flush=True)
    rng = np.random.default_rng(tokens + hq)
    kv = rng.standard_normal(tokens * 2 * hkv * 128).astype(np.float16).view(np.uint16)
    q = rng.standard_normal(hq * 128).astype(np.float32)
    expect = O.attention_reference(kv, q, tokens, hq, hkv, 128, SCALE)
    out = hip.attention_contiguous(to_dev(kv.view(np.int16)).view(torch.uint16), to_dev(q), tokens, hq, hkv, SCALE)
    torch.cuda.synchronize()
    assert_close_2e3(out.cpu().numpy(), expect)


def test_bad_page_is_flagged_not_read(hip):
    case = make_case(46, 1, 16, 8, [32 * 8])
    sel = np.zeros((1, 8, 4), np.int32)
    sel[0, :, :] = [0, 1, 2, 3]
    cnt = np.full((1, 8), 4, np.int32)
    kv = device_kv(case)
    kv.block_table[0, 2] = case.num_pages + 1000  # out of range: must be skipped
    st = status_tensor()
    hip.sparse_decode_attention(kv, to_dev(case.query), to_dev(sel), to_dev(cnt), SCALE, status=st)
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_BAD_PAGE


@pytest.mark.parametrize("hq", [16, 32, 64])
def test_split_phase_partial_and_merge(hip, hq):
    """Hits-first schedule: attend one part of the selection (with the tail),
    then the rest, then merge; equals attention over the whole selection."""
    print(f"case: hq={hq}", flush=True)
    case = make_case(47, 3, hq, 8, [32 * 60 + 7, 32 * 41, 32 * 80 + 31])
    sel, cnt = O.paged_score_select(case.query, case.reps, case.sealed, 3, hq, 8, D, 8, case.rep_stride, 8, 24, 2,
                                    3)
    expect = O.paged_sparse_attention(case.pool, PAGE, case.table, case.seq_len, case.sealed, sel, cnt, 8,
                                      case.query, 3, hq, 8, D, SCALE)
    # split every (seq, group) list into its even and odd positions
    first = np.full_like(sel, -1)
    second = np.full_like(sel, -1)
    c1 = np.zeros_like(cnt)
    c2 = np.zeros_like(cnt)
    for b in range(3):
        for g in range(8):
            ids = sel[b, g, : cnt[b, g]]
            a, z = ids[0::2], ids[1::2]
            first[b, g, : len(a)] = a
            second[b, g, : len(z)] = z
            c1[b, g], c2[b, g] = len(a), len(z)
    kv = device_kv(case)
    total = 3
    ws, _ = hip.attention_workspace(kv, total)
    q = to_dev(case.query)
    st = status_tensor()
    hip.sparse_decode_attention_partial(kv, q, to_dev(first), to_dev(c1), SCALE, True, ws, 0, 2, total, status=st)
    hip.sparse_decode_attention_partial(kv, q, to_dev(second), to_dev(c2), SCALE, False, ws, 2, 1, total, status=st)
    out = torch.empty((3, hq, D), dtype=torch.float32, device="cuda")
    hip.attention_merge(kv, ws, total, out)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    assert_close_2e3(out.cpu().numpy(), expect)
