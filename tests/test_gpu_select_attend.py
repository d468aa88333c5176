"""GPU parity: the fused score + select + attend launch (sa_hip_select_attend).

Its selection must be bit-exact with the oracle (which is bit-exact with the
reference's select_shared_blocks, cpp/src/selection.cpp:96-147, per KV
group) and its attention within 2e-3 of the oracle's fp32 attention
(attention_reference, cpp/src/attention_reference.cpp:55-96).  The fused
kernel runs the same attention code as the separate attention kernel, with
the pages visited in another order, so their outputs agree to fp32 rounding.

decode_step adds the append + seal (kv_lifecycle_main.cpp:31-45, 92-113;
append_fp16_kv, qwen_layer_main.cpp:270-281) to the same launch: page bytes,
representatives and counters must be bit-exact with the oracle after every
step."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import assert_close_2e3, device_kv, status_tensor, to_dev
from paged_case import D, PAGE, make_case

pytestmark = pytest.mark.gpu

SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128)))


def oracle_step(case, budget, init, local, sel_stride, budgets=None):
    esel = np.full((case.batch, case.hkv, sel_stride), -1, np.int32)
    ecnt = np.zeros((case.batch, case.hkv), np.int32)
    for b in range(case.batch):
        bud = budget if budgets is None else int(budgets[b])
        s_, c_ = O.paged_score_select(case.query[b:b + 1], case.reps[b:b + 1], case.sealed[b:b + 1], 1, case.hq,
                                      case.hkv, D, case.rep_heads, case.rep_stride, case.hkv, bud, init, local,
                                      sel_stride=sel_stride)
        esel[b], ecnt[b] = s_[0], c_[0]
    expect = O.paged_sparse_attention(case.pool, PAGE, case.table, case.seq_len, case.sealed, esel, ecnt, case.hkv,
                                      case.query, case.batch, case.hq, case.hkv, D, SCALE)
    return esel, ecnt, expect


def run_fused(hip, case, budget, init, local, sel_stride=None, budgets=None, splits=1):
    sel_stride = sel_stride or budget
    kv = device_kv(case)
    st = status_tensor()
    q = to_dev(case.query)
    bud = None if budgets is None else to_dev(budgets)
    sel, cnt, out = hip.select_attend(kv, q, case.hkv, budget, init, local, SCALE, status=st, sel_stride=sel_stride,
                                      budgets=bud, splits=splits)
    # the same step as two separate launches
    sel2, cnt2 = hip.score_select(kv, q, case.hkv, budget, init, local, status=st, sel_stride=sel_stride,
                                  budgets=bud)
    out2 = hip.sparse_decode_attention(kv, q, sel2, cnt2, SCALE, splits=splits, status=st)
    torch.cuda.synchronize()
    return (sel.cpu().numpy(), cnt.cpu().numpy(), out.cpu().numpy(), sel2.cpu().numpy(), cnt2.cpu().numpy(),
            out2.cpu().numpy(), int(st.item()), hip.select_attend_fused(kv, case.hkv, splits))


def check(hip, case, budget, init, local, sel_stride=None, budgets=None, splits=1, expect_fused=True):
    sel_stride = sel_stride or budget
    sel, cnt, out, sel2, cnt2, out2, status, fused = run_fused(hip, case, budget, init, local, sel_stride, budgets,
                                                               splits)
    assert status == 0
    assert fused == expect_fused
    esel, ecnt, expect = oracle_step(case, budget, init, local, sel_stride, budgets)
    assert np.array_equal(cnt, ecnt)
    assert np.array_equal(cnt2, ecnt)
    for b in range(case.batch):
        for g in range(case.hkv):
            c = int(ecnt[b, g])
            assert sel[b, g, :c].tolist() == esel[b, g, :c].tolist(), (b, g)
            assert sel2[b, g, :c].tolist() == esel[b, g, :c].tolist(), (b, g)
    assert np.isfinite(out).all()
    assert_close_2e3(out, expect)
    close_fp32(out, out2)


def close_fp32(a, b):
    """Same attention computed with another page order: fp32 rounding only."""
    err = np.abs(a.astype(np.float64) - b)
    assert (err <= 1e-5 + 1e-5 * np.abs(b)).all(), f"max diff {err.max():.3e}"


@pytest.mark.parametrize("group,hkv,rep_heads", [(2, 8, None), (2, 8, 16), (1, 8, None), (2, 4, None), (4, 8, None),
                                                 (4, 8, 32), (4, 4, None)])
def test_fused_shapes(hip, group, hkv, rep_heads):
    print(f"case: group={group} hkv={hkv} rep_heads={rep_heads}", flush=True)
    case = make_case(700 + group + hkv, 4, group * hkv, hkv, [32 * 512 + 7, 32 * 300 + 17, 32 * 64, 32 * 13 + 31],
                     planted=8, rep_heads=rep_heads)
    check(hip, case, 64, 4, 8)


@pytest.mark.parametrize("hq", [32, 64])
def test_fused_at_four_fallback_at_eight_heads_per_kv_head(hip, hq):
    """G=4 (Qwen3-8B shape) runs fused (LDS-staged pages, q.K on the matrix
    cores); G=8 runs as the two launches; results are the same."""
    case = make_case(710 + hq, 3, hq, 8, [32 * 200 + 3, 32 * 90, 32 * 20 + 1], planted=8)
    check(hip, case, 32, 2, 4, expect_fused=hq == 32)


def test_four_heads_odd_rep_stride_runs_separately(hip):
    """The fused kernel at G=4 reads two representatives per 8-byte load: an
    odd rep_stride takes the two launches, with the same results."""
    case = make_case(709, 2, 32, 8, [32 * 60 + 5, 32 * 33], rep_stride=67, planted=4)
    check(hip, case, 24, 2, 4, expect_fused=False)


def test_fused_split_request_runs_separately(hip):
    case = make_case(711, 2, 16, 8, [32 * 150 + 5, 32 * 40])
    check(hip, case, 24, 2, 4, splits=3, expect_fused=False)


@pytest.mark.parametrize("hq", [16, 32])
@pytest.mark.parametrize("lengths", [[5, 31, 32, 33], [32 * 3, 32 * 11 + 2, 32 * 12, 32 * 17 + 31]])
def test_short_sequences_overlap_and_clamp(hip, lengths, hq):
    """No sealed block, init/local overlap, budget >= blocks."""
    print(f"case: lengths={lengths} hq={hq}", flush=True)
    case = make_case(712, len(lengths), hq, 8, lengths)
    check(hip, case, 12, 4, 8)


@pytest.mark.parametrize("hq", [16, 32])
def test_many_blocks_and_ties(hip, hq):
    """4096 blocks per sequence (several compaction chunks) and quantised
    representatives with many equal scores."""
    case = make_case(713, 2, hq, 8, [32 * 4096, 32 * 1537 + 9])
    rng = np.random.default_rng(9)
    case.reps[:] = (rng.integers(-1, 2, size=case.reps.shape) * 0.5).astype(np.float32)
    case.query[:] = (rng.integers(-1, 2, size=case.query.shape) * 0.25).astype(np.float32)
    check(hip, case, 128, 4, 8)


def test_four_heads_keys_past_first_slot(hip):
    """4 query heads per KV head with 5000 sealed blocks: the keys (20 KB)
    reach into the second page slot, so that slot's wave stays out of the
    forced-block walk during the selection."""
    case = make_case(717, 2, 8, 2, [32 * 5000 + 7, 32 * 4096 + 31], planted=4)
    check(hip, case, 64, 4, 8)


@pytest.mark.parametrize("hq", [16, 32])
@pytest.mark.parametrize("lengths", [[32 * 256 + 5, 32 * 257, 32 * 512, 32 * 513 + 1],
                                     [32 * 768 + 31, 32 * 1024 + 1, 32 * 1025]])
def test_list_length_boundaries_with_ties(hip, lengths, hq):
    """Lists of 256, 257, 512, 513, 768, 1024 and 1025 blocks (the edges of
    the one-wave selection's 4/8/12/16 keys per lane and its LDS fallback)
    with quantised scores: many equal keys at the threshold, many zeros."""
    print(f"case: lengths={lengths} hq={hq}", flush=True)
    case = make_case(714, len(lengths), hq, 8, lengths)
    rng = np.random.default_rng(14)
    case.reps[:] = (rng.integers(-1, 2, size=case.reps.shape) * 0.5).astype(np.float32)
    case.query[:] = (rng.integers(-1, 2, size=case.query.shape) * 0.25).astype(np.float32)
    check(hip, case, 64, 4, 8)


@pytest.mark.parametrize("hq", [16, 32])
def test_stress_budgets_outliers(hip, hq):
    """Mixed lengths, a shared fragmented pool, per-sequence budgets in
    {16, 64, all blocks} and 1% of tokens at +-60000."""
    rng = np.random.default_rng(714)
    batch = 8
    lengths = (rng.integers(1024, 8192, size=batch) // 32 * 32).astype(np.int64)
    case = make_case(715, batch, hq, 8, lengths.tolist(), outliers=0.01, spare_pages=64)
    n_blocks = case.sealed.astype(np.int64)
    choice = rng.integers(0, 3, size=batch)
    budgets = np.where(choice == 0, 16, np.where(choice == 1, 64, n_blocks)).astype(np.int32)
    budgets[0] = n_blocks[0]
    print(f"case: lengths={lengths.tolist()} budgets={budgets.tolist()}", flush=True)
    check(hip, case, 64, 4, 8, sel_stride=int(n_blocks.max()), budgets=budgets)


def test_capacity_and_bad_budget_flags(hip):
    """A sequence with more sealed blocks than rep_stride selects nothing and
    attends its tail only; a bad per-sequence budget is flagged the same way
    as by score_select."""
    case = make_case(716, 2, 16, 8, [32 * 40 + 3, 32 * 30])
    kv = device_kv(case)
    q = to_dev(case.query)
    st = status_tensor()
    budgets = to_dev(np.array([20, 10], np.int32))  # 10 < init + local
    sel, cnt, out = hip.select_attend(kv, q, 8, 20, 4, 8, SCALE, status=st, sel_stride=20, budgets=budgets)
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_BAD_BUDGET
    c = cnt.cpu().numpy()
    assert (c[1] == 0).all() and (c[0] == 20).all()
    kv.sealed.copy_(to_dev(np.array([case.rep_stride + 1, 30], np.int32)))
    kv.seq_len.copy_(to_dev(np.array([32 * (case.rep_stride + 1) + 3, 32 * 30], np.int32)))
    st.zero_()
    sel, cnt, out = hip.select_attend(kv, q, 8, 20, 4, 8, SCALE, status=st, sel_stride=20)
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_CAPACITY
    assert (cnt.cpu().numpy()[0] == 0).all()


# ---- decode_step: append + seal + select + attend ----------------------------

def oracle_decode(case, k, v, local_tokens, budget, init, local, sel_stride, k16=None, v16=None):
    """The oracle's step: append, seal, then select + attend per KV group."""
    if k16 is not None:
        O.paged_append(case.pool, PAGE, case.table, case.seq_len, k16=k16, v16=v16, batch=case.batch, hkv=case.hkv,
                       d=D)
    else:
        O.paged_append(case.pool, PAGE, case.table, case.seq_len, k=k, v=v, batch=case.batch, hkv=case.hkv, d=D)
    O.paged_seal(case.pool, PAGE, case.table, case.seq_len, case.sealed, case.generation, case.reps,
                 case.rep_heads, case.rep_stride, case.batch, case.hq, case.hkv, D, local_tokens)
    return oracle_step(case, budget, init, local, sel_stride)


def check_state(kv, case):
    from gpu_util import pool_numpy
    assert np.array_equal(kv.seq_len.cpu().numpy(), case.seq_len)
    assert np.array_equal(kv.sealed.cpu().numpy(), case.sealed)
    assert np.array_equal(kv.generation.cpu().numpy(), case.generation)
    assert np.array_equal(pool_numpy(kv), case.pool)
    assert np.array_equal(kv.reps.cpu().numpy().view(np.uint32), case.reps.view(np.uint32))


@pytest.mark.parametrize("local_tokens,rep_heads,hq", [(0, None, 16), (32, None, 16), (0, 16, 16), (0, None, 32),
                                                      (32, 32, 32)])
def test_decode_steps_bit_exact(hip, local_tokens, rep_heads, hq):
    """40 decode steps across seal boundaries (tails start at 30, 0 and 13
    tokens), each step one launch; state, ids and outputs checked per step."""
    print(f"case: local_tokens={local_tokens} rep_heads={rep_heads} hq={hq}", flush=True)
    case = make_case(720 + local_tokens + hq, 3, hq, 8, [32 * 70 + 30, 32 * 20, 32 * 9 + 13], table_stride=80,
                     local_tokens=local_tokens, rep_heads=rep_heads, planted=4)
    kv = device_kv(case)
    assert hip.select_attend_fused(kv, 8)  # G=2 and G=4 both run as one launch
    ws, _ = hip.decode_step_workspace(kv)
    st = status_tensor()
    rng = np.random.default_rng(11)
    budget, init, local = 16, 2, 3
    for step in range(40):
        k = (rng.standard_normal((3, 8, D)) * 2).astype(np.float32)
        v = (rng.standard_normal((3, 8, D)) * 2).astype(np.float32)
        case.query[:] = rng.standard_normal(case.query.shape).astype(np.float32)
        sel, cnt, out = hip.decode_step(kv, to_dev(k), to_dev(v), local_tokens, to_dev(case.query), 8, budget, init,
                                        local, SCALE, ws, status=st)
        esel, ecnt, expect = oracle_decode(case, k, v, local_tokens, budget, init, local, budget)
        torch.cuda.synchronize()
        assert int(st.item()) == 0, step
        got_sel, got_cnt = sel.cpu().numpy(), cnt.cpu().numpy()
        assert np.array_equal(got_cnt, ecnt), step
        for b in range(3):
            for g in range(8):
                assert got_sel[b, g, : ecnt[b, g]].tolist() == esel[b, g, : ecnt[b, g]].tolist(), (step, b, g)
        assert_close_2e3(out.cpu().numpy(), expect)
        if step % 13 == 0 or step == 39:
            check_state(kv, case)
    assert int(ws[:kv.batch].abs().sum().item()) == 0, "arrival counters must be left at zero"


def test_decode_step_f16_and_three_launch_fallback(hip):
    """Raw FP16 input at G=2 and G=4 (fused), and G=8 (fallback: three
    launches) give the oracle's state and outputs."""
    for hq, seed in ((16, 730), (32, 731), (64, 733)):
        case = make_case(seed, 2, hq, 8, [32 * 40 + 31, 32 * 12 + 2], table_stride=48)
        kv = device_kv(case)
        assert hip.select_attend_fused(kv, 8) == (hq in (16, 32))
        ws, _ = hip.decode_step_workspace(kv)
        st = status_tensor()
        rng = np.random.default_rng(seed)
        for step in range(3):
            k16 = (rng.standard_normal((2, 8, D)) * 3).astype(np.float16).view(np.uint16)
            v16 = (rng.standard_normal((2, 8, D)) * 3).astype(np.float16).view(np.uint16)
            sel, cnt, out = hip.decode_step(kv, to_dev(k16.view(np.int16)).view(torch.uint16),
                                            to_dev(v16.view(np.int16)).view(torch.uint16), 0, to_dev(case.query), 8,
                                            12, 2, 2, SCALE, ws, status=st)
            esel, ecnt, expect = oracle_decode(case, None, None, 0, 12, 2, 2, 12, k16=k16, v16=v16)
            torch.cuda.synchronize()
            assert int(st.item()) == 0
            assert np.array_equal(cnt.cpu().numpy(), ecnt)
            got_sel = sel.cpu().numpy()
            for b in range(2):
                for g in range(8):
                    assert got_sel[b, g, : ecnt[b, g]].tolist() == esel[b, g, : ecnt[b, g]].tolist()
            assert_close_2e3(out.cpu().numpy(), expect)
        check_state(kv, case)


def test_decode_step_capacity_leaves_counters(hip):
    """No page for the new token: flagged, nothing appended or sealed, and the
    step still selects and attends the existing tokens."""
    case = make_case(732, 2, 16, 8, [32 * 4, 32 * 2 + 5], table_stride=4)
    kv = device_kv(case)
    ws, _ = hip.decode_step_workspace(kv)
    st = status_tensor()
    z = torch.zeros((2, 8, D), dtype=torch.float32, device="cuda")
    sel, cnt, out = hip.decode_step(kv, z, z, 0, to_dev(case.query), 8, 4, 1, 1, SCALE, ws, status=st)
    torch.cuda.synchronize()
    assert int(st.item()) & hip.STATUS_CAPACITY
    assert kv.seq_len.cpu().numpy().tolist() == [32 * 4, 32 * 2 + 6]
    esel, ecnt, expect = oracle_step_after_partial_append(case)
    assert np.array_equal(cnt.cpu().numpy(), ecnt)
    assert_close_2e3(out.cpu().numpy(), expect)
    assert int(ws[:kv.batch].abs().sum().item()) == 0


def oracle_step_after_partial_append(case):
    """Sequence 0 has no page left (unchanged); sequence 1 appends a zero token."""
    z = np.zeros((1, 8, D), np.float32)
    seq1 = case.seq_len[1:2].copy()
    O.paged_append(case.pool, PAGE, case.table[1:2], seq1, k=z, v=z, batch=1, hkv=8, d=D)
    case.seq_len[1] = seq1[0]
    return oracle_step(case, 4, 1, 1, 4)


def test_decode_step_graph_replays(hip):
    """One decode step captured in a HIP graph and replayed 5 times (each
    replay appends the captured token again and advances the counters), with
    eager work and synchronisations between replays, equals 5 eager steps on
    a copy of the state: same bytes, counters, ids and outputs, bit for bit."""
    case = make_case(740, 4, 16, 8, [32 * 60 + 29, 32 * 33, 32 * 12 + 3, 32 * 70 + 31], table_stride=80, planted=4)
    rng = np.random.default_rng(41)
    k = to_dev((rng.standard_normal((4, 8, D)) * 2).astype(np.float32))
    v = to_dev((rng.standard_normal((4, 8, D)) * 2).astype(np.float32))
    q = to_dev(case.query)
    outs = []
    for mode in ("eager", "graph"):
        kv = device_kv(case)
        ws, _ = hip.decode_step_workspace(kv)
        sel = torch.full((4, 8, 16), -1, dtype=torch.int32, device="cuda")
        cnt = torch.zeros((4, 8), dtype=torch.int32, device="cuda")
        out = torch.zeros((4, 16, D), dtype=torch.float32, device="cuda")
        st = status_tensor()
        step = lambda: hip.decode_step(kv, k, v, 0, q, 8, 16, 2, 3, SCALE, ws, selected=sel, counts=cnt, out=out,
                                       status=st)
        history = []
        if mode == "eager":
            for _ in range(5):
                step()
                torch.cuda.synchronize()
                history.append((sel.clone(), cnt.clone(), out.clone()))
        else:
            side = torch.cuda.Stream()
            with torch.cuda.stream(side):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=side):
                    step()
            torch.cuda.synchronize()
            for _ in range(5):
                g.replay()
                torch.cuda.synchronize()
                _ = (out * 2).sum().item()  # eager work between replays
                history.append((sel.clone(), cnt.clone(), out.clone()))
        assert int(st.item()) == 0
        assert int(ws[:kv.batch].abs().sum().item()) == 0
        outs.append((history, kv.seq_len.cpu().numpy(), kv.sealed.cpu().numpy(), kv.generation.cpu().numpy(),
                     kv.pool.view(torch.int16).cpu().numpy(), kv.reps.cpu().numpy()))
    (he, *se), (hg, *sg) = outs
    for a, b in zip(se, sg):
        assert np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))
    for (s1, c1, o1), (s2, c2, o2) in zip(he, hg):
        assert torch.equal(c1, c2) and torch.equal(s1, s2) and torch.equal(o1, o2)
    assert int(outs[0][1][3]) == 32 * 70 + 31 + 5  # five tokens appended, a seal on the way


def test_decode_steps_key_channel_outliers_four_heads(hip):
    """The Qwen3-8B decode step's data through its default kernel: 32 query /
    8 KV heads (the fused, LDS-staged G = 4 launch), keys with 4 of 128
    channels scaled x8 (post-RoPE key outliers, in the pool and in every
    appended token), 1024+ sealed blocks per sequence, budget 64 = 4 init +
    8 local + 52 dynamic; 24 decode steps with seals on the way.  Ids and
    state bit-exact, attention within 2e-3 of the oracle on every step."""
    lengths = [32 * 1024 + 20, 32 * 1100 + 30, 32 * 1040 + 9]
    print(f"case: G=4 channel outliers lengths={lengths}", flush=True)
    case = make_case(761, 3, 32, 8, lengths, table_stride=1112, channel_scale=(4, 8.0))
    kv = device_kv(case)
    budget, init, local = 64, 4, 8
    assert hip.select_attend_fused(kv, 8)
    ws, _ = hip.decode_step_workspace(kv)
    st = status_tensor()
    rng = np.random.default_rng(62)
    seals = 0
    for step in range(24):
        k = rng.standard_normal((3, 8, D)).astype(np.float32)
        k[..., :4] *= 8.0
        v = rng.standard_normal((3, 8, D)).astype(np.float32)
        case.query[:] = rng.standard_normal(case.query.shape).astype(np.float32)
        before = case.sealed.copy()
        sel, cnt, out = hip.decode_step(kv, to_dev(k), to_dev(v), 0, to_dev(case.query), 8, budget, init, local,
                                        SCALE, ws, status=st)
        esel, ecnt, expect = oracle_decode(case, k, v, 0, budget, init, local, budget)
        seals += int((case.sealed - before).sum())
        torch.cuda.synchronize()
        assert int(st.item()) == 0, step
        got_sel, got_cnt = sel.cpu().numpy(), cnt.cpu().numpy()
        assert np.array_equal(got_cnt, ecnt), step
        assert (ecnt == budget).all()
        for b in range(3):
            for g in range(8):
                assert got_sel[b, g, :budget].tolist() == esel[b, g, :budget].tolist(), (step, b, g)
        assert_close_2e3(out.cpu().numpy(), expect)
        if step in (0, 12, 23):
            check_state(kv, case)
    assert seals == 3  # one seal each, after 12, 2 and 23 appends
    assert int(ws[:kv.batch].abs().sum().item()) == 0


def test_decode_steps_qwen3_06b_shape_two_heads(hip):
    """The Qwen3-0.6B decode step through the kernel the headline bench
    times: 16 query / 8 KV heads (the fused G = 2 launch with the append),
    512+ sealed blocks per sequence in permuted pages, budget 64 = 4 init +
    8 local + 52 dynamic, 8 planted blocks per KV head; 24 decode steps with
    seals on the way.  Ids and state bit-exact, attention within 2e-3 of the
    oracle on every step."""
    lengths = [32 * 512 + 20, 32 * 530 + 30, 32 * 600 + 9, 32 * 515 + 31]
    print(f"case: G=2 Qwen3-0.6B heads, lists of 512+ blocks, lengths={lengths}", flush=True)
    case = make_case(771, 4, 16, 8, lengths, table_stride=620, planted=8)
    kv = device_kv(case)
    budget, init, local = 64, 4, 8
    assert hip.select_attend_fused(kv, 8)
    ws, _ = hip.decode_step_workspace(kv)
    st = status_tensor()
    rng = np.random.default_rng(63)
    seals = 0
    for step in range(24):
        k = rng.standard_normal((4, 8, D)).astype(np.float32)
        v = rng.standard_normal((4, 8, D)).astype(np.float32)
        # the query drifts a little, so the planted blocks keep scoring high
        case.query[:] = case.query + 0.1 * rng.standard_normal(case.query.shape).astype(np.float32)
        before = case.sealed.copy()
        sel, cnt, out = hip.decode_step(kv, to_dev(k), to_dev(v), 0, to_dev(case.query), 8, budget, init, local,
                                        SCALE, ws, status=st)
        esel, ecnt, expect = oracle_decode(case, k, v, 0, budget, init, local, budget)
        seals += int((case.sealed - before).sum())
        torch.cuda.synchronize()
        assert int(st.item()) == 0, step
        got_sel, got_cnt = sel.cpu().numpy(), cnt.cpu().numpy()
        assert np.array_equal(got_cnt, ecnt), step
        assert (ecnt == budget).all()
        for b in range(4):
            for g in range(8):
                assert got_sel[b, g, :budget].tolist() == esel[b, g, :budget].tolist(), (step, b, g)
        assert_close_2e3(out.cpu().numpy(), expect)
        if step in (0, 11, 23):
            check_state(kv, case)
    assert seals == 4  # after 12, 2, 23 and 1 appends
    assert int(ws[:kv.batch].abs().sum().item()) == 0


def test_c1_shape_shared_selection_then_attention(hip):
    """The reference's C1/C2 single-layer case at its own shape: 1 sequence,
    16 query / 8 KV heads, 2048 tokens (64 blocks), 4 planted blocks whose
    keys are 0.5 x the query of their head group plus noise, one block set
    shared by all 16 query heads with budget 16 = init 1 + local 2 + 13
    dynamic (selection_main.cpp:178-181), then attention over the 512
    selected tokens.  Ids bit-exact in every selection form (the planted
    blocks among them), attention within 2e-3 of the oracle over the paged
    pool and, after packing the 16 blocks (gather_pages, the placement of
    read_blocks_fixed), over the 512 contiguous tokens against the oracle's
    attention_reference on the packed bytes."""
    case = make_case(770, 1, 16, 8, [2048], table_stride=66)
    rng = np.random.default_rng(77)
    planted = [9, 22, 37, 50]
    f16 = case.pool.view(np.float16)
    for g in range(8):
        qmean = case.query[0, 2 * g:2 * g + 2].mean(axis=0)
        for blk in planted:
            noise = rng.standard_normal((PAGE, D)).astype(np.float32)
            f16[case.table[0, blk], :, 0, g, :] = (0.5 * qmean[None, :] + 0.5 * noise).astype(np.float16)
    case.sealed[:] = 0
    case.generation[:] = 0
    case.reps[:] = 0
    O.paged_seal(case.pool, PAGE, case.table, case.seq_len, case.sealed, case.generation, case.reps, 8,
                 case.rep_stride, 1, 16, 8, D, 0)
    assert int(case.sealed[0]) == 64
    budget, init, local = 16, 1, 2
    esel, ecnt = O.paged_score_select(case.query, case.reps, case.sealed, 1, 16, 8, D, 8, case.rep_stride, 1, budget,
                                      init, local)
    ids = esel[0, 0, :16].tolist()
    assert ecnt[0, 0] == 16 and set(planted) <= set(ids) and 0 in ids and {62, 63} <= set(ids)
    expect = O.paged_sparse_attention(case.pool, PAGE, case.table, case.seq_len, case.sealed, esel, ecnt, 1,
                                      case.query, 1, 16, 8, D, SCALE)
    kv = device_kv(case)
    q = to_dev(case.query)
    st = status_tensor()
    forms = {"single": hip.score_select(kv, q, 1, budget, init, local, status=st),
             "split": hip.score_select_split(kv, q, 1, budget, init, local, status=st)[:2]}
    sel_f, cnt_f, out_f = hip.select_attend(kv, q, 1, budget, init, local, SCALE, status=st)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    for name, (sel, cnt) in forms.items():
        assert cnt.cpu().numpy().tolist() == [[16]], name
        assert sel.cpu().numpy()[0, 0].tolist() == ids, name
    assert sel_f.cpu().numpy()[0, 0].tolist() == ids
    assert_close_2e3(out_f.cpu().numpy(), expect)
    sel, cnt = forms["single"]
    for splits in (1, 2, 4):
        out = hip.sparse_decode_attention(kv, q, sel, cnt, SCALE, splits=splits, status=st)
        torch.cuda.synchronize()
        assert_close_2e3(out.cpu().numpy(), expect)
    # the reference's C2 flow: pack the selected blocks, attend the 512 tokens
    pages = to_dev(case.table[0, ids].astype(np.int32))
    packed = torch.zeros((16, case.page_elems), dtype=torch.int16, device="cuda").view(torch.uint16)
    hip.gather_pages(kv.pool, kv.page_bytes, kv.num_pages, pages, packed, status=st)
    out_c = hip.attention_contiguous(packed.view(-1), q[0], 512, 16, 8, SCALE)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    packed_np = packed.view(torch.int16).cpu().numpy().view(np.uint16)
    ref = O.attention_reference(packed_np, case.query[0], 512, 16, 8, D, SCALE)
    assert np.abs(out_c.cpu().numpy().astype(np.float64) - ref).max() <= 2e-5
    assert_close_2e3(ref[None], expect)
