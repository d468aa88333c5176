"""GPU parity: the paged path at head dimensions other than 128.

The reference's selection and attention take any head_dim
(select_shared_blocks, cpp/src/selection.cpp:96-147; attention_reference,
cpp/src/attention_reference.cpp:55-96); the pool's append and mean-key seal
follow append_fp16_kv (cpp/src/qwen_layer_main.cpp:270-281) and the tail
lifecycle (cpp/src/kv_lifecycle_main.cpp:92-113).  At head_dim 64, 96 and 256
(any multiple of 8 up to 512 is accepted) the library runs its general
kernels: append + seal one workgroup per sequence, the scoring one lane per
block, the attention over the page list with the tile arithmetic of the
contiguous general kernel.  Bars: pool bytes, counters and representative
bits equal the oracle's; selected ids and score bits equal the oracle's;
attention within 2e-3 of the oracle; the decode step over steps that seal
blocks holds all three."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import assert_close_2e3, status_tensor, to_dev

pytestmark = pytest.mark.gpu

PAGE = 32


class State:
    """A paged pool of `batch` sequences in random page order, numpy side."""

    def __init__(self, seed, batch, hq, hkv, d, lengths, local=0, table_stride=None, rep_heads=None):
        rng = np.random.default_rng(seed)
        self.rng = rng
        self.batch, self.hq, self.hkv, self.d = batch, hq, hkv, d
        self.table_stride = table_stride or max((n + PAGE - 1) // PAGE for n in lengths) + 4
        self.num_pages = batch * self.table_stride
        self.rep_heads = rep_heads or hkv
        self.rep_stride = (self.table_stride + 31) // 32 * 32
        self.table = rng.permutation(self.num_pages).astype(np.int32).reshape(batch, self.table_stride)
        self.pool = rng.standard_normal((self.num_pages, PAGE, 2, hkv, d)).astype(np.float16).view(np.uint16)
        self.seq_len = np.array(lengths, np.int32)
        self.sealed = np.zeros(batch, np.int32)
        self.gen = np.zeros(batch, np.int32)
        self.reps = np.zeros((batch, self.rep_heads, d, self.rep_stride), np.float32)
        O.paged_seal(self.pool, PAGE, self.table, self.seq_len, self.sealed, self.gen, self.reps, self.rep_heads,
                     self.rep_stride, batch, hq, hkv, d, local)

    def device(self, hip):
        pool = torch.from_numpy(self.pool.view(np.int16).copy()).cuda().view(torch.uint16)
        kv = hip.PagedKV(self.batch, self.hq, self.hkv, self.table_stride, num_pages=self.num_pages,
                         rep_heads=self.rep_heads, rep_stride=self.rep_stride, head_dim=self.d, pool=pool)
        kv.block_table.copy_(to_dev(self.table))
        kv.seq_len.copy_(to_dev(self.seq_len))
        kv.sealed.copy_(to_dev(self.sealed))
        kv.generation.copy_(to_dev(self.gen))
        kv.reps.copy_(to_dev(self.reps))
        return kv

    def check_device(self, kv):
        assert np.array_equal(kv.pool.view(torch.int16).cpu().numpy().view(np.uint16), self.pool), "pool bytes"
        assert np.array_equal(kv.seq_len.cpu().numpy(), self.seq_len)
        assert np.array_equal(kv.sealed.cpu().numpy(), self.sealed)
        assert np.array_equal(kv.generation.cpu().numpy(), self.gen)
        got = kv.reps.cpu().numpy()
        for b in range(self.batch):
            n = int(self.sealed[b])
            assert np.array_equal(got[b, ..., :n].view(np.uint32), self.reps[b, ..., :n].view(np.uint32)), b


@pytest.mark.parametrize("d,hq,hkv,rep_heads,local", [(64, 16, 8, None, 0), (96, 8, 4, 8, 5),
                                                      (256, 8, 2, None, 3)])
def test_append_seal_general_head_dim(hip, d, hq, hkv, rep_heads, local):
    """Appends (fp32 converted round-to-nearest-even, then FP16 bits) over 40
    steps that seal blocks: pool bytes, lengths, sealed counts, generations
    and representative bits equal the oracle's after every step."""
    print(f"case: append_seal d={d} hq={hq} hkv={hkv} rep_heads={rep_heads} local={local}", flush=True)
    st = State(10 + d, 3, hq, hkv, d, [32 * 5 + 31, 32 * 2 + 3, 7], local=local, rep_heads=rep_heads)
    kv = st.device(hip)
    status = status_tensor()
    for step in range(40):
        k = st.rng.standard_normal((st.batch, hkv, d)).astype(np.float32)
        v = st.rng.standard_normal((st.batch, hkv, d)).astype(np.float32)
        if step % 3 == 2:
            k16, v16 = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
            hip.append_seal(kv, to_dev(k16.view(np.int16)).view(torch.uint16),
                            to_dev(v16.view(np.int16)).view(torch.uint16), local, status=status)
            O.paged_append(st.pool, PAGE, st.table, st.seq_len, k16=k16, v16=v16, batch=st.batch, hkv=hkv, d=d)
        else:
            hip.append_seal(kv, to_dev(k), to_dev(v), local, status=status)
            O.paged_append(st.pool, PAGE, st.table, st.seq_len, k=k, v=v, batch=st.batch, hkv=hkv, d=d)
        O.paged_seal(st.pool, PAGE, st.table, st.seq_len, st.sealed, st.gen, st.reps, st.rep_heads,
                     st.rep_stride, st.batch, hq, hkv, d, local)
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        st.check_device(kv)


@pytest.mark.parametrize("d,hq,hkv,rep_heads,lengths", [(64, 8, 4, None, [32 * 9 + 4, 32 * 3]),
                                                       (96, 8, 4, 8, [32 * 70 + 4, 32 * 3, 32 * 41 + 31]),
                                                       (256, 16, 8, None, [32 * 40 + 1, 32 * 17]),
                                                       (512, 4, 2, None, [32 * 12 + 7]),
                                                       (8, 4, 4, None, [32 * 33, 5])])
def test_seal_only_general_head_dim(hip, d, hq, hkv, rep_heads, lengths):
    """sa_hip_seal (no append) on a prefill (the bulk seal, spread over
    blocks and KV heads): every block the tail rule releases is sealed, with
    the oracle's representative bits and counters."""
    print(f"case: bulk seal d={d} hq={hq} hkv={hkv} rep_heads={rep_heads} lengths={lengths}", flush=True)
    st = State(31 + d, len(lengths), hq, hkv, d, lengths, rep_heads=rep_heads)
    kv = st.device(hip)
    kv.sealed.zero_()
    kv.generation.zero_()
    st.sealed[:] = 0
    st.gen[:] = 0
    st.reps[:] = 0
    kv.reps.zero_()
    status = status_tensor()
    hip.seal(kv, 2, status=status)
    O.paged_seal(st.pool, PAGE, st.table, st.seq_len, st.sealed, st.gen, st.reps, st.rep_heads, st.rep_stride,
                 st.batch, st.hq, st.hkv, st.d, 2)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    st.check_device(kv)


@pytest.mark.parametrize("d,hq,hkv,groups,rep_heads", [(64, 16, 8, 8, None), (64, 16, 8, 1, None),
                                                       (96, 8, 4, 4, 8), (256, 32, 8, 1, None),
                                                       (8, 4, 4, 2, None)])
def test_selection_general_head_dim(hip, d, hq, hkv, groups, rep_heads):
    """The split selection (and the one-workgroup entry point, which hands
    the scores over the same way at these head dims): ids and score bits
    equal the oracle's; the chunked form refuses the head_dim."""
    print(f"case: selection d={d} hq={hq} hkv={hkv} groups={groups}", flush=True)
    st = State(40 + d + groups, 3, hq, hkv, d, [32 * 700 + 5, 32 * 60, 32 * 9 + 1], rep_heads=rep_heads)
    kv = st.device(hip)
    q = st.rng.standard_normal((st.batch, hq, d)).astype(np.float32)
    budget, init, local = 40, 2, 4
    esel, ecnt, esc = O.paged_score_select(q, st.reps, st.sealed, st.batch, hq, hkv, d, st.rep_heads,
                                           st.rep_stride, groups, budget, init, local, want_scores=True)
    for form in ("split", "single"):
        status = status_tensor()
        scores = torch.zeros((st.batch, groups, st.rep_stride), dtype=torch.float32, device="cuda")
        fn = hip.score_select_split if form == "split" else hip.score_select
        res = fn(kv, to_dev(q), groups, budget, init, local, scores=scores, status=status)
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        sel, cnt = res[0].cpu().numpy(), res[1].cpu().numpy()
        assert np.array_equal(cnt, ecnt), form
        for b in range(st.batch):
            n = int(st.sealed[b])
            for g in range(groups):
                assert sel[b, g, : cnt[b, g]].tolist() == esel[b, g, : ecnt[b, g]].tolist(), (form, b, g)
                assert np.array_equal(scores.cpu().numpy()[b, g, :n].view(np.uint32),
                                      esc[b, g, :n].view(np.uint32)), (form, b, g)
    ws, _ = hip.score_select_chunked_workspace(kv, groups, budget, init, local)
    with pytest.raises(hip.SaHipError):
        hip.score_select_chunked(kv, to_dev(q), groups, budget, init, local, ws)


@pytest.mark.parametrize("d,hq,hkv,groups,splits", [(64, 16, 8, 8, 1), (64, 16, 8, 8, 3), (96, 32, 8, 1, 2),
                                                    (256, 8, 2, 2, 4), (512, 4, 4, 4, 1), (16, 8, 1, 1, 2)])
def test_attention_general_head_dim(hip, d, hq, hkv, groups, splits):
    """Attention over the oracle's selection plus the tail (a partial tail
    page, an empty tail, a sequence with nothing sealed): within 2e-3 of
    the oracle, with 1 to 4 splits merged in split order."""
    print(f"case: attention d={d} hq={hq} hkv={hkv} groups={groups} splits={splits}", flush=True)
    st = State(70 + d + splits, 3, hq, hkv, d, [32 * 50 + 17, 32 * 20, 21])
    kv = st.device(hip)
    q = st.rng.standard_normal((st.batch, hq, d)).astype(np.float32)
    budget = 12
    esel, ecnt = O.paged_score_select(q, st.reps, st.sealed, st.batch, hq, hkv, d, st.rep_heads, st.rep_stride,
                                      groups, budget, 1, 2)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    expect = O.paged_sparse_attention(st.pool, PAGE, st.table, st.seq_len, st.sealed, esel, ecnt, groups, q,
                                      st.batch, hq, hkv, d, scale)
    status = status_tensor()
    out = hip.sparse_decode_attention(kv, to_dev(q), to_dev(esel), to_dev(ecnt), scale, splits=splits,
                                      status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    assert_close_2e3(out.cpu().numpy().reshape(expect.shape), expect)


def test_attention_general_head_dim_bad_block_flagged(hip):
    """A selected id past the sealed blocks is flagged (bad block) and
    skipped; the other sequence's output is untouched by it."""
    st = State(90, 2, 8, 4, 64, [32 * 10 + 3, 32 * 12])
    kv = st.device(hip)
    q = st.rng.standard_normal((st.batch, 8, 64)).astype(np.float32)
    esel, ecnt = O.paged_score_select(q, st.reps, st.sealed, st.batch, 8, 4, 64, 4, st.rep_stride, 4, 6, 1, 1)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(64)))
    expect = O.paged_sparse_attention(st.pool, PAGE, st.table, st.seq_len, st.sealed, esel, ecnt, 4, q, st.batch,
                                      8, 4, 64, scale)
    bad = esel.copy()
    bad[0, 1, 0] = 999
    status = status_tensor()
    out = hip.sparse_decode_attention(kv, to_dev(q), to_dev(bad), to_dev(ecnt), scale, splits=2, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) & hip.STATUS_BAD_BLOCK
    assert_close_2e3(out.cpu().numpy()[1], expect.reshape(out.shape)[1])


@pytest.mark.parametrize("d,hq,hkv,groups,splits,local,f16", [
    (64, 16, 8, 8, 1, 0, False), (96, 8, 4, 1, 2, 4, False), (256, 16, 4, 4, 3, 0, False),
    (96, 8, 4, 4, 1, 4, False), (256, 16, 4, 4, 1, 0, True), (8, 4, 4, 4, 1, 0, False),
    (200, 8, 8, 8, 1, 3, False), (64, 32, 8, 8, 1, 0, True), (64, 16, 8, 8, 2, 0, False)])
def test_decode_steps_general_head_dim(hip, d, hq, hkv, groups, splits, local, f16):
    """sa_hip_decode_step at another head_dim over 36 steps that seal blocks:
    one launch (decode_kernel_rows: selection per KV group, splits 1) or its
    launches in sequence (append + seal, scoring, selection, attention);
    state bit-exact, ids equal, attention within 2e-3 of the oracle at every
    step, fp32 and FP16 token input."""
    print(f"case: decode steps d={d} hq={hq} hkv={hkv} groups={groups} splits={splits} f16={f16}", flush=True)
    st = State(120 + d, 2, hq, hkv, d, [32 * 30 + 29, 32 * 8 + 2], local=local)
    kv = st.device(hip)
    assert hip.select_attend_fused(kv, groups, splits) == (groups == hkv and splits == 1)
    budget, init, loc = 16, 1, 2
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    ws, _ = hip.decode_step_workspace(kv, splits)
    status = status_tensor()
    for step in range(36):
        k = st.rng.standard_normal((st.batch, hkv, d)).astype(np.float32)
        v = st.rng.standard_normal((st.batch, hkv, d)).astype(np.float32)
        q = st.rng.standard_normal((st.batch, hq, d)).astype(np.float32)
        if f16:
            k16, v16 = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
            kd = to_dev(k16.view(np.int16)).view(torch.uint16)
            vd = to_dev(v16.view(np.int16)).view(torch.uint16)
        else:
            kd, vd = to_dev(k), to_dev(v)
        sel, cnt, out = hip.decode_step(kv, kd, vd, local, to_dev(q), groups, budget, init, loc,
                                        scale, ws, splits=splits, status=status)
        if f16:
            O.paged_append(st.pool, PAGE, st.table, st.seq_len, k16=k16, v16=v16, batch=st.batch, hkv=hkv, d=d)
        else:
            O.paged_append(st.pool, PAGE, st.table, st.seq_len, k=k, v=v, batch=st.batch, hkv=hkv, d=d)
        O.paged_seal(st.pool, PAGE, st.table, st.seq_len, st.sealed, st.gen, st.reps, st.rep_heads, st.rep_stride,
                     st.batch, hq, hkv, d, local)
        esel, ecnt = O.paged_score_select(q, st.reps, st.sealed, st.batch, hq, hkv, d, st.rep_heads,
                                          st.rep_stride, groups, budget, init, loc)
        expect = O.paged_sparse_attention(st.pool, PAGE, st.table, st.seq_len, st.sealed, esel, ecnt, groups, q,
                                          st.batch, hq, hkv, d, scale)
        torch.cuda.synchronize()
        assert int(status.item()) == 0, step
        assert np.array_equal(cnt.cpu().numpy(), ecnt), step
        assert np.array_equal(sel.cpu().numpy(), esel), step
        assert_close_2e3(out.cpu().numpy().reshape(expect.shape), expect)
    st.check_device(kv)


def test_general_head_dim_refusals(hip):
    """Entry points built for head_dim 128 only refuse another one with an
    error (no launch): the fused select-attend, the chunked attention, and
    the allocation-free step; a head_dim that is not a multiple of 8 is
    refused everywhere."""
    st = State(150, 1, 8, 4, 64, [32 * 6])
    kv = st.device(hip)
    q = to_dev(st.rng.standard_normal((1, 8, 64)).astype(np.float32))
    with pytest.raises(hip.SaHipError):
        hip.select_attend(kv, q, 4, 8, 1, 1, 0.125)
    sel = torch.zeros((1, 4, 8), dtype=torch.int32, device="cuda")
    cnt = torch.zeros((1, 4), dtype=torch.int32, device="cuda")
    with pytest.raises(hip.SaHipError):
        hip.sparse_decode_attention_chunked(kv, q, sel, cnt, 0.125, 2, 4)
    bad = State(151, 1, 8, 4, 12, [32 * 2])
    kvb = bad.device(hip)
    with pytest.raises(hip.SaHipError):
        hip.score_select_split(kvb, to_dev(bad.rng.standard_normal((1, 8, 12)).astype(np.float32)), 4, 8, 1, 1)
