"""GPU: sa_hip_read_step_bytes, the decode step's bytes read with no
arithmetic (the bandwidth reference the bench sets beside the attention
kernels).  Its output, the XOR of every 32-bit word read per (sequence, KV
head), is checked bit for bit against the same XOR over the case's numpy
arrays: the representative rows of the sealed blocks, the selected pages'
K/V slices of the head and the unsealed tail."""
import numpy as np
import pytest
import torch

from gpu_util import device_kv, status_tensor, to_dev
from paged_case import PAGE, make_case

pytestmark = pytest.mark.gpu


def expect_xor(case, sel, cnt, select_groups):
    pool32 = case.pool.view(np.uint32).reshape(case.num_pages, PAGE, 2, case.hkv, 64)
    reps32 = case.reps.view(np.uint32)
    per = case.hkv // select_groups
    sel_stride = sel.shape[-1]
    out = np.zeros((case.batch, case.hkv), np.uint32)
    xor = np.bitwise_xor.reduce
    for b in range(case.batch):
        s, n = int(case.sealed[b]), int(case.seq_len[b])
        for h in range(case.hkv):
            x = np.uint32(0)
            for r in range(h, case.rep_heads, case.hkv):
                if s:
                    x ^= xor(reps32[b, r, :, :s].ravel())
            for blk in sel[b, h // per, :min(int(cnt[b, h // per]), sel_stride)]:
                if 0 <= blk < s:
                    x ^= xor(pool32[case.table[b, blk], :, :, h, :].ravel())
            for t in range(s * PAGE, n):
                x ^= xor(pool32[case.table[b, t // PAGE], t % PAGE, :, h, :].ravel())
            out[b, h] = x
    return out


def random_lists(rng, case, select_groups, sel_stride):
    sel = np.full((case.batch, select_groups, sel_stride), -1, np.int32)
    cnt = np.zeros((case.batch, select_groups), np.int32)
    for b in range(case.batch):
        s = int(case.sealed[b])
        for g in range(select_groups):
            c = int(rng.integers(0, min(s, sel_stride) + 1)) if s else 0
            sel[b, g, :c] = rng.choice(s, size=c, replace=False)
            cnt[b, g] = c
    return sel, cnt


@pytest.mark.parametrize("hq,hkv,select_groups,rep_heads,local", [
    (16, 8, 8, None, 0),      # one list per KV head, mean-key reps per KV head (the decode step's layout)
    (32, 8, 2, None, 32),     # lists shared by 4 KV heads, a tail spanning two pages
    (16, 8, 8, 16, 0),        # representatives per query head
    (8, 8, 8, None, 0),
])
def test_read_step_bytes_xor(hip, hq, hkv, select_groups, rep_heads, local):
    lengths = [0, 31, 32, 32 * 9 + 17, 32 * 40, 32 * 75 + 3, 32 * 3 + 1]
    case = make_case(401 + hq + select_groups, len(lengths), hq, hkv, lengths, rep_heads=rep_heads,
                     local_tokens=local)
    rng = np.random.default_rng(hq * 7 + select_groups)
    sel_stride = 64
    sel, cnt = random_lists(rng, case, select_groups, sel_stride)
    print(f"case: read_step_bytes hq={hq} hkv={hkv} groups={select_groups} rep_heads={case.rep_heads} "
          f"local={local} sealed={case.sealed.tolist()}", flush=True)
    kv = device_kv(case)
    st = status_tensor()
    got = hip.read_step_bytes(kv, to_dev(sel), to_dev(cnt), select_groups, status=st)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    assert np.array_equal(got.cpu().numpy().view(np.uint32), expect_xor(case, sel, cnt, select_groups))


def test_read_step_bytes_skips_and_flags_bad_ids(hip):
    """Ids outside the sealed range are skipped and flagged (kStatusBadBlock);
    counts above sel_stride read sel_stride entries."""
    case = make_case(431, 3, 16, 8, [32 * 20, 32 * 6 + 5, 32 * 12])
    sel_stride = 8
    sel = np.tile(np.arange(sel_stride, dtype=np.int32), (3, 8, 1))
    # sequence 1 holds 6 sealed blocks: its ids 6 and 7 (the tail's block and
    # one past it) are outside the sealed range in every list
    sel[2, 5, 0] = -1
    cnt = np.full((3, 8), sel_stride, np.int32)
    cnt[0, 0] = 1000    # clamped to sel_stride
    kv = device_kv(case)
    st = status_tensor()
    got = hip.read_step_bytes(kv, to_dev(sel), to_dev(cnt), 8, status=st)
    torch.cuda.synchronize()
    assert int(st.item()) == 2
    assert np.array_equal(got.cpu().numpy().view(np.uint32), expect_xor(case, sel, cnt, 8))
