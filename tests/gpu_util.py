"""Copy a PagedCase (numpy) into a solidattention_amd.PagedKV on cuda:0."""
from __future__ import annotations

import numpy as np
import torch

import solidattention_amd as sa

ATOL = 2e-3
RTOL = 2e-3


def to_dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def device_kv(case) -> sa.PagedKV:
    assert case.pool.shape == (case.num_pages, 32, 2, case.hkv, 128)
    assert case.table.max() < case.num_pages and case.table.min() >= 0
    pool = torch.from_numpy(case.pool.view(np.int16)).cuda().view(torch.uint16)
    kv = sa.PagedKV(case.batch, case.hq, case.hkv, case.table_stride, num_pages=case.num_pages,
                    rep_heads=case.rep_heads, rep_stride=case.rep_stride, pool=pool)
    kv.block_table.copy_(to_dev(case.table))
    kv.seq_len.copy_(to_dev(case.seq_len))
    kv.sealed.copy_(to_dev(case.sealed))
    kv.generation.copy_(to_dev(case.generation))
    kv.reps.copy_(to_dev(case.reps))
    return kv


def pool_numpy(kv: sa.PagedKV) -> np.ndarray:
    return kv.pool.view(torch.int16).cpu().numpy().view(np.uint16)


def assert_close_2e3(got, expect):
    """The north-star bar: within 2e-3 absolute or relative."""
    got = np.asarray(got, np.float64)
    expect = np.asarray(expect, np.float64)
    err = np.abs(got - expect)
    ok = (err <= ATOL) | (err <= RTOL * np.abs(expect))
    if not ok.all():
        i = int(np.argmax(np.where(ok, 0, err)))
        raise AssertionError(f"{(~ok).sum()} of {ok.size} outside 2e-3; worst idx {i}: got {got.ravel()[i]} "
                             f"expect {expect.ravel()[i]}")


def status_tensor():
    return torch.zeros(1, dtype=torch.int32, device="cuda")
