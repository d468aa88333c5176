"""Seeded paged-KV scenarios shared by the CPU oracle tests and the GPU parity
tests (numpy arrays; the GPU tests copy them to device memory)."""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

import oracle as O

PAGE = 32
D = 128


@dataclass
class PagedCase:
    batch: int
    hq: int
    hkv: int
    table_stride: int
    num_pages: int
    pool: np.ndarray          # uint16 [num_pages, 32, 2, hkv, D]
    table: np.ndarray         # int32 [batch, table_stride]
    seq_len: np.ndarray       # int32 [batch]
    sealed: np.ndarray        # int32 [batch]
    generation: np.ndarray    # int32 [batch]
    reps: np.ndarray          # float32 [batch, rep_heads, D, rep_stride]
    query: np.ndarray         # float32 [batch, hq, D]
    rep_heads: int
    rep_stride: int
    local_tokens: int = 0
    extra: dict = field(default_factory=dict)

    @property
    def page_elems(self):
        return PAGE * 2 * self.hkv * D


def make_case(seed, batch, hq, hkv, lengths, table_stride=None, rep_heads=None, local_tokens=0,
              spare_pages=3, outliers=0.0, planted=0, channel_scale=None, rep_stride=None):
    """Random FP16 KV in a randomly permuted page pool; sequences hold
    `lengths` tokens; every block past the local tail is sealed with the
    mean-key representative (computed by the oracle's seal)."""
    rng = np.random.default_rng(seed)
    lengths = np.asarray(lengths, np.int64)
    need = [(int(n) + PAGE - 1) // PAGE for n in lengths]
    table_stride = table_stride or max(max(need) + 2, 1)
    total = sum(table_stride for _ in range(batch)) + spare_pages
    num_pages = total
    perm = rng.permutation(num_pages).astype(np.int32)
    table = perm[: batch * table_stride].reshape(batch, table_stride).copy()
    pool = (rng.standard_normal((num_pages, PAGE, 2, hkv, D)) * 1.0).astype(np.float16)
    if channel_scale is not None:
        ch, factor = channel_scale
        pool[:, :, 0, :, :ch] = (pool[:, :, 0, :, :ch].astype(np.float32) * factor).astype(np.float16)
    if outliers > 0:
        mask = rng.random((num_pages, PAGE)) < outliers
        sign = np.where(rng.random((num_pages, PAGE, 2, hkv, D)) < 0.5, -1.0, 1.0).astype(np.float16)
        big = (sign * np.float16(60000)).astype(np.float16)
        pool = np.where(mask[:, :, None, None, None], big, pool).astype(np.float16)
    pool = pool.view(np.uint16)
    query = rng.standard_normal((batch, hq, D)).astype(np.float32)
    if planted:
        g = hq // hkv
        for b in range(batch):
            full = int(lengths[b]) // PAGE
            if full == 0:
                continue
            for kvh in range(hkv):
                qmean = query[b, kvh * g:(kvh + 1) * g].mean(axis=0)
                for blk in rng.choice(full, size=min(planted, full), replace=False):
                    page = table[b, blk]
                    noise = rng.standard_normal((PAGE, D)).astype(np.float32) * 0.5
                    pool.view(np.float16)[page, :, 0, kvh, :] = (0.5 * qmean[None, :] + noise).astype(np.float16)
    rep_heads = rep_heads or hkv
    rep_stride = rep_stride or (table_stride + 3) // 4 * 4
    reps = np.zeros((batch, rep_heads, D, rep_stride), np.float32)
    seq_len = lengths.astype(np.int32).copy()
    sealed = np.zeros(batch, np.int32)
    generation = np.zeros(batch, np.int32)
    O.paged_seal(pool, PAGE, table, seq_len, sealed, generation, reps, rep_heads, rep_stride, batch, hq, hkv,
                 D, local_tokens)
    return PagedCase(batch, hq, hkv, table_stride, num_pages, pool, table, seq_len, sealed, generation, reps,
                     query, rep_heads, rep_stride, local_tokens)


def oracle_select_attend(case, budget, init, local, sel_stride, scale, budgets=None):
    """The oracle's per-KV-group selection and sparse attention of one step."""
    esel = np.full((case.batch, case.hkv, sel_stride), -1, np.int32)
    ecnt = np.zeros((case.batch, case.hkv), np.int32)
    for b in range(case.batch):
        bud = budget if budgets is None else int(budgets[b])
        s_, c_ = O.paged_score_select(case.query[b:b + 1], case.reps[b:b + 1], case.sealed[b:b + 1], 1, case.hq,
                                      case.hkv, D, case.rep_heads, case.rep_stride, case.hkv, bud, init, local,
                                      sel_stride=sel_stride)
        esel[b], ecnt[b] = s_[0], c_[0]
    expect = O.paged_sparse_attention(case.pool, PAGE, case.table, case.seq_len, case.sealed, esel, ecnt, case.hkv,
                                      case.query, case.batch, case.hq, case.hkv, D, scale)
    return esel, ecnt, expect


def oracle_online_append_seal(case, ring, k, v, query, local_tokens, window, topk, use_ref=False):
    """The InfLLM online seal on the oracle (the reference's P1.3c.4 step,
    online_seal_main.cpp:41-44): append one token per sequence, keep its
    decode queries in ring[b][h][pos % ring_tokens], then seal while the tail
    holds local_tokens + 32 tokens, each sealed block's representative of
    query head h being build_local_causal_representatives over that block
    alone (its 32 keys and the 32 queries of its tokens)."""
    ring_tokens = ring.shape[2]
    pos = case.seq_len.copy()
    O.paged_append(case.pool, PAGE, case.table, case.seq_len, k=k, v=v, batch=case.batch, hkv=case.hkv, d=D)
    for b in range(case.batch):
        if case.seq_len[b] > pos[b]:
            ring[b, :, pos[b] % ring_tokens, :] = query[b]
    for b in range(case.batch):
        while case.seq_len[b] >= (case.sealed[b] + 1) * PAGE + local_tokens:
            n = int(case.sealed[b])
            block_kv = case.pool[case.table[b, n]]  # [32][2][hkv][128]: the reference's token format
            slots = [(n * PAGE + t) % ring_tokens for t in range(PAGE)]
            block_q = np.ascontiguousarray(ring[b][:, slots, :])  # [hq][32][128]
            vals, _ = O.local_causal_representatives(block_q, block_kv, PAGE, case.hq, case.hkv, D, PAGE, window,
                                                     topk, use_ref=use_ref)
            case.reps[b, :, :, n] = vals[:, 0, :]
            case.sealed[b] += 1
            case.generation[b] += 1
