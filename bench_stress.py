"""Mixed-length stress workload (bench.py --workload stress).

Qwen3-0.6B attention shape (16 query / 8 KV heads, head_dim 128), batch 128
sequences whose contexts are drawn uniformly from [1024, 65536] tokens
(rounded down to 32), pages drawn at random from one shared fragmented pool,
a per-sequence budget of 16, 64 or every sealed block (512 / 2048 tokens /
full context), K/V ~ N(0,1) FP16 with 1% of tokens set to +-60000.

A step = for each layer: append one K/V token per sequence (+seal when a
page fills), score + select per KV group under the per-sequence budgets,
and sparse GQA decode attention with each (sequence, KV head) page list cut
into fixed-size chunks (one workgroup each, log-sum-exp merge), so a
2048-page list and a 17-page one cost by their length.  The pool of one
layer holds ~17 GiB; the layer count defaults to 4 (per-layer figures do
not depend on it: nothing of a layer stays in cache for the next).

Reported: µs/layer, tokens/s, achieved HBM GB/s of the attention kernel
(selected KV + tail + q/out + ids per launch) and of the layer, a full-size
parity check (selection bit-exact, attention within 2e-3 of the oracle,
full-budget sequences within 2e-3 of dense attention), and the oracle's
single-thread time on a bounded sample of sequences.
"""
from __future__ import annotations

import json
import os
import sys
import time

PAGE = 32
D = 128
HBM_PEAK_GBPS = 8000.0


def log(msg):
    print(f"[stress] {msg}", file=sys.stderr, flush=True)


class StressLayer:
    """One layer's paged pool (shared, fragmented), tables, representatives
    and per-step inputs, all resident in HBM."""

    def __init__(self, sa, np, torch, lengths, hq, hkv, layer, seed, total_steps):
        batch = len(lengths)
        need = (lengths + total_steps + PAGE - 1) // PAGE
        table_stride = int(need.max())
        num_pages = int(need.sum()) + 64
        kv = sa.PagedKV(batch, hq, hkv, table_stride, num_pages=num_pages)
        lseed = seed + 7919 * layer
        g = torch.Generator(device="cpu")
        g.manual_seed(lseed)
        perm = torch.randperm(num_pages, generator=g, dtype=torch.int64).to(torch.int32)
        table = torch.full((batch, table_stride), -1, dtype=torch.int32)
        first = 0
        for b in range(batch):
            n = int(need[b])
            table[b, :n] = perm[first:first + n]
            first += n
        kv.block_table.copy_(table)
        sa.fill_synthetic_f16(kv.pool.view(-1), lseed, 0)
        # 1% of tokens: every K and V element set to +-60000
        gg = torch.Generator(device="cuda")
        gg.manual_seed(lseed + 5)
        tok = kv.pool.view(torch.float16).view(num_pages * PAGE, 2 * hkv * D)
        hit = (torch.rand(num_pages * PAGE, generator=gg, device="cuda") < 0.01).nonzero().squeeze(1)
        sign = torch.randint(0, 2, (hit.numel(), 2 * hkv * D), generator=gg, device="cuda", dtype=torch.int8)
        tok[hit] = (sign.to(torch.float16) * 2 - 1) * 60000.0
        del sign, hit
        q = torch.empty((total_steps, batch, hq, D), dtype=torch.float32, device="cuda")
        sa.fill_synthetic_f32(q.view(-1), lseed + 1, 0)
        knew = torch.empty((total_steps, batch, hkv, D), dtype=torch.float32, device="cuda")
        vnew = torch.empty_like(knew)
        sa.fill_synthetic_f32(knew.view(-1), lseed + 2, 0)
        sa.fill_synthetic_f32(vnew.view(-1), lseed + 3, 0)
        kv.seq_len.copy_(torch.from_numpy(lengths.astype(np.int32)))
        sa.seal(kv, 0)
        self.kv, self.q, self.knew, self.vnew = kv, q, knew, vnew
        self.batch, self.hq, self.hkv = batch, hq, hkv


def run(args):
    import numpy as np
    import torch

    import solidattention_amd as sa

    B, HQ, HKV = 128, 16, 8
    INIT, LOCAL = 4, 8
    layers = args.layers or 4
    chunk = args.chunk if args.chunk is not None else 128
    torch.cuda.set_device(0)
    rng = np.random.default_rng(args.seed)
    lengths = (rng.integers(1024, 65536 + 1, size=B) // PAGE * PAGE).astype(np.int64)
    blocks = lengths // PAGE
    klass = rng.integers(0, 3, size=B)
    sel_stride = int(blocks.max())
    budgets = np.where(klass == 0, 16, np.where(klass == 1, 64, sel_stride)).astype(np.int32)
    total_steps = args.warmup + args.steps
    log(f"setup: {layers} layers, batch {B}, contexts {lengths.min()}..{lengths.max()} "
        f"(mean {lengths.mean():.0f}), budgets 16/64/full = {(klass == 0).sum()}/{(klass == 1).sum()}/"
        f"{(klass == 2).sum()}, chunk {chunk}")
    t0 = time.time()
    L = [StressLayer(sa, np, torch, lengths, HQ, HKV, l, args.seed, total_steps) for l in range(layers)]
    torch.cuda.synchronize()
    log(f"setup done in {time.time() - t0:.1f}s; pool {L[0].kv.pool.numel() * 2 * layers / 2**30:.1f} GiB")

    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    budgets_d = torch.from_numpy(budgets).cuda()
    selected = torch.full((B, HKV, sel_stride), -1, dtype=torch.int32, device="cuda")
    counts = torch.zeros((B, HKV), dtype=torch.int32, device="cuda")
    out = torch.empty((B, HQ, D), dtype=torch.float32, device="cuda")
    if chunk > 0:
        # enough chunks for the longest list (every sealed block + the tail page)
        max_chunks = max(2, (sel_stride + 1 + chunk - 1) // chunk)
        splits = max_chunks
    else:
        max_chunks = 0
        splits = args.splits or sa.default_splits(B, HKV, int(blocks.mean()), HQ)
    ws_bytes = max(sa.lib().sa_hip_attention_workspace_bytes(B, HQ, HKV, D, splits),
                   sa.lib().sa_hip_attention_chunked_workspace_bytes(B, HQ, HKV, D, max_chunks)
                   if chunk > 0 and not getattr(args, "chunk_grid_order", False) else 0)
    workspace = torch.zeros(max(ws_bytes // 4, 1), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    # mixed lengths: the chunked selection (long lists spread over workgroups)
    select_mode = getattr(args, "select", "auto")
    if select_mode == "auto":
        select_mode = "chunked"
    split_select = select_mode == "split"
    scores = (torch.zeros((B, HKV, L[0].kv.rep_stride), dtype=torch.float32, device="cuda")
              if split_select else None)
    select_ws = (sa.score_select_chunked_workspace(L[0].kv, HKV, sel_stride, INIT, LOCAL, sel_stride)[0]
                 if select_mode == "chunked" else None)

    def attend(ly, s):
        if chunk > 0:
            sa.sparse_decode_attention_chunked(ly.kv, ly.q[s], selected, counts, scale, chunk, max_chunks, out=out,
                                               workspace=workspace, status=status)
        else:
            sa.sparse_decode_attention(ly.kv, ly.q[s], selected, counts, scale, out=out, splits=splits,
                                       workspace=workspace, status=status)

    def layer_step(ly, s, e=None):
        if e: e[0].record(stream)
        sa.append_seal(ly.kv, ly.knew[s], ly.vnew[s], 0, status=status)
        if e: e[1].record(stream)
        if split_select:
            sa.score_select_split(ly.kv, ly.q[s], HKV, sel_stride, INIT, LOCAL, selected=selected, counts=counts,
                                  scores=scores, status=status, sel_stride=sel_stride, budgets=budgets_d)
        elif select_ws is not None:
            sa.score_select_chunked(ly.kv, ly.q[s], HKV, sel_stride, INIT, LOCAL, select_ws, selected=selected,
                                    counts=counts, status=status, sel_stride=sel_stride, budgets=budgets_d)
        else:
            sa.score_select(ly.kv, ly.q[s], HKV, sel_stride, INIT, LOCAL, selected=selected, counts=counts,
                            status=status, sel_stride=sel_stride, budgets=budgets_d)
        if e: e[2].record(stream)
        attend(ly, s)
        if e: e[3].record(stream)

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps * layers)]
    for s in range(args.warmup):
        for ly in L:
            layer_step(ly, s)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(args.steps):
        s = args.warmup + i
        for l, ly in enumerate(L):
            layer_step(ly, s, ev[i * layers + l])
    end.record(stream)
    torch.cuda.synchronize()
    if int(status.item()) != 0:
        raise SystemExit(f"device status flagged {int(status.item())}")
    ms = start.elapsed_time(end)
    ms_per_step = ms / args.steps
    us_per_layer = ms_per_step * 1000.0 / layers
    app = 1000.0 * np.mean([e[0].elapsed_time(e[1]) for e in ev])
    sel = 1000.0 * np.mean([e[1].elapsed_time(e[2]) for e in ev])
    att = 1000.0 * np.mean([e[2].elapsed_time(e[3]) for e in ev])

    # attention alone, back to back over the layers (last step's inputs and
    # the last layer's selection: the counts do not depend on the layer)
    s_last = total_steps - 1
    reps = 4
    start.record(stream)
    for _ in range(reps):
        for ly in L:
            attend(ly, s_last)
    end.record(stream)
    torch.cuda.synchronize()
    kernel_us = 1000.0 * start.elapsed_time(end) / (reps * layers)
    if int(status.item()) != 0:
        raise SystemExit(f"device status flagged {int(status.item())}")

    kv = L[-1].kv
    seq_len = kv.seq_len.cpu().numpy().astype(np.int64)
    sealed = kv.sealed.cpu().numpy().astype(np.int64)
    cnt = counts.cpu().numpy().astype(np.int64)
    tail = seq_len - sealed * PAGE
    tok_bytes = 2 * D * 2
    att_bytes = int(cnt.sum() * PAGE * tok_bytes + tail.sum() * HKV * tok_bytes + B * HQ * D * 4 * 2 + cnt.sum() * 4)
    rep_bytes = int(sealed.sum() * HKV * D * 4)
    append_bytes = B * HKV * D * 2 * (4 + 2)
    layer_bytes = att_bytes + rep_bytes + append_bytes
    achieved = att_bytes / (kernel_us * 1e-6) / 1e9
    log(f"layer {us_per_layer:.1f} us (append {app:.1f} / select {sel:.1f} / attention {att:.1f}); attention "
        f"back-to-back {kernel_us:.1f} us = {achieved:.0f} GB/s over {att_bytes / 1e9:.2f} GB")

    parity = check(sa, np, torch, L[-1], selected, counts, out, budgets, sel_stride, INIT, LOCAL, scale, s_last,
                   args.check_seqs, klass, chunk, max_chunks, splits, workspace, status)
    cpu = None if args.no_cpu_baseline else cpu_baseline(np, torch, L[0], budgets, sel_stride, INIT, LOCAL, scale)
    kernel = "sparse_decode_attention_kernel<2>"
    line = {
        "metric": "mixed-length sparse decode µs/layer + achieved HBM GB/s (Qwen3-0.6B shape, B=128, "
                  "contexts 1K-64K, budgets 512/2048/full)",
        "value": round(us_per_layer, 3), "unit": "us/layer", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16 KV, fp32 math",
        "data": "synthetic (seeded N(0,1) FP16 KV, 1% of tokens +-60000, fragmented shared page pool)",
        "config": {"workload": "mixed-length decode step: append+seal, score+select under per-sequence budgets, "
                               "chunked sparse GQA attention", "layers": layers, "batch": B, "query_heads": HQ,
                   "kv_heads": HKV, "head_dim": D, "context_min": int(lengths.min()),
                   "context_max": int(lengths.max()), "context_mean": float(lengths.mean()),
                   "budget_blocks": {"16": int((klass == 0).sum()), "64": int((klass == 1).sum()),
                                     "full": int((klass == 2).sum())},
                   "init_blocks": INIT, "local_blocks": LOCAL, "chunk_pages": chunk, "max_chunks": max_chunks,
                   "splits": splits, "selection": select_mode},
        "tokens_per_s": round(B / (ms_per_step * 1e-3), 1),
        "achieved_layer_hbm_gbps": round(layer_bytes / (us_per_layer * 1e-6) / 1e9, 1),
        "kernels_us": {"attention": round(kernel_us, 3), "attention_in_step": round(att, 3),
                       "score_select": round(sel, 3), "append_seal": round(app, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(kernel, chunk),
                     "kernel": kernel,
                     "algorithmic_bytes": att_bytes, "launch_us": round(kernel_us, 3)},
        "parity": parity, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def measured_traffic(kernel, chunk):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary of this workload (128-page chunks); None for other schedules."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "attention_chunked_stress-b128-mixed.traffic.json")
    if chunk != 128 or not os.path.exists(path):
        return None
    with open(path) as f:
        entry = json.load(f).get("kernels", {}).get(kernel)
    return None if entry is None else entry.get("traffic_bytes_per_launch")


def _host_pages(np, torch, kv, seqs):
    """The pages of `seqs` copied to the host, with their tables remapped."""
    seq_len = kv.seq_len[seqs].cpu().numpy()
    npages = int((seq_len.max() + PAGE - 1) // PAGE)
    table = kv.block_table[seqs].cpu().numpy()[:, :npages]
    used = np.unique(table[table >= 0])
    pool = kv.pool.view(torch.int16)[torch.from_numpy(used).cuda().long()].cpu().numpy().view(np.uint16)
    lookup = np.zeros(int(used.max()) + 1, np.int32)
    lookup[used] = np.arange(used.size, dtype=np.int32)
    table_l = np.where(table >= 0, lookup[np.maximum(table, 0)], 0).astype(np.int32)
    return pool, np.ascontiguousarray(table_l), seq_len


def check(sa, np, torch, ly, selected, counts, out, budgets, sel_stride, init, local, scale, s, n_check, klass,
          chunk, max_chunks, splits, workspace, status):
    """Full-size spot check on the last layer (n_check 0 skips it): the
    longest and the shortest sequence and the first of each budget class,
    selection bit-exact and
    attention within 2e-3 of the oracle; full-budget sequences also within
    2e-3 of dense attention over every token."""
    import oracle as O
    if n_check <= 0:
        return None
    kv = ly.kv
    seq_all = kv.seq_len.cpu().numpy()
    picks = [int(np.argmax(seq_all)), int(np.argmin(seq_all))]
    for c in range(3):
        idx = np.nonzero(klass == c)[0]
        if idx.size:
            picks.append(int(idx[0]))
    picks = sorted(set(picks))
    q = ly.q[s][picks].cpu().numpy()
    sealed = kv.sealed[picks].cpu().numpy()
    reps = np.ascontiguousarray(kv.reps[picks].cpu().numpy())
    got_sel = selected[picks].cpu().numpy()
    got_cnt = counts[picks].cpu().numpy()
    got = out[picks].cpu().numpy()
    pool, table_l, seq_len = _host_pages(np, torch, kv, picks)
    sel_ok, att_err, dense_err = True, 0.0, 0.0
    att_ok, dense_ok = True, True
    n = len(picks)
    esel = np.full((n, ly.hkv, sel_stride), -1, np.int32)
    ecnt = np.zeros((n, ly.hkv), np.int32)
    for i, b in enumerate(picks):
        s_, c_ = O.paged_score_select(q[i:i + 1], reps[i:i + 1], sealed[i:i + 1], 1, ly.hq, ly.hkv, D,
                                      kv.rep_heads, kv.rep_stride, ly.hkv, int(budgets[b]), init, local,
                                      sel_stride=sel_stride)
        esel[i], ecnt[i] = s_[0], c_[0]
    sel_ok = bool(np.array_equal(got_cnt, ecnt)) and all(
        np.array_equal(got_sel[i, g, : ecnt[i, g]], esel[i, g, : ecnt[i, g]]) for i in range(n) for g in range(ly.hkv))
    expect = O.paged_sparse_attention(pool, PAGE, table_l, seq_len, sealed, esel, ecnt, ly.hkv, q, n, ly.hq, ly.hkv,
                                      D, scale)
    err = np.abs(got.astype(np.float64) - expect)
    att_ok = bool(((err <= 2e-3) | (err <= 2e-3 * np.abs(expect))).all()) and bool(np.isfinite(got).all())
    att_err = float(err.max())
    full = [i for i, b in enumerate(picks) if klass[b] == 2]
    for i in full:
        ntok = int(seq_len[i])
        pages = [pool[table_l[i, p]].reshape(PAGE, -1) for p in range((ntok + PAGE - 1) // PAGE)]
        dense = O.attention_reference(np.concatenate(pages)[:ntok].ravel(), q[i], ntok, ly.hq, ly.hkv, D, scale)
        e = np.abs(got[i].astype(np.float64) - dense)
        dense_ok = dense_ok and bool(((e <= 2e-3) | (e <= 2e-3 * np.abs(dense))).all())
        dense_err = max(dense_err, float(e.max()))
    return {"sequences": picks, "contexts": [int(x) for x in seq_len], "selection_bit_exact": sel_ok,
            "attention_within_2e-3": att_ok, "attention_max_abs_err": att_err,
            "full_budget_sequences": len(full), "full_budget_equals_dense_within_2e-3": dense_ok,
            "dense_max_abs_err": dense_err}


def cpu_baseline(np, torch, ly, budgets, sel_stride, init, local, scale):
    """The oracle's restatement of the reference CPU path (score + select +
    pack + attention per (sequence, KV group)), one thread, on every 16th
    sequence of one layer (8 of 128: a mix of contexts and budgets), scaled
    by 16 to the full batch."""
    import oracle as O
    kv = ly.kv
    picks = list(range(0, ly.batch, 16))
    q = ly.q[0][picks].cpu().numpy()
    sealed = kv.sealed[picks].cpu().numpy()
    reps = np.ascontiguousarray(kv.reps[picks].cpu().numpy())
    pool, table_l, seq_len = _host_pages(np, torch, kv, picks)
    n = len(picks)
    t0 = time.perf_counter()
    loops = 0
    while True:
        for i, b in enumerate(picks):
            s_, c_ = O.paged_score_select(q[i:i + 1], reps[i:i + 1], sealed[i:i + 1], 1, ly.hq, ly.hkv, D,
                                          kv.rep_heads, kv.rep_stride, ly.hkv, int(budgets[b]), init, local,
                                          sel_stride=sel_stride)
            O.paged_sparse_attention(pool, PAGE, table_l[i:i + 1], seq_len[i:i + 1], sealed[i:i + 1], s_, c_,
                                     ly.hkv, q[i:i + 1], 1, ly.hq, ly.hkv, D, scale)
        loops += 1
        el = time.perf_counter() - t0
        if el > 10.0 or loops >= 100:
            break
    per_layer_us = el / loops * (ly.batch / n) * 1e6
    return {"value": round(per_layer_us, 1), "unit": "us/layer", "cores": 1, "kind": "port",
            "sample": f"every 16th sequence ({n} of {ly.batch}, contexts {int(seq_len.min())}..{int(seq_len.max())}) "
                      f"of one layer x {loops} repeats (score+select+gather+attention per KV group, oracle C "
                      f"restatement, 1 thread), scaled by {ly.batch // n}",
            "nproc": os.cpu_count()}
