#!/usr/bin/env python3
"""Decode-step benchmark of the KV-cache hot path on one MI355X.

Workload (default): Qwen3-0.6B attention shape, 28 layers, batch 64
sequences of 16384 tokens, FP16 KV in a paged HBM pool (32-token pages,
block tables randomly permuted per sequence), budget 64 blocks per KV group
(4 init + 8 local + 52 dynamic), 8 planted high-score blocks per (sequence,
KV head).  A step = for each layer: append one K/V token per sequence (+seal
and representative update when a page fills), score + select per KV group,
sparse GQA decode attention over the selected blocks plus the tail.

Prints one JSON line: µs/layer (value), tokens/s, achieved HBM GB/s of the
decode-step kernel against MI355X peak (with a measured page-copy bandwidth
beside it), and the CPU baseline (the reference's own CPU functions, compiled from
its sources, timed on a bounded sample).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "solidattention-repro_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
PAGE = 32
D = 128

METRICS = {
    "qwen3-0.6b-b64-16k": "sparse decode-attn µs/layer + achieved HBM GB/s (Qwen3-0.6B shape, B=64, 16K)",
    "qwen3-8b-b32-32k": "sparse decode-attn µs/layer + achieved HBM GB/s (Qwen3-8B shape, B=32, 32K)",
}

CONFIGS = {
    # name: (layers, batch, query_heads, kv_heads, context, budget, init, local, planted, model)
    "qwen3-0.6b-b64-16k": (28, 64, 16, 8, 16384, 64, 4, 8, 8, "Qwen3-0.6B"),
    "qwen3-8b-b32-32k": (36, 32, 32, 8, 32768, 64, 4, 8, 8, "Qwen3-8B"),
}
# key channels scaled up in every key (pool, planted blocks, appended tokens):
# (channels, factor), the post-RoPE key outliers of the Qwen3-8B shape
KEY_OUTLIERS = {"qwen3-8b-b32-32k": (4, 8.0)}
# the generator of fill_synthetic_*: an Irwin-Hall(4) sum of four 16-bit
# uniforms, centred and scaled to unit variance (bounded at +-3.46)
GENERATOR = "Irwin-Hall(4) approximately normal, mean 0, variance 1, bounded at +-3.46"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=8)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="qwen3-0.6b-b64-16k", choices=sorted(CONFIGS))
    ap.add_argument("--layers", type=int, default=None, help="override the layer count")
    ap.add_argument("--splits", type=int, default=0, help="attention splits per (seq, KV head); 0 = library default")
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-seqs", type=int, default=0, help="sequences in the CPU sample (0 = auto)")
    ap.add_argument("--check-seqs", type=int, default=2, help="sequences parity-checked against the oracle")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches only (no HIP graph replay)")
    ap.add_argument("--launches", type=int, default=1, choices=[1, 2, 3],
                    help="kernel launches per layer: 1 = the fused decode step (append + seal + select + attend), "
                         "2 = append_seal then the fused select + attend, 3 = append_seal, score_select, attention "
                         "(1 and 2 fall back to 3 where the fused kernel does not apply)")
    ap.add_argument("--prefetch-blocks", type=int, default=128,
                    help="store workload: blocks per store -> pool prefetch batch")
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "correction", "represent", "stress", "store", "layer", "shared", "head_dim"],
                    help="decode: the headline decode step; correction: long-context miss correction "
                         "(Qwen3-8B shape, B=8, 128K context, 128-block budget, ~75%% history coverage); "
                         "represent: InfLLM prefill representatives (16K-token prompt, window 32, top 4); "
                         "stress: B=128 mixed contexts 1K-64K, budgets 512/2048/full, +-60000 outliers; "
                         "store: seal writeback behind decoding and store -> pool prefetch; "
                         "layer: decode step with its q/k/v producer and o-proj consumer; "
                         "shared: one block set over all heads, 1 sequence x 2048 tokens, one launch vs split; "
                         "head_dim: the decode step and bulk seal at head_dim 64 / 128 / 256")
    ap.add_argument("--select", default="auto", choices=["auto", "single", "split", "chunked"],
                    help="separate selection launch: one workgroup per list, scoring split over 256-block "
                         "workgroups (two launches), lists in chunks of 1024-2048 blocks (one launch), or the default "
                         "(stress workload: chunked; decode workload: the library's preference)")
    ap.add_argument("--chunk", type=int, default=None,
                    help="stress workload: pages per attention chunk (0 = split schedule instead)")
    ap.add_argument("--chunk-grid-order", action="store_true",
                    help="stress workload: chunked attention in grid order (a workspace without room for the "
                         "longest-first schedule)")
    ap.add_argument("--microbatches", type=int, default=1,
                    help="layer workload: the batch in this many parts, each a chain of layers on its own stream")
    ap.add_argument("--separate-producer", action="store_true",
                    help="layer workload: the q/k/v producer as its own call before the decode step (else the "
                         "decode step runs the producer's epilogue: sa_hip_decode_step_qkv)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="PAGES",
                    help="also run one plain page copy of PAGES pages (HBM counter calibration)")
    return ap.parse_args()


class Layer:
    """One layer's device state: paged pool, tables, representatives, and the
    per-step inputs (q, new K/V) already resident in HBM."""

    def __init__(self, sa, torch, cfg, layer, args, total_steps):
        layers, batch, hq, hkv, ctx, budget, init, local, planted, _ = cfg
        self.batch, self.hq, self.hkv = batch, hq, hkv
        table_stride = (ctx + total_steps + PAGE - 1) // PAGE + 1
        num_pages = batch * table_stride
        seed = args.seed + 7919 * layer
        kv = sa.PagedKV(batch, hq, hkv, table_stride, num_pages=num_pages)
        g = torch.Generator(device="cpu")
        g.manual_seed(seed)
        perm = torch.randperm(num_pages, generator=g, dtype=torch.int64).to(torch.int32)
        kv.block_table.copy_(perm.view(batch, table_stride))
        sa.fill_synthetic_f16(kv.pool.view(-1), seed, 0)
        # one query per sequence, held over every step, so that the planted
        # blocks below score high in every timed step (new K/V per step)
        q0 = torch.empty((batch, hq, D), dtype=torch.float32, device="cuda")
        sa.fill_synthetic_f32(q0.view(-1), seed + 1, 0)
        q = q0.unsqueeze(0).expand(total_steps, batch, hq, D)
        knew = torch.empty((total_steps, batch, hkv, D), dtype=torch.float32, device="cuda")
        vnew = torch.empty_like(knew)
        sa.fill_synthetic_f32(knew.view(-1), seed + 2, 0)
        sa.fill_synthetic_f32(vnew.view(-1), seed + 3, 0)
        # planted high-score blocks: keys = 0.5 * mean(q of the group) + 0.5 * noise
        if planted:
            full = ctx // PAGE
            # distinct blocks per (sequence, head): a block drawn twice would be
            # written twice by one index assignment, and which write lands is
            # not defined on the GPU
            blocks = torch.rand((batch, hkv, full), generator=g).argsort(dim=-1)[..., :planted].cuda()
            grp = hq // hkv
            qmean = q0.view(batch, hkv, grp, D).mean(dim=2)  # [B, Hkv, D]
            pool16 = kv.pool.view(torch.float16)  # [pages, 32, 2, Hkv, D]
            noise = torch.empty((batch, hkv, planted, PAGE, D), dtype=torch.float32, device="cuda")
            sa.fill_synthetic_f32(noise.view(-1), seed + 4, 0)
            pages = torch.gather(kv.block_table.to(torch.int64), 1, blocks.view(batch, -1)).view(batch, hkv, planted)
            heads = torch.arange(hkv, device="cuda").view(1, hkv, 1).expand(batch, hkv, planted)
            vals = (0.5 * qmean[:, :, None, None, :] + 0.5 * noise).to(torch.float16)
            pool16[pages.reshape(-1), :, 0, heads.reshape(-1), :] = vals.reshape(-1, PAGE, D)
        outliers = KEY_OUTLIERS.get(getattr(args, "config", None))
        if outliers:
            # every key of the pool and every appended key: the first
            # `channels` channels scaled (exact in FP16: a power of two)
            ch, factor = outliers
            pool16 = kv.pool.view(torch.float16).view(-1, PAGE, 2, hkv, D)
            pool16[:, :, 0, :, :ch] *= factor
            knew[..., :ch] *= factor
        kv.seq_len.fill_(ctx)
        # the prefill's bulk seal: every whole page gets its representative
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        sa.seal(kv, 0)
        e1.record()
        self.seal_events = (e0, e1)
        self.kv, self.q, self.knew, self.vnew = kv, q, knew, vnew
        self.budget, self.init, self.local = budget, init, local
        self.selected = torch.full((batch, hkv, budget), -1, dtype=torch.int32, device="cuda")
        self.counts = torch.zeros((batch, hkv), dtype=torch.int32, device="cuda")
        self.out = torch.empty((batch, hq, D), dtype=torch.float32, device="cuda")


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "the benchmark runs on one GPU: the KV-cache hot path is measured at its "
                                   "real per-GPU shape; --gpus must be 1"}))
        sys.exit(2)
    if args.workload == "correction":
        import bench_correction
        bench_correction.run(args)
        return
    if args.workload == "represent":
        import bench_represent
        bench_represent.run(args)
        return
    if args.workload == "stress":
        import bench_stress
        bench_stress.run(args)
        return
    if args.workload == "store":
        import bench_store
        bench_store.run(args)
        return
    if args.workload == "head_dim":
        import bench_head_dim
        bench_head_dim.run(args)
        return
    if args.workload == "shared":
        import bench_shared
        bench_shared.run(args)
        return
    if args.workload == "layer":
        import bench_layer
        bench_layer.run(args)
        return
    import numpy as np
    import torch

    import solidattention_amd as sa

    cfg = list(CONFIGS[args.config])
    if args.layers:
        cfg[0] = args.layers
    layers, batch, hq, hkv, ctx, budget, init, local, planted, model = cfg
    graph = not args.no_graph
    # eager timed steps, then (graph mode) one capture-warmup step and the
    # graph-replayed timed steps; every step appends one token per layer
    total_steps = args.warmup + args.steps + ((args.steps + 1) if graph else 0)
    torch.cuda.set_device(0)
    log(f"setup {args.config}: layers={layers} batch={batch} ctx={ctx} budget={budget}")
    t0 = time.time()
    L = [Layer(sa, torch, cfg, l, args, total_steps) for l in range(layers)]
    torch.cuda.synchronize()
    log(f"setup done in {time.time() - t0:.1f}s; pool {L[0].kv.pool.numel() * 2 * layers / 2**30:.1f} GiB")

    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    pages_hint = budget + 2
    # the fused launch (splits 1) where it applies and fills the device; the
    # separate attention launch splits its page lists by default_splits
    fused_ok = (args.splits in (0, 1) and sa.select_attend_fused(L[0].kv, hkv, 1, sel_stride=budget)
                and (args.splits == 1 or sa.select_attend_default_splits(L[0].kv, hkv, budget) == 1))
    splits = args.splits or sa.default_splits(batch, hkv, pages_hint, hq)
    ws_bytes = sa.lib().sa_hip_attention_workspace_bytes(batch, hq, hkv, D, splits)
    workspace = torch.zeros(max(ws_bytes // 4, 1), dtype=torch.float32, device="cuda")
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    stream = torch.cuda.current_stream()

    n_ev = total_steps * layers
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(n_ev)]

    launches = args.launches if fused_ok else 3
    if launches < 3:
        splits = 1
    step_ws, _ = sa.decode_step_workspace(L[0].kv, 1)
    split_select = args.select == "split" or (
        args.select == "auto" and sa.score_select_split_preferred(L[0].kv, hkv, budget, init, local))
    scores = (torch.zeros((batch, hkv, L[0].kv.rep_stride), dtype=torch.float32, device="cuda")
              if split_select else None)
    select_ws = (sa.score_select_chunked_workspace(L[0].kv, hkv, budget, init, local)[0]
                 if args.select == "chunked" else None)

    def layer_launches(ly, s, e=None):
        """One layer of one decode step; e = 4 timing events (append, select, attention)."""
        if e: e[0].record(stream)
        if launches == 1:
            sa.decode_step(ly.kv, ly.knew[s], ly.vnew[s], 0, ly.q[s], hkv, budget, init, local, scale, step_ws,
                           selected=ly.selected, counts=ly.counts, out=ly.out, splits=1, status=status)
            if e:
                for x in e[1:]:
                    x.record(stream)
            return
        sa.append_seal(ly.kv, ly.knew[s], ly.vnew[s], 0, status=status)
        if e: e[1].record(stream)
        if launches == 2:
            sa.select_attend(ly.kv, ly.q[s], hkv, budget, init, local, scale, selected=ly.selected,
                             counts=ly.counts, out=ly.out, splits=1, status=status)
            if e: e[2].record(stream)
        else:
            if split_select:
                sa.score_select_split(ly.kv, ly.q[s], hkv, budget, init, local, selected=ly.selected,
                                      counts=ly.counts, scores=scores, status=status)
            elif select_ws is not None:
                sa.score_select_chunked(ly.kv, ly.q[s], hkv, budget, init, local, select_ws, selected=ly.selected,
                                        counts=ly.counts, status=status)
            else:
                sa.score_select(ly.kv, ly.q[s], hkv, budget, init, local, selected=ly.selected, counts=ly.counts,
                                status=status)
            if e: e[2].record(stream)
            sa.sparse_decode_attention(ly.kv, ly.q[s], ly.selected, ly.counts, scale, out=ly.out, splits=splits,
                                       workspace=workspace, status=status)
        if e: e[3].record(stream)

    def step(s, record):
        for l, ly in enumerate(L):
            layer_launches(ly, s, ev[s * layers + l] if record else None)

    if args.calibrate_copy:
        # a plain copy of known size: PAGES x 128 KiB read and written once
        n = args.calibrate_copy
        src_pages = torch.arange(n, dtype=torch.int32, device="cuda")
        dst = torch.empty((n, L[0].kv.page_bytes // 2), dtype=torch.int16, device="cuda").view(torch.uint16)
        sa.gather_pages(L[0].kv.pool, L[0].kv.page_bytes, L[0].kv.num_pages, src_pages, dst)
        torch.cuda.synchronize()
        log(f"calibration copy: {n * L[0].kv.page_bytes} bytes read and written by gather_pages_kernel")
        del dst
    for s in range(args.warmup):
        step(s, record=False)
    torch.cuda.synchronize()
    log("warmup done")
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    eager_first = args.warmup
    start.record(stream)
    for s in range(eager_first, eager_first + args.steps):
        step(s, record=True)
    end.record(stream)
    torch.cuda.synchronize()
    eager_ms = start.elapsed_time(end)
    last_step = eager_first + args.steps - 1
    graph_ms = None
    if graph:
        # one HIP graph per decode step (28 layers x append/select/attention
        # launches); capture records, it does not execute
        first = eager_first + args.steps
        graphs = []
        for s in range(first, first + args.steps + 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step(s, record=False)
            graphs.append(g)
        graphs[0].replay()  # warm replay (step `first`)
        torch.cuda.synchronize()
        gstream = torch.cuda.current_stream()
        start.record(gstream)
        for g in graphs[1:]:
            g.replay()
        end.record(gstream)
        torch.cuda.synchronize()
        graph_ms = start.elapsed_time(end)
        last_step = first + args.steps
    if int(status.item()) != 0:
        raise SystemExit(f"device status flagged {int(status.item())}")
    total_ms = graph_ms if graph else eager_ms
    ms_per_step = total_ms / args.steps
    us_per_layer = ms_per_step * 1000.0 / layers
    app, sel, att = [], [], []
    for s in range(eager_first, eager_first + args.steps):
        for l in range(layers):
            e = ev[s * layers + l]
            app.append(e[0].elapsed_time(e[1]))
            sel.append(e[1].elapsed_time(e[2]))
            att.append(e[2].elapsed_time(e[3]))
    att_us = 1000.0 * sum(att) / len(att)
    sel_us = 1000.0 * sum(sel) / len(sel)
    app_us = 1000.0 * sum(app) / len(app)

    # duration of the dominant kernel for the roofline, from the timed region
    # itself (HIP events on the bench stream).  One launch per layer: the
    # decode-step kernel is the only kernel of the step, so its average launch
    # duration is the timed region over steps x layers launches (graph
    # replay; it includes the dispatch gap between consecutive launches, so
    # it bounds the kernel trace's average from above).  Eager, or two or
    # three launches: the events around each launch of the eager timed steps.
    if launches == 1:
        kernel_us = us_per_layer if graph else app_us
        assert kernel_us * layers <= ms_per_step * 1000.0 * (1 + 1e-9) or not graph
    else:
        kernel_us = sel_us if launches == 2 else att_us

    seal_us = 1000.0 * sum(ly.seal_events[0].elapsed_time(ly.seal_events[1]) for ly in L) / layers
    seal_bytes = batch * (ctx // PAGE) * (PAGE * hkv * D * 2 + hkv * D * 4)
    log(f"prefill bulk seal: {seal_us:.1f} us per layer ({seal_bytes / (seal_us * 1e-6) / 1e9:.0f} GB/s over the "
        f"keys read and representatives written)")
    copy_ref = copy_reference(sa, torch, L[0].kv, args.seed)
    read_ref = read_reference(sa, np, torch, L[-1], hkv)

    # algorithmic bytes of one launch: selected KV + tail KV + q + out + ids,
    # plus the fp32 representatives of every sealed block (select+attend) and
    # the appended token (decode step: fp32 K/V read, FP16 K/V written)
    seq_len = L[-1].kv.seq_len.cpu().numpy().astype(np.int64)
    sealed = L[-1].kv.sealed.cpu().numpy().astype(np.int64)
    counts = L[-1].counts.cpu().numpy().astype(np.int64)
    tail = seq_len - sealed * PAGE
    kv_tok_bytes = 2 * D * 2  # K+V of one KV head, FP16
    att_bytes = int(counts.sum() * PAGE * kv_tok_bytes + (tail.sum() * hkv) * kv_tok_bytes +
                    batch * hq * D * 4 * 2 + counts.sum() * 8)
    rep_bytes = int(sealed.sum() * hkv * D * 4)
    append_bytes = batch * hkv * D * 2 * (4 + 2)
    layer_bytes = att_bytes + rep_bytes + append_bytes
    kernel_bytes = {1: layer_bytes, 2: att_bytes + rep_bytes, 3: att_bytes}[launches]
    achieved = kernel_bytes / (kernel_us * 1e-6) / 1e9
    layer_gbps = layer_bytes / (us_per_layer * 1e-6) / 1e9
    if launches == 1:
        log(f"1 launch per layer: decode step {kernel_us:.2f} us per launch in the timed region ({achieved:.0f} "
            f"GB/s); eager with events around each launch {app_us:.2f} us; layer {us_per_layer:.2f} us")
    else:
        log(f"{launches} launches per layer: dominant kernel {kernel_us:.2f} us per launch ({achieved:.0f} GB/s); "
            f"eager append {app_us:.2f} / select {sel_us:.2f} / attention {att_us:.2f} us; "
            f"layer {us_per_layer:.2f} us")
    log(f"copy reference: gather_pages_kernel {copy_ref['gbps']:.0f} GB/s over {copy_ref['bytes']} bytes")
    log(f"read reference: read_step_bytes_kernel {read_ref['gbps']:.0f} GB/s over {read_ref['bytes']} bytes")
    grp = hq // hkv
    if grp == 4:  # the LDS-staged one-launch kernel (4 query heads per KV head)
        kernel_name = {1: "decode_kernel_staged<4,true,false,false>", 2: "decode_kernel_staged<4,false,false,false>",
                       3: "sparse_decode_attention_kernel<4>"}[launches]
    else:
        kernel_name = {1: f"decode_kernel<{grp},{grp},true,false,false>", 2: f"decode_kernel<{grp},{grp},false,false,false>",
                       3: f"sparse_decode_attention_kernel<{grp}>"}[launches]
    traffic, traffic_run = measured_traffic(args.config, kernel_name)

    parity = check_parity(sa, np, torch, L[-1], args, scale, hkv, budget, init, local, last_step)
    cpu = None if args.no_cpu_baseline else cpu_baseline(np, torch, L[0], args, budget, init, local, scale)

    line = {
        "metric": METRICS[args.config],
        "value": round(us_per_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 KV, fp32 math",
        "data": f"synthetic: seeded FP16 KV and fp32 queries from the {GENERATOR} generator, one query per "
                f"sequence held over the steps, {planted} planted high-score blocks per (sequence, KV head) "
                "against it, new K/V every step, randomly permuted page tables"
                + ("" if not KEY_OUTLIERS.get(args.config) else
                   f", keys with {KEY_OUTLIERS[args.config][0]} of 128 channels scaled x"
                   f"{KEY_OUTLIERS[args.config][1]:g} (pool and appended tokens)"),
        "config": {"workload": f"{model} attention shape decode step: append+seal, score+select, sparse GQA "
                               f"attention", "layers": layers, "batch": batch, "query_heads": hq,
                   "kv_heads": hkv, "head_dim": D, "context": ctx, "budget_blocks": budget,
                   "init_blocks": init, "local_blocks": local, "page_tokens": PAGE, "splits": splits,
                   "launches_per_layer": launches,
                   "selection": None if launches < 3 else ("split" if split_select else
                                                          "chunked" if select_ws is not None else "single")},
        "tokens_per_s": round(batch / (ms_per_step * 1e-3), 1),
        "launch": "hip graph per decode step" if graph else "eager",
        "eager_us_per_layer": round(eager_ms * 1000.0 / args.steps / layers, 3),
        "achieved_layer_hbm_gbps": round(layer_gbps, 1),
        "prefill_seal": {"us_per_layer": round(seal_us, 1), "bytes_per_layer": seal_bytes,
                         "gbps": round(seal_bytes / (seal_us * 1e-6) / 1e9, 1)},
        "kernels_us": ({"decode_step": round(kernel_us, 3), "decode_step_eager": round(app_us, 3)}
                       if launches == 1 else
                       {"select_attend": round(kernel_us, 3), "select_attend_in_step": round(sel_us, 3),
                        "append_seal": round(app_us, 3)} if launches == 2 else
                       {"attention": round(kernel_us, 3), "attention_in_step": round(att_us, 3),
                        "score_select": round(sel_us, 3), "append_seal": round(app_us, 3)}),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic, "traffic_run": traffic_run,
                     "kernel": kernel_name, "algorithmic_bytes": kernel_bytes,
                     "launch_us": round(kernel_us, 3),
                     "launch_timing": ("graph-replayed timed region / (steps x layers)" if launches == 1 and graph
                                       else "events around each launch in the eager timed steps"),
                     "copy_reference": copy_ref, "read_reference": read_ref,
                     "frac_of_read_reference": round(achieved / read_ref["gbps"], 4)},
        "parity": parity,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def read_reference(sa, np, torch, ly, hkv, reps=5):
    """A measured bandwidth reference on the decode step's own access
    pattern: read_step_bytes_kernel reads, for every (sequence, KV head) of
    the layer's last step, the representatives of the sealed blocks, the K/V
    slices of the selected pages and the tail, with no arithmetic but an XOR
    of the words read, timed with HIP events over `reps` launches on the
    bench stream.  Its rate is what the memory system gives this pattern of
    reads; the decode step's rate over it says how much the kernel's own
    structure costs."""
    kv = ly.kv
    out = sa.read_step_bytes(kv, ly.selected, ly.counts, hkv)  # warm
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        sa.read_step_bytes(kv, ly.selected, ly.counts, hkv, out=out)
    end.record(stream)
    torch.cuda.synchronize()
    us = 1000.0 * start.elapsed_time(end) / reps
    seq_len = kv.seq_len.cpu().numpy().astype(np.int64)
    sealed = kv.sealed.cpu().numpy().astype(np.int64)
    counts = np.minimum(ly.counts.cpu().numpy().astype(np.int64), ly.selected.shape[-1])
    kv_tok_bytes = 2 * D * 2  # K+V of one KV head, FP16
    nbytes = int(sealed.sum() * kv.rep_heads * D * 4 + counts.sum() * PAGE * kv_tok_bytes +
                 (seq_len - sealed * PAGE).sum() * hkv * kv_tok_bytes)
    gbps = nbytes / (us * 1e-6) / 1e9
    return {"kernel": "read_step_bytes_kernel",
            "what": "the layer's representatives, selected page slices and tails read with no arithmetic",
            "bytes": nbytes, "us": round(us, 2), "gbps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4)}


def copy_reference(sa, torch, kv, seed, pages=4096, reps=5):
    """A measured bandwidth reference on the same pool: gather_pages_kernel
    copying `pages` whole 128 KiB pages, drawn in random order from the pool,
    into a contiguous buffer (each byte read once and written once), timed
    with HIP events over `reps` launches on the bench stream.  A copy mixes
    reads and writes, so a read-dominated kernel can exceed it: it is a
    reference point on the same box, not a ceiling."""
    n = min(pages, int(kv.num_pages))
    g = torch.Generator(device="cpu")
    g.manual_seed(seed + 17)
    src = torch.randperm(int(kv.num_pages), generator=g)[:n].to(torch.int32).cuda()
    dst = torch.empty((n, kv.page_bytes // 2), dtype=torch.int16, device="cuda").view(torch.uint16)
    sa.gather_pages(kv.pool, kv.page_bytes, kv.num_pages, src, dst)  # warm
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        sa.gather_pages(kv.pool, kv.page_bytes, kv.num_pages, src, dst)
    end.record(stream)
    torch.cuda.synchronize()
    us = 1000.0 * start.elapsed_time(end) / reps
    nbytes = 2 * n * kv.page_bytes
    del dst
    return {"kernel": "gather_pages_kernel", "what": f"copy of {n} random pool pages (read + write)",
            "bytes": nbytes, "us": round(us, 2), "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}


def measured_traffic(config, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary for this workload (FETCH_SIZE scaled by the copy-kernel
    calibration, plus WRITE_SIZE), and that counter run's own algorithmic
    bytes per launch and their ratio (the counter run is a short run of its
    own, whose steps hold slightly different tails than this run's last
    step); (None, None) when no summary matches."""
    path = os.path.join(ROOT, "profiles", f"decode_step_{config}.traffic.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        entry = json.load(f).get("kernels", {}).get(kernel)
    if entry is None:
        return None, None
    return entry.get("traffic_bytes_per_launch"), {
        "algorithmic_bytes_per_launch": entry.get("algorithmic_bytes_per_launch"),
        "traffic_over_algorithmic": entry.get("traffic_over_algorithmic"),
        "source": os.path.relpath(path, ROOT)}


def check_parity(sa, np, torch, ly, args, scale, hkv, budget, init, local, s):
    """Full-size spot check: for a few sequences of the last layer, the selection
    (bit-exact) and attention (2e-3) against the oracle on the device bytes."""
    import oracle as O
    n = min(args.check_seqs, ly.batch)
    if n <= 0:
        return None
    kv = ly.kv
    seqs = list(range(n))
    table = kv.block_table[seqs].cpu().numpy()
    seq_len = kv.seq_len[seqs].cpu().numpy()
    sealed = kv.sealed[seqs].cpu().numpy()
    used = np.unique(table[:, : int(((seq_len.max() + PAGE - 1) // PAGE))])
    pool = kv.pool.view(torch.int16)[torch.from_numpy(used).cuda().long()].cpu().numpy().view(np.uint16)
    remap = {int(p): i for i, p in enumerate(used)}
    table_l = np.vectorize(lambda p: remap.get(int(p), 0))(table).astype(np.int32)
    reps = kv.reps[seqs].cpu().numpy()
    q = ly.q[s][seqs].cpu().numpy()
    esel, ecnt = O.paged_score_select(q, reps, sealed, n, ly.hq, hkv, D, kv.rep_heads, kv.rep_stride, hkv, budget,
                                      init, local)
    got_sel = ly.selected[seqs].cpu().numpy()
    got_cnt = ly.counts[seqs].cpu().numpy()
    sel_ok = bool(np.array_equal(got_cnt, ecnt)) and all(
        np.array_equal(got_sel[b, g, : ecnt[b, g]], esel[b, g, : ecnt[b, g]]) for b in range(n) for g in range(hkv))
    expect = O.paged_sparse_attention(pool, PAGE, table_l, seq_len, sealed, esel, ecnt, hkv, q, n, ly.hq, hkv, D,
                                      scale)
    got = ly.out[seqs].cpu().numpy()
    err = np.abs(got.astype(np.float64) - expect)
    att_ok = bool(((err <= 2e-3) | (err <= 2e-3 * np.abs(expect))).all())
    return {"sequences": n, "selection_bit_exact": sel_ok, "attention_within_2e-3": att_ok,
            "attention_max_abs_err": float(err.max())}


def cpu_baseline(np, torch, ly, args, budget, init, local, scale):
    """The reference CPU path on a bounded sample of sequences of the same
    workload, reported per layer of the full batch by scaling with batch /
    sample: on one thread (as the reference runs), and with one thread per
    sequence over the host's cores.  Per (sequence, KV group) it runs the
    reference's select_shared_blocks (cpp/src/selection.cpp:96-147) over the
    group's query heads, packs the selected blocks of that KV head plus the
    tail contiguously (the placement of read_blocks_fixed,
    uring_reader.cpp:87-95) and runs its attention_reference
    (cpp/src/attention_reference.cpp:55-96).  kind "reference": the
    reference's own functions compiled from its sources (oracle/_ref);
    kind "port": the oracle's bit-identical C restatement where oracle/_ref
    was not built.  ctypes releases the interpreter lock during each call."""
    from concurrent.futures import ThreadPoolExecutor

    import oracle as O
    use_ref = O.ref_available()
    kv = ly.kv
    batch, hq, hkv = ly.batch, ly.hq, ly.hkv
    grp = hq // hkv
    threads = max(1, min(len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count(),
                         16, batch))
    n = args.cpu_sample_seqs or threads
    seqs = list(range(n))
    table = kv.block_table[seqs].cpu().numpy()
    seq_len = kv.seq_len[seqs].cpu().numpy()
    sealed = kv.sealed[seqs].cpu().numpy()
    used = np.unique(table[:, : int(((seq_len.max() + PAGE - 1) // PAGE))])
    pool = kv.pool.view(torch.int16)[torch.from_numpy(used).cuda().long()].cpu().numpy().view(np.uint16)
    lookup = np.zeros(int(used.max()) + 1, np.int32)
    lookup[used] = np.arange(used.size, dtype=np.int32)
    table_l = np.ascontiguousarray(lookup[np.clip(table, 0, used.max())].astype(np.int32))
    reps = kv.reps[seqs].cpu().numpy()  # [n][rep_heads][D][rep_stride]
    q = np.ascontiguousarray(ly.q[0][seqs].cpu().numpy())
    gpu_sel = ly.selected[seqs].cpu().numpy()
    gpu_cnt = ly.counts[seqs].cpu().numpy()
    # the reference's representative layout, [query head][block][D] per group
    # (a layout change done once, outside the timed region)
    rep_g = {}
    for b in range(n):
        nb = int(sealed[b])
        for g in range(hkv):
            rows = [reps[b, g if kv.rep_heads == hkv else g * grp + j, :, :nb].T for j in range(grp)]
            rep_g[b, g] = np.ascontiguousarray(np.stack(rows), dtype=np.float32)
    q_g = {(b, g): np.ascontiguousarray(q[b, g * grp:(g + 1) * grp]) for b in range(n) for g in range(hkv)}

    def unit(b, g):
        nb = int(sealed[b])
        ids, _ = O.select_shared_blocks(q_g[b, g], rep_g[b, g], grp, nb, D, budget, init, local, use_ref=use_ref)
        tail = int(seq_len[b]) - nb * PAGE
        tokens = len(ids) * PAGE + tail
        packed = np.empty((tokens, 2, 1, D), np.uint16)
        packed[: len(ids) * PAGE] = pool[table_l[b, ids], :, :, g:g + 1, :].reshape(-1, 2, 1, D)
        if tail:
            tp = pool[table_l[b, nb:nb + (tail + PAGE - 1) // PAGE], :, :, g:g + 1, :].reshape(-1, 2, 1, D)
            packed[len(ids) * PAGE:] = tp[:tail]
        O.attention_reference(packed, q_g[b, g], tokens, grp, 1, D, scale, use_ref=use_ref)
        return ids

    # cross-check: the reference's ids for the sample equal the GPU's selection
    ids_equal = all(unit(b, g).tolist() == gpu_sel[b, g, : gpu_cnt[b, g]].tolist()
                    for b in range(min(n, 2)) for g in range(hkv))

    def one(b):
        for g in range(hkv):
            unit(b, g)

    # one thread: the first two sequences, repeated for ~10 s at most
    t0 = time.perf_counter()
    loops = 0
    while True:
        one(0)
        one(1 % n)
        loops += 1
        el = time.perf_counter() - t0
        if el > 10.0 or loops >= 1000:
            break
    single_us = el / (2 * loops) * batch * 1e6
    # every core: the n sequences at once, repeated for ~5 s at most
    with ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(one, range(n)))  # warm
        t0 = time.perf_counter()
        rounds = 0
        while True:
            list(ex.map(one, range(n)))
            rounds += 1
            el = time.perf_counter() - t0
            if el > 5.0 or rounds >= 200:
                break
    multi_us = el / (rounds * n) * batch * 1e6
    what = ("the reference's select_shared_blocks + pack + attention_reference (oracle/_ref, built from its "
            "sources)" if use_ref else "the oracle's C restatement of select_shared_blocks + pack + "
            "attention_reference")
    return {"value": round(multi_us, 1), "unit": "us/layer", "cores": threads,
            "kind": "reference" if use_ref else "port",
            "sample": f"{n} of {batch} sequences of one layer (all {hkv} KV groups each), one per thread on "
                      f"{threads} threads, x {rounds} rounds, scaled to {batch} sequences; per group: {what}",
            "single_thread": {"value": round(single_us, 1), "cores": 1,
                              "sample": f"2 sequences x {loops} repeats on one thread, scaled to {batch}"},
            "ids_equal_gpu_selection": bool(ids_equal),
            "host_cpu": _cpu_model(), "nproc": os.cpu_count()}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    main()
