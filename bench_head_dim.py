"""Head-dimension workload (bench.py --workload head_dim).

The decode step and the prefill's bulk seal of the Qwen3-0.6B attention
shape (16 query / 8 KV heads, batch 64, 16384-token contexts, budget 64 =
init 4 + local 8 + 52) at head_dim 64, 128 and 256: 128 runs the tuned
one-launch step, the others the general kernels in sequence (append + seal,
scoring, selection, token-row attention).  Each head_dim builds its own pool
(synthetic FP16 keys and values in a randomly permuted page table), seals
it, then times `steps` decode steps eagerly and `steps` more as one HIP graph
(HIP events around the timed steps; every step appends one token).  Reported per head_dim: µs per step (graphs; eager beside it) and the
algorithmic bytes rate (representatives + selected pages), the bulk seal's
time, and the status word.
"""
from __future__ import annotations

import json
import sys

PAGE = 32


def log(msg):
    print(f"[head_dim] {msg}", file=sys.stderr, flush=True)


def run(args):
    import numpy as np
    import torch

    import bench
    import solidattention_amd as sa

    batch, hq, hkv, ctx, budget, init, local = 64, 16, 8, 16384, 64, 4, 8
    steps, warmup = args.steps, args.warmup
    torch.cuda.set_device(0)
    results = {}
    for d in (64, 128, 256):
        ts = (ctx + 3 * steps + warmup + PAGE - 1) // PAGE + 2
        kv = sa.PagedKV(batch, hq, hkv, ts, num_pages=batch * ts, head_dim=d)
        g = torch.Generator(device="cpu")
        g.manual_seed(args.seed + d)
        kv.block_table.copy_(torch.randperm(batch * ts, generator=g, dtype=torch.int64).to(torch.int32).view(batch, ts))
        sa.fill_synthetic_f16(kv.pool.view(-1), args.seed + d, 0)
        kv.seq_len.fill_(ctx)
        q = torch.empty((batch, hq, d), dtype=torch.float32, device="cuda")
        sa.fill_synthetic_f32(q.view(-1), args.seed + d + 1, 0)
        k = torch.empty((2 * steps + warmup, batch, hkv, d), dtype=torch.float32, device="cuda")
        v = torch.empty_like(k)
        sa.fill_synthetic_f32(k.view(-1), args.seed + d + 2, 0)
        sa.fill_synthetic_f32(v.view(-1), args.seed + d + 3, 0)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        sa.seal(kv, 0)
        e1.record()
        torch.cuda.synchronize()
        seal_us = 1000.0 * e0.elapsed_time(e1)
        splits = sa.select_attend_default_splits(kv, hkv, budget)
        ws, _ = sa.decode_step_workspace(kv, splits)
        st = torch.zeros(1, dtype=torch.int32, device="cuda")
        sel = torch.full((batch, hkv, budget), -1, dtype=torch.int32, device="cuda")
        cnt = torch.zeros((batch, hkv), dtype=torch.int32, device="cuda")
        out = torch.empty((batch, hq, d), dtype=torch.float32, device="cuda")
        scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))

        def step(s):
            sa.decode_step(kv, k[s], v[s], 0, q, hkv, budget, init, local, scale, ws, selected=sel, counts=cnt,
                           out=out, splits=splits, status=st)

        for s in range(warmup):
            step(s)
        torch.cuda.synchronize()
        # eager steps, then the same number of steps as one HIP graph (every
        # step appends its own token; the graph is replayed once to warm up)
        e0.record()
        for s in range(warmup, warmup + steps):
            step(s)
        e1.record()
        torch.cuda.synchronize()
        eager_us = 1000.0 * e0.elapsed_time(e1) / steps
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for s in range(warmup + steps, warmup + 2 * steps):
                step(s)
        gr.replay()  # warm replay
        torch.cuda.synchronize()
        e0.record()
        gr.replay()
        e1.record()
        torch.cuda.synchronize()
        us = 1000.0 * e0.elapsed_time(e1) / steps
        del gr
        blocks = ctx // PAGE
        alg = batch * hkv * (blocks * d * 4 + budget * PAGE * 2 * d * 2)
        results[str(d)] = {
            "us_per_step": round(us, 2),
            "eager_us_per_step": round(eager_us, 2),
            "algorithmic_gbps": round(alg / us / 1e3, 1),
            "fused_one_launch": bool(sa.select_attend_fused(kv, hkv, splits, sel_stride=budget)),
            "bulk_seal_us": round(seal_us, 1),
            "status": int(st.item()),
        }
        log(f"head_dim {d}: {results[str(d)]}")
        del kv, k, v, ws
        torch.cuda.empty_cache()
    line = {
        "metric": "decode step µs/layer by head_dim (Qwen3-0.6B heads, B=64, 16K)",
        "value": results["64"]["us_per_step"],
        "unit": "us/layer",
        "higher_is_better": False,
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "dtype": "fp16 KV, fp32 math",
        "data": f"synthetic ({bench.GENERATOR}), randomly permuted page tables",
        "config": {"workload": "decode step at head_dim 64 / 128 / 256", "batch": batch, "heads": f"{hq}/{hkv}",
                   "context": ctx, "budget": f"{init} + {local} + {budget - init - local}",
                   "timing": "one HIP graph of the timed steps, events around its replay (eager_us_per_step: "
                             "the same number of eager steps)"},
        "by_head_dim": results,
    }
    print(json.dumps(line), flush=True)
    if any(r["status"] for r in results.values()):
        raise SystemExit("device status flagged")
