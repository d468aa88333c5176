"""Shared-selection workload (bench.py --workload shared).

The reference's single-sequence shared case (one block set over all 16 query
heads, budget 16 = init 1 + local 2 + 13 dynamic; selection_main.cpp:178-181,
pipeline_main.cpp:480-499) as a decode loop: Qwen3-0.6B heads (16 query / 8
KV, head_dim 128), 28 layers, one sequence with a 2048-token context (64
blocks, 4 planted blocks per KV head), one token appended per layer and step.

Timed two ways, each on its own copy of the same state and as HIP graphs of
whole decode steps:
  * one launch per layer (decode_kernel_shared: every workgroup of the
    sequence scores the whole shared set, selects, and attends its KV head);
  * the split launches (append + seal, score + select, attention + merge).
Reported: µs per layer-step of each, and, on the last step, the two paths'
ids equal, their outputs within fp32 rounding, and their states (pool,
representatives, counters) equal bit for bit.  Parity with the oracle is in
tests/test_gpu_shared_step.py.
"""
from __future__ import annotations

import json
import sys
import time

D = 128


def log(msg):
    print(f"[shared] {msg}", file=sys.stderr, flush=True)


def run(args):
    import numpy as np
    import torch

    import bench
    import solidattention_amd as sa

    layers = args.layers or 28
    batch, hq, hkv, ctx, budget, init, local, planted = 1, 16, 8, 2048, 16, 1, 2, 4
    cfg = [layers, batch, hq, hkv, ctx, budget, init, local, planted, "Qwen3-0.6B"]
    steps, warmup = args.steps, args.warmup
    total_steps = warmup + steps + 1
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream()
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    results = {}
    for mode, splits in (("one_launch", 1), ("split_launches", 2)):
        L = [bench.Layer(sa, torch, cfg, l, args, total_steps) for l in range(layers)]
        fused = sa.select_attend_fused(L[0].kv, 1, splits, sel_stride=budget)
        assert fused == (splits == 1), (mode, fused)
        ws, _ = sa.decode_step_workspace(L[0].kv, splits)
        sel = torch.full((layers, batch, 1, budget), -1, dtype=torch.int32, device="cuda")
        cnt = torch.zeros((layers, batch, 1), dtype=torch.int32, device="cuda")
        out = torch.empty((layers, batch, hq, D), dtype=torch.float32, device="cuda")

        def step(s):
            for l, ly in enumerate(L):
                sa.decode_step(ly.kv, ly.knew[s], ly.vnew[s], 0, ly.q[s], 1, budget, init, local, scale, ws,
                               selected=sel[l], counts=cnt[l], out=out[l], splits=splits, status=status)

        for s in range(warmup):
            step(s)
        torch.cuda.synchronize()
        graphs = []
        for s in range(warmup, warmup + steps + 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step(s)
            graphs.append(g)
        graphs[0].replay()  # warm replay
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for g in graphs[1:]:
            g.replay()
        end.record(stream)
        torch.cuda.synchronize()
        ms = start.elapsed_time(end)
        if int(status.item()) != 0:
            raise SystemExit(f"{mode}: device status flagged {int(status.item())}")
        results[mode] = {
            "us_per_layer": 1000.0 * ms / (steps * layers),
            "sel": sel.cpu().numpy(), "cnt": cnt.cpu().numpy(), "out": out.cpu().numpy(),
            "state": [(ly.kv.pool.clone(), ly.kv.reps.clone(), ly.kv.seq_len.clone(), ly.kv.sealed.clone())
                      for ly in L],
        }
        log(f"{mode}: {results[mode]['us_per_layer']:.2f} us per layer-step")
        del graphs, L
        torch.cuda.synchronize()

    a, b = results["one_launch"], results["split_launches"]
    ids_equal = bool(np.array_equal(a["sel"], b["sel"]) and np.array_equal(a["cnt"], b["cnt"]))
    diff = np.abs(a["out"].astype(np.float64) - b["out"])
    out_close = bool((diff <= 1e-5 + 1e-5 * np.abs(b["out"])).all())
    state_equal = all(all(bool(torch.equal(x, y)) for x, y in zip(sa_, sb_)) for sa_, sb_ in zip(a["state"], b["state"]))
    line = {
        "metric": "shared-selection decode step µs/layer (one launch vs split launches)",
        "value": round(a["us_per_layer"], 3),
        "unit": "us/layer",
        "higher_is_better": False,
        "split_launches_us_per_layer": round(b["us_per_layer"], 3),
        "speedup": round(b["us_per_layer"] / a["us_per_layer"], 3),
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "dtype": "fp16 KV, fp32 math",
        "data": f"synthetic ({bench.GENERATOR}: pool, query and new K/V; 4 planted blocks per KV head)",
        "config": {"workload": "shared selection, one sequence", "heads": f"{hq}/{hkv}/{D}", "layers": layers,
                   "batch": batch, "context": ctx, "budget": f"{init} + {local} + {budget - init - local}",
                   "select_groups": 1, "timing": "HIP graph per decode step"},
        "parity": {"ids_equal": ids_equal, "out_within_fp32_rounding": out_close, "out_max_diff": float(diff.max()),
                   "state_equal": state_equal},
    }
    print(json.dumps(line), flush=True)
    if not (ids_equal and out_close and state_equal):
        raise SystemExit("the one-launch and split-launch paths disagree")
