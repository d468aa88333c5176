"""InfLLM prefill-representative workload (bench.py --workload represent).

Qwen3-0.6B attention shape (16 query / 8 KV heads, head_dim 128), one
sequence's 16384-token prompt per layer, local window 32, top-4 keys per
32-token block: the reference's build_local_causal_representatives with the
settings of its C2.1 driver (selection_main.cpp:159-162), scaled from 512 to
16384 tokens.  A step builds the representatives of `layers` layers (one
call each, inputs resident in HBM), writing them into the d-major layout
the selection reads.

Reported: µs per layer and prompt tokens per second; achieved GB/s and
GFLOP/s of the call (algorithmic bytes: queries, keys, the probabilities
written and read back once, the outputs; flops: one multiply and one add per
(query, key, dim) of every window); the reference builder's single-thread
time on a 512-token sample (oracle/_ref, built from the reference's sources;
the oracle's restatement where that is absent; the reference publishes 51.5 ms for 512 tokens on an
i9-14900HX, docs/cpp-versions/C2.1-infllm-selection-uring.md:58); and a
parity check of the last layer against the oracle's builder with the same
exponential (bit-exact) and of a 512-token prefix against the reference's
builder arithmetic.
"""
from __future__ import annotations

import json
import os
import sys
import time

D = 128


def log(msg):
    print(f"[represent] {msg}", file=sys.stderr, flush=True)


def run(args):
    import numpy as np
    import torch

    import solidattention_amd as sa

    HQ, HKV, T, W, K = 16, 8, 16384, 32, 4
    layers = args.layers or 28
    blocks = T // 32
    rep_stride = (blocks + 3) // 4 * 4
    torch.cuda.set_device(0)
    dev = torch.device("cuda")
    t0 = time.time()
    pq, kv, reps = [], [], []
    for layer in range(layers):
        seed = args.seed + 7919 * layer
        q = torch.empty((HQ, T, D), dtype=torch.float32, device=dev)
        sa.fill_synthetic_f32(q.view(-1), seed, 0)
        k = torch.empty((T, 2, HKV, D), dtype=torch.int16, device=dev).view(torch.uint16)
        sa.fill_synthetic_f16(k.view(-1), seed + 1, 0)
        pq.append(q)
        kv.append(k)
        reps.append(torch.zeros((HQ, D, rep_stride), dtype=torch.float32, device=dev))
    nbytes = sa.lib().sa_hip_local_causal_workspace_bytes(T, HQ, W)
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    offs = torch.empty((HQ, blocks, K), dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    log(f"setup {layers} layers in {time.time() - t0:.1f}s")
    stream = torch.cuda.current_stream()
    C = sa.C

    def call(layer):
        sa.check(sa.lib().sa_hip_local_causal_representatives(
            sa._ptr(pq[layer]), sa._ptr(kv[layer]), T, HQ, HKV, D, 32, W, K, None, sa._ptr(offs),
            sa._ptr(reps[layer]), rep_stride, None, sa._ptr(ws), nbytes, sa._stream(stream)),
            "local_causal_representatives")

    for s in range(args.warmup):
        for layer in range(layers):
            call(layer)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for s in range(args.steps):
        for layer in range(layers):
            call(layer)
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    us_per_layer = ms * 1000.0 / (args.steps * layers)

    alg_bytes = HQ * T * D * 4 + T * HKV * D * 2 + 2 * HQ * T * W * 4 + HQ * T * 4 * 2 + HQ * blocks * (D * 4 + K * 4)
    # window sizes are W except for the first W-1 queries of the prompt
    pairs = HQ * (T * W - W * (W - 1) // 2)
    flops = 2 * pairs * D
    parity = check(sa, np, torch, pq[-1], kv[-1], reps[-1], offs, HQ, HKV, T, W, K, blocks, rep_stride)
    cpu = None if args.no_cpu_baseline else cpu_baseline(np, HQ, HKV, W, K)
    line = {
        "metric": "InfLLM prefill representatives µs/layer (Qwen3-0.6B shape, 16K-token prompt, window 32, top 4)",
        "value": round(us_per_layer, 3), "unit": "us/layer", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "higher_is_better": False, "dtype": "fp32 math, fp16 keys",
        "data": "synthetic (seeded N(0,1) queries and FP16 keys)",
        "config": {"workload": "local-causal representatives of one 16K-token prompt per layer", "layers": layers,
                   "query_heads": HQ, "kv_heads": HKV, "head_dim": D, "tokens": T, "local_window": W,
                   "topk": K, "block_tokens": 32},
        "prompt_tokens_per_s": round(T / (us_per_layer * 1e-6), 1),
        "achieved_gbps": round(alg_bytes / (us_per_layer * 1e-6) / 1e9, 1),
        "achieved_gflops": round(flops / (us_per_layer * 1e-6) / 1e9, 1),
        "algorithmic_bytes": alg_bytes, "flops": flops,
        "parity": parity, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def check(sa, np, torch, pq, kv, reps, offs, HQ, HKV, T, W, K, blocks, rep_stride):
    """Last layer vs the oracle's builder with the same exponential, on a
    4096-token prefix (bit-exact reps and offsets), so the check finishes in
    seconds."""
    import oracle as O
    n = 4096
    got_reps = reps[:, :, : n // 32].cpu().numpy()
    got_offs = offs[:, : n // 32].cpu().numpy()
    # the prefix's representatives do not depend on later tokens except through
    # the received mass of the last window: compare the blocks before it
    q = pq[:, :n].cpu().numpy()
    k = kv[:n].view(torch.int16).cpu().numpy().view(np.uint16)
    vals, eoffs, _ = O.local_causal_representatives_restated(q, k, n, HQ, HKV, D, 32, W, K)
    full = n // 32 - (W + 31) // 32  # blocks whose tokens' windows end inside the prefix
    reps_ok = bool(np.array_equal(got_reps[:, :, :full].transpose(0, 2, 1).view(np.uint32),
                                  vals[:, :full].view(np.uint32)))
    offs_ok = bool(np.array_equal(got_offs[:, :full], eoffs[:, :full].astype(np.int32)))
    return {"prefix_tokens": n, "blocks_checked": full, "representatives_bit_exact": reps_ok,
            "offsets_exact": offs_ok}


def cpu_baseline(np, HQ, HKV, W, K):
    """The reference's build_local_causal_representatives (selection.cpp:12-94)
    on the host, one thread, on a 512-token prompt (the reference's C2.1
    size), scaled linearly to 16384 tokens.  kind "reference": the
    reference's own function compiled from its sources (oracle/_ref); kind
    "port": the oracle's C restatement (libm expf) where oracle/_ref is
    absent."""
    import oracle as O
    use_ref = O.ref_available()
    rng = np.random.default_rng(5)
    T = 512
    pq = rng.standard_normal(HQ * T * D).astype(np.float32)
    kv = rng.standard_normal(T * 2 * HKV * D).astype(np.float16).view(np.uint16)
    t0 = time.perf_counter()
    loops = 0
    while True:
        O.local_causal_representatives(pq, kv, T, HQ, HKV, D, 32, W, K, use_ref=use_ref)
        loops += 1
        el = time.perf_counter() - t0
        if el > 10.0 or loops >= 200:
            break
    per_512 = el / loops
    what = ("the reference's builder, oracle/_ref built from its sources" if use_ref
            else "the oracle's C restatement, libm expf")
    return {"value": round(per_512 * 1e6 * (16384 / 512), 1), "unit": "us/layer", "cores": 1,
            "kind": "reference" if use_ref else "port",
            "sample": f"512-token prompt x {loops} repeats ({what}, 1 thread), "
                      f"{per_512 * 1e3:.2f} ms each, scaled linearly to 16384 tokens",
            "nproc": os.cpu_count()}
