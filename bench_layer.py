"""Attention-layer decode step with its query producer and output consumer
(bench.py --workload layer).

Qwen3-0.6B attention shape (hidden 1024, 16 query / 8 KV heads, head_dim
128), batch 64 sequences of 16384 tokens, budget 64 blocks (4 + 8 + 52),
fp32 weights.  One layer step = two calls, four launches: the decode step
fed by its q/k/v producer (sa_hip_decode_step_qkv: the K-slice partial
projections with the RMSNorm of the hidden rows folded in, then the
one-launch decode step whose workgroups first add their heads' slices and
apply head RMS norm and RoPE at the sequence's position, then append k/v,
seal, score + select and attend) -> the o-projection (partials, then their
sum with the residual add).  With --separate-producer the producer is its own
call (partials, then a reduce launch) before the decode step: three calls,
five launches, the same bits.  Every layer's output is the next layer's
input; inputs and weights are resident in HBM.

Reported: µs per layer (HIP graph of one step over all layers), the
components (event-bracketed eager launches), the projections' achieved HBM
GB/s (fp32 weights read once per step plus their partial sums), a parity
spot check of the last layer against the oracle, and the oracle's
single-thread time for the producer and consumer of one layer.
"""
from __future__ import annotations

import json
import sys
import time

D = 128


def log(msg):
    print(f"[layer] {msg}", file=sys.stderr, flush=True)


def run(args):
    import numpy as np
    import torch

    import bench
    import solidattention_amd as sa

    layers = args.layers or 8
    cfg = list(bench.CONFIGS["qwen3-0.6b-b64-16k"])
    cfg[0] = layers
    _, batch, hq, hkv, ctx, budget, init, local, planted, _ = cfg
    hidden = 1024
    torch.cuda.set_device(0)
    total_steps = args.warmup + 2 * args.steps + 2
    t0 = time.time()
    L = [bench.Layer(sa, torch, cfg, l, args, total_steps) for l in range(layers)]
    W = []
    for l in range(layers):
        seed = args.seed + 104729 * (l + 1)

        def rnd(shape, scale, off):
            t = torch.empty(shape, dtype=torch.float32, device="cuda")
            sa.fill_synthetic_f32(t.view(-1), seed + off, 0)
            return t * scale

        W.append(dict(inorm=1 + 0.1 * rnd((hidden,), 1.0, 1), wq=rnd((hq * D, hidden), hidden ** -0.5, 2),
                      wk=rnd((hkv * D, hidden), hidden ** -0.5, 3), wv=rnd((hkv * D, hidden), hidden ** -0.5, 4),
                      qn=1 + 0.1 * rnd((D,), 1.0, 5), kn=1 + 0.1 * rnd((D,), 1.0, 6),
                      wo=rnd((hidden, hq * D), (hq * D) ** -0.5, 7)))
    h0 = torch.empty((batch, hidden), dtype=torch.float32, device="cuda")
    sa.fill_synthetic_f32(h0.view(-1), args.seed + 11, 0)
    torch.cuda.synchronize()
    log(f"setup {layers} layers in {time.time() - t0:.1f}s")

    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    q = torch.empty((batch, hq, D), dtype=torch.float32, device="cuda")
    k = torch.empty((batch, hkv, D), dtype=torch.float32, device="cuda")
    v = torch.empty_like(k)
    hs = [torch.empty((batch, hidden), dtype=torch.float32, device="cuda") for _ in range(layers + 1)]
    stream = torch.cuda.current_stream()
    # micro-batches: the batch's sequences in `mb` equal parts, each its own
    # chain of layers on its own stream (the parts share no state, so one
    # part's latency-bound projections run beside another's decode step)
    mb = max(1, int(getattr(args, "microbatches", 1) or 1))
    if batch % mb:
        raise SystemExit(f"--microbatches {mb} does not divide the batch of {batch}")
    part = batch // mb
    fused_producer = not getattr(args, "separate_producer", False)
    parts = []
    for i in range(mb):
        a, b = i * part, (i + 1) * part
        kvs = [ly.kv.sequences(a, b) for ly in L]
        parts.append(dict(
            rows=slice(a, b), kvs=kvs, stream=None if i == 0 else torch.cuda.Stream(),
            ws=sa.decode_step_workspace(kvs[0], 1)[0],
            # the projections' K-slice partial tiles
            qkv_ws=torch.empty(sa.lib().sa_hip_qkv_workspace_bytes(part, hidden, hq, hkv) // 4,
                               dtype=torch.float32, device="cuda"),
            lin_ws=torch.empty(sa.lib().sa_hip_linear_workspace_bytes(part, hq * D, hidden) // 4,
                               dtype=torch.float32, device="cuda")))

    def layer_step(l, pt, ev=None):
        # part 0 runs on the current stream (the capture stream under graph
        # capture); the others on their own streams, forked from it
        ly, w, r = L[l], W[l], pt["rows"]
        st = pt["stream"] or torch.cuda.current_stream()
        kv = pt["kvs"][l]
        if ev: ev[0].record(st)
        # RMSNorm + q/k/v + head RMS + RoPE; the new token's position is the
        # sequence's length before the append
        if fused_producer:
            # the producer's partials, then the decode step running its
            # epilogue (two launches)
            sa.decode_step_qkv(kv, hs[l][r], w["wq"], w["wk"], w["wv"], w["qn"], w["kn"], kv.seq_len, q[r], k[r],
                               v[r], pt["qkv_ws"], 0, hkv, budget, init, local, scale, pt["ws"],
                               input_norm=w["inorm"], input_eps=1e-6, selected=ly.selected[r], counts=ly.counts[r],
                               out=ly.out[r], splits=1, status=status, stream=st)
            if ev: ev[1].record(st)
        else:
            sa.qkv_project(hs[l][r], w["wq"], w["wk"], w["wv"], w["qn"], w["kn"], kv.seq_len, hq, hkv, q=q[r],
                           k=k[r], v=v[r], workspace=pt["qkv_ws"], input_norm=w["inorm"], input_eps=1e-6, stream=st)
            if ev: ev[1].record(st)
            sa.decode_step(kv, k[r], v[r], 0, q[r], hkv, budget, init, local, scale, pt["ws"],
                           selected=ly.selected[r], counts=ly.counts[r], out=ly.out[r], splits=1, status=status,
                           stream=st)
        if ev: ev[2].record(st)
        sa.linear(ly.out[r].reshape(part, hq * D), w["wo"], hs[l][r], out=hs[l + 1][r], workspace=pt["lin_ws"],
                  stream=st)
        if ev: ev[3].record(st)

    def step(ev=None):
        cur = torch.cuda.current_stream()
        hs[0].copy_(h0)
        for pt in parts[1:]:
            pt["stream"].wait_stream(cur)
        for l in range(layers):
            for i, pt in enumerate(parts):
                layer_step(l, pt, None if ev is None or i else ev[l])
        for pt in parts[1:]:
            cur.wait_stream(pt["stream"])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(layers)] for _ in range(args.steps)]
    for s in range(args.steps):
        step(evs[s])
    torch.cuda.synchronize()
    comp = np.array([[[e[i].elapsed_time(e[i + 1]) for i in range(3)] for e in evs[s]] for s in range(args.steps)])
    comp_us = comp.reshape(-1, 3).mean(axis=0) * 1000.0

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(args.steps):
        g.replay()
    b.record(stream)
    torch.cuda.synchronize()
    us_per_layer = a.elapsed_time(b) * 1000.0 / (args.steps * layers)
    if int(status.item()) != 0:
        raise SystemExit(f"device status flagged {int(status.item())}")

    # algorithmic bytes: the fp32 weights read once, the activations in and out
    qkv_bytes = (hq + 2 * hkv) * D * hidden * 4 + hidden * 4 + batch * (hidden + (hq + 2 * hkv) * D) * 4
    o_bytes = hidden * hq * D * 4 + batch * (hq * D + 2 * hidden) * 4
    parity = check(sa, np, torch, L[-1], W[-1], hs, q, k, v, layers, batch, hq, hkv, hidden)
    cpu = None if args.no_cpu_baseline else cpu_baseline(np, batch, hq, hkv, hidden)
    line = {
        "metric": "attention-layer decode step µs/layer incl. q/k/v producer and o-proj consumer (Qwen3-0.6B "
                  "shape, B=64, 16K)",
        "value": round(us_per_layer, 3), "unit": "us/layer", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "higher_is_better": False, "dtype": "fp32 weights and math, fp16 KV",
        "data": f"synthetic: seeded weights and hidden rows, FP16 KV from the {bench.GENERATOR} generator, "
                "planted blocks",
        "config": {"workload": "RMSNorm + q/k/v projections + head RMS + RoPE -> decode step -> o-proj + residual",
                   "producer": "partials launch, epilogue inside the decode step" if fused_producer
                   else "partials launch + reduce launch, then the decode step",
                   "layers": layers, "batch": batch, "hidden": hidden, "query_heads": hq,
                   "kv_heads": hkv, "head_dim": D, "context": ctx, "budget_blocks": budget,
                   "microbatches": mb, "streams": mb},
        "tokens_per_s": round(batch / (us_per_layer * layers * 1e-6), 1),
        "components_us": ({"decode_step_qkv": round(comp_us[0], 3)} if fused_producer else
                          {"qkv_project_rms": round(comp_us[0], 3), "decode_step": round(comp_us[1], 3)}) |
                         {"o_proj": round(comp_us[2], 3),
                          "timing": "events around each call of the first micro-batch in eager steps"},
        "projections": ({} if fused_producer else
                        {"qkv_bytes": qkv_bytes, "qkv_gbps": round(qkv_bytes / (comp_us[0] * 1e-6) / 1e9, 1)}) |
                       {"o_bytes": o_bytes, "o_gbps": round(o_bytes / (comp_us[2] * 1e-6) / 1e9, 1)},
        "parity": parity, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def check(sa, np, torch, ly, w, hs, q, k, v, layers, batch, hq, hkv, hidden):
    """The last layer of the last replay: q/k/v from its input and the o-proj
    output against the oracle (the attention output is the device's, checked
    against the oracle by the decode-step parity)."""
    import oracle as O
    h_in = hs[layers - 1].cpu().numpy()
    exn = O.rms_norm(h_in, w["inorm"].cpu().numpy())
    wq, wk, wv = (w[n].cpu().numpy() for n in ("wq", "wk", "wv"))
    pos = (ly.kv.seq_len.cpu().numpy() - 1).astype(np.int32)  # the position the last step appended at
    eq = O.qk_norm_rope(O.linear(exn, wq).reshape(batch, hq, 128), w["qn"].cpu().numpy(), pos)
    ek = O.qk_norm_rope(O.linear(exn, wk).reshape(batch, hkv, 128), w["kn"].cpu().numpy(), pos)
    ev = O.linear(exn, wv).reshape(batch, hkv, 128)
    out = O.linear(ly.out.view(batch, -1).cpu().numpy(), w["wo"].cpu().numpy(), h_in)

    def rel(a, b):
        return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))

    r = {"q_rel_err": rel(q.cpu().numpy(), eq), "k_rel_err": rel(k.cpu().numpy(), ek),
         "v_rel_err": rel(v.cpu().numpy(), ev), "o_proj_rel_err": rel(hs[layers].cpu().numpy(), out)}
    r["within_bars"] = bool(r["q_rel_err"] < 2e-5 and r["k_rel_err"] < 2e-5 and r["v_rel_err"] < 1e-5
                            and r["o_proj_rel_err"] < 1e-5)
    return r


def cpu_baseline(np, batch, hq, hkv, hidden):
    """The oracle's producer (rms_norm, three projections, head RMS + RoPE)
    and consumer (o-proj + residual) for all 64 rows of one layer, one
    thread, float64 sums."""
    import oracle as O
    rng = np.random.default_rng(3)
    x = rng.standard_normal((batch, hidden)).astype(np.float32)
    g = np.ones(hidden, np.float32)
    wq = rng.standard_normal((hq * D, hidden)).astype(np.float32)
    wk = rng.standard_normal((hkv * D, hidden)).astype(np.float32)
    wo = rng.standard_normal((hidden, hq * D)).astype(np.float32)
    pos = np.arange(batch, dtype=np.int32)
    t = time.perf_counter()
    xn = O.rms_norm(x, g)
    q = O.qk_norm_rope(O.linear(xn, wq).reshape(batch, hq, D), np.ones(D, np.float32), pos)
    k = O.qk_norm_rope(O.linear(xn, wk).reshape(batch, hkv, D), np.ones(D, np.float32), pos)
    O.linear(xn, wk)  # the value projection has the key projection's shape
    O.linear(q.reshape(batch, -1), wo, x)
    el = time.perf_counter() - t
    del k
    return {"value": round(el * 1e6, 1), "unit": "us/layer", "cores": 1, "kind": "port",
            "sample": f"producer + consumer of one layer, {batch} rows (oracle C restatement, float64 sums, "
                      "1 thread)"}
