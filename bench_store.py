"""Store-tier workload (bench.py --workload store).

Two measurements of the host store tier around the HBM pool, Qwen3-0.6B
shape (16 query / 8 KV heads, head_dim 128, 128 KiB pages), batch 64,
16384-token contexts:

1. Seal writeback behind decoding: `layers` layers decode `steps` tokens with
   the one-launch decode step; whenever a page seals (every sequence, every
   32 tokens) the sealed pages are copied to pinned staging on a copy stream
   behind the step (sa_hip_pages_to_host_async) and written to the main store
   file by its I/O threads (sa_store_submit_writes, O_DIRECT) while the next
   steps run.  Reported: µs per layer-step with and without the writeback,
   the pages written and the write rate, and a byte check of every written
   block against the pool.
2. Store -> pool prefetch: batches of `prefetch_blocks` blocks of one layer
   read from the store into pinned staging and copied into pool pages on a
   copy stream (sa_hip_fill_pages_async), the next batch's read overlapping
   the current copies; reported as GB/s of the read, the copy and the whole
   bridge.
The reference's tier runs on io_uring and a local SSD; the figures here are
those of the host's file system (wherever the store file lies), so they
describe the bridge, not a drive.
"""
from __future__ import annotations

import json
import os
import sys
import tempfile
import time

PAGE = 32
D = 128


def log(msg):
    print(f"[store] {msg}", file=sys.stderr, flush=True)


def run(args):
    import numpy as np
    import torch

    import bench
    import solidattention_amd as sa

    layers = args.layers or 4
    steps = max(args.steps, 64)
    cfg = list(bench.CONFIGS["qwen3-0.6b-b64-16k"])
    cfg[0] = layers
    _, batch, hq, hkv, ctx, budget, init, local, planted, _ = cfg
    torch.cuda.set_device(0)
    total_steps = 2 * steps + args.warmup
    t0 = time.time()
    L = [bench.Layer(sa, torch, cfg, l, args, total_steps) for l in range(layers)]
    torch.cuda.synchronize()
    log(f"setup {layers} layers in {time.time() - t0:.1f}s")
    page_bytes = L[0].kv.page_bytes
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws, _ = sa.decode_step_workspace(L[0].kv, 1)
    compute = torch.cuda.current_stream()
    copy = torch.cuda.Stream()

    # segment of (layer, sequence): blocks sealed during the run
    seals_max = total_steps // PAGE + 2
    tmpdir = tempfile.mkdtemp(prefix="sa_store_bench_", dir=os.environ.get("TMPDIR", "/tmp"))
    path = os.path.join(tmpdir, "main-kv-store.bin")
    # layer segment: block b * seals_max + k = the k-th block sequence b sealed in the run
    store = sa.MainStore(path, layers, batch * seals_max, page_bytes, create=True, direct=True, threads=8)
    log(f"store {path}: {store.nbytes / 2**20:.0f} MiB, O_DIRECT {store.direct}")
    # two bursts of seals (every sequence of every layer) fit in the ring;
    # when the drive cannot keep up with the seal rate the ring fills and the
    # decode loop waits for the writes
    ring_pages = 2 * layers * batch
    staging = torch.empty(ring_pages * page_bytes, dtype=torch.uint8).pin_memory()
    tables = [ly.kv.block_table.cpu().numpy() for ly in L]

    def step(s):
        for ly in L:
            sa.decode_step(ly.kv, ly.knew[s], ly.vnew[s], 0, ly.q[s], hkv, budget, init, local, scale, ws,
                           selected=ly.selected, counts=ly.counts, out=ly.out, splits=1, status=status)

    seq_len0 = int(L[0].kv.seq_len[0].item())
    for s in range(args.warmup):
        step(s)
    # first use of the copy stream, its events, the staging kernel and the
    # store threads (queue creation and code loading cost milliseconds once)
    for li in range(layers):
        w_after, w_done = torch.cuda.Event(), torch.cuda.Event()
        w_after.record(compute)
        w_done.record(copy)
        sa.pages_to_host_async(L[li].kv.pool, page_bytes, L[li].kv.num_pages, tables[li][:, 0].astype(np.int32),
                               staging[: batch * page_bytes], copy, after_event=w_after, done_event=w_done)
        w_done.synchronize()
    store.wait(store.submit_writes(0, [b * seals_max + seals_max - 1 for b in range(batch)],
                                   staging[: batch * page_bytes]))
    torch.cuda.synchronize()

    def submit(p):
        """The store writes of a staged group (one block per sequence)."""
        li, blk, dst = p[3], p[4], p[5]
        p[1] = [store.submit_writes(li, [b * seals_max + blk for b in range(batch)], dst)]

    def finish(p):
        p[0].synchronize()
        if not p[1]:
            submit(p)
        for bid in p[1]:
            store.wait(bid)

    def timed(first, n, writeback):
        """n decode steps from step `first`; with writeback, every step that
        seals pages stages them and hands them to the store threads."""
        pending = []  # (done event, batch ids of the store writes not yet submitted)
        written = []
        head = 0
        t = time.perf_counter()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(compute)
        for s in range(first, first + n):
            step(s)
            tokens = seq_len0 + s + 1  # every sequence holds the same length
            if writeback and tokens % PAGE == 0:
                sealed_idx = tokens // PAGE - 1
                after = torch.cuda.Event()
                after.record(compute)
                for li in range(layers):
                    pages = tables[li][:, sealed_idx].astype(np.int32)
                    if head + batch > ring_pages:
                        head = 0
                    # the ring slot is free once its earlier writes are done
                    for p in [p for p in pending if p[2] == head]:
                        finish(p)
                        pending.remove(p)
                    done = torch.cuda.Event()
                    done.record(copy)  # created before its use as a record target
                    dst = staging[head * page_bytes:(head + batch) * page_bytes]
                    sa.pages_to_host_async(L[li].kv.pool, page_bytes, L[li].kv.num_pages, pages, dst, copy,
                                           after_event=after, done_event=done)
                    blk = (tokens - seq_len0 - 1) // PAGE  # seals of the run so far
                    pending.append([done, [], head, li, blk, dst])
                    written.append((li, sealed_idx, blk, head))
                    head += batch
            # hand landed copies to the store threads without blocking the loop
            for p in pending:
                if not p[1] and p[0].query():
                    submit(p)
        e1.record(compute)
        torch.cuda.synchronize()
        gpu_ms = e0.elapsed_time(e1)
        for p in pending:
            finish(p)
        store.sync()
        wall_ms = (time.perf_counter() - t) * 1000.0
        return gpu_ms, wall_ms, written

    first = args.warmup
    base_gpu, base_wall, _ = timed(first, steps, False)
    wb_gpu, wb_wall, written = timed(first + steps, steps, True)
    if int(status.item()) != 0:
        raise SystemExit(f"device status flagged {int(status.item())}")
    pages_written = len(written) * batch
    # check: every written block equals its pool page
    ok = True
    buf = np.zeros(page_bytes, np.uint8)
    for li, sealed_idx, blk, _ in written:
        for b in (0, batch // 2, batch - 1):
            store.read(li, [b * seals_max + blk], buf)
            page = int(tables[li][b, sealed_idx])
            dev = L[li].kv.pool.view(torch.uint8).view(-1, page_bytes)[page].cpu().numpy()
            ok = ok and bool(np.array_equal(buf, dev))

    # ---- store -> pool prefetch bandwidth ----------------------------------
    nblk = args.prefetch_blocks
    batches = 8
    pf_store = sa.MainStore(os.path.join(tmpdir, "prefetch.bin"), batches, nblk, page_bytes, create=True,
                            direct=True, threads=8)
    src = torch.empty(nblk * page_bytes, dtype=torch.uint8).pin_memory()
    rng = np.random.default_rng(7)
    src.numpy()[:] = rng.integers(0, 256, size=src.numel(), dtype=np.uint8)
    for bl in range(batches):
        pf_store.write(bl, range(nblk), src)
    pf_store.sync()
    stage = [torch.empty(nblk * page_bytes, dtype=torch.uint8).pin_memory() for _ in range(2)]
    pool = L[0].kv.pool
    dst_pages = np.arange(nblk, dtype=np.int32)  # overwritten pages of layer 0 (the decode run is over)
    read_ms = 0.0
    ev = [torch.cuda.Event() for _ in range(2)]
    for e in ev:
        e.record(copy)  # created before the library records them
    cp0, cp1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t = time.perf_counter()
    bid = pf_store.submit_reads(0, range(nblk), stage[0])
    cp0.record(copy)
    for bl in range(batches):
        r0 = time.perf_counter()
        pf_store.wait(bid)
        read_ms += (time.perf_counter() - r0) * 1000.0
        cur = stage[bl % 2]
        sa.fill_pages_async(pool, page_bytes, dst_pages, cur.data_ptr(), np.arange(nblk), copy, ev[bl % 2])
        if bl + 1 < batches:
            nxt = (bl + 1) % 2
            ev[nxt].synchronize()  # that buffer's previous copies have landed
            bid = pf_store.submit_reads(bl + 1, range(nblk), stage[nxt])
    cp1.record(copy)
    copy.synchronize()
    bridge_ms = (time.perf_counter() - t) * 1000.0
    moved = batches * nblk * page_bytes
    copy_ms = cp0.elapsed_time(cp1)
    pf_ok = bool(torch.equal(pool.view(torch.uint8).view(-1, page_bytes)[:nblk].reshape(-1).cpu(), src))
    line = {
        "workload": "store tier: seal writeback behind decoding and store -> pool prefetch (Qwen3-0.6B shape, "
                    "B=64, 16K context, 128 KiB pages)",
        "layers": layers, "steps": steps,
        "o_direct": store.direct, "bounced_blocks": store.bounced + pf_store.bounced,
        "writeback": {
            "us_per_layer_step_without": round(base_gpu * 1000.0 / steps / layers, 3),
            "us_per_layer_step_with": round(wb_gpu * 1000.0 / steps / layers, 3),
            "wall_ms_without": round(base_wall, 1), "wall_ms_with": round(wb_wall, 1),
            "pages_written": pages_written, "bytes_written": pages_written * page_bytes,
            "write_gbps_over_wall": round(pages_written * page_bytes / (wb_wall * 1e-3) / 1e9, 3),
            "written_blocks_equal_pool_pages": ok,
        },
        "prefetch": {
            "blocks_per_batch": nblk, "batches": batches, "bytes": moved,
            "bridge_gbps": round(moved / (bridge_ms * 1e-3) / 1e9, 3),
            "read_wait_ms": round(read_ms, 2), "copy_stream_ms": round(copy_ms, 2),
            "pool_pages_equal_store_blocks": pf_ok,
        },
    }
    print(json.dumps(line), flush=True)
    pf_store.close()
    store.close()
    for f in ("main-kv-store.bin", "prefetch.bin"):
        try:
            os.remove(os.path.join(tmpdir, f))
        except OSError:
            pass
    os.rmdir(tmpdir)
