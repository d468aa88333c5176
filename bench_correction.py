"""Long-context miss-correction workload (bench.py --workload correction).

Runs the self-checking C++ driver tests/cpp/correction_check (built by
__graft_entry__.build()), whose per-layer loop is the reference's P1
history-correction loop (cpp/src/pipeline_main.cpp:752-924) over the C++ API
of include/solidattention/hip_kv.hpp: Qwen3-8B attention shape, batch 8,
131072 tokens (4096 blocks per sequence), budget 128 blocks (4 init + 8 local
+ 116 dynamic), one block set per sequence (the reference's shared
selection), the layer's whole KV in pinned host memory and 130 page slots
per sequence in HBM.  Each KV head has 16 planted blocks (4 runs of 4) that
move one block position per step, so the previous step's selection covers
99 / 128 = 0.7734 of the next one by construction.

Four schedules run on the same recorded steps (each replayed from the same
state, so each sees the same misses): serial (the reference's host barrier
on the fills, then one attention), serial_split (host barrier, then the
split arithmetic: hits, misses, merge), overlapped (hits attended while the
copy stream fills the misses, device-side wait, misses, merge) with one
hipMemcpyAsync per page, and overlapped_gather (the fills as one kernel over
the pinned store's device mapping).  Reported per layer: the host wall time
of the whole loop (host leg included), the host leg alone (compare_prediction,
table and list updates), the selection, the device critical path and the
fill bandwidth.  The driver's checks (exit status 2 on a failure): the same
misses in every schedule, the closed-form planted selection at every step,
overlapped == serial_split bit for bit (the reference's exact bar,
pipeline_main.cpp:1123), serial within 2e-3 of serial_split, and against the
oracle after the last step: selection ids, resident set, slot bytes and
attention (2e-3).
"""
from __future__ import annotations

import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(ROOT, "tests", "cpp", "correction_check")


def log(msg):
    print(f"[correction] {msg}", file=sys.stderr, flush=True)


def run(args, batch=None, context=None, timeout=1100):
    """Run the driver; returns its JSON line (printed on stdout).  Raises
    SystemExit on a failed check or an error, after printing the line."""
    if not os.path.exists(EXE):
        raise SystemExit("tests/cpp/correction_check is not built: run __graft_entry__.build()")
    cmd = [EXE, "--layers", str(args.layers or 2), "--steps", str(args.steps), "--warmup", str(args.warmup),
           "--seed", str(args.seed)]
    if batch:
        cmd += ["--batch", str(batch)]
    if context:
        cmd += ["--context", str(context)]
    log(" ".join(cmd[1:]))
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=sys.stderr, text=True, timeout=timeout)
    lines = [x for x in r.stdout.splitlines() if x.startswith("{")]
    if not lines:
        raise SystemExit(f"correction_check printed no result (exit {r.returncode})")
    line = json.loads(lines[-1])
    print(json.dumps(line), flush=True)
    if r.returncode != 0:
        failed = [k for k, v in line.get("checks", {}).items() if v is False]
        raise SystemExit(f"correction_check exit {r.returncode}; failed checks: {failed}")
    return line
