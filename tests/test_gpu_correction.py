"""GPU: the composed long-context miss-correction workload (Qwen3-8B shape,
batch 8, 131072 tokens = 4096 blocks per sequence, budget 128 blocks, ~75%
history coverage) run end to end through bench_correction at one layer.

Every step appends and seals, selects on the GPU, diffs the selection
against the resident set (compare_prediction, pipeline_main.cpp:686-717),
fills the misses from pinned memory on a copy stream, attends the hits while
the copies run and merges.  bench_correction then checks, for all 8
sequences: the selection equals the oracle's bit for bit, the resident set
equals the selection (the reference's corrected == oracle,
pipeline_main.cpp:704-715), every slot's bytes equal its store block, the
attention is within 2e-3 of the oracle on the resident pages, and the
overlapped (pipelined) schedule equals the serial one within 2e-3 on the same
state (the reference's serial-vs-pipelined acceptance,
pipeline_main.cpp:1090-1123; the merge order differs, so not bit for bit)."""
from types import SimpleNamespace

import pytest

pytestmark = pytest.mark.gpu


def test_correction_workload_one_layer(hip):
    import bench_correction
    print("case: correction workload, layers=1 steps=2 warmup=1 accept_steps=3", flush=True)
    line = bench_correction.run(SimpleNamespace(layers=1, steps=2, warmup=1, seed=20261202, accept_steps=3))
    c = line["checks"]
    assert c["sequences"] == 8
    assert c["selection_equals_oracle"] and c["resident_set_equals_selection"] and c["slot_bytes_equal_store"]
    assert c["attention_within_2e-3"], c["attention_max_abs_err"]
    assert c["serial_equals_pipelined_within_2e-3"], c["serial_pipelined_max_abs_err"]
    assert c["accept_layer_steps"] == 3
    # the drifting queries keep the history prediction near its 75% design point
    assert 0.55 <= line["history_coverage"] <= 0.95, line["history_coverage"]
    for sched in line["schedules"].values():
        assert sched["misses_per_layer"] > 0
