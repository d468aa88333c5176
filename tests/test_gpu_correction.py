"""GPU: the long-context miss-correction workload end to end, through the
self-checking C++ driver tests/cpp/correction_check (the reference's P1
history-correction loop, pipeline_main.cpp:752-924, over hip_kv.hpp).

Planted blocks drift one block position per step, so the previous step's
selection covers 99 / 128 of the next by construction.  Four schedules
(serial, serial_split, overlapped, overlapped_gather) replay the same steps
from the same state.  The driver checks: every schedule sees the same misses;
every step's selection is the closed-form planted set; the overlapped
schedules equal serial_split bit for bit (the reference's exact
serial-vs-pipelined bar, pipeline_main.cpp:1123); the one-pass serial
attention is within 2e-3 of the split; and, after the last step, the
selection equals the oracle's (bit-exact ids), the resident set equals the
selection (the reference's corrected == oracle, pipeline_main.cpp:704-715),
every slot's bytes equal its store block and the attention is within 2e-3 of
the oracle on the resident pages."""
from types import SimpleNamespace

import pytest

pytestmark = pytest.mark.gpu

DESIGNED = 99 / 128


def check_line(line, sequences):
    c = line["checks"]
    assert c["sequences"] == sequences
    for key in ("same_misses_every_schedule", "selection_equals_planted_set",
                "overlapped_equals_serial_split_bitwise", "overlapped_gather_equals_serial_split_bitwise",
                "serial_single_pass_within_2e-3_of_split", "selection_equals_oracle", "resident_set_equals_selection",
                "slot_bytes_equal_store", "attention_within_2e-3_of_oracle"):
        assert c[key] is True, (key, c)
    assert c["device_status"] == "0" or c["device_status"] == 0
    assert abs(line["history_coverage"] - DESIGNED) < 1e-9, line["history_coverage"]
    misses = {s["misses_per_layer"] for s in line["schedules"].values()}
    assert len(misses) == 1, misses


def test_correction_long_context_one_layer(hip):
    """The full shape (batch 8, 131072 tokens) at one layer, 3 timed steps."""
    import bench_correction
    print("case: correction_check layers=1 steps=3 warmup=1 batch=8 context=131072", flush=True)
    line = bench_correction.run(SimpleNamespace(layers=1, steps=3, warmup=1, seed=20261202))
    check_line(line, 8)
    assert line["schedules"]["serial"]["misses_per_layer"] == 8 * 29


def test_correction_two_layers_short_context(hip):
    """Two layers (their steps interleaved, one copy stream and one fill
    event shared by the layers) at 16384 tokens, batch 2."""
    import bench_correction
    print("case: correction_check layers=2 steps=4 warmup=2 batch=2 context=16384", flush=True)
    line = bench_correction.run(SimpleNamespace(layers=2, steps=4, warmup=2, seed=7), batch=2, context=16384)
    check_line(line, 4)
    assert line["schedules"]["overlapped"]["misses_per_layer"] == 2 * 29
